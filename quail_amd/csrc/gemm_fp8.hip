// FP8 (OCP e4m3) block-scaled GEMM on gfx950 MFMA:
//   C[m, n] = sum_kb sa[kb, m] * sb[n/128, kb] * sum_{k in kb} A[m, k] * B[n, k]
// with A = activations [M, K] (1x128 per-token scales, column-major storage)
// and B = weights [N, K] (128x128 block scales), fp32 accumulation. Two
// epilogues: bf16 C, or (gate_up projection) y = silu(gate) * up over the two
// halves of B's rows, quantized per 1x128 group to e4m3 + fp32 scales.
//
// One v_mfma_scale_f32_16x16x128_f8f6f4 consumes exactly one 128-deep K block,
// so each MFMA starts from zero and its 16x16 result is promoted into the fp32
// accumulator with the block's combined scale (one FMA per output) - the
// per-block scales never have to be powers of two. The MFMA computes
// C^T = B A^T: its row operand is the weight tile, so a lane's four outputs are
// four consecutive n of one m and the activation scale is one value per lane.
//
// Structure (one workgroup of 8 waves per CU, persistent):
//   - tile = 256 tokens x 256 weight rows (two 128-row blocks). Wave w owns
//     tokens 32w .. 32w+31 and all 256 weight rows, so a token's whole output
//     row segment lives in one wave (what the fused SiLU epilogue needs).
//   - the workgroup walks its tiles as one stream of 128-deep K steps. Weight
//     blocks reach LDS by DMA (buffer_load ... lds) NS-1 = 3 steps ahead into a
//     4-stage ring. Each wave DMAs its own 32 tokens' activation block one step
//     ahead into a 4 KiB LDS region only it touches, and loads the scales
//     straight into VGPRs two steps ahead. Loads cross tile boundaries, so a
//     tile's first blocks arrive during the previous tile. Every load is a DMA
//     of whole 128-byte rows: loading activation fragments straight into
//     VGPRs touches 16 half-used lines per instruction and measured ~25 % of
//     the step.
//   - every wave issues exactly LOADS = 12 vector-memory loads per step, all
//     as inline asm, one between consecutive MFMA pairs, in the order
//     activation DMA (step s+1), weight DMA (s+3), scales (s+2). The wait at
//     the end of step s is vmcnt(8): everything but this step's weight DMA
//     and scales has landed, the activation block of step s+1 included, whose
//     fragments are then read into VGPRs. A wait counts stores too; loads
//     complete in order among themselves, so a count that leaves only the
//     last eight loads in flight also leaves no older load in flight,
//     whatever the stores do. A tile's epilogue issues its stores right after
//     that wait, so they have a whole step to drain before the next one.
//   - one barrier per step: it publishes stage s (every wave's DMA share has
//     landed) and frees stage s-1 for the DMA of step s+3. The first two
//     weight fragments of step s+1 are read at the end of step s.
//   - the epilogue stages its output through the wave's activation region,
//     after that region's fragments for the next step are in VGPRs and before
//     the next step's activation DMA overwrites it.
//   - tiles are ordered so each XCD's L2 works on a contiguous group of them.
#include "common.h"

#include <cstddef>
#include <type_traits>

namespace qh {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

namespace gemm {
constexpr int BM = 256;         // tile tokens
constexpr int BR = 256;         // tile weight rows
constexpr int BK = 128;         // K block: one MFMA, one scale block
constexpr int NS = 4;           // weight stages in LDS
constexpr int PA = 2;           // scale blocks in flight ahead
constexpr int STAGE = BR * BK;  // 32 KiB
constexpr int A_WAVE = 32 * BK; // 4 KiB: a wave's 32 tokens of one K block
constexpr int LOADS = 12;       // vector-memory loads per wave per step
constexpr int XCDS = 8;
enum { kStoreBf16 = 0, kSiluQuant = 1, kQkvRope = 2 };
}  // namespace gemm

// The qkv projection's fused epilogue (kQkvRope): per-head q/k RMSNorm +
// NeoX rotary on the tile's two heads, then q to q_out, k and v to their
// rows (k_out, v_out) or, with row_dst, straight into the arena's K and V^T
// pages (arena row row_dst[m] = page * page_tokens + slot).
struct QkvRope {
  const int64_t* positions;  // [M]
  const uint16_t* cos_sin;   // [max_pos, 128] bf16: cos | sin
  int max_pos;
  const uint16_t* q_w;       // [128] bf16
  const uint16_t* k_w;
  float eps;
  int n_q, n_kv;             // heads; both even (two heads per 256-column tile)
  uint16_t* q_out;           // [M, ld_q]
  long ld_q;
  uint16_t* k_out;           // [M, ld_kv] (row mode)
  uint16_t* v_out;
  long ld_kv;
  uint16_t* k_pool;          // arena mode: [pages, n_kv, page_tokens, 128]
  uint16_t* v_pool;          //             [pages, n_kv, 128, page_tokens]
  const int64_t* row_dst;    // [M] or nullptr (row mode)
  int page_tokens;
};

struct GemmArgs {
  const uint8_t* A;
  long lda;
  const float* sa;
  const uint8_t* B;
  long ldb;
  const float* sb;
  void* C;        // bf16 [M, N] (kStoreBf16) or e4m3 [M, N/2] (kSiluQuant)
  long ldc;       // elements of C's type
  float* scales;  // kSiluQuant: [N/256, M]
  int M, N, K;
  int ue8m0;
  int group_m;    // tile rows per column sweep (see launch_gemm)
  QkvRope rope;   // kQkvRope only
};

// Raw buffer descriptor: byte-addressed, `bytes` long; accesses past the end
// read zero / are dropped.
__device__ __forceinline__ i32x4 buffer_rsrc(const void* base, uint32_t bytes) {
  const uint64_t b = (uint64_t)base;
  return (i32x4){(int)(uint32_t)b, (int)(uint32_t)(b >> 32), (int)bytes, 0x00020000};
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// silu(gate) * up of one GEMM output pair, with both rounded to bf16 first:
// the same arithmetic as silu_mul_quant_kernel on a bf16 gate_up tensor.
__device__ __forceinline__ float silu_mul_bf16(float gate_acc, float up_acc) {
  return silu_mul(round_bf16(gate_acc), round_bf16(up_acc));
}

// HW: the activation and weight scales are UE8M0 (powers of two). The MFMA
// then applies them itself through its E8M0 scale operands and accumulates
// across K blocks in place, with no promotion FMAs: the exponent byte of an
// fp32 power of two 2^e is e + 127, which is the E8M0 encoding of 2^e.
template <int EPI, bool HW>
__global__ __launch_bounds__(512, 1) void fp8_gemm_kernel(GemmArgs p) {
  using namespace gemm;
  // weight stages, then one activation region per wave (160 KiB in all)
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NS * STAGE + 8 * A_WAVE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int g = lane >> 4;
  const int M = p.M;
  const int nk = p.K / BK;
  const long lda = p.lda, ldb = p.ldb;

  // ---- tiles of this workgroup --------------------------------------------
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = p.N / BR;
  const int n_tiles = tiles_m * tiles_n;
  const int per_xcd = n_tiles / XCDS;
  const int G = gridDim.x;
  const int my_tiles = (n_tiles - (int)blockIdx.x + G - 1) / G;

  // linear tile t -> (tile row, tile column): XCD-contiguous chunks, then
  // group_m tile rows per column sweep
  const int group_m = p.group_m;
  auto coords = [&](int t, int& tm, int& tn) __attribute__((always_inline)) {
    if (t < per_xcd * XCDS) t = (t % XCDS) * per_xcd + t / XCDS;
    const int in_group = group_m * tiles_n;
    const int first_m = (t / in_group) * group_m;
    const int gsize = min(tiles_m - first_m, group_m);
    tm = first_m + (t % in_group) % gsize;
    tn = (t % in_group) / gsize;
  };
  // first weight row of 128-row half h of tile column tn
  auto weight_row = [&](int tn, int h) __attribute__((always_inline)) {
    return EPI == kSiluQuant ? h * (p.N / 2) + 128 * tn : 256 * tn + 128 * h;
  };

  // A position in the step stream; advancing past the last step stays there
  // (the loads of those steps are repeats nobody reads).
  struct Cursor {
    int tl, kb, tm, tn;
  };
  auto start = [&](Cursor& c) __attribute__((always_inline)) {
    c.tl = 0;
    c.kb = 0;
    coords((int)blockIdx.x, c.tm, c.tn);
  };
  auto advance = [&](Cursor& c) __attribute__((always_inline)) {
    if (++c.kb == nk) {
      if (c.tl + 1 < my_tiles) {
        c.kb = 0;
        ++c.tl;
        coords((int)blockIdx.x + c.tl * G, c.tm, c.tn);
      } else {
        c.kb = nk - 1;
      }
    }
  };

  // ---- loads ----------------------------------------------------------------
  // Weight DMA: instruction i (0..3) fills LDS block 8*i + wave of the stage,
  // i.e. tile rows 64*i + 8*wave + lane/8 (half i/2); lane l writes physical
  // chunk l%8 of its row, which holds logical chunk (l%8) ^ (row%8).
  const i32x4 rb = buffer_rsrc(p.B, (uint32_t)((long)p.N * ldb));
  const uint32_t offb = (uint32_t)(8 * wave + (lane >> 3)) * (uint32_t)ldb +
                        (uint32_t)((((lane & 7) ^ (lane >> 3)) & 7) * 16);
  auto dma = [&](const Cursor& c, int stage, int i) __attribute__((always_inline)) {
    const uint32_t dst = lds_addr(lds + stage * STAGE + (8 * i + wave) * 1024);
    const uint32_t so = (uint32_t)(weight_row(c.tn, i >> 1) + 64 * (i & 1)) * (uint32_t)ldb +
                        (uint32_t)c.kb * BK;
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "buffer_load_dwordx4 %1, %2, %3 offen lds"
        :
        : "s"(dst), "v"(offb), "s"(rb), "s"(so)
        : "memory", "m0");
  };

  // Activation DMA: instruction i (0..3) fills rows 8i .. 8i+7 of the wave's
  // region, i.e. tokens 32*wave + 8i + lane/8 of the tile, with the weight
  // blocks' chunk swizzle. Tokens past M lie outside the descriptor and read
  // zero. Then the two activation scales of the lane's tokens and the two
  // weight-block scales of the tile, straight into VGPRs.
  uint8_t* const areg = lds + NS * STAGE + wave * A_WAVE;
  const uint32_t offa = (uint32_t)(32 * wave + (lane >> 3)) * (uint32_t)lda +
                        (uint32_t)((((lane & 7) ^ (lane >> 3)) & 7) * 16);
  const uint32_t srow = 4u * (uint32_t)(32 * wave + (lane & 15));
  const i32x4 rsa = buffer_rsrc(p.sa, (uint32_t)nk * (uint32_t)M * 4u);
  const i32x4 rsb = buffer_rsrc(p.sb, (uint32_t)(p.N / 128) * (uint32_t)nk * 4u);
  struct ALoad {
    i32x4 ra;
    uint32_t k0, ks, kw0, kw1;
  };
  auto a_args = [&](const Cursor& c) __attribute__((always_inline)) {
    ALoad L;
    const int m0 = c.tm * BM;
    L.ra = buffer_rsrc(p.A + (long)m0 * lda, (uint32_t)((long)min(M - m0, BM) * lda));
    L.k0 = (uint32_t)c.kb * BK;
    L.ks = ((uint32_t)c.kb * (uint32_t)M + (uint32_t)m0) * 4u;
    L.kw0 = ((uint32_t)(weight_row(c.tn, 0) / 128) * (uint32_t)nk + (uint32_t)c.kb) * 4u;
    L.kw1 = ((uint32_t)(weight_row(c.tn, 1) / 128) * (uint32_t)nk + (uint32_t)c.kb) * 4u;
    return L;
  };
  auto adma = [&](const ALoad& L, int i) __attribute__((always_inline)) {
    const uint32_t dst = lds_addr(areg + i * 1024);
    const uint32_t so = L.k0 + (uint32_t)(8 * i) * (uint32_t)lda;
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "buffer_load_dwordx4 %1, %2, %3 offen lds"
        :
        : "s"(dst), "v"(offa), "s"(L.ra), "s"(so)
        : "memory", "m0");
  };
  auto s_load = [&](const ALoad& L, int op, float* sv, float* wv) __attribute__((always_inline)) {
    switch (op) {
      case 0:
        asm volatile("buffer_load_dword %0, %1, %2, %3 offen"
                     : "=v"(sv[0]) : "v"(srow), "s"(rsa), "s"(L.ks) : "memory");
        break;
      case 1:
        asm volatile("buffer_load_dword %0, %1, %2, %3 offen offset:64"
                     : "=v"(sv[1]) : "v"(srow), "s"(rsa), "s"(L.ks) : "memory");
        break;
      case 2:
        asm volatile("buffer_load_dword %0, off, %1, %2"
                     : "=v"(wv[0]) : "s"(rsb), "s"(L.kw0) : "memory");
        break;
      case 3:
        asm volatile("buffer_load_dword %0, off, %1, %2"
                     : "=v"(wv[1]) : "s"(rsb), "s"(L.kw1) : "memory");
        break;
    }
  };

  // Fragment i of a stage or of a wave's activation region: lane reads row
  // 16*i + lane%16, logical chunks g and g+4; row % 8 == lane % 8, so the
  // swizzle is per lane. A region's fragments 0 and 1 are the wave's two
  // 16-token halves.
  const int frow = (lane & 15) * BK;
  const int c_lo = ((g ^ (lane & 7)) & 7) * 16;
  const int c_hi = (((g + 4) ^ (lane & 7)) & 7) * 16;
  auto frag = [&](const uint8_t* st, int i) __attribute__((always_inline)) {
    const uint8_t* q = st + i * 16 * BK + frow;
    const i32x4 lo = *reinterpret_cast<const i32x4*>(q + c_lo);
    const i32x4 hi = *reinterpret_cast<const i32x4*>(q + c_hi);
    return (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };

  // ---- state ------------------------------------------------------------------
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc[16][2];  // [n-tile][token half]
#pragma unroll
  for (int i = 0; i < 16; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = zero;
  float sav[PA + 1][2], sbv[PA + 1][2];
  // kQkvRope: the positions of the lane's two tokens (rows lane % 16 and
  // lane % 16 + 16 of the wave), loaded at the tile's first step (low words
  // of the int64 positions; rows past M read 0)
  int pos_pf[2] = {0, 0};

  // ---- epilogues --------------------------------------------------------------
  // A lane holds 4 consecutive columns of one token per n-tile, so storing
  // straight from registers writes 16 scattered 32-byte pieces per
  // instruction, which measured ~16k cycles per tile. Instead each wave
  // stages part of its output at a time in its own LDS slice (rows padded
  // so that the writes are bank-conflict free) and stores whole 128-byte row
  // segments, 16 bytes per lane. The slice is the wave's activation region, free
  // between the read of its fragments and the next activation DMA. The output
  // is stored non-temporal: no later step of this kernel reads it, and left
  // in L2 it would evict the activation and weight blocks the concurrent
  // tiles share (1-4 % faster at 65k tokens).
  uint8_t* const slice = areg;
  // One token half j of the tile as bf16 rows, in four passes, one per
  // column quarter qd (n-tiles 4qd .. 4qd+3): every lane writes its 4 x 4
  // columns of row lane % 16 into 16 staged rows of 64 columns (row pitch
  // 144 bytes: each half-wave's 8-byte writes cover all 64 banks once),
  // then each lane reads back 16 bytes and the wave stores 8 whole 128-byte
  // row segments per instruction. seg(k, R, qd) is the 128-byte destination
  // of staged row R (tile row 32 wave + 16 j + R, R = 8 k + lane / 8) and
  // quarter qd.
  auto store_half_bf16 = [&](const Cursor& c, int j, auto seg) __attribute__((always_inline)) {
    constexpr int ROWB = 128 + 16;
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      uint8_t* w = slice + (lane & 15) * ROWB + 8 * g;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int i = 4 * qd + ii;
        // v_cvt_pk_bf16_f32: round-to-nearest-even, as f32_to_bf16
        typedef float f32x2_t __attribute__((ext_vector_type(2)));
        const f32x2_t x0 = {acc[i][j][0], acc[i][j][1]}, x1 = {acc[i][j][2], acc[i][j][3]};
        const bf16x2 p0 = __builtin_convertvector(x0, bf16x2);
        const bf16x2 p1 = __builtin_convertvector(x1, bf16x2);
        *reinterpret_cast<uint2*>(w + 32 * ii) =
            make_uint2(__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1));
      }
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int R = 8 * k + (lane >> 3), chunk = lane & 7;
        const uint4 v = *reinterpret_cast<const uint4*>(slice + R * ROWB + chunk * 16);
        const int m = c.tm * BM + 32 * wave + 16 * j + R;
        if (m < M)
          __builtin_nontemporal_store(__builtin_bit_cast(i32x4, v),
                                      reinterpret_cast<i32x4*>(seg(k, R, qd) + chunk * 16));
      }
    }
  };
  auto zero_acc = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = zero;
  };
  auto store_bf16 = [&](const Cursor& c) __attribute__((always_inline)) {
    uint8_t* C = (uint8_t*)p.C;
    const long ldc_b = p.ldc * 2;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const long row0 = c.tm * BM + 32 * wave + 16 * j;
      store_half_bf16(c, j, [&](int k, int R, int qd) __attribute__((always_inline)) {
        return C + (row0 + R) * ldc_b + (long)c.tn * BR * 2 + qd * 128;
      });
    }
    zero_acc();
  };
  // kQkvRope: the tile holds two heads (n-tiles 0-7 and 8-15); tile columns
  // below n_q / 2 are q heads, then n_kv / 2 of k heads, then v heads. On q
  // and k tiles each token's head is normed and rotated in registers, as
  // qk_norm_rope does (common.h: the shared summation order; a lane holds
  // columns 16 ib + 4 g + r of its token, the NeoX partner d + 64 in n-tile
  // ib + 4 of the same lane), and the bf16 rows go to q_out, k_out or the
  // arena's K page rows. v tiles are stored as rows, or transposed into the
  // arena's V^T pages.
  auto store_qkv_rope = [&](const Cursor& c) __attribute__((always_inline)) {
    // the epilogue's arguments are read here, through a pointer the
    // compiler cannot see through, so they do not occupy scalar registers
    // across the main loop
    typedef const __attribute__((address_space(4))) QkvRope ConstRope;
    const __attribute__((address_space(4))) uint8_t* ka =
        (const __attribute__((address_space(4))) uint8_t*)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(ka));
    ConstRope& R = *reinterpret_cast<ConstRope*>(ka + offsetof(GemmArgs, rope));
    const int qt = R.n_q >> 1, kt = (R.n_q + R.n_kv) >> 1;
    const int tn = c.tn;
    const int base_row = c.tm * BM + 32 * wave;
    const bool arena = R.row_dst != nullptr;
    constexpr int PT = 16;  // arena page tokens (checked at launch)
    if (tn < kt) {
      const bool is_q = tn < qt;
      const uint16_t* wt = is_q ? R.q_w : R.k_w;
      // the cos / sin of the lane's columns 16 ib + 4 g .. +3 in the first
      // head half (ib < 4) of token half j (the positions came with the
      // tile's first step)
      uint2 craw[4], sraw[4];
      auto load_cs = [&](int j) __attribute__((always_inline)) {
        int pos = pos_pf[j];
        pos = pos < 0 ? 0 : (pos >= R.max_pos ? R.max_pos - 1 : pos);
        const uint16_t* cs = R.cos_sin + (long)pos * 128;
#pragma unroll
        for (int ib = 0; ib < 4; ++ib) {
          craw[ib] = *reinterpret_cast<const uint2*>(cs + 16 * ib + 4 * g);
          sraw[ib] = *reinterpret_cast<const uint2*>(cs + 64 + 16 * ib + 4 * g);
        }
      };
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        load_cs(j);
        // the two heads' inverse RMS (n-tiles 0-7 and 8-15), each phase on
        // its own: scheduled across, the phases' loads and temporaries
        // overlap and the registers run out
        float rstd[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          __builtin_amdgcn_sched_barrier(0);
          float qs[8];
#pragma unroll
          for (int ib = 0; ib < 8; ++ib) {
            f32x4& v = acc[8 * hh + ib][j];
            float x0 = v[0], x1 = v[1], x2 = v[2], x3 = v[3];
            round_bf16_pair(x0, x1);
            round_bf16_pair(x2, x3);
            v = (f32x4){x0, x1, x2, x3};
            qs[ib] = sumsq4(x0, x1, x2, x3);
          }
          const float sg = ((qs[0] + qs[1]) + (qs[2] + qs[3])) + ((qs[4] + qs[5]) + (qs[6] + qs[7]));
          // S_g + S_(g^1) (lanes l and l ^ 16), then + the other pair (l ^ 32)
          rstd[hh] = head_rstd(xor32_sum(xor16_sum(sg)), R.eps);
        }
        // norm + rotation per 16-column block pair (ib, ib + 4): the weights
        // and cos / sin of the block unpacked once for both heads
#pragma unroll
        for (int ib = 0; ib < 4; ++ib) {
          __builtin_amdgcn_sched_barrier(0);
          const uint2 wl = *reinterpret_cast<const uint2*>(wt + 16 * ib + 4 * g);
          const uint2 wh = *reinterpret_cast<const uint2*>(wt + 16 * (ib + 4) + 4 * g);
          const uint32_t wlo[2] = {wl.x, wl.y}, whi[2] = {wh.x, wh.y};
          const uint32_t cw[2] = {craw[ib].x, craw[ib].y};
          const uint32_t sw[2] = {sraw[ib].x, sraw[ib].y};
          float wa[4], wb[4], cr[4], sr[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int sh = 16 * (r & 1);
            wa[r] = bf16_to_f32((wlo[r >> 1] >> sh) & 0xffffu);
            wb[r] = bf16_to_f32((whi[r >> 1] >> sh) & 0xffffu);
            cr[r] = bf16_to_f32((cw[r >> 1] >> sh) & 0xffffu);
            sr[r] = bf16_to_f32((sw[r >> 1] >> sh) & 0xffffu);
          }
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            f32x4& lo = acc[8 * hh + ib][j];
            f32x4& hi = acc[8 * hh + ib + 4][j];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float a0 = head_norm(lo[r], rstd[hh], wa[r]);
              const float b0 = head_norm(hi[r], rstd[hh], wb[r]);
              lo[r] = rope_first(a0, b0, cr[r], sr[r]);
              hi[r] = rope_second(b0, a0, cr[r], sr[r]);
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);
        const long row0 = base_row + 16 * j;
        if (is_q) {
          uint8_t* Q = (uint8_t*)R.q_out;
          store_half_bf16(c, j, [&](int k, int Rr, int qd) __attribute__((always_inline)) {
            return Q + (row0 + Rr) * R.ld_q * 2 + (long)tn * BR * 2 + qd * 128;
          });
        } else if (arena) {
          // byte offset in the K pool of the page row of each staged row this
          // lane stores (head 0 of the tile)
          long kofs[2];
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            const int m = base_row + 16 * j + 8 * k + (lane >> 3);
            const long r = m < M ? R.row_dst[m] : 0;
            kofs[k] = (((r >> 4) * R.n_kv + 2 * (tn - qt)) * PT + (r & (PT - 1))) * 256;
          }
          uint8_t* KP = (uint8_t*)R.k_pool;
          store_half_bf16(c, j, [&](int k, int Rr, int qd) __attribute__((always_inline)) {
            return KP + kofs[k] + (qd >> 1) * (PT * 256) + (qd & 1) * 128;
          });
        } else {
          uint8_t* KR = (uint8_t*)R.k_out;
          store_half_bf16(c, j, [&](int k, int Rr, int qd) __attribute__((always_inline)) {
            return KR + (row0 + Rr) * R.ld_kv * 2 + (long)(tn - qt) * BR * 2 + qd * 128;
          });
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i][j] = zero;
        __builtin_amdgcn_sched_barrier(0);
      }
    } else if (!arena) {
      uint8_t* VR = (uint8_t*)R.v_out;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const long row0 = base_row + 16 * j;
        store_half_bf16(c, j, [&](int k, int Rr, int qd) __attribute__((always_inline)) {
          return VR + (row0 + Rr) * R.ld_kv * 2 + (long)(tn - kt) * BR * 2 + qd * 128;
        });
      }
      zero_acc();
    } else {
      // V^T pages: per token half j, head hh and 64-column half dh, the
      // lane's 16 values of token lane % 16 go to LDS rows [token][d] (pitch
      // 136 bytes: 8-byte aligned, and the transposed reads of 16 tokens at
      // one d fall in 16 distinct banks), then lane (dr = lane / 16,
      // e = lane % 16) writes token e at d = 4 dd + dr: consecutive tokens in
      // consecutive slots of a page land in one 32-byte page row per
      // instruction
      constexpr int VP = 136;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int e = lane & 15;
        const int m = base_row + 16 * j + e;
        const long r = m < M ? R.row_dst[m] : 0;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const long h = 2 * (tn - kt) + hh;
          uint16_t* vcol = R.v_pool + ((r >> 4) * R.n_kv + h) * 128 * PT + (r & (PT - 1));
#pragma unroll
          for (int dh = 0; dh < 2; ++dh) {
            __builtin_amdgcn_sched_barrier(0);
            uint8_t* w = slice + e * VP + 8 * g;
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
              const f32x4 v = acc[8 * hh + 4 * dh + ii][j];
              typedef float f32x2_t __attribute__((ext_vector_type(2)));
              const f32x2_t x0 = {v[0], v[1]}, x1 = {v[2], v[3]};
              const bf16x2 p0 = __builtin_convertvector(x0, bf16x2);
              const bf16x2 p1 = __builtin_convertvector(x1, bf16x2);
              *reinterpret_cast<uint2*>(w + 32 * ii) =
                  make_uint2(__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1));
            }
            // the wave's own slice: its writes above precede these reads
            uint16_t* vd = vcol + (long)(64 * dh + (lane >> 4)) * PT;
            const uint8_t* rd = slice + e * VP + 2 * (lane >> 4);
#pragma unroll
            for (int dd = 0; dd < 16; ++dd) {
              if ((dd & 3) == 0) __builtin_amdgcn_sched_barrier(0);
              const uint16_t x = *reinterpret_cast<const uint16_t*>(rd + 8 * dd);
              if (m < M) vd[64 * dd] = x;
            }
          }
        }
      }
      zero_acc();
    }
  };
  // silu(gate) * up for the tile's 128 output columns 128*tn .. (n-tiles 0-7
  // hold gate, 8-15 the matching up), one 1x128 quantization group per token:
  // a token's 128 values sit in the four lanes lane%16 + 16*g'.
  auto store_silu_quant = [&](const Cursor& c) __attribute__((always_inline)) {
    constexpr int ROWB = 128 + 16;  // one 128-column e4m3 row + pad
    uint8_t* out = (uint8_t*)p.C;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int m_row = c.tm * BM + 32 * wave + 16 * j;
      float amax = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int r = 0; r < 4; r += 2) {
          // silu_mul_bf16 on two columns, their gate and up values rounded
          // to bf16 a pair at a time
          float g0 = acc[i][j][r], g1 = acc[i][j][r + 1];
          float u0 = acc[i + 8][j][r], u1 = acc[i + 8][j][r + 1];
          round_bf16_pair(g0, g1);
          round_bf16_pair(u0, u1);
          const float y0 = silu_mul(g0, u0), y1 = silu_mul(g1, u1);
          acc[i][j][r] = y0;
          acc[i][j][r + 1] = y1;
          amax = fmaxf(amax, fabsf(y0));
          amax = fmaxf(amax, fabsf(y1));
        }
      amax = fmaxf(amax, __shfl_xor(amax, 16, kWave));
      amax = fmaxf(amax, __shfl_xor(amax, 32, kWave));
      const float scale = group_scale(amax, p.ue8m0 != 0);
      const double rinv = recip_exact(scale);
      uint8_t* w = slice + (lane & 15) * ROWB + 4 * g;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t b = quant_e4m3_x4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3],
                                         rinv);
        *reinterpret_cast<uint32_t*>(w + 16 * i) = b;
        acc[i][j] = zero;
        acc[i + 8][j] = zero;
      }
      if (g == 0 && m_row + (lane & 15) < M) p.scales[(long)c.tn * M + m_row + (lane & 15)] = scale;
      // the 16 staged rows, eight whole 128-byte rows per instruction
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int R = 8 * q + (lane >> 3), chunk = lane & 7;
        const uint4 v = *reinterpret_cast<const uint4*>(slice + R * ROWB + chunk * 16);
        if (m_row + R < M)
          __builtin_nontemporal_store(
              __builtin_bit_cast(i32x4, v),
              reinterpret_cast<i32x4*>(out + (long)(m_row + R) * p.ldc + 128 * c.tn + chunk * 16));
      }
    }
  };
  auto epilogue = [&](const Cursor& c) __attribute__((always_inline)) {
    if constexpr (EPI == kSiluQuant) store_silu_quant(c);
    else if constexpr (EPI == kQkvRope) store_qkv_rope(c);
    else store_bf16(c);
  };

  // ---- prologue -----------------------------------------------------------------
  // weight stages 0 and 1, the activation block and scales of step 0, then
  // weight stage 2 and the scales of step 1; the wait leaves those last
  // eight loads in flight
  Cursor cd, cn, ca, cc;  // weight DMA (step s+3), activation DMA (s+1), scales (s+2), compute (s)
  start(cd);
  start(cn);
  start(ca);
  start(cc);
#pragma unroll
  for (int s = 0; s < 2; ++s) {
#pragma unroll
    for (int i = 0; i < 4; ++i) dma(cd, s, i);
    advance(cd);
  }
  {
    const ALoad L = a_args(cn);
#pragma unroll
    for (int i = 0; i < 4; ++i) adma(L, i);
    advance(cn);
  }
  {
    const ALoad L = a_args(ca);
#pragma unroll
    for (int op = 0; op < 4; ++op) s_load(L, op, sav[0], sbv[0]);
    advance(ca);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) dma(cd, 2, i);
  advance(cd);
  {
    const ALoad L = a_args(ca);
#pragma unroll
    for (int op = 0; op < 4; ++op) s_load(L, op, sav[1], sbv[1]);
    advance(ca);
  }
  asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  wg_barrier();

  // carried across steps: the activation fragments and the first two weight
  // fragments of the step, and the last two products of the previous step
  // with their scales
  v8i xa0 = frag(areg, 0), xa1 = frag(areg, 1);
  v8i bf = frag(lds, 0), bn = frag(lds, 1);
  f32x4 tp0 = zero, tp1 = zero;  // products two and one MFMAs back
  float s_last0 = 0.f, s_last1 = 0.f;

  auto step = [&](auto slot_c, int s) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_c)::value;
    constexpr int nslot = (slot + PA) % (PA + 1);
    // stage s: every wave's DMA share landed before its wait at the end of
    // step s-1; the barrier publishes it and frees stage s-1
    asm volatile("" : "+v"(sav[slot][0]), "+v"(sav[slot][1]), "+v"(sbv[slot][0]),
                 "+v"(sbv[slot][1]));
    wg_barrier();
    // the activation fragments were read from the region at the end of step
    // s-1 (and an epilogue may have staged through it since): all of that is
    // done before this step's activation DMA overwrites the region
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if constexpr (EPI == kQkvRope) {
      // issued before the step's twelve loads, so the wait at the end of
      // the step (all but the last eight loads) covers them
      if (cc.kb == 0) {
        // rows past M read the last row (their outputs are not stored)
        const int m = cc.tm * BM + 32 * wave + (lane & 15);
        const int64_t* pp = p.rope.positions;
        const int64_t* p0 = pp + min(m, M - 1);
        const int64_t* p1 = pp + min(m + 16, M - 1);
        asm volatile("global_load_dword %0, %2, off\n\t"
                     "global_load_dword %1, %3, off"
                     : "=v"(pos_pf[0]), "=v"(pos_pf[1]) : "v"(p0), "v"(p1) : "memory");
      }
    }
    const ALoad Ln = a_args(cn);
    const ALoad Ls = a_args(ca);
    const int dstage = (s + NS - 1) % NS;
    float sc[2][2];  // [token half][weight half]
    int ea[2], eb[2];  // E8M0 exponents (HW): token half, weight half
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      sc[j][0] = sav[slot][j] * sbv[slot][0];
      sc[j][1] = sav[slot][j] * sbv[slot][1];
      ea[j] = (int)((__builtin_bit_cast(uint32_t, sav[slot][j]) >> 23) & 0xffu);
      eb[j] = (int)((__builtin_bit_cast(uint32_t, sbv[slot][j]) >> 23) & 0xffu);
    }
    const uint8_t* st = lds + (s % NS) * STAGE;
    const uint8_t* st_next = lds + ((s + 1) % NS) * STAGE;
    const v8i xa[2] = {xa0, xa1};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      // fragments two n-tiles ahead; the last two are step s+1's first, from
      // a stage the previous barrier already covered
      const v8i bnn = i < 14 ? frag(st, i + 2) : frag(st_next, i - 14);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if constexpr (HW) {
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              bf, xa[j], acc[i][j], 0, 0, 0, eb[i >> 3], 0, ea[j]);
        } else {
          const f32x4 t = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              bf, xa[j], zero, 0, 0, 0, 127, 0, 127);
          // promote the product two MFMAs back: its MFMA finished while the
          // one in between ran, so the FMAs co-issue with the MFMA pipe
          // instead of waiting on it (one MFMA back, they wait)
          const int q = 2 * i + j - 2;
          if (q >= 0) {
  #pragma unroll
            for (int r = 0; r < 4; ++r) acc[q >> 1][q & 1][r] += tp0[r] * sc[q & 1][(q >> 1) >> 3];
          } else {
            const float sl = q == -2 ? s_last0 : s_last1;
  #pragma unroll
            for (int r = 0; r < 4; ++r) acc[15][q + 2][r] += tp0[r] * sl;
          }
          tp0 = tp1;
          tp1 = t;
        }
      }
      // the step's twelve loads, one per n-tile: activation DMA for step
      // s+1, weight DMA for step s+3, then scales for step s+2
      if (i < 4) adma(Ln, i);
      else if (i < 8) dma(cd, dstage, i - 4);
      else if (i < 12) s_load(Ls, i - 8, sav[nslot], sbv[nslot]);
      bf = bn;
      bn = bnn;
      // issue order: MFMA, the two fragment reads, the FMAs of the product
      // two back, MFMA, FMAs. Left alone, the scheduler puts both MFMAs
      // last and their products' FMAs first in the next group, where they
      // wait for the MFMAs instead of running beside them.
      if constexpr (HW) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      } else {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    s_last0 = sc[0][1];
    s_last1 = sc[1][1];
    // everything but this step's weight DMA and scales has landed: the
    // activation block of step s+1, and weight stage s+2 of this wave
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    xa0 = frag(areg, 0);
    xa1 = frag(areg, 1);
    if (cc.kb == nk - 1) {
      if constexpr (!HW) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          acc[15][0][r] += tp0[r] * s_last0;
          acc[15][1][r] += tp1[r] * s_last1;
        }
        tp0 = tp1 = zero;
        s_last0 = s_last1 = 0.f;
      }
      // the region is free once the fragments are in VGPRs
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      epilogue(cc);
    }
    advance(cc);
    advance(cn);
    advance(ca);
    advance(cd);
  };

  const int S = my_tiles * nk;
  static_assert(PA == 2, "the step loop is unrolled for three scale slots");
  for (int s = 0; s < S; s += 3) {
    step(std::integral_constant<int, 0>{}, s);
    if (s + 1 < S) step(std::integral_constant<int, 1>{}, s + 1);
    if (s + 2 < S) step(std::integral_constant<int, 2>{}, s + 2);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no DMA outlives the workgroup
}


// Tile order. Each XCD's 32 CUs run 32 consecutive tiles of its chunk at a
// time, group_m tile rows x 32/group_m tile columns. A wave of tiles re-reads
// its weight blocks from beyond L2 once per group of tile rows and its
// activation blocks once per wave of tile columns. group_m = 4 (4 x 8 tiles)
// was the measured best or within 2 % of it among 1/2/4/8/16 for every
// Qwen3-4B projection at 102,400 tokens, the fused gate_up included.
template <int EPI, bool HW = false>
static int launch_gemm(GemmArgs a, qh_stream_t stream, const char* what) {
  const int tiles_n = a.N / gemm::BR;
  const int tiles = ((a.M + gemm::BM - 1) / gemm::BM) * tiles_n;
  const int grid = min(tiles, device_cus());
  a.group_m = 4;
  hipLaunchKernelGGL((fp8_gemm_kernel<EPI, HW>), dim3(grid), dim3(512), 0, (hipStream_t)stream,
                     a);
  return launch_status(what);
}

// Byte ranges the kernel addresses through 32-bit buffer offsets.
static bool offsets_fit(int M, int N, int K, long lda, long ldb) {
  const long lim = 0x7fffffffL;
  return (long)N * ldb < lim && 256L * lda < lim && (long)(K / 128) * M * 4 < lim;
}

}  // namespace qh

using namespace qh;

static int gemm_nt(const void* A, long lda, const float* sa, const void* B, long ldb,
                   const float* sb, void* C, long ldc, int M, int N, int K, bool hw,
                   qh_stream_t stream, const char* what) {
  QH_REQUIRE(M >= 0 && N > 0 && K > 0, "%s: M=%d N=%d K=%d", what, M, N, K);
  QH_REQUIRE(N % gemm::BR == 0, "%s: N=%d must be a multiple of 256", what, N);
  QH_REQUIRE(K % gemm::BK == 0, "%s: K=%d must be a multiple of 128", what, K);
  QH_REQUIRE(lda >= K && ldb >= K && ldc >= N, "%s: leading dimensions", what);
  QH_REQUIRE(lda % 16 == 0 && ldb % 16 == 0 && ldc % 4 == 0,
             "%s: lda/ldb must be multiples of 16 bytes, ldc of 4 elements", what);
  QH_REQUIRE(offsets_fit(M, N, K, lda, ldb), "%s: operands exceed 2 GiB offsets", what);
  if (M == 0) return QH_OK;
  QH_REQUIRE(A && sa && B && sb && C, "%s: null pointer", what);
  GemmArgs a{(const uint8_t*)A, lda, sa, (const uint8_t*)B, ldb, sb, C, ldc, nullptr,
             M, N, K, 0, 0, {}};
  return hw ? launch_gemm<gemm::kStoreBf16, true>(a, stream, what)
            : launch_gemm<gemm::kStoreBf16, false>(a, stream, what);
}

static int gemm_silu_quant(const void* A, long lda, const float* sa, const void* B, long ldb,
                           const float* sb, int M, int I, int K, void* out_q, long ld_out,
                           float* scales, int ue8m0, bool hw, qh_stream_t stream,
                           const char* what) {
  QH_REQUIRE(M >= 0 && I > 0 && K > 0, "%s: M=%d I=%d K=%d", what, M, I, K);
  QH_REQUIRE(I % 128 == 0, "%s: I=%d must be a multiple of 128", what, I);
  QH_REQUIRE(K % gemm::BK == 0, "%s: K=%d must be a multiple of 128", what, K);
  QH_REQUIRE(lda >= K && ldb >= K && ld_out >= I, "%s: leading dimensions", what);
  QH_REQUIRE(lda % 16 == 0 && ldb % 16 == 0 && ld_out % 4 == 0,
             "%s: lda/ldb must be multiples of 16 bytes, ld_out of 4", what);
  QH_REQUIRE(offsets_fit(M, 2 * I, K, lda, ldb), "%s: operands exceed 2 GiB offsets", what);
  if (M == 0) return QH_OK;
  QH_REQUIRE(A && sa && B && sb && out_q && scales, "%s: null pointer", what);
  GemmArgs a{(const uint8_t*)A, lda, sa, (const uint8_t*)B, ldb, sb, out_q, ld_out, scales,
             M, 2 * I, K, ue8m0, 0, {}};
  return hw ? launch_gemm<gemm::kSiluQuant, true>(a, stream, what)
            : launch_gemm<gemm::kSiluQuant, false>(a, stream, what);
}

static int gemm_qkv_rope(const void* A, long lda, const float* sa, const void* B, long ldb,
                         const float* sb, int M, int K, int n_q, int n_kv,
                         const int64_t* positions, const void* cos_sin, int max_pos,
                         const void* q_w, const void* k_w, float eps, void* q_out, long ld_q,
                         void* k_out, void* v_out, long ld_kv, void* k_pool, void* v_pool,
                         const int64_t* row_dst, int page_tokens, bool arena, bool hw,
                         qh_stream_t stream, const char* what) {
  QH_REQUIRE(M >= 0 && K > 0 && n_q > 0 && n_kv > 0, "%s: M=%d K=%d n_q=%d n_kv=%d", what, M,
             K, n_q, n_kv);
  QH_REQUIRE(n_q % 2 == 0 && n_kv % 2 == 0 && n_q % n_kv == 0,
             "%s: n_q=%d and n_kv=%d must be even (two 128-wide heads per tile)", what, n_q, n_kv);
  QH_REQUIRE(K % gemm::BK == 0, "%s: K=%d must be a multiple of 128", what, K);
  QH_REQUIRE(max_pos > 0, "%s: max_pos=%d", what, max_pos);
  const int N = (n_q + 2 * n_kv) * 128;
  QH_REQUIRE(lda >= K && ldb >= K && lda % 16 == 0 && ldb % 16 == 0,
             "%s: lda/ldb must be >= K and multiples of 16 bytes", what);
  QH_REQUIRE(ld_q >= n_q * 128 && ld_q % 8 == 0, "%s: ld_q=%ld", what, ld_q);
  QH_REQUIRE(offsets_fit(M, N, K, lda, ldb), "%s: operands exceed 2 GiB offsets", what);
  if (arena) {
    QH_REQUIRE(page_tokens == 16, "%s: page_tokens=%d (the arena's pages hold 16 tokens)", what,
               page_tokens);
  } else {
    QH_REQUIRE(ld_kv >= n_kv * 128 && ld_kv % 8 == 0, "%s: ld_kv=%ld", what, ld_kv);
  }
  if (M == 0) return QH_OK;
  QH_REQUIRE(A && sa && B && sb && positions && cos_sin && q_w && k_w && q_out,
             "%s: null pointer", what);
  QH_REQUIRE(arena ? (k_pool && v_pool) : (k_out && v_out), "%s: null k/v destination", what);
  GemmArgs a{(const uint8_t*)A, lda, sa, (const uint8_t*)B, ldb, sb, nullptr, 0, nullptr,
             M, N, K, 0, 0, {}};
  a.rope = QkvRope{positions, (const uint16_t*)cos_sin, max_pos, (const uint16_t*)q_w,
                   (const uint16_t*)k_w, eps, n_q, n_kv, (uint16_t*)q_out, ld_q,
                   (uint16_t*)k_out, (uint16_t*)v_out, ld_kv, (uint16_t*)k_pool,
                   (uint16_t*)v_pool, row_dst, page_tokens};
  return hw ? launch_gemm<gemm::kQkvRope, true>(a, stream, what)
            : launch_gemm<gemm::kQkvRope, false>(a, stream, what);
}

extern "C" int qh_fp8_gemm_qkv_rope(const void* A, long lda, const float* sa, const void* B,
                                    long ldb, const float* sb, int M, int K, int n_q,
                                    int n_kv, const int64_t* positions, const void* cos_sin,
                                    int max_pos, const void* q_w, const void* k_w, float eps,
                                    void* q_out, long ld_q, void* k_out, void* v_out,
                                    long ld_kv, int ue8m0_scales, qh_stream_t stream) {
  return gemm_qkv_rope(A, lda, sa, B, ldb, sb, M, K, n_q, n_kv, positions, cos_sin, max_pos,
                       q_w, k_w, eps, q_out, ld_q, k_out, v_out, ld_kv, nullptr, nullptr,
                       nullptr, 16, false, ue8m0_scales != 0, stream, "fp8_gemm_qkv_rope");
}

extern "C" int qh_fp8_gemm_qkv_rope_kv(const void* A, long lda, const float* sa,
                                       const void* B, long ldb, const float* sb, int M, int K,
                                       int n_q, int n_kv, const int64_t* positions,
                                       const void* cos_sin, int max_pos, const void* q_w,
                                       const void* k_w, float eps, void* q_out, long ld_q,
                                       void* k_pool, void* v_pool, const int64_t* row_dst,
                                       int page_tokens, int ue8m0_scales,
                                       qh_stream_t stream) {
  QH_REQUIRE(row_dst != nullptr || M == 0, "fp8_gemm_qkv_rope_kv: row_dst is null");
  return gemm_qkv_rope(A, lda, sa, B, ldb, sb, M, K, n_q, n_kv, positions, cos_sin, max_pos,
                       q_w, k_w, eps, q_out, ld_q, nullptr, nullptr, 0, k_pool, v_pool, row_dst,
                       page_tokens, true, ue8m0_scales != 0, stream, "fp8_gemm_qkv_rope_kv");
}

extern "C" int qh_fp8_gemm_nt(const void* A, long lda, const float* sa, const void* B,
                              long ldb, const float* sb, void* C, long ldc, int M, int N,
                              int K, qh_stream_t stream) {
  return gemm_nt(A, lda, sa, B, ldb, sb, C, ldc, M, N, K, false, stream, "fp8_gemm_nt");
}

extern "C" int qh_fp8_gemm_nt_ue8m0(const void* A, long lda, const float* sa, const void* B,
                                    long ldb, const float* sb, void* C, long ldc, int M,
                                    int N, int K, qh_stream_t stream) {
  return gemm_nt(A, lda, sa, B, ldb, sb, C, ldc, M, N, K, true, stream, "fp8_gemm_nt_ue8m0");
}

extern "C" int qh_fp8_gemm_silu_quant(const void* A, long lda, const float* sa,
                                      const void* B, long ldb, const float* sb, int M,
                                      int I, int K, void* out_q, long ld_out,
                                      float* scales, int ue8m0, qh_stream_t stream) {
  return gemm_silu_quant(A, lda, sa, B, ldb, sb, M, I, K, out_q, ld_out, scales, ue8m0, false,
                         stream, "fp8_gemm_silu_quant");
}

extern "C" int qh_fp8_gemm_silu_quant_ue8m0(const void* A, long lda, const float* sa,
                                            const void* B, long ldb, const float* sb, int M,
                                            int I, int K, void* out_q, long ld_out,
                                            float* scales, qh_stream_t stream) {
  return gemm_silu_quant(A, lda, sa, B, ldb, sb, M, I, K, out_q, ld_out, scales, 1, true,
                         stream, "fp8_gemm_silu_quant_ue8m0");
}
