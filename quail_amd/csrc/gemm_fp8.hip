// FP8 (OCP e4m3) block-scaled GEMM on gfx950 MFMA:
//   C[m, n] = sum_kb sa[kb, m] * sb[n/128, kb] * sum_{k in kb} A[m, k] * B[n, k]
// with A = activations [M, K] (1x128 per-token scales, column-major storage)
// and B = weights [N, K] (128x128 block scales), fp32 accumulation, bf16 out.
//
// One v_mfma_scale_f32_16x16x128_f8f6f4 consumes exactly one 128-deep K block,
// so each MFMA starts from zero and its 16x16 result is promoted into the fp32
// accumulator with the block's combined scale (one FMA per output) - the
// per-block scales never have to be powers of two. The MFMA computes
// C^T = B A^T: its row operand is the weight tile, so a lane's four outputs are
// four consecutive n of one m (8-byte bf16 stores) and the activation scale is
// one value per lane.
//
// Workgroup tile 256 x 256 x 128 with 8 waves (4 along M x 2 along N, 64 x 128
// per wave). Operand tiles move global -> LDS by DMA (no staging registers)
// into two LDS stages of 2 x 32 KiB; the next K block's DMA and scales are in
// flight while the current block computes; one barrier per K block. Tiles are
// mapped so that each XCD's L2 sees a contiguous group of them.
#include "common.h"

namespace qh {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

namespace gemm {
constexpr int BM = 256, BN = 256, BK = 128;
constexpr int ROW = BK;                  // LDS row: 128 fp8 bytes, no padding
constexpr int TILE_BYTES = 256 * ROW;    // one operand, one stage: 32 KiB
constexpr int GROUP_M = 8;
constexpr int XCDS = 8;
}  // namespace gemm


// LDS rows hold their eight 16-byte chunks XOR-swizzled by row % 8. A
// fragment read (16 consecutive rows; lane group g = lane/16 reads logical
// chunks g and g+4) is then free of bank conflicts on gfx950's 64-bank LDS,
// as measured with a ds_read_b128 probe over candidate patterns (a
// (row / 2) % 8 swizzle runs at half rate).
__device__ __forceinline__ int swz(int row, int chunk) {
  return chunk ^ (row & 7);
}

typedef int i32x4 __attribute__((ext_vector_type(4)));

// Raw buffer descriptor over a tile's rows (byte-addressed, stride 0; the
// range check is left open because the caller clamps row indices).
__device__ __forceinline__ i32x4 tile_rsrc(const uint8_t* base) {
  const uint64_t b = (uint64_t)base;
  return (i32x4){(int)(uint32_t)b, (int)(uint32_t)(b >> 32), 0x7fffffff, 0x00020000};
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Per-lane byte offsets of the four DMA rows a lane fetches in one K block of
// a 256-row operand tile. Wave instruction i fills the contiguous 1 KiB LDS
// block blk = 8*i + wave (8 rows); lane l writes its 16 bytes at 16*l of it,
// i.e. row 8*blk + l/8, physical chunk l%8, which holds logical chunk
// swz(row, l%8) of that row.
__device__ __forceinline__ void tile_offsets(long ld, int row0, int row_max, int wave,
                                             int lane, uint32_t off[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (8 * i + wave) * 8 + (lane >> 3);
    const int grow = min(row0 + r, row_max);
    off[i] = (uint32_t)(grow - row0) * (uint32_t)ld + (uint32_t)(swz(r, lane & 7) * 16);
  }
}

// One K block (bytes k0 .. k0+127 of each row) global -> LDS with
// buffer_load_dwordx4 ... lds (M0 = LDS block base). Issued as inline asm so
// the compiler does not treat the LDS reads of the other stage as dependent
// on it; the consumer waits with s_waitcnt vmcnt(0) + a barrier.
__device__ __forceinline__ void load_tile_lds(i32x4 rsrc, const uint32_t off[4], uint32_t k0,
                                              const uint8_t* tile, int wave) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t dst = lds_addr(tile + (8 * i + wave) * 1024);
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "buffer_load_dwordx4 %1, %2, %3 offen lds"
        :
        : "s"(dst), "v"(off[i]), "s"(rsrc), "s"(k0)
        : "memory", "m0");
  }
}

__global__ __launch_bounds__(512, 1) void fp8_gemm_nt_kernel(
    const uint8_t* __restrict__ A, long lda, const float* __restrict__ sa,
    const uint8_t* __restrict__ B, long ldb, const float* __restrict__ sb,
    uint16_t* __restrict__ C, long ldc, int M, int N, int K) {
  using namespace gemm;
  // [stage][A | B][256 rows x 128 B]
  __shared__ __attribute__((aligned(1024))) uint8_t lds[4 * TILE_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int wm = wave & 3, wn = wave >> 2;

  // ---- tile mapping: XCD-contiguous, then grouped along M -----------------
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = N / BN;
  const int n_tiles = tiles_m * tiles_n;
  int pid = blockIdx.x;
  {
    const int per_xcd = n_tiles / XCDS;
    if (pid < per_xcd * XCDS) pid = (pid % XCDS) * per_xcd + pid / XCDS;
  }
  const int in_group = GROUP_M * tiles_n;
  const int group = pid / in_group;
  const int first_m = group * GROUP_M;
  const int gsize = min(tiles_m - first_m, GROUP_M);
  const int tm = first_m + (pid % in_group) % gsize;
  const int tn = (pid % in_group) / gsize;
  const int m0 = tm * BM, n0 = tn * BN;
  const int nk = K / BK;

  f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // activation-scale offsets (bytes) of the rows this lane's outputs belong
  // to, one per m-tile; rows past M read row M-1 (their outputs are dropped)
  uint32_t srow[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) srow[j] = 4u * min(m0 + 64 * wm + 16 * j + (lane & 15), M - 1);
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      (void*)sa, 0, 0x7fffffff, 0x00020000);
  const int nblk = (n0 + 128 * wn) / 128;
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  const int g = lane >> 4;
  const i32x4 ra = tile_rsrc(A + (long)m0 * lda);
  const i32x4 rb = tile_rsrc(B + (long)n0 * ldb);
  uint32_t offa[4], offb[4];
  tile_offsets(lda, m0, M - 1, wave, lane, offa);
  tile_offsets(ldb, n0, N - 1, wave, lane, offb);


  // Scales: s_cur holds this K block's combined per-lane scales; the next
  // block's raw activation scales and weight scale are loaded one step ahead
  // and only multiplied when they become current, so their loads never make
  // the compiler wait in the middle of a step.
  float s_cur[4], sa_nxt[4], sb_nxt;
  auto load_scales = [&](int kb) {
    sb_nxt = sb[(long)nblk * nk + kb];
    const uint32_t kboff = 4u * (uint32_t)kb * (uint32_t)M;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      sa_nxt[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                rsa, srow[j], kboff, 0));
  };

  // Fragment reads: lane reads row base + 16*t + lane%16, logical chunks g and
  // g+4 (K bytes [16g, 16g+16) and [64+16g, 64+16g+16) - both operands use the
  // same K order, so the MFMA sums the same products). For every such row
  // row % 8 == lane % 8, so the swizzle is per lane and the rows differ by
  // immediate offsets of 16 * 128 bytes.
  const int frag_lo = (lane & 15) * ROW + ((g ^ (lane & 7)) * 16);
  const int frag_hi = (lane & 15) * ROW + (((g + 4) ^ (lane & 7)) * 16);
  auto frag = [&](const uint8_t* tile, int row16) {
    const uint8_t* p = tile + row16 * 16 * ROW;
    uint4 lo = *reinterpret_cast<const uint4*>(p + frag_lo);
    uint4 hi = *reinterpret_cast<const uint4*>(p + frag_hi);
    return (v8i){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                 (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  };

  // One K block from LDS stage (la, lb): 32 MFMAs, each promoted into acc one
  // MFMA later (the promotion of (i, j) is issued behind the MFMA of the next
  // pair, so no FMA stalls on the MFMA it reads). Two weight fragments are
  // live at a time: the scheduler is fenced per n-tile to keep it that way.
  auto compute = [&](const uint8_t* la, const uint8_t* lb) {
    v8i xf[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) xf[j] = frag(la, 4 * wm + j);
    v8i wf = frag(lb, 8 * wn);
    f32x4 tp = zero;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v8i wf_n = wf;
      if (i < 7) wf_n = frag(lb, 8 * wn + i + 1);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 t = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
            wf, xf[j], zero, 0, 0, 0, 127, 0, 127);
        const int q = 4 * i + j - 1;  // the previous pair
        if (q >= 0) {
#pragma unroll
          for (int r2 = 0; r2 < 4; ++r2) acc[q >> 2][q & 3][r2] += tp[r2] * s_cur[q & 3];
        }
        tp = t;
      }
      wf = wf_n;
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int r2 = 0; r2 < 4; ++r2) acc[7][3][r2] += tp[r2] * s_cur[3];
  };

  // One pipeline step: wait for this stage's DMA (and for every wave to leave
  // the other stage), queue the next block's scales and DMA into the other
  // stage, then compute this stage.
  auto step = [&](int kb, const uint8_t* la, const uint8_t* lb, const uint8_t* na,
                  const uint8_t* nb) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) s_cur[j] = sa_nxt[j] * sb_nxt;
    if (kb + 1 < nk) {
      load_scales(kb + 1);
      const uint32_t k1 = (uint32_t)(kb + 1) * BK;
      load_tile_lds(ra, offa, k1, na, wave);
      load_tile_lds(rb, offb, k1, nb, wave);
    }
    compute(la, lb);
  };

  load_scales(0);
  load_tile_lds(ra, offa, 0, lds, wave);
  load_tile_lds(rb, offb, 0, lds + TILE_BYTES, wave);
  for (int kb = 0; kb < nk; ++kb) {
    const uint8_t* cur = lds + (kb & 1) * 2 * TILE_BYTES;
    const uint8_t* nxt = lds + ((kb + 1) & 1) * 2 * TILE_BYTES;
    step(kb, cur, cur + TILE_BYTES, nxt, nxt + TILE_BYTES);
  }

  // ---- epilogue: lane holds C[m][n .. n+3] for each (i, j) ------------------
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = m0 + 64 * wm + 16 * j + (lane & 15);
    if (m >= M) continue;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int n = n0 + 128 * wn + 16 * i + 4 * g;
      // v_cvt_pk_bf16_f32: round-to-nearest-even, as f32_to_bf16
      const bf16x2 p0 = {(__bf16)acc[i][j][0], (__bf16)acc[i][j][1]};
      const bf16x2 p1 = {(__bf16)acc[i][j][2], (__bf16)acc[i][j][3]};
      const uint32_t w0 = __builtin_bit_cast(uint32_t, p0);
      const uint32_t w1 = __builtin_bit_cast(uint32_t, p1);
      *reinterpret_cast<uint2*>(C + (long)m * ldc + n) = make_uint2(w0, w1);
    }
  }
}

}  // namespace qh

using namespace qh;

extern "C" int qh_fp8_gemm_nt(const void* A, long lda, const float* sa, const void* B,
                              long ldb, const float* sb, void* C, long ldc, int M, int N,
                              int K, qh_stream_t stream) {
  QH_REQUIRE(M >= 0 && N > 0 && K > 0, "fp8_gemm_nt: M=%d N=%d K=%d", M, N, K);
  QH_REQUIRE(N % gemm::BN == 0, "fp8_gemm_nt: N=%d must be a multiple of 256", N);
  QH_REQUIRE(K % gemm::BK == 0, "fp8_gemm_nt: K=%d must be a multiple of 128", K);
  QH_REQUIRE(lda >= K && ldb >= K && ldc >= N, "fp8_gemm_nt: leading dimensions");
  QH_REQUIRE(lda % 16 == 0 && ldb % 16 == 0 && ldc % 4 == 0,
             "fp8_gemm_nt: lda/ldb must be multiples of 16 bytes, ldc of 4 elements");
  if (M == 0) return QH_OK;
  QH_REQUIRE(A && sa && B && sb && C, "fp8_gemm_nt: null pointer");
  const int tiles = ((M + gemm::BM - 1) / gemm::BM) * (N / gemm::BN);
  hipLaunchKernelGGL(fp8_gemm_nt_kernel, dim3(tiles), dim3(512), 0,
                     (hipStream_t)stream, (const uint8_t*)A, lda, sa, (const uint8_t*)B,
                     ldb, sb, (uint16_t*)C, ldc, M, N, K);
  return launch_status("fp8_gemm_nt");
}
