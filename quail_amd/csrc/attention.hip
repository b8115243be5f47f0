// Varlen attention on bf16 MFMA (gfx950 v_mfma_f32_32x32x16_bf16).
//
// attn_fwd_kernel serves the contiguous-row call (tree call A: K/V are the
// chunk's own rows); attn_paged_kernel further down serves the paged calls.
//
// One workgroup = one q-tile of 32 query rows of one sequence x 4 query heads
// that share one KV head (GQA packs the 4 heads into the 4 waves, so each K/V
// tile is fetched from HBM once for all of them). Per 64-key tile:
//   S^T = K Q^T   (M = keys, N = queries, K = head dim): each lane ends up
//                 holding 16 keys of ONE query, so the row max / row sum of the
//                 online softmax are in-lane plus one cross-half shuffle.
//   O^T += V^T P^T (M = head dim, N = queries, K = keys): P^T comes straight
//                 from the S^T registers (a fixed key permutation inside each
//                 16-key step, mirrored when V^T fragments are read).
// K tiles are staged in LDS as [key][d]; V tiles as V^T [d][key] (the row
// V is transposed on its way into LDS).
#include "common.h"

#include <mutex>
#include <type_traits>

namespace qh {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace attn {
constexpr int BQ = 32;          // query rows per tile
constexpr int BKV = 64;         // keys per KV tile
constexpr int D = 128;          // head dim
constexpr int HPW = 4;          // query heads per workgroup (one per wave)
constexpr int K_LD = D + 8;     // LDS row stride of K (elements): 272 B
constexpr int VT_LD = BKV + 4;  // LDS row stride of V^T (elements): 136 B
constexpr int PAGE = 16;
}  // namespace attn

namespace ntree {
constexpr int RES = 8;          // node tiles held in LDS: 256 keys, 128 KiB of K and V^T
constexpr int RING = 2;         // LDS stages of the streamed tiles
constexpr int ITEM_KEYS = 128;  // fixed work of a q-tile (Q load, epilogue) in keys
constexpr int QROWS = 64;       // query rows of a q-tile (two halves of 32, one per wave set)
}  // namespace ntree

struct AttnParams {
  const uint16_t* q;
  long ldq;
  int q_rows_total;
  const int64_t* q_rows;
  const uint16_t* k_pool;
  const uint16_t* v_pool;
  int pool_pages;
  const int32_t* table;
  int table_width;
  const uint16_t* k_rows;
  const uint16_t* v_rows;
  int kv_rows_total;
  const int32_t* cu_k;
  const int32_t* cu_q;
  const int32_t* kv_len;
  int n_seqs;
  int n_q;
  int n_kv;
  float scale_log2;  // softmax_scale * log2(e)
  uint16_t* out;
  long ldo;
  float* lse;
  long lse_stride;
  const int32_t* tile_off;  // [n_seqs + 1] exclusive scan of q-tiles
  // fp8 output (attn_paged_kernel with FP8OUT): e4m3 [n_out, n_q*128] and
  // per-(row, head) scales [n_q, n_out]
  uint8_t* out_q;
  long ld_out_q;
  float* out_scales;
  int n_out;
  int ue8m0;
};

// Exclusive scan of per-sequence q-tile counts into tile_off[0..n_seqs].
__global__ __launch_bounds__(1024) void attn_tile_scan_kernel(
    const int32_t* __restrict__ cu_q, int n_seqs, int32_t* __restrict__ tile_off) {
  __shared__ int32_t warp_sums[16];
  __shared__ int32_t carry;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  for (int base = 0; base < n_seqs; base += 1024) {
    const int s = base + threadIdx.x;
    int v = 0;
    if (s < n_seqs) {
      const int c = cu_q[s + 1] - cu_q[s];
      v = c > 0 ? (c + attn::BQ - 1) / attn::BQ : 0;
    }
    // inclusive scan within the wave
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (lane == 63) warp_sums[wid] = x;
    __syncthreads();
    int wave_off = 0;
    for (int w = 0; w < wid; ++w) wave_off += warp_sums[w];
    const int c0 = carry;
    if (s < n_seqs) tile_off[s] = c0 + wave_off + x - v;
    __syncthreads();
    if (threadIdx.x == 1023) carry = c0 + wave_off + x;
    __syncthreads();
  }
  if (threadIdx.x == 0) tile_off[n_seqs] = carry;
}

// The node-resident tree kernel's two exclusive scans over the segments of
// cu_a: q-tiles into tile_off[0..n_seg] and work into seg_cost[0..n_seg].
// A segment of c rows reading a node of nk keys has v = ceil(c / 64)
// q-tiles of QROWS = 64 rows; q-tile j (heaviest first) attends nk +
// (j == 0 ? c : 64 (v - j)) keys, and each q-tile also counts ITEM_KEYS for
// its Q load and epilogue: v (nk + ITEM_KEYS) + c + 32 (v - 1) v in all. The workgroups cut the
// q-tiles into runs of equal work from these.
__global__ __launch_bounds__(1024) void attn_tree_scan_kernel(
    const int32_t* __restrict__ cu_a, const int32_t* __restrict__ seg_read,
    const int32_t* __restrict__ read_used, int n_reads, int n_seg,
    int32_t* __restrict__ tile_off, long long* __restrict__ seg_cost) {
  __shared__ int32_t wsum_t[16];
  __shared__ long long wsum_c[16];
  __shared__ int32_t carry_t;
  __shared__ long long carry_c;
  if (threadIdx.x == 0) {
    carry_t = 0;
    carry_c = 0;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  for (int base = 0; base < n_seg; base += 1024) {
    const int s = base + threadIdx.x;
    int v = 0;
    long long c = 0;
    if (s < n_seg) {
      const int count = cu_a[s + 1] - cu_a[s];
      v = count > 0 ? (count + ntree::QROWS - 1) / ntree::QROWS : 0;
      if (v > 0) {
        const int r = seg_read[s];
        const int nk = (r >= 0 && r < n_reads) ? max(0, read_used[r]) : 0;
        c = (long long)v * (nk + ntree::ITEM_KEYS) + count + (ntree::QROWS / 2LL) * (v - 1) * v;
      }
    }
    int x = v;
    long long y = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int xo = __shfl_up(x, o, 64);
      const long long yo = __shfl_up(y, o, 64);
      if (lane >= o) {
        x += xo;
        y += yo;
      }
    }
    if (lane == 63) {
      wsum_t[wid] = x;
      wsum_c[wid] = y;
    }
    __syncthreads();
    int ot = 0;
    long long oc = 0;
    for (int w = 0; w < wid; ++w) {
      ot += wsum_t[w];
      oc += wsum_c[w];
    }
    const int ct = carry_t;
    const long long cc = carry_c;
    if (s < n_seg) {
      tile_off[s] = ct + ot + x - v;
      seg_cost[s] = cc + oc + y - c;
    }
    __syncthreads();
    if (threadIdx.x == 1023) {
      carry_t = ct + ot + x;
      carry_c = cc + oc + y;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    tile_off[n_seg] = carry_t;
    seg_cost[n_seg] = carry_c;
  }
}

// The sequence of q-tile b: the largest s in [0, n) with off[s] <= b, where
// off is non-decreasing and off[0] = 0 <= b. A 64-way search: each round the
// wave's lanes load 64 evenly spaced candidates at once and a ballot picks
// the last one <= b, so n <= 4096 takes two dependent loads where a binary
// search of scalar loads takes twelve (each an L2 round trip, paid before a
// workgroup can start its first DMA). Every lane of the wave must call it.
template <typename T>
__device__ __forceinline__ int last_le(const T* __restrict__ off, int n, T b, int lane) {
  int lo = 0, span = n;  // off[lo] <= b; the answer lies in [lo, lo + span)
  while (span > 1) {
    const int step = (span + 63) >> 6;
    const int idx = lo + lane * step;
    const bool ok = lane * step < span && off[idx] <= b;
    const unsigned long long m = __builtin_amdgcn_ballot_w64(ok);
    const int k = 63 - __builtin_clzll(m);  // lane 0 always holds (off[lo] <= b)
    lo += k * step;
    span = min(step, span - k * step);
  }
  return __builtin_amdgcn_readfirstlane(lo);
}
__device__ __forceinline__ int tile_seq(const int32_t* __restrict__ off, int n, int b, int lane) {
  return last_le<int32_t>(off, n, b, lane);
}

// The work item (q-tile b, head group y) of workgroup (bx, by). The hardware
// deals the workgroups of a launch to the 8 XCDs round-robin in linear order
// (x fastest), so linear id L runs on XCD L % 8. When the head groups split
// evenly over the XCDs, XCD x takes head groups x*per .. x*per + per - 1
// (per = gy / 8) and walks q-tiles in issue order (heaviest first within a
// sequence): its L2 then holds the K/V pages of its own KV heads only, and
// the q-tiles of one sequence, which read the same pages, run there back to
// back. Otherwise the head group is L % gy. Either way the map is a
// bijection of [0, gx) x [0, gy). The launchers keep gx * gy below 2^31, so
// L is a 32-bit index; per is a power of two for every head count in use
// (8 and 16 head groups), which makes the map shifts and masks instead of a
// scalar division routine ahead of the first load.
__device__ __forceinline__ void xcd_item(int bx, int by, int gx, int gy, int& b, int& y) {
  const uint32_t L = (uint32_t)by * (uint32_t)gx + (uint32_t)bx;
  if ((gy & 7) == 0) {
    const uint32_t per = (uint32_t)gy >> 3;
    const uint32_t r = L >> 3;
    uint32_t rq, rr;
    if ((per & (per - 1)) == 0) {
      rq = r >> __builtin_ctz(per);
      rr = r & (per - 1);
    } else {
      rq = r / per;
      rr = r - rq * per;
    }
    y = (int)((L & 7) * per + rr);
    b = (int)rq;
  } else {
    y = (int)(L % (uint32_t)gy);
    b = (int)(L / (uint32_t)gy);
  }
}

// x / d for wave-uniform x >= 0 and d > 0: a shift when d is a power of two
// (the GQA group sizes in use), a division otherwise.
__device__ __forceinline__ int udiv_uniform(int x, int d) {
  return (d & (d - 1)) == 0 ? (int)((uint32_t)x >> __builtin_ctz((uint32_t)d))
                            : (int)((uint32_t)x / (uint32_t)d);
}

template <bool CAUSAL>
__global__ __launch_bounds__(256) void attn_fwd_kernel(AttnParams p) {
  using namespace attn;
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[BKV * K_LD];
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[D * VT_LD];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int half = lane >> 5;   // which 4-row half of each 8-row MFMA group
  const int col = lane & 31;    // query column of the S^T / O^T tiles

  // ---- which sequence and q-tile -------------------------------------------
  int b, hy;
  xcd_item(blockIdx.x, blockIdx.y, gridDim.x, gridDim.y, b, hy);
  const int total_tiles = p.tile_off[p.n_seqs];
  if (b >= total_tiles) return;
  const int s = tile_seq(p.tile_off, p.n_seqs, b, lane);
  const int q0 = p.cu_q[s];
  const int count = p.cu_q[s + 1] - q0;
  const int n_tiles = (count + BQ - 1) / BQ;
  const int tq = n_tiles - 1 - (b - p.tile_off[s]);  // heaviest tile first
  const int i0 = tq * BQ;
  const int kv_len = p.kv_len[s];

  const int group = udiv_uniform(p.n_q, p.n_kv);
  const int hq = hy * HPW + wave;
  const int hk = udiv_uniform(hy * HPW, group);

  // keys this tile reads: causal rows i attend keys < kv_len - count + i + 1
  int kv_end = kv_len;
  if (CAUSAL) {
    const int last = min(i0 + BQ, count) - 1;
    kv_end = min(kv_len, kv_len - count + last + 1);
  }
  if (kv_end < 0) kv_end = 0;

  // ---- Q fragments (B operand of S^T = K Q^T) --------------------------------
  // lane holds Q[query col][16*st + 8*half .. +7] for st = 0..7
  bf16x8_t qf[8];
  {
    const int i = i0 + col;
    const bool valid = i < count;
    long row = q0 + i;
    if (valid && p.q_rows) row = p.q_rows[row];
    const bool ok = valid && row >= 0 && row < p.q_rows_total;
    const uint16_t* qp = p.q + row * p.ldq + (long)hq * D + 8 * half;
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      bf16x8 v;
      if (ok) v = load8(qp + 16 * st);
      else v.w[0] = v.w[1] = v.w[2] = v.w[3] = 0;
      qf[st] = *reinterpret_cast<bf16x8_t*>(&v);
    }
  }

  f32x16 acc_o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int a = 0; a < 16; ++a) acc_o[db][a] = 0.f;
  float m_run = -INFINITY;  // running max (log2 domain), same in both halves
  float l_run = 0.f;        // running sum of this lane's keys

  // query row limit for the mask (exclusive): keys < lim are visible
  const int my_i = i0 + col;
  const int lim = CAUSAL ? min(kv_len, kv_len - count + my_i + 1) : kv_len;

  const int n_kv_tiles = (kv_end + BKV - 1) / BKV;

  // ---- staging: 4 x 16 B of K and 4 x 16 B of V per thread per tile ---------
  bf16x8 kreg[4], vreg[4];
  auto load_tile = [&](int kt) {
    const int key0 = kt * BKV;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // instruction i covers keys 16i .. 16i+15 of the tile
      const int key = key0 + 16 * i + (tid >> 4);
      const int kc = (tid & 15) * 8;
      bf16x8 kv;
      kv.w[0] = kv.w[1] = kv.w[2] = kv.w[3] = 0;
      bf16x8 vv;
      vv.w[0] = vv.w[1] = vv.w[2] = vv.w[3] = 0;
      if (key < kv_end) {
        const long row = (long)p.cu_k[s] + key;
        if (row >= 0 && row < p.kv_rows_total) {
          kv = load8(p.k_rows + (row * p.n_kv + hk) * D + kc);
          vv = load8(p.v_rows + (row * p.n_kv + hk) * D + kc);
        }
      }
      kreg[i] = kv;
      vreg[i] = vv;
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = 16 * i + (tid >> 4);
      const int kc = (tid & 15) * 8;
      store8(k_lds + key * K_LD + kc, kreg[i]);
      // row-layout V: 8 consecutive d of one key, transposed into V^T
#pragma unroll
      for (int e = 0; e < 8; ++e)
        vt_lds[(kc + e) * VT_LD + key] =
            (uint16_t)((vreg[i].w[e >> 1] >> ((e & 1) * 16)) & 0xffffu);
    }
  };

  if (n_kv_tiles > 0) load_tile(0);
  for (int kt = 0; kt < n_kv_tiles; ++kt) {
    __syncthreads();  // previous tile's LDS reads are done
    store_tile();
    if (kt + 1 < n_kv_tiles) load_tile(kt + 1);
    __syncthreads();

    // ---- S^T = K Q^T over two 32-key blocks -------------------------------
    f32x16 sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int a = 0; a < 16; ++a) sacc[kb][a] = 0.f;
      const uint16_t* kp = k_lds + (32 * kb + col) * K_LD + 8 * half;
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        bf16x8_t af = *reinterpret_cast<const bf16x8_t*>(kp + 16 * st);
        sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, qf[st], sacc[kb], 0, 0, 0);
      }
    }
    // ---- mask, scale, online softmax --------------------------------------
    const int key0 = kt * BKV;
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int a = 0; a < 16; ++a) {
        const int key = key0 + 32 * kb + 8 * (a >> 2) + 4 * half + (a & 3);
        const float v = key < lim ? sacc[kb][a] * p.scale_log2 : -INFINITY;
        sacc[kb][a] = v;
        tmax = fmaxf(tmax, v);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = (m_new == -INFINITY) ? 1.f : exp2f(m_run - m_new);
    float psum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int a = 0; a < 16; ++a) {
        const float e = (m_new == -INFINITY) ? 0.f : exp2f(sacc[kb][a] - m_new);
        sacc[kb][a] = e;
        psum += e;
      }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int a = 0; a < 16; ++a) acc_o[db][a] *= alpha;

    // ---- O^T += V^T P^T over four 16-key steps ----------------------------
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int kb = t >> 1, b0 = 2 * (t & 1);
      bf16x8_t pf;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pf[r] = (__bf16)sacc[kb][4 * b0 + r];
        pf[4 + r] = (__bf16)sacc[kb][4 * (b0 + 1) + r];
      }
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const uint16_t* vp = vt_lds + (32 * db + col) * VT_LD + 16 * t + 4 * half;
        uint2 lo = *reinterpret_cast<const uint2*>(vp);
        uint2 hi = *reinterpret_cast<const uint2*>(vp + 8);
        uint32_t w4[4] = {lo.x, lo.y, hi.x, hi.y};
        bf16x8_t vf = *reinterpret_cast<bf16x8_t*>(w4);
        acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, acc_o[db], 0, 0, 0);
      }
    }
  }

  // ---- epilogue -----------------------------------------------------------
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  if (my_i >= count) return;
  const long qi = q0 + my_i;
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  uint16_t* op = p.out + qi * p.ldo + (long)hq * D;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * db + 8 * g + 4 * half;
      uint32_t w0 = f32_to_bf16(acc_o[db][4 * g + 0] * inv) |
                    (f32_to_bf16(acc_o[db][4 * g + 1] * inv) << 16);
      uint32_t w1 = f32_to_bf16(acc_o[db][4 * g + 2] * inv) |
                    (f32_to_bf16(acc_o[db][4 * g + 3] * inv) << 16);
      *reinterpret_cast<uint2*>(op + d) = make_uint2(w0, w1);
    }
  if (p.lse && half == 0) {
    const float lse = l_tot > 0.f ? (m_run + log2f(l_tot)) * 0.69314718055994531f : -INFINITY;
    p.lse[(long)hq * p.lse_stride + qi] = lse;
  }
}


// ---------------------------------------------------------------------------
// Paged attention, DMA-fed (the unified path and tree call B).
//
// Same workgroup decomposition as attn_fwd_kernel (32 queries x 4 GQA heads,
// one wave per head) but with 32-key tiles that reach LDS by DMA
// (buffer_load ... lds) straight from the arena's 4 KiB page blocks, in a
// 3-stage ring two tiles ahead, and with about half the registers, so three
// workgroups share a CU. Per tile each wave issues exactly four vector-memory
// loads - its four 1 KiB DMA pieces of tile t+2 (wave w moves K (w < 2) or
// V^T (w >= 2) of page w % 2) - and one scalar load, the page id it needs
// for tile t+3, so every wait is vmcnt(4).
//
// LDS stage: K [32 keys][128 d] with 16-byte chunks XOR-swizzled by
// (key % 16) ^ (key / 16); V^T [2 pages][128 d][16 slots] with the two
// 16-byte halves of a d row swapped when (d / 8) is odd. The swizzles are
// applied by choosing which global chunk each DMA lane fetches.
//
// The S^T MFMA row i reads key kperm(i) (bits 2 and 3 swapped), so that in
// each 16-key P.V step a lane's eight P values are eight consecutive keys -
// exactly sacc[8t .. 8t+7] - and its V^T fragment is one 16-byte read.
// Pages past the sequence read zeros (zero-length descriptor); the V slots
// past kv_end of a partial last page are zeroed in LDS, so P = 0 never meets
// a NaN.

namespace pattn {
constexpr int BQ = 32;
constexpr int BKV = 32;
constexpr int D = 128;
constexpr int HPW = 4;
constexpr int PAGE = 16;
constexpr int NST = 3;             // LDS stages
constexpr int HALF = BKV * D * 2;  // 8 KiB: K or V^T of one tile
constexpr int STAGE = 2 * HALF;
}  // namespace pattn

// The fp8 epilogue's store of one wave's 32 x 128 e4m3 block. A lane holds
// row `col` of the q-tile, bytes d = 32*db + 8*g + 4*half .. +3 in w[db][g];
// stored straight from there, every 4-byte store touches 32 rows. The block
// goes through the wave's own padded LDS rows (`stage`, 32 x 144 bytes) and
// leaves as whole 128-byte rows, 8 rows per 16-byte-per-lane store. Rows at
// or past `rows` are not written. The caller has ended every wave's use of
// the LDS area first.
__device__ __forceinline__ void store_fp8_rows(uint8_t* stage, const uint32_t (&w)[4][4],
                                               int lane, uint8_t* out, long ld, int rows) {
  constexpr int ROWB = 144;
  const int col = lane & 31, half = lane >> 5;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *reinterpret_cast<uint32_t*>(stage + col * ROWB + 32 * db + 8 * g + 4 * half) = w[db][g];
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int row = 8 * k + (lane >> 3), chunk = lane & 7;
    const uint4 v = *reinterpret_cast<const uint4*>(stage + row * ROWB + 16 * chunk);
    if (row < rows) *reinterpret_cast<uint4*>(out + row * ld + 16 * chunk) = v;
  }
}

__device__ __forceinline__ int kperm(int i) {
  return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1);
}
__device__ __forceinline__ int kswz(int key) { return (key & 15) ^ (key >> 4); }

// A row's maximum over the tile's 32 keys, unscaled: the lane's 16 scores
// and its partner lane's (lane ^ 32) through IEEE maximum (v_maximum3_f32,
// two scores per instruction), which needs no quieting of the MFMA results
// as fmaxf's maxNum lowering does.
__device__ __forceinline__ float tile_row_max(const f32x16& s) {
  float m = __builtin_elementwise_maximum(s[0], s[1]);
#pragma unroll
  for (int a = 2; a < 16; ++a) m = __builtin_elementwise_maximum(m, s[a]);
  return xor32_maximum(m);
}

// l += the row sum of 8 probabilities as the bf16 values the P.V MFMA
// multiplies (v_dot2_f32_bf16 against (1, 1), two per instruction): the
// normaliser sums exactly the P the numerator does.
__device__ __forceinline__ float add_row_sum(const bf16x8_t& pf, float l) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t one = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
  for (int k = 0; k < 4; ++k)
    l = __builtin_amdgcn_fdot2_f32_bf16((bf16x2_t){pf[2 * k], pf[2 * k + 1]}, one, l, false);
  return l;
}

typedef int pi32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ pi32x4 attn_rsrc(const void* base, uint32_t bytes) {
  const uint64_t b = (uint64_t)base;
  return (pi32x4){(int)(uint32_t)b, (int)(uint32_t)(b >> 32), (int)bytes, 0x00020000};
}

template <bool CAUSAL, bool FP8OUT>
__global__ __launch_bounds__(256, 3) void attn_paged_kernel(AttnParams p) {
  using namespace pattn;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NST * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int col = lane & 31;

  // ---- sequence and q-tile (heaviest tile of a sequence first) -------------
  int b, hy;
  xcd_item(blockIdx.x, blockIdx.y, gridDim.x, gridDim.y, b, hy);
  const int total_tiles = p.tile_off[p.n_seqs];
  if (b >= total_tiles) return;
  const int s = tile_seq(p.tile_off, p.n_seqs, b, lane);
  const int q0 = p.cu_q[s];
  const int count = p.cu_q[s + 1] - q0;
  const int n_qt = (count + BQ - 1) / BQ;
  const int i0 = (n_qt - 1 - (b - p.tile_off[s])) * BQ;
  const int kv_len = p.kv_len[s];
  const int group = udiv_uniform(p.n_q, p.n_kv);
  const int hq = hy * HPW + wave;
  const int hk = udiv_uniform(hy * HPW, group);
  int kv_end = kv_len;
  if (CAUSAL) kv_end = min(kv_len, kv_len - count + min(i0 + BQ, count));
  kv_end = max(kv_end, 0);
  const int n_tiles = (kv_end + BKV - 1) / BKV;
  const int my_i = i0 + col;
  const int lim = CAUSAL ? min(kv_len, kv_len - count + my_i + 1) : kv_len;

  // ---- DMA roles ------------------------------------------------------------
  const int region = wave >> 1;  // 0: K, 1: V^T
  const int pit = wave & 1;      // page within the tile
  uint32_t voff[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int P = 1024 * c + 16 * lane;  // byte position in the LDS page block
    if (region == 0) {
      const int r16 = P >> 8, pc = (P >> 4) & 15;
      voff[c] = (uint32_t)(r16 * 256 + ((pc ^ kswz(16 * pit + r16)) * 16));
    } else {
      const int d = P >> 5, ph = (P >> 4) & 1;
      voff[c] = (uint32_t)(d * 32 + ((ph ^ ((d >> 3) & 1)) * 16));
    }
  }
  const uint16_t* pool = region ? p.v_pool : p.k_pool;
  const long tab_row = (long)s * p.table_width;
  // page index of this wave's page in tile t, clamped into the table row
  auto tab_off = [&](int t) __attribute__((always_inline)) {
    const int pidx = min(2 * t + pit, p.table_width - 1);
    return (uint32_t)((tab_row + pidx) * 4);
  };
  // this wave's four DMA pieces of tile t into `stage` (= t % NST)
  auto dma_tile = [&](int t, int page_id, int stage) __attribute__((always_inline)) {
    const int pidx = 2 * t + pit;
    const bool live = t < n_tiles && pidx < p.table_width && pidx * PAGE < kv_end &&
                      page_id >= 0 && page_id < p.pool_pages;
    const int slots = live ? min(PAGE, kv_end - pidx * PAGE) : 0;
    const uint32_t bytes = region ? (live ? 4096u : 0u) : (uint32_t)slots * 256u;
    const uint16_t* blk = pool + ((long)(live ? page_id : 0) * p.n_kv + hk) * (PAGE * D);
    const pi32x4 rs = attn_rsrc(blk, bytes);
    const uint32_t base =
        (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)(
            lds + stage * STAGE + region * HALF + pit * 4096);
#pragma unroll
    for (int c = 0; c < 4; ++c)
      asm volatile(
          "s_mov_b32 m0, %0\n\t"
          "buffer_load_dwordx4 %1, %2, 0 offen lds"
          :
          : "s"(base + 1024 * c), "v"(voff[c]), "s"(rs)
          : "memory", "m0");
  };

  // ---- Q fragments: lane holds Q[query col][16*st + 8*half .. +7] -----------
  typedef int qi32x4 __attribute__((ext_vector_type(4)));
  qi32x4 qraw[8];
  {
    long row = q0 + my_i;
    bool ok = my_i < count;
    if (ok && p.q_rows) row = p.q_rows[row];
    ok = ok && row >= 0 && row < p.q_rows_total;
    const uint32_t qoff = ok ? (uint32_t)(row * p.ldq * 2 + (long)hq * D * 2 + 16 * half)
                             : 0x80000000u;
    const pi32x4 rq = attn_rsrc(p.q, (uint32_t)((long)p.q_rows_total * p.ldq * 2));
#pragma unroll
    for (int st = 0; st < 8; ++st)
      asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen offset:%3"
                   : "=v"(qraw[st]) : "v"(qoff), "s"(rq), "i"(32 * st) : "memory");
  }

  // ---- prologue: page ids of tiles 0..2 (scalar), DMA of tiles 0 and 1 -------
  // The page ids are scalar loads through the constant address space: as
  // vector loads behind the Q loads, their vmcnt waits also waited for Q, so
  // the first DMA went out only after a whole Q round trip.
  int pg0 = -1, pg1 = -1, pg2 = -1;
  if (n_tiles > 0) {
    const __attribute__((address_space(4))) int32_t* tab =
        (const __attribute__((address_space(4))) int32_t*)(uintptr_t)(p.table);
    pg0 = tab[tab_row + min(pit, p.table_width - 1)];
    pg1 = tab[tab_row + min(2 + pit, p.table_width - 1)];
    pg2 = tab[tab_row + min(4 + pit, p.table_width - 1)];
    dma_tile(0, pg0, 0);
    dma_tile(1, pg1, 1);
  }
  asm volatile("s_waitcnt vmcnt(4)" ::: "memory");  // Q and tile 0 landed
  asm volatile("" : "+v"(qraw[0]), "+v"(qraw[1]), "+v"(qraw[2]), "+v"(qraw[3]),
               "+v"(qraw[4]), "+v"(qraw[5]), "+v"(qraw[6]), "+v"(qraw[7]));
  bf16x8_t qf[8];
#pragma unroll
  for (int st = 0; st < 8; ++st) qf[st] = __builtin_bit_cast(bf16x8_t, qraw[st]);

  f32x16 acc_o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int a = 0; a < 16; ++a) acc_o[db][a] = 0.f;
  float m_run = -1e30f;   // finite floor: see the softmax note in the tile loop
  float l_run = 0.f;
  const float inv_scale = __builtin_amdgcn_rcpf(p.scale_log2);
  float m_thr = (m_run + 8.0f) * inv_scale;
  int pg_next = pg2;  // page id for the DMA of tile t+2

  const int kq = kperm(col);  // key row this lane's S^T row reads
  const int ksw = kswz(kq);
  // K fragment st of a stage sits at kbase + ((32 st) ^ kx): the chunk
  // swizzle (2 st + half) ^ ksw splits into a half-chunk fixed per lane and a
  // permutation of the 32-byte chunk pairs. V^T fragment (pt, db) sits at
  // vbase + 4096 pt + 1024 db (its half swap depends on col only). Each LDS
  // address is then the stage's offset (a scalar) plus a lane offset plus an
  // immediate.
  const uint32_t kbase = (uint32_t)(kq * 256 + ((half ^ (ksw & 1)) * 16));
  const uint32_t kx = (uint32_t)((ksw >> 1) * 32);
  const uint32_t vbase = (uint32_t)(col * 32 + ((half ^ ((col >> 3) & 1)) * 16));
  // the causal mask of a boundary tile: element a holds key key0 + 8 half +
  // kc(a), with kc(a) = kperm(8 (a / 4) + (a % 4)) a compile-time constant
  auto step = [&](int t, int stage) __attribute__((always_inline)) {
    // tile t's DMA (issued two tiles back) and the page id of tile t+2
    // (issued first last tile) have landed; tile t+1's DMA may be in flight
    asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    const int page_t2 = pg_next;
    // stage t visible to all (every wave waited for its share above); stage
    // t-1 free. A plain barrier: __syncthreads' fence would also wait for
    // the DMA of tile t+1.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    wg_barrier();
    dma_tile(t + 2, page_t2, stage == 0 ? 2 : stage - 1);

    uint8_t* st_base = lds + stage * STAGE;
    const int key0 = t * BKV;
    // a partial last page: zero its V^T slots past kv_end
    if (key0 + BKV > kv_end && ((kv_end & (PAGE - 1)) != 0)) {
      const int zpit = (kv_end - key0) >> 4;
      const int valid = kv_end & (PAGE - 1);
      if (zpit < 2) {
        const int d = tid >> 1, ph = tid & 1;
        const int lh = ph ^ ((d >> 3) & 1);
        uint16_t* vp = reinterpret_cast<uint16_t*>(st_base + HALF + zpit * 4096 + d * 32 + ph * 16);
        bf16x8 v = load8(vp);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (8 * lh + e >= valid) v.set(e, 0);
        store8(vp, v);
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      wg_barrier();
    }

    // ---- S^T = K Q^T ---------------------------------------------------------
    f32x16 sacc;
#pragma unroll
    for (int a = 0; a < 16; ++a) sacc[a] = 0.f;
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const bf16x8_t af = *reinterpret_cast<const bf16x8_t*>(
          st_base + (kbase + (((uint32_t)(32 * st)) ^ kx)));
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, qf[st], sacc, 0, 0, 0);
    }
    // ---- mask (boundary tiles only), online softmax (log2 domain) ---------
    // every key of a tile is visible to every row when the tile ends before
    // both the sequence and the first row's causal limit
    const int first_lim = CAUSAL ? kv_len - count + i0 + 1 : kv_len;
    if (key0 + BKV > min(kv_len, first_lim)) {
      const int L = lim - key0 - 8 * half;
#pragma unroll
      for (int a = 0; a < 16; ++a) {
        const int kc = kperm(8 * (a >> 2) + (a & 3));
        if (kc >= L) sacc[a] = -INFINITY;
      }
    }
    // The running maximum moves only when a row's tile maximum exceeds it by
    // more than 8 (probabilities up to 2^8 against it are exact in the fp32
    // sums and lose nothing in bf16), so the rescale of the accumulator is
    // skipped on most tiles; m_run starts at a finite floor, so exp2 of a
    // masked score is 0 and no -inf arithmetic needs a guard. The test
    // compares the unscaled maximum with m_thr = (m_run + 8) / scale (set
    // whenever m_run moves). On the first tile the accumulator and the sum
    // are still zero, so the rescale is skipped outright.
    const float traw = tile_row_max(sacc);
    const bool grow = traw > m_thr;
    if (t == 0) {
      m_run = grow ? traw * p.scale_log2 : m_run;
      m_thr = (m_run + 8.0f) * inv_scale;
    } else if (__builtin_amdgcn_ballot_w64(grow)) {
      const float m_new = grow ? traw * p.scale_log2 : m_run;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      m_thr = (m_run + 8.0f) * inv_scale;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int a = 0; a < 16; ++a) acc_o[db][a] *= alpha;
    }
#pragma unroll
    for (int a = 0; a < 16; ++a)
      sacc[a] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[a], p.scale_log2, -m_run));

    // ---- O^T += V^T P^T over the tile's two pages ----------------------------
#pragma unroll
    for (int pt = 0; pt < 2; ++pt) {
      bf16x8_t pf;
#pragma unroll
      for (int e = 0; e < 8; ++e) pf[e] = (__bf16)sacc[8 * pt + e];
      l_run = add_row_sum(pf, l_run);
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const bf16x8_t vf = *reinterpret_cast<const bf16x8_t*>(
            st_base + HALF + pt * 4096 + db * 1024 + vbase);
        acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, acc_o[db], 0, 0, 0);
      }
    }
    // the page id of tile t+3 by a scalar load (the table is read-only for
    // the kernel: constant address space), issued last so that its latency
    // hides behind the next tile's DMA wait. A vector load, whose result the
    // compiler would wait for with vmcnt(0) - it cannot see the DMA loads -
    // drained the DMA ring at every tile.
    pg_next = ((const __attribute__((address_space(4))) int32_t*)(uintptr_t)(p.table))[
        tab_off(t + 3) / 4];
  };
  for (int t = 0, stage = 0; t < n_tiles; ++t, stage = stage == NST - 1 ? 0 : stage + 1)
    step(t, __builtin_amdgcn_readfirstlane(stage));
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no DMA outlives the workgroup

  // ---- epilogue -------------------------------------------------------------
  const float l_tot = xor32_sum(l_run);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  const long qi = q0 + my_i;
  if constexpr (FP8OUT) {
    // the bf16 output, quantized per (row, head) 128-wide group exactly as
    // group_quant would quantize it; the group's other 64 values sit in the
    // partner lane (lane ^ 32)
    float amax = 0.f;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int a = 0; a < 16; a += 2) {
        float v0 = acc_o[db][a] * inv, v1 = acc_o[db][a + 1] * inv;
        round_bf16_pair(v0, v1);
        acc_o[db][a] = v0;
        acc_o[db][a + 1] = v1;
        amax = fmaxf(amax, fabsf(v0));
        amax = fmaxf(amax, fabsf(v1));
      }
    amax = xor32_max(amax);
    const float scale = group_scale(amax, p.ue8m0 != 0);
    const double rinv = recip_exact(scale);
    uint32_t w[4][4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        w[db][g] = quant_e4m3_x4(acc_o[db][4 * g], acc_o[db][4 * g + 1], acc_o[db][4 * g + 2],
                                 acc_o[db][4 * g + 3], rinv);
    // every wave is past its last read of the stages (and every DMA landed)
    // before the stages become staging rows
    wg_barrier();
    store_fp8_rows(lds + wave * 32 * 144, w, lane,
                   p.out_q + (long)(q0 + i0) * p.ld_out_q + (long)hq * D, p.ld_out_q,
                   count - i0);
    if (my_i >= count) return;
    if (half == 0) p.out_scales[(long)hq * p.n_out + qi] = scale;
  } else {
    if (my_i >= count) return;
    uint16_t* op = p.out + qi * p.ldo + (long)hq * D;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * db + 8 * g + 4 * half;
        uint32_t w0 = f32_to_bf16(acc_o[db][4 * g + 0] * inv) |
                      (f32_to_bf16(acc_o[db][4 * g + 1] * inv) << 16);
        uint32_t w1 = f32_to_bf16(acc_o[db][4 * g + 2] * inv) |
                      (f32_to_bf16(acc_o[db][4 * g + 3] * inv) << 16);
        *reinterpret_cast<uint2*>(op + d) = make_uint2(w0, w1);
      }
  }
  if (p.lse && half == 0) {
    const float lse = l_tot > 0.f ? (m_run + log2f(l_tot)) * 0.69314718055994531f : -INFINITY;
    p.lse[(long)hq * p.lse_stride + qi] = lse;
  }
}


// ---------------------------------------------------------------------------
// Tree attention, fused (the tree path's call A + call B + merge in one pass).
//
// The chunk's rows form causal segments (cu_a). A segment may read a node:
// resident arena pages every one of its rows attends in full (a parent's
// shared prefix, or a kept anchor's document) - seg_read[s] names the read
// sequence (page table row, used keys) or is -1. One workgroup = 32 rows of
// one segment x the 4 query heads of one KV head; it walks the node's pages
// (non-causal) and then the segment's own rows (causal) as one stream of
// 32-key tiles with one online softmax, so no LSE, second output or merge
// pass exists, and q-tiles of the rows under one node run back to back, so
// the node's pages are fetched from HBM once and served from L2 after.
//
// Node tiles reach LDS exactly as in attn_paged_kernel (K and V^T page
// blocks by DMA). Own tiles are the chunk's contiguous K/V rows
// [T, n_kv, 128], also by DMA: K into the same swizzled [key][d] layout,
// V into [key][d] rows whose 16-byte chunks are XOR-swizzled by 4 (key % 4);
// the P.V operand (8 consecutive keys of one d per lane) is then read with
// two ds_read_b64_tr_b16. Within a 16-lane group, that instruction hands
// lane i element i % 4 of the 8-byte rows addressed by lanes i/4, 4 + i/4,
// 8 + i/4 and 12 + i/4, so lane r addresses key kbase + r/4 at
// d = dbase + 4 (r % 4) and lane i receives keys kbase .. kbase+3 of
// d = dbase + i.
struct TreeParams {
  const uint16_t* q;
  long ldq;
  int n_rows;                 // T: chunk rows (q, k_rows, v_rows, outputs)
  const uint16_t* k_rows;
  const uint16_t* v_rows;
  long ld_kv;                 // elements per row of k_rows / v_rows (n_kv * 128)
  const int32_t* cu_a;        // [n_seg + 1]
  const int32_t* seg_read;    // [n_seg]: read sequence or -1
  int n_seg;
  const uint16_t* k_pool;
  const uint16_t* v_pool;
  int pool_pages;
  const int32_t* table;       // [n_reads, table_width]
  int table_width;
  const int32_t* read_used;   // [n_reads]
  int n_reads;
  int n_q;
  int n_kv;
  float scale_log2;
  uint16_t* out;              // bf16 [T, n_q*128] (row stride ldo), or
  long ldo;
  uint8_t* out_q;             // e4m3 [T, n_q*128] + scales [n_q, T]
  long ld_out_q;
  float* out_scales;
  int ue8m0;
  const int32_t* tile_off;    // [n_seg + 1] exclusive scan of q-tiles
  const long long* seg_cost;  // [n_seg + 1] exclusive scan of work (node-resident kernel)
};

__device__ __forceinline__ int vswz(int key) { return 4 * (key & 3); }

typedef short ts16x4 __attribute__((ext_vector_type(4)));

template <bool FP8OUT>
__global__ __launch_bounds__(256, 3) void attn_tree_kernel(TreeParams p) {
  using namespace pattn;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NST * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int col = lane & 31;

  // ---- segment and q-tile (heaviest q-tile of a segment first) -------------
  int b, hy;
  xcd_item(blockIdx.x, blockIdx.y, gridDim.x, gridDim.y, b, hy);
  const int total_tiles = p.tile_off[p.n_seg];
  if (b >= total_tiles) return;
  const int s = tile_seq(p.tile_off, p.n_seg, b, lane);
  const int q0 = p.cu_a[s];
  const int count = p.cu_a[s + 1] - q0;
  const int n_qt = (count + BQ - 1) / BQ;
  const int i0 = (n_qt - 1 - (b - p.tile_off[s])) * BQ;
  const int group = udiv_uniform(p.n_q, p.n_kv);
  const int hq = hy * HPW + wave;
  const int hk = udiv_uniform(hy * HPW, group);
  int r = p.seg_read[s];
  if (r >= p.n_reads) r = -1;
  const int node_keys = r >= 0 ? max(0, p.read_used[r]) : 0;
  const int n1 = (node_keys + BKV - 1) / BKV;          // node tiles
  const int own_keys = min(count, i0 + BQ);            // causal: rows < i0 + 32
  const int n_tiles = n1 + (own_keys + BKV - 1) / BKV;
  const int my_i = i0 + col;
  // what the epilogue needs, pinned to VGPRs: held as scalars across the
  // tile loops they were spilled to VGPR lanes and read back by v_readlane
  int ep_row0 = q0 + i0, ep_rows = count - i0, ep_hq = hq, ep_stage = wave * 32 * 144;
  asm volatile("" : "+v"(ep_row0), "+v"(ep_rows), "+v"(ep_hq), "+v"(ep_stage));

  // ---- DMA roles: wave (region, pit) moves K (region 0) or V (region 1) of
  // keys 16 pit .. 16 pit + 15 of a tile, as four 1 KiB pieces -------------
  const int region = wave >> 1;
  const int pit = wave & 1;
  const uint32_t row_bytes = (uint32_t)p.ld_kv * 2u;
  // Lane byte offsets of DMA piece c (bytes 1024 c + 16 lane of the wave's
  // 4 KiB block): key r16 = 4c + lane/16 of the wave's 16, physical chunk
  // lane % 16, which holds logical chunk (lane % 16) ^ swizzle(key). K's
  // swizzle kswz(16 pit + r16) = r16 ^ pit; own V's vswz = 4 (r16 % 4) =
  // 4 (lane / 16); a node V^T row d = 32c + lane/2 swaps its halves when
  // (d / 8) is odd, i.e. when (lane / 16) is odd. Computed per piece from
  // the lane, to keep registers for the tile loop: the lane id is re-read
  // (v_mbcnt, opaque to the compiler) at every DMA, so none of these offsets
  // is held across the loop - held, they were spilled, and the reload's
  // vmcnt(0) wait drained the DMA ring before every tile.
  struct LaneOff {
    uint32_t k_chunk, own_v_chunk, node_v_off, own_row;
    int l16;
  };
  auto lane_offsets = [&]() __attribute__((always_inline)) {
    int ln;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
    LaneOff o;
    o.l16 = ln >> 4;
    const int pc = ln & 15;
    o.k_chunk = (uint32_t)((pc ^ o.l16 ^ pit) * 16);  // XOR 64 c per piece
    o.own_v_chunk = (uint32_t)((pc ^ (4 * o.l16)) * 16);
    o.node_v_off = (uint32_t)((ln >> 1) * 32 + (((ln & 1) ^ (o.l16 & 1)) * 16));
    o.own_row = (uint32_t)o.l16 * row_bytes + (uint32_t)hk * 256u;
    return o;
  };
  auto voff_node = [&](const LaneOff& o, int c) __attribute__((always_inline)) {
    return region == 0 ? (uint32_t)((4 * c + o.l16) * 256) + (o.k_chunk ^ (uint32_t)(64 * c))
                       : o.node_v_off + (uint32_t)(1024 * c);
  };
  auto voff_own = [&](const LaneOff& o, int c) __attribute__((always_inline)) {
    return o.own_row + (uint32_t)(4 * c) * row_bytes +
           (region == 0 ? (o.k_chunk ^ (uint32_t)(64 * c)) : o.own_v_chunk);
  };
  const uint16_t* pool = region ? p.v_pool : p.k_pool;
  const uint16_t* own_rows = region ? p.v_rows : p.k_rows;
  const long tab_row = (long)(r >= 0 ? r : 0) * p.table_width;
  auto tab_off = [&](int t) __attribute__((always_inline)) {
    const int pidx = min(2 * t + pit, p.table_width - 1);
    return (uint32_t)((tab_row + max(pidx, 0)) * 4);
  };
  // this wave's four DMA pieces of tile t into `stage` (= t % NST)
  auto dma_tile = [&](int t, int page_id, int stage) __attribute__((always_inline)) {
    const uint32_t base =
        (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)(
            lds + stage * STAGE + region * HALF + pit * 4096);
    const LaneOff lo = lane_offsets();
    if (t < n1) {
      const int pidx = 2 * t + pit;
      const bool live = pidx < p.table_width && pidx * PAGE < node_keys && page_id >= 0 &&
                        page_id < p.pool_pages;
      const int slots = live ? min(PAGE, node_keys - pidx * PAGE) : 0;
      const uint32_t bytes = region ? (live ? 4096u : 0u) : (uint32_t)slots * 256u;
      const uint16_t* blk = pool + ((long)(live ? page_id : 0) * p.n_kv + hk) * (PAGE * D);
      const pi32x4 rs = attn_rsrc(blk, bytes);
#pragma unroll
      for (int c = 0; c < 4; ++c)
        asm volatile(
            "s_mov_b32 m0, %0\n\t"
            "buffer_load_dwordx4 %1, %2, 0 offen lds"
            :
            : "s"(base + 1024 * c), "v"(voff_node(lo, c)), "s"(rs)
            : "memory", "m0");
    } else {
      // own keys 32 (t - n1) + 16 pit + 0..15: chunk rows q0 + those keys;
      // rows past the chunk (or past the tiles) read zero
      const long row0 = (long)q0 + 32L * (t - n1) + 16 * pit;
      const bool live = t < n_tiles && row0 < p.n_rows;
      const long rows_left = live ? (long)p.n_rows - row0 : 0;
      const pi32x4 rs = attn_rsrc(own_rows + (live ? row0 : 0) * p.ld_kv,
                                  (uint32_t)(rows_left * (long)row_bytes));
#pragma unroll
      for (int c = 0; c < 4; ++c)
        asm volatile(
            "s_mov_b32 m0, %0\n\t"
            "buffer_load_dwordx4 %1, %2, 0 offen lds"
            :
            : "s"(base + 1024 * c), "v"(voff_own(lo, c)), "s"(rs)
            : "memory", "m0");
    }
  };

  // ---- Q fragments: lane holds Q[query col][16*st + 8*half .. +7] -----------
  typedef int qi32x4 __attribute__((ext_vector_type(4)));
  qi32x4 qraw[8];
  {
    const long row = (long)q0 + my_i;
    const bool ok = my_i < count && row < p.n_rows;
    const uint32_t qoff = ok ? (uint32_t)(row * p.ldq * 2 + (long)hq * D * 2 + 16 * half)
                             : 0x80000000u;
    const pi32x4 rq = attn_rsrc(p.q, (uint32_t)((long)p.n_rows * p.ldq * 2));
#pragma unroll
    for (int st = 0; st < 8; ++st)
      asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen offset:%3"
                   : "=v"(qraw[st]) : "v"(qoff), "s"(rq), "i"(32 * st) : "memory");
  }

  // ---- prologue: page ids of node tiles 0..2 (scalar), DMA of tiles 0, 1 -----
  // scalar loads through the constant address space (see attn_paged_kernel)
  auto page_of = [&](int t) __attribute__((always_inline)) {
    const __attribute__((address_space(4))) int32_t* tab =
        (const __attribute__((address_space(4))) int32_t*)(uintptr_t)(p.table);
    return (r >= 0 && t < n1) ? tab[tab_row + min(2 * t + pit, p.table_width - 1)] : -1;
  };
  const int pg0 = page_of(0), pg1 = page_of(1), pg2 = page_of(2);
  dma_tile(0, pg0, 0);
  dma_tile(1, pg1, 1);
  asm volatile("s_waitcnt vmcnt(4)" ::: "memory");  // Q and tile 0 landed
  asm volatile("" : "+v"(qraw[0]), "+v"(qraw[1]), "+v"(qraw[2]), "+v"(qraw[3]),
               "+v"(qraw[4]), "+v"(qraw[5]), "+v"(qraw[6]), "+v"(qraw[7]));
  bf16x8_t qf[8];
#pragma unroll
  for (int st = 0; st < 8; ++st) qf[st] = __builtin_bit_cast(bf16x8_t, qraw[st]);

  f32x16 acc_o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int a = 0; a < 16; ++a) acc_o[db][a] = 0.f;
  float m_run = -1e30f;   // finite floor: see the softmax note in the tile loop
  float l_run = 0.f;
  const float inv_scale = __builtin_amdgcn_rcpf(p.scale_log2);
  float m_thr = (m_run + 8.0f) * inv_scale;
  int pg_next = pg2;

  // own-tile P.V operand addresses (see the note above the kernel): lane
  // group G = lane / 16 covers d = 32 db + 16 (G % 2) + lane % 16 and keys
  // 16 pt + 8 (G / 2) + 4 u + 0..3; lane addresses key + (lane % 16) / 4
  // byte offset of that address within the tile's V rows at db = 0: key
  // tr_key's row, logical chunk 2 (G % 2) + (lane % 4) / 2 XOR the row's
  // vswz (a lane constant: vswz(key) = 4 (key % 4) and 16 pt + 4 u keeps
  // key % 4), half (lane % 2); block db only XORs 4 db into the chunk, i.e.
  // 64 db into the byte offset
  const int gi = lane & 15;
  const int tr_key = 8 * (lane >> 5) + (gi >> 2);
  const uint32_t tr_off = (uint32_t)(tr_key * 256 +
                                     (((2 * ((lane >> 4) & 1) + ((gi & 3) >> 1)) ^ vswz(tr_key)) * 16) +
                                     (gi & 1) * 8);

  // K fragment st at kbase + ((32 st) ^ kx) of a stage and node V^T
  // fragment (pt, db) at vbase + 4096 pt + 1024 db, as in attn_paged_kernel.
  // kbase and kx are recomputed per tile from the lane id (as the DMA
  // offsets are): held across the loop, with the eight fragment offsets the
  // compiler derives from them, they pushed the kernel into spills.
  const uint32_t vbase = (uint32_t)(col * 32 + ((half ^ ((col >> 3) & 1)) * 16));
  // one 32-key tile in `stage`; NODE is the phase (the two phases' P.V
  // operands differ)
  auto tile = [&](int t, int stage, auto node_c) __attribute__((always_inline)) {
    constexpr bool node = decltype(node_c)::value;
    asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    const int page_t2 = pg_next;
    // stage t visible to all (every wave waited for its share above); stage
    // t-1 free. A plain barrier: __syncthreads' fence would also wait for
    // the DMA of tile t+1.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    wg_barrier();
    dma_tile(t + 2, page_t2, stage == 0 ? 2 : stage - 1);

    uint8_t* st_base = lds + stage * STAGE;
    const int key0 = node ? t * BKV : (t - n1) * BKV;
    // a partial last node page: zero its V^T slots past node_keys
    if (node && key0 + BKV > node_keys && ((node_keys & (PAGE - 1)) != 0)) {
      const int zpit = (node_keys - key0) >> 4;
      const int valid = node_keys & (PAGE - 1);
      if (zpit < 2) {
        const int d = tid >> 1, ph = tid & 1;
        const int lh = ph ^ ((d >> 3) & 1);
        uint16_t* vp = reinterpret_cast<uint16_t*>(st_base + HALF + zpit * 4096 + d * 32 + ph * 16);
        bf16x8 v = load8(vp);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (8 * lh + e >= valid) v.set(e, 0);
        store8(vp, v);
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      wg_barrier();
    }

    // ---- S^T = K Q^T ---------------------------------------------------------
    f32x16 sacc;
#pragma unroll
    for (int a = 0; a < 16; ++a) sacc[a] = 0.f;
    int ln;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
    const int kq = kperm(ln & 31);
    const int ksw = kswz(kq);
    const uint32_t kbase = (uint32_t)(kq * 256 + (((ln >> 5) ^ (ksw & 1)) * 16));
    const uint32_t kx = (uint32_t)((ksw >> 1) * 32);
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const bf16x8_t af = *reinterpret_cast<const bf16x8_t*>(
          st_base + (kbase + (((uint32_t)(32 * st)) ^ kx)));
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, qf[st], sacc, 0, 0, 0);
    }
    // ---- mask (boundary tiles only), online softmax (log2 domain) ---------
    // a node tile needs the mask only past node_keys; an own tile only where
    // it reaches past the q-tile's first row (the causal diagonal)
    const bool need_mask = node ? key0 + BKV > node_keys : key0 + BKV - 1 > i0;
    if (need_mask) {
      // element a holds key key0 + 8 half + kperm(8 (a / 4) + a % 4)
      const int L = (node ? node_keys : my_i + 1) - key0 - 8 * half;
#pragma unroll
      for (int a = 0; a < 16; ++a) {
        const int kc = kperm(8 * (a >> 2) + (a & 3));
        if (kc >= L) sacc[a] = -INFINITY;
      }
    }
    // The running maximum moves only when a row's tile maximum exceeds it by
    // more than 8 (probabilities up to 2^8 against it are exact in the fp32
    // sums and lose nothing in bf16), so the rescale of the accumulator is
    // skipped on most tiles; m_run starts at a finite floor, so exp2 of a
    // masked score is 0 and no -inf arithmetic needs a guard. The test
    // compares the unscaled maximum with m_thr = (m_run + 8) / scale (set
    // whenever m_run moves).
    const float traw = tile_row_max(sacc);
    const bool grow = traw > m_thr;
    if (__builtin_amdgcn_ballot_w64(grow)) {
      const float m_new = grow ? traw * p.scale_log2 : m_run;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      m_thr = (m_run + 8.0f) * inv_scale;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int a = 0; a < 16; ++a) acc_o[db][a] *= alpha;
    }
#pragma unroll
    for (int a = 0; a < 16; ++a)
      sacc[a] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[a], p.scale_log2, -m_run));

    // ---- O^T += V^T P^T over the tile's two 16-key steps ---------------------
#pragma unroll
    for (int pt = 0; pt < 2; ++pt) {
      bf16x8_t pf;
#pragma unroll
      for (int e = 0; e < 8; ++e) pf[e] = (__bf16)sacc[8 * pt + e];
      l_run = add_row_sum(pf, l_run);
      if constexpr (node) {
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const bf16x8_t vf = *reinterpret_cast<const bf16x8_t*>(
              st_base + HALF + pt * 4096 + db * 1024 + vbase);
          acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, acc_o[db], 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          ts16x4 part[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            auto a = (__attribute__((address_space(3))) ts16x4*)(
                (__attribute__((address_space(3))) uint8_t*)(
                    (const __attribute__((address_space(3))) void*)(st_base + HALF)) +
                (16 * pt + 4 * u) * 256 + (tr_off ^ (uint32_t)(64 * db)));
            part[u] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(a);
          }
          const ts16x4 x0 = part[0], x1 = part[1];
          typedef short ts16x8 __attribute__((ext_vector_type(8)));
          const ts16x8 both = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
          const bf16x8_t vf = __builtin_bit_cast(bf16x8_t, both);
          acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, acc_o[db], 0, 0, 0);
          // 16 wait states before anything may reuse vf's registers: without
          // them the next ds_read_b64_tr_b16 refilling these registers
          // corrupted this MFMA's A operand (wrong, run-to-run varying
          // results on gfx950; the ds_read_b128 fragments of the node path
          // never showed it). The padding sits inside the MFMA's own
          // 32-cycle issue window.
          __builtin_amdgcn_sched_barrier(0);
          asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    // the page id of node tile t+3 by a scalar load, last (as attn_paged_kernel)
    pg_next = (r >= 0 && t + 3 < n1)
                  ? ((const __attribute__((address_space(4))) int32_t*)(uintptr_t)(p.table))[
                        tab_off(t + 3) / 4]
                  : 0;
  };
  int stage = 0;
  for (int t = 0; t < n1; ++t, stage = stage == NST - 1 ? 0 : stage + 1)
    tile(t, __builtin_amdgcn_readfirstlane(stage), std::true_type{});
  for (int t = n1; t < n_tiles; ++t, stage = stage == NST - 1 ? 0 : stage + 1)
    tile(t, __builtin_amdgcn_readfirstlane(stage), std::false_type{});
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no DMA outlives the workgroup

  // ---- epilogue -------------------------------------------------------------
  const float l_tot = xor32_sum(l_run);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  const long qi = (long)ep_row0 + col;
  if constexpr (FP8OUT) {
    float amax = 0.f;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int a = 0; a < 16; a += 2) {
        float v0 = acc_o[db][a] * inv, v1 = acc_o[db][a + 1] * inv;
        round_bf16_pair(v0, v1);
        acc_o[db][a] = v0;
        acc_o[db][a + 1] = v1;
        amax = fmaxf(amax, fabsf(v0));
        amax = fmaxf(amax, fabsf(v1));
      }
    amax = xor32_max(amax);
    // the output parameters, read here (late_params: not held across the loop)
    const auto* E = late_params<TreeParams>();
    const float scale = group_scale(amax, E->ue8m0 != 0);
    const double rinv = recip_exact(scale);
    uint32_t w[4][4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        w[db][g] = quant_e4m3_x4(acc_o[db][4 * g], acc_o[db][4 * g + 1], acc_o[db][4 * g + 2],
                                 acc_o[db][4 * g + 3], rinv);
    // every wave is past its last read of the stages (and every DMA landed)
    // before the stages become staging rows
    wg_barrier();
    store_fp8_rows(lds + ep_stage, w, lane,
                   E->out_q + (long)ep_row0 * E->ld_out_q + (long)ep_hq * D, E->ld_out_q,
                   ep_rows);
    if (col >= ep_rows) return;
    if (half == 0) E->out_scales[(long)ep_hq * E->n_rows + qi] = scale;
  } else {
    if (col >= ep_rows) return;
    const auto* E = late_params<TreeParams>();
    uint16_t* op = E->out + qi * E->ldo + (long)ep_hq * D;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * db + 8 * g + 4 * half;
        uint32_t w0 = f32_to_bf16(acc_o[db][4 * g + 0] * inv) |
                      (f32_to_bf16(acc_o[db][4 * g + 1] * inv) << 16);
        uint32_t w1 = f32_to_bf16(acc_o[db][4 * g + 2] * inv) |
                      (f32_to_bf16(acc_o[db][4 * g + 3] * inv) << 16);
        *reinterpret_cast<uint2*>(op + d) = make_uint2(w0, w1);
      }
  }
}

// Tree attention with each node's K and V^T resident in LDS: the result of
// attn_tree_kernel (every causal segment attends its node in full and its
// own rows causally, under one softmax), organised so that a node is moved
// into LDS once per workgroup for all the q-tiles of the workgroup that read
// it, instead of once per q-tile.
//
// One 8-wave workgroup per CU, persistent: waves 0-3 take rows 0-31 and
// waves 4-7 rows 32-63 of a 64-row q-tile, each wave one of the 4 query
// heads of head group hy = w % n_hy (two waves per SIMD). Workgroup w walks
// the q-tiles whose work (the seg_cost scan) falls in the (w / n_hy)-th of W
// equal parts, in segment order, heaviest q-tile of a segment first. LDS holds RES = 8
// stages of 16 KiB (a 32-key tile's K and V^T, laid out as a DMA stage of
// attn_tree_kernel) for node keys 0..255, and a RING = 2 stage ring for the
// rest: node keys past 256 (from their pages) and the q-tile's own rows.
// When a q-tile reads another node than the one resident, its first 8
// tiles are loaded (one wait, one barrier) and the V^T slots past the end of
// a partial last page are zeroed once. The resident tiles then need no DMA,
// wait or barrier; the streamed tiles use the ring with one barrier each,
// their DMA one tile ahead (the first two are issued before the resident
// phase). The epilogue stages its fp8 rows in the ring.
template <bool FP8OUT>
__global__ __launch_bounds__(512, 1) void attn_tree_node_kernel(TreeParams p) {
  using namespace pattn;
  using ntree::QROWS;
  using ntree::RES;
  using ntree::RING;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[(RES + RING) * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rh = wave >> 2;  // row half of the q-tile
  const int half = lane >> 5;
  const int col = lane & 31;

  // ---- this workgroup's run of q-tiles -------------------------------------
  const int n_hy = p.n_q / HPW;
  const int W = (int)gridDim.x / n_hy;
  const int hy = (int)blockIdx.x % n_hy;
  const int wj = (int)blockIdx.x / n_hy;
  if (wj >= W) return;
  const int group = udiv_uniform(p.n_q, p.n_kv);
  const int hq = hy * HPW + (wave & 3);
  const int hk = udiv_uniform(hy * HPW, group);
  const long long C = p.seg_cost[p.n_seg];
  const int total = p.tile_off[p.n_seg];
  auto node_of = [&](int s) __attribute__((always_inline)) {
    const int r = p.seg_read[s];
    return (r >= 0 && r < p.n_reads) ? r : -1;
  };
  // the first q-tile (index into the tile_off numbering) whose work starts
  // at or after `target`
  auto first_item = [&](long long target) __attribute__((always_inline)) {
    if (target >= C) return total;
    const int s = last_le<long long>(p.seg_cost, p.n_seg + 1, target, lane);
    const int count = p.cu_a[s + 1] - p.cu_a[s];
    const int n_qt = (count + QROWS - 1) / QROWS;
    const int r = node_of(s);
    const long long per = (long long)(r >= 0 ? max(0, p.read_used[r]) : 0) + ntree::ITEM_KEYS;
    const long long c0 = p.seg_cost[s];
    int j = 0;
    while (j < n_qt) {
      const long long e =
          c0 + (long long)j * per +
          (j > 0 ? count + (long long)QROWS * ((long long)(j - 1) * n_qt - (long long)(j - 1) * j / 2)
                 : 0LL);
      if (e >= target) break;
      ++j;
    }
    return p.tile_off[s] + j;
  };
  const int k0 = first_item(C * wj / W);
  const int k1 = first_item(C * (wj + 1) / W);
  if (k0 >= k1) return;

  // ---- DMA roles, as attn_tree_kernel with the work halved: wave (region,
  // pit, sub) moves pieces 2 sub and 2 sub + 1 (1 KiB each) of K (region 0)
  // or V (region 1) of keys 16 pit .. 16 pit + 15 of a tile; the lane
  // offsets are loop-invariant (computed from the lane id at each DMA
  // instead, the kernel measured 4 % slower)
  const int region = (wave >> 1) & 1;
  const int pit = wave & 1;
  const int sub = wave >> 2;
  const uint32_t row_bytes = (uint32_t)p.ld_kv * 2u;
  uint32_t vo_node[2], vo_own[2];
  {
    const int l16 = lane >> 4;
    const int pc = lane & 15;
    const uint32_t k_chunk = (uint32_t)((pc ^ l16 ^ pit) * 16);
    const uint32_t own_v_chunk = (uint32_t)((pc ^ (4 * l16)) * 16);
    const uint32_t node_v_off = (uint32_t)((lane >> 1) * 32 + (((lane & 1) ^ (l16 & 1)) * 16));
    const uint32_t own_row = (uint32_t)l16 * row_bytes + (uint32_t)hk * 256u;
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
      const int c = 2 * sub + cc;
      vo_node[cc] = region == 0 ? (uint32_t)((4 * c + l16) * 256) + (k_chunk ^ (uint32_t)(64 * c))
                                : node_v_off + (uint32_t)(1024 * c);
      vo_own[cc] = own_row + (uint32_t)(4 * c) * row_bytes +
                   (region == 0 ? (k_chunk ^ (uint32_t)(64 * c)) : own_v_chunk);
    }
  }
  const uint16_t* pool = region ? p.v_pool : p.k_pool;
  const uint16_t* own_rows = region ? p.v_rows : p.k_rows;
  const __attribute__((address_space(4))) int32_t* tab =
      (const __attribute__((address_space(4))) int32_t*)(uintptr_t)(p.table);
  const pi32x4 rq = attn_rsrc(p.q, (uint32_t)((long)p.n_rows * p.ldq * 2));

  // ---- fragment addressing (as attn_tree_kernel) ---------------------------
  const int kq = kperm(col);
  const int ksw = kswz(kq);
  const uint32_t kbase = (uint32_t)(kq * 256 + ((half ^ (ksw & 1)) * 16));
  const uint32_t kx = (uint32_t)((ksw >> 1) * 32);
  const uint32_t vbase = (uint32_t)(col * 32 + ((half ^ ((col >> 3) & 1)) * 16));
  const int gi = lane & 15;
  const int tr_key = 8 * (lane >> 5) + (gi >> 2);
  const uint32_t tr_off = (uint32_t)(tr_key * 256 +
                                     (((2 * ((lane >> 4) & 1) + ((gi & 3) >> 1)) ^ vswz(tr_key)) * 16) +
                                     (gi & 1) * 8);
  const float inv_scale = __builtin_amdgcn_rcpf(p.scale_log2);

  f32x16 acc_o[4];
  float m_run, l_run, m_thr;
  bf16x8_t qf[8];
  // One 32-key tile from LDS at st_base: S^T = K Q^T, mask, online softmax,
  // O^T += V^T P^T. NODE selects the P.V operand form: a node tile holds
  // V^T rows (ds_read_b128), an own tile V rows (ds_read_b64_tr_b16).
  auto compute = [&](const uint8_t* st_base, bool need_mask, int L, auto node_c)
      __attribute__((always_inline)) {
    constexpr bool node = decltype(node_c)::value;
    f32x16 sacc;
#pragma unroll
    for (int a = 0; a < 16; ++a) sacc[a] = 0.f;
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const bf16x8_t af = *reinterpret_cast<const bf16x8_t*>(
          st_base + (kbase + (((uint32_t)(32 * st)) ^ kx)));
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, qf[st], sacc, 0, 0, 0);
    }
    if (need_mask) {
      // element a holds key key0 + 8 half + kperm(8 (a / 4) + a % 4); L is
      // the number of visible keys from key0 + 8 half on
#pragma unroll
      for (int a = 0; a < 16; ++a) {
        const int kc = kperm(8 * (a >> 2) + (a & 3));
        if (kc >= L) sacc[a] = -INFINITY;
      }
    }
    // the running maximum moves only past m_run + 8 (see attn_tree_kernel)
    const float traw = tile_row_max(sacc);
    const bool grow = traw > m_thr;
    if (__builtin_amdgcn_ballot_w64(grow)) {
      const float m_new = grow ? traw * p.scale_log2 : m_run;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      m_thr = (m_run + 8.0f) * inv_scale;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int a = 0; a < 16; ++a) acc_o[db][a] *= alpha;
    }
#pragma unroll
    for (int a = 0; a < 16; ++a)
      sacc[a] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[a], p.scale_log2, -m_run));
#pragma unroll
    for (int pt = 0; pt < 2; ++pt) {
      bf16x8_t pf;
#pragma unroll
      for (int e = 0; e < 8; ++e) pf[e] = (__bf16)sacc[8 * pt + e];
      l_run = add_row_sum(pf, l_run);
      if constexpr (node) {
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const bf16x8_t vf = *reinterpret_cast<const bf16x8_t*>(
              st_base + HALF + pt * 4096 + db * 1024 + vbase);
          acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, acc_o[db], 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          ts16x4 part[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            auto a = (__attribute__((address_space(3))) ts16x4*)(
                (__attribute__((address_space(3))) uint8_t*)(
                    (const __attribute__((address_space(3))) void*)(st_base + HALF)) +
                (16 * pt + 4 * u) * 256 + (tr_off ^ (uint32_t)(64 * db)));
            part[u] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(a);
          }
          const ts16x4 x0 = part[0], x1 = part[1];
          typedef short ts16x8 __attribute__((ext_vector_type(8)));
          const ts16x8 both = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
          const bf16x8_t vf = __builtin_bit_cast(bf16x8_t, both);
          acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, acc_o[db], 0, 0, 0);
          // the wait states attn_tree_kernel needs after this MFMA before
          // its A-operand registers are refilled
          __builtin_amdgcn_sched_barrier(0);
          asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  };

  // Zero the V^T slots of a partial last node page (the one holding key
  // node_keys - 1, in the tile at st_base that starts at key0): a masked key
  // has P = 0, and 0 times a NaN left in the arena would still be NaN.
  auto zero_tail = [&](uint8_t* st_base, int key0, int node_keys) __attribute__((always_inline)) {
    const int zpit = (node_keys - key0) >> 4;
    const int valid = node_keys & (PAGE - 1);
    if (zpit < 2 && tid < 256) {
      const int d = tid >> 1, ph = tid & 1;
      const int lh = ph ^ ((d >> 3) & 1);
      uint16_t* vp = reinterpret_cast<uint16_t*>(st_base + HALF + zpit * 4096 + d * 32 + ph * 16);
      bf16x8 v = load8(vp);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (8 * lh + e >= valid) v.set(e, 0);
      store8(vp, v);
    }
  };

  int s = tile_seq(p.tile_off, p.n_seg, k0, lane);
  int cur_r = -2;  // the node resident in stages 0 .. RES-1 (-2: none yet)
  for (int k = k0; k < k1; ++k) {
    while (p.tile_off[s + 1] <= k) ++s;
    const int q0 = p.cu_a[s];
    const int count = p.cu_a[s + 1] - q0;
    const int n_qt = (count + QROWS - 1) / QROWS;
    const int i0 = (n_qt - 1 - (k - p.tile_off[s])) * QROWS;
    const int i0w = i0 + 32 * rh;  // this wave's first row
    const bool live_w = i0w < count;
    const int r = node_of(s);
    const int node_keys = r >= 0 ? max(0, p.read_used[r]) : 0;
    const int n1 = (node_keys + BKV - 1) / BKV;
    const int nres = min(n1, RES);
    const int own_keys = min(count, i0 + QROWS);
    const int n_tiles = n1 + (own_keys + BKV - 1) / BKV;
    const int n_str = n_tiles - nres;
    const int my_i = i0w + col;
    const long tab_row = (long)(r >= 0 ? r : 0) * p.table_width;
    auto page_of = [&](int t) __attribute__((always_inline)) {
      return (r >= 0 && t < n1) ? tab[tab_row + min(2 * t + pit, p.table_width - 1)] : -1;
    };
    // this wave's four DMA pieces of tile t (of this q-tile's sequence: node
    // tiles, then own tiles) into stage stg
    auto dma_tile = [&](int t, int page_id, int stg) __attribute__((always_inline)) {
      const uint32_t base =
          (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)(
              lds + stg * STAGE + region * HALF + pit * 4096 + 2048 * sub);
      if (t < n1) {
        const int pidx = 2 * t + pit;
        const bool live = pidx < p.table_width && pidx * PAGE < node_keys && page_id >= 0 &&
                          page_id < p.pool_pages;
        const int slots = live ? min(PAGE, node_keys - pidx * PAGE) : 0;
        const uint32_t bytes = region ? (live ? 4096u : 0u) : (uint32_t)slots * 256u;
        const uint16_t* blk = pool + ((long)(live ? page_id : 0) * p.n_kv + hk) * (PAGE * D);
        const pi32x4 rs = attn_rsrc(blk, bytes);
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
          asm volatile(
              "s_mov_b32 m0, %0\n\t"
              "buffer_load_dwordx4 %1, %2, 0 offen lds"
              :
              : "s"(base + 1024 * cc), "v"(vo_node[cc]), "s"(rs)
              : "memory", "m0");
      } else {
        // own keys 32 (t - n1) + 16 pit + 0..15: chunk rows q0 + those keys;
        // rows past the chunk (or past the tiles) read zero
        const long row0 = (long)q0 + 32L * (t - n1) + 16 * pit;
        const bool live = t < n_tiles && row0 < p.n_rows;
        const long rows_left = live ? (long)p.n_rows - row0 : 0;
        const pi32x4 rs = attn_rsrc(own_rows + (live ? row0 : 0) * p.ld_kv,
                                    (uint32_t)(rows_left * (long)row_bytes));
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
          asm volatile(
              "s_mov_b32 m0, %0\n\t"
              "buffer_load_dwordx4 %1, %2, 0 offen lds"
              :
              : "s"(base + 1024 * cc), "v"(vo_own[cc]), "s"(rs)
              : "memory", "m0");
      }
    };

    // ---- Q: lane holds Q[query col][16*st + 8*half .. +7] -------------------
    typedef int qi32x4 __attribute__((ext_vector_type(4)));
    qi32x4 qraw[8];
    {
      const long row = (long)q0 + my_i;
      const bool ok = my_i < count && row < p.n_rows;
      const uint32_t qoff = ok ? (uint32_t)(row * p.ldq * 2 + (long)hq * D * 2 + 16 * half)
                               : 0x80000000u;
      // s_nop 4 first: the descriptor may come from an SGPR the compiler
      // restores by v_readlane just before (a VALU write that a VMEM read
      // needs 5 wait states after, which the compiler does not insert
      // ahead of inline asm)
#pragma unroll
      for (int st = 0; st < 8; ++st)
        asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2, 0 offen offset:%3"
                     : "=v"(qraw[st]) : "v"(qoff), "s"(rq), "i"(32 * st) : "memory");
    }

    // ---- the node's first RES tiles into LDS, unless already there ----------
    if (r != cur_r) {
      for (int t = 0; t < nres; ++t) dma_tile(t, page_of(t), t);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      wg_barrier();
      if ((node_keys & (PAGE - 1)) != 0 && (node_keys - 1) / BKV < RES) {
        const int tl = (node_keys - 1) / BKV;
        zero_tail(lds + tl * STAGE, tl * BKV, node_keys);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        wg_barrier();
      }
      cur_r = r;
    }

    // ---- the first two streamed tiles into the ring ------------------------
    dma_tile(nres, page_of(nres), RES);
    dma_tile(nres + 1, page_of(nres + 1), RES + 1);
    asm volatile("s_waitcnt vmcnt(4)" ::: "memory");  // Q landed
    asm volatile("" : "+v"(qraw[0]), "+v"(qraw[1]), "+v"(qraw[2]), "+v"(qraw[3]),
                 "+v"(qraw[4]), "+v"(qraw[5]), "+v"(qraw[6]), "+v"(qraw[7]));
#pragma unroll
    for (int st = 0; st < 8; ++st) qf[st] = __builtin_bit_cast(bf16x8_t, qraw[st]);
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int a = 0; a < 16; ++a) acc_o[db][a] = 0.f;
    m_run = -1e30f;  // finite floor: see attn_tree_kernel
    l_run = 0.f;
    m_thr = (m_run + 8.0f) * inv_scale;

    // ---- resident node tiles: no DMA, no wait, no barrier --------------------
    if (live_w) {
      for (int t = 0; t < nres; ++t) {
        const int key0 = t * BKV;
        compute(lds + t * STAGE, key0 + BKV > node_keys, node_keys - key0 - 8 * half,
                std::true_type{});
      }
    }

    // ---- streamed tiles: node tiles past RES, then own tiles -----------------
    int pg_next = page_of(nres + 2);
    for (int u = 0; u < n_str; ++u) {
      const int t = nres + u;
      if (u == 0)
        asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      // tile u visible to all; everyone is past tile u - 1, whose stage the
      // DMA of tile u + 1 now refills
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      wg_barrier();
      if (u >= 1) {
        dma_tile(t + 1, pg_next, RES + ((u + 1) & 1));
        pg_next = page_of(t + 2);
      }
      uint8_t* st_base = lds + (RES + (u & 1)) * STAGE;
      if (t < n1) {
        const int key0 = t * BKV;
        if (key0 + BKV > node_keys && (node_keys & (PAGE - 1)) != 0) {
          zero_tail(st_base, key0, node_keys);
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          wg_barrier();
        }
        if (live_w)
          compute(st_base, key0 + BKV > node_keys, node_keys - key0 - 8 * half,
                  std::true_type{});
      } else {
        // own tiles wholly past this wave's rows are skipped (all masked)
        const int key0 = (t - n1) * BKV;
        if (live_w && key0 <= i0w + 31)
          compute(st_base, key0 + BKV - 1 > i0w, my_i + 1 - key0 - 8 * half, std::false_type{});
      }
    }
    // every DMA of this q-tile landed (also the unused second prefetch) and
    // every wave is past its last read of the ring before it stages rows
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    wg_barrier();

    // ---- epilogue -----------------------------------------------------------
    const float l_tot = xor32_sum(l_run);
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    const long qi = q0 + my_i;
    if constexpr (FP8OUT) {
      float amax = 0.f;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int a = 0; a < 16; a += 2) {
          float v0 = acc_o[db][a] * inv, v1 = acc_o[db][a + 1] * inv;
          round_bf16_pair(v0, v1);
          acc_o[db][a] = v0;
          acc_o[db][a + 1] = v1;
          amax = fmaxf(amax, fabsf(v0));
          amax = fmaxf(amax, fabsf(v1));
        }
      amax = xor32_max(amax);
      // the output parameters, read here (late_params: not held across the loop)
      const auto* E = late_params<TreeParams>();
      const float scale = group_scale(amax, E->ue8m0 != 0);
      const double rinv = recip_exact(scale);
      uint32_t w[4][4];
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          w[db][g] = quant_e4m3_x4(acc_o[db][4 * g], acc_o[db][4 * g + 1], acc_o[db][4 * g + 2],
                                   acc_o[db][4 * g + 3], rinv);
      uint8_t* const out_rows = E->out_q + (long)(q0 + i0w) * E->ld_out_q + (long)hq * D;
      // the ring holds the staging rows of 4 waves at a time
      if (rh == 0)
        store_fp8_rows(lds + RES * STAGE + (wave & 3) * 32 * 144, w, lane, out_rows,
                       E->ld_out_q, count - i0w);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      wg_barrier();
      if (rh == 1)
        store_fp8_rows(lds + RES * STAGE + (wave & 3) * 32 * 144, w, lane, out_rows,
                       E->ld_out_q, count - i0w);
      if (my_i < count && half == 0) E->out_scales[(long)hq * E->n_rows + qi] = scale;
    } else {
      if (my_i < count) {
        const auto* E = late_params<TreeParams>();
        uint16_t* op = E->out + qi * E->ldo + (long)hq * D;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int d = 32 * db + 8 * g + 4 * half;
            uint32_t w0 = f32_to_bf16(acc_o[db][4 * g + 0] * inv) |
                          (f32_to_bf16(acc_o[db][4 * g + 1] * inv) << 16);
            uint32_t w1 = f32_to_bf16(acc_o[db][4 * g + 2] * inv) |
                          (f32_to_bf16(acc_o[db][4 * g + 3] * inv) << 16);
            *reinterpret_cast<uint2*>(op + d) = make_uint2(w0, w1);
          }
      }
    }
    // the staged rows are read back before the next q-tile's DMA refills the ring
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    wg_barrier();
  }
}

}  // namespace qh

using namespace qh;

// tile_off [n_seqs + 1] int32, then (node-resident tree calls) seg_cost
// [n_seqs + 1] int64 at the next 16-byte boundary. The paged and streaming
// calls use tile_off only (paged_workspace_bytes); the query returns what
// every call needs.
static size_t seg_cost_offset(int n_seqs) {
  return ((size_t)(n_seqs + 1) * sizeof(int32_t) + 15) & ~(size_t)15;
}
static size_t paged_workspace_bytes(int n_seqs) {
  return (size_t)(n_seqs + 1) * sizeof(int32_t) + 256;
}
extern "C" size_t qh_attention_workspace_bytes(int n_seqs) {
  return seg_cost_offset(n_seqs) + (size_t)(n_seqs + 1) * sizeof(long long) + 256;
}

// Shared by qh_attention and qh_attention_fp8: checks, tile scan, launch.
static int attention_launch(const void* q, long ldq, int q_rows_total, const int64_t* q_rows,
                            const void* k_pool, const void* v_pool, int pool_pages,
                            const int32_t* table, int table_width, int page_tokens,
                            const void* k_rows, const void* v_rows, int kv_rows_total,
                            const int32_t* cu_k, const int32_t* cu_q, const int32_t* kv_len,
                            int n_seqs, int n_queries, int max_q, int n_q, int n_kv, int d,
                            float softmax_scale, int causal, void* out, long ldo, float* lse,
                            long lse_stride, void* out_q, long ld_out_q, float* out_scales,
                            int ue8m0, void* workspace, size_t workspace_bytes,
                            qh_stream_t stream) {
  QH_REQUIRE(d == attn::D, "attention: head_dim %d unsupported (128 only)", d);
  QH_REQUIRE(n_q > 0 && n_kv > 0 && n_q % n_kv == 0 && (n_q / n_kv) % attn::HPW == 0,
             "attention: n_q=%d n_kv=%d needs a GQA group that is a multiple of 4", n_q, n_kv);
  QH_REQUIRE(n_seqs >= 0 && n_queries >= 0 && max_q >= 0, "attention: negative sizes");
  if (n_seqs == 0 || n_queries == 0) return QH_OK;
  // the kernels index their workgroups (q-tile bound x head groups) in 32 bits
  QH_REQUIRE(((long)n_queries / attn::BQ + n_seqs) * (n_q / attn::HPW) < (1L << 31),
             "attention: %d queries in %d sequences x %d heads exceed 2^31 workgroups",
             n_queries, n_seqs, n_q);
  const bool fp8 = out_q != nullptr;
  QH_REQUIRE(q && cu_q && kv_len && (fp8 ? out_scales != nullptr : out != nullptr),
             "attention: null pointer");
  QH_REQUIRE(ldq >= (long)n_q * d && ldq % 8 == 0, "attention: row stride ldq=%ld", ldq);
  if (fp8)
    QH_REQUIRE(ld_out_q >= (long)n_q * d && ld_out_q % 16 == 0,
               "attention: fp8 row stride %ld", ld_out_q);
  else
    QH_REQUIRE(ldo >= (long)n_q * d && ldo % 8 == 0, "attention: row stride ldo=%ld", ldo);
  const bool paged = table != nullptr;
  if (paged) {
    QH_REQUIRE(k_pool && v_pool && pool_pages > 0 && table_width > 0,
               "attention: paged call without pools/table");
    // the paged kernel addresses q and the table through 32-bit buffer offsets
    QH_REQUIRE((long)q_rows_total * ldq * 2 < 0x80000000L &&
                   (long)n_seqs * table_width * 4 < 0x80000000L,
               "attention: q (%d rows) or page table exceeds 2 GiB", q_rows_total);
    QH_REQUIRE(page_tokens == attn::PAGE, "attention: page_tokens %d unsupported (16 only)",
               page_tokens);
  } else {
    QH_REQUIRE(!fp8, "attention: fp8 output needs the paged path");
    QH_REQUIRE(k_rows && v_rows && cu_k && kv_rows_total > 0,
               "attention: contiguous call without k_rows/v_rows/cu_k");
  }
  QH_REQUIRE(workspace && workspace_bytes >= paged_workspace_bytes(n_seqs),
             "attention: workspace of %zu bytes needed", paged_workspace_bytes(n_seqs));
  QH_REQUIRE(((uintptr_t)workspace & 15) == 0, "attention: workspace must be 16-byte aligned");
  int32_t* tile_off = (int32_t*)workspace;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(attn_tile_scan_kernel, dim3(1), dim3(1024), 0, st, cu_q, n_seqs, tile_off);
  int rc = launch_status("attention tile scan");
  if (rc) return rc;

  AttnParams p;
  p.q = (const uint16_t*)q;
  p.ldq = ldq;
  p.q_rows_total = q_rows_total;
  p.q_rows = q_rows;
  p.k_pool = (const uint16_t*)k_pool;
  p.v_pool = (const uint16_t*)v_pool;
  p.pool_pages = pool_pages;
  p.table = table;
  p.table_width = table_width;
  p.k_rows = (const uint16_t*)k_rows;
  p.v_rows = (const uint16_t*)v_rows;
  p.kv_rows_total = kv_rows_total;
  p.cu_k = cu_k;
  p.cu_q = cu_q;
  p.kv_len = kv_len;
  p.n_seqs = n_seqs;
  p.n_q = n_q;
  p.n_kv = n_kv;
  p.scale_log2 = softmax_scale * 1.4426950408889634f;
  p.out = (uint16_t*)out;
  p.ldo = ldo;
  p.lse = lse;
  p.lse_stride = lse_stride;
  p.tile_off = tile_off;
  p.out_q = (uint8_t*)out_q;
  p.ld_out_q = ld_out_q;
  p.out_scales = out_scales;
  p.n_out = n_queries;
  p.ue8m0 = ue8m0;
  // upper bound on the q-tiles: sum ceil(c/32) <= n_queries/32 + n_seqs
  const long max_tiles = (long)n_queries / attn::BQ + n_seqs;
  dim3 grid((unsigned)max_tiles, (unsigned)(n_q / attn::HPW));
  if (paged) {
    if (fp8) {
      if (causal) hipLaunchKernelGGL((attn_paged_kernel<true, true>), grid, dim3(256), 0, st, p);
      else hipLaunchKernelGGL((attn_paged_kernel<false, true>), grid, dim3(256), 0, st, p);
    } else {
      if (causal) hipLaunchKernelGGL((attn_paged_kernel<true, false>), grid, dim3(256), 0, st, p);
      else hipLaunchKernelGGL((attn_paged_kernel<false, false>), grid, dim3(256), 0, st, p);
    }
  } else {
    if (causal) hipLaunchKernelGGL((attn_fwd_kernel<true>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((attn_fwd_kernel<false>), grid, dim3(256), 0, st, p);
  }
  return launch_status("attention");
}

extern "C" int qh_attention(const void* q, long ldq, int q_rows_total, const int64_t* q_rows,
                            const void* k_pool, const void* v_pool, int pool_pages,
                            const int32_t* table, int table_width, int page_tokens,
                            const void* k_rows, const void* v_rows, int kv_rows_total,
                            const int32_t* cu_k, const int32_t* cu_q, const int32_t* kv_len,
                            int n_seqs, int n_queries, int max_q, int n_q, int n_kv, int d,
                            float softmax_scale, int causal, void* out, long ldo, float* lse,
                            long lse_stride, void* workspace, size_t workspace_bytes,
                            qh_stream_t stream) {
  return attention_launch(q, ldq, q_rows_total, q_rows, k_pool, v_pool, pool_pages, table,
                          table_width, page_tokens, k_rows, v_rows, kv_rows_total, cu_k, cu_q,
                          kv_len, n_seqs, n_queries, max_q, n_q, n_kv, d, softmax_scale, causal,
                          out, ldo, lse, lse_stride, nullptr, 0, nullptr, 0, workspace,
                          workspace_bytes, stream);
}

extern "C" int qh_attention_fp8(const void* q, long ldq, int q_rows_total,
                                const int64_t* q_rows, const void* k_pool, const void* v_pool,
                                int pool_pages, const int32_t* table, int table_width,
                                int page_tokens, const int32_t* cu_q, const int32_t* kv_len,
                                int n_seqs, int n_queries, int max_q, int n_q, int n_kv, int d,
                                float softmax_scale, int causal, void* out_q, long ld_out_q,
                                float* scales, int ue8m0, void* workspace,
                                size_t workspace_bytes, qh_stream_t stream) {
  QH_REQUIRE(n_seqs == 0 || n_queries == 0 || (table && out_q && scales),
             "attention_fp8: paged call needs table, out_q, scales");
  return attention_launch(q, ldq, q_rows_total, q_rows, k_pool, v_pool, pool_pages, table,
                          table_width, page_tokens, nullptr, nullptr, 0, nullptr, cu_q, kv_len,
                          n_seqs, n_queries, max_q, n_q, n_kv, d, softmax_scale, causal,
                          nullptr, 0, nullptr, 0, out_q, ld_out_q, scales, ue8m0, workspace,
                          workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// qh_attention_fp8_noalloc: qh_attention_fp8 with its q-tile scan in a
// file-scope device array instead of a caller workspace, for callers that
// cannot allocate. Each GPU holds its own copy of `scratch` (512 KiB) until
// the process ends; its address on a device is looked up once, with that
// device current, and kept per device. The scan kernel writes every entry
// a launch reads (tile_off[0..n_seqs]), so nothing needs clearing between
// calls. Calls that overlap on one GPU (two streams, two host threads)
// share the array and race.
namespace {

constexpr int kScratchSeqs = 131072;               // sequences one call may carry
constexpr int kScratchWords = kScratchSeqs + 128;  // + the scan's total and 256 B slack

__device__ __align__(256) int32_t scratch[kScratchWords];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
int32_t* g_scratch_ptr[kMaxDevices] = {};

// The current device's copy of `scratch` (its device address), looked up once.
int scratch_on_current_device(int32_t** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) {
    set_error("attention_fp8_noalloc: hipGetDevice failed: %s", hipGetErrorString(err));
    return QH_E_HIP;
  }
  QH_REQUIRE(dev >= 0 && dev < kMaxDevices, "attention_fp8_noalloc: device %d out of range",
             dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr) {
      set_error("attention_fp8_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                dev, hipGetErrorString(err));
      return QH_E_HIP;
    }
    g_scratch_ptr[dev] = static_cast<int32_t*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return QH_OK;
}

}  // namespace

extern "C" int qh_attention_fp8_noalloc(const void* q, long ldq, int q_rows_total,
                                        const int64_t* q_rows, const void* k_pool,
                                        const void* v_pool, int pool_pages,
                                        const int32_t* table, int table_width,
                                        int page_tokens, const int32_t* cu_q,
                                        const int32_t* kv_len, int n_seqs, int n_queries,
                                        int max_q, int n_q, int n_kv, int d,
                                        float softmax_scale, int causal, void* out_q,
                                        long ld_out_q, float* scales, int ue8m0,
                                        qh_stream_t stream) {
  QH_REQUIRE(n_seqs >= 0 && n_seqs <= kScratchSeqs,
             "attention_fp8_noalloc: %d sequences; the static scratch holds at most %d",
             n_seqs, kScratchSeqs);
  int32_t* ws = nullptr;
  const int rc = scratch_on_current_device(&ws);
  if (rc) return rc;
  return qh_attention_fp8(q, ldq, q_rows_total, q_rows, k_pool, v_pool, pool_pages, table,
                          table_width, page_tokens, cu_q, kv_len, n_seqs, n_queries, max_q,
                          n_q, n_kv, d, softmax_scale, causal, out_q, ld_out_q, scales, ue8m0,
                          ws, (size_t)kScratchWords * sizeof(int32_t), stream);
}

// Shared by qh_tree_attention (streaming kernel) and
// qh_tree_attention_resident (node-resident kernel): checks, scan, launch.
static int tree_attention_launch(const void* q, long ldq, int n_rows, const void* k_rows,
                                 const void* v_rows, long ld_kv, const int32_t* cu_a,
                                 const int32_t* seg_read, int n_seg, const void* k_pool,
                                 const void* v_pool, int pool_pages, const int32_t* table,
                                 int table_width, const int32_t* read_used, int n_reads,
                                 int page_tokens, int n_q, int n_kv, int d,
                                 float softmax_scale, void* out, long ldo, void* out_q,
                                 long ld_out_q, float* scales, int ue8m0, void* workspace,
                                 size_t workspace_bytes, qh_stream_t stream, bool resident) {
  QH_REQUIRE(d == attn::D, "tree_attention: head_dim %d unsupported (128 only)", d);
  QH_REQUIRE(n_q > 0 && n_kv > 0 && n_q % n_kv == 0 && (n_q / n_kv) % attn::HPW == 0,
             "tree_attention: n_q=%d n_kv=%d needs a GQA group that is a multiple of 4",
             n_q, n_kv);
  QH_REQUIRE(n_rows >= 0 && n_seg >= 0 && n_reads >= 0, "tree_attention: negative sizes");
  if (n_rows == 0 || n_seg == 0) return QH_OK;
  // the streaming kernel indexes its workgroups (q-tile bound x head groups) in 32 bits
  QH_REQUIRE(((long)n_rows / attn::BQ + n_seg) * (n_q / attn::HPW) < (1L << 31),
             "tree_attention: %d rows in %d segments x %d heads exceed 2^31 workgroups",
             n_rows, n_seg, n_q);
  const bool fp8 = out_q != nullptr;
  QH_REQUIRE(q && k_rows && v_rows && cu_a && seg_read && (fp8 ? scales != nullptr : out != nullptr),
             "tree_attention: null pointer");
  QH_REQUIRE(ldq >= (long)n_q * d && ldq % 8 == 0, "tree_attention: row stride ldq=%ld", ldq);
  QH_REQUIRE(ld_kv >= (long)n_kv * d && ld_kv % 8 == 0, "tree_attention: row stride ld_kv=%ld",
             ld_kv);
  if (fp8)
    QH_REQUIRE(ld_out_q >= (long)n_q * d && ld_out_q % 16 == 0,
               "tree_attention: fp8 row stride %ld", ld_out_q);
  else
    QH_REQUIRE(ldo >= (long)n_q * d && ldo % 8 == 0, "tree_attention: row stride ldo=%ld", ldo);
  if (n_reads > 0)
    QH_REQUIRE(k_pool && v_pool && pool_pages > 0 && table && table_width > 0 && read_used,
               "tree_attention: reads without pools, table or used");
  QH_REQUIRE(page_tokens == attn::PAGE, "tree_attention: page_tokens %d unsupported (16 only)",
             page_tokens);
  // the kernel addresses q, the rows and the table through 32-bit buffer offsets
  QH_REQUIRE((long)n_rows * ldq * 2 < 0x80000000L && (long)n_rows * ld_kv * 2 < 0x80000000L &&
                 (long)n_reads * table_width * 4 < 0x80000000L,
             "tree_attention: q, k/v rows or page table exceed 2 GiB");
  const size_t ws_need = resident ? qh_attention_workspace_bytes(n_seg) : paged_workspace_bytes(n_seg);
  QH_REQUIRE(workspace && workspace_bytes >= ws_need, "tree_attention: workspace of %zu bytes needed",
             ws_need);
  QH_REQUIRE(((uintptr_t)workspace & 15) == 0, "tree_attention: workspace must be 16-byte aligned");
  int32_t* tile_off = (int32_t*)workspace;
  long long* seg_cost = (long long*)((char*)workspace + seg_cost_offset(n_seg));
  hipStream_t st = (hipStream_t)stream;
  if (resident) {
    QH_REQUIRE((long)table_width * page_tokens <= ntree::RES * pattn::BKV,
               "tree_attention_resident: page-table rows of %d pages exceed the %d resident keys",
               table_width, ntree::RES * pattn::BKV);
  }
  if (resident)
    hipLaunchKernelGGL(attn_tree_scan_kernel, dim3(1), dim3(1024), 0, st, cu_a, seg_read,
                       read_used, n_reads, n_seg, tile_off, seg_cost);
  else
    hipLaunchKernelGGL(attn_tile_scan_kernel, dim3(1), dim3(1024), 0, st, cu_a, n_seg, tile_off);
  int rc = launch_status("tree attention tile scan");
  if (rc) return rc;
  TreeParams p;
  p.q = (const uint16_t*)q;
  p.ldq = ldq;
  p.n_rows = n_rows;
  p.k_rows = (const uint16_t*)k_rows;
  p.v_rows = (const uint16_t*)v_rows;
  p.ld_kv = ld_kv;
  p.cu_a = cu_a;
  p.seg_read = seg_read;
  p.n_seg = n_seg;
  p.k_pool = (const uint16_t*)k_pool;
  p.v_pool = (const uint16_t*)v_pool;
  p.pool_pages = pool_pages;
  p.table = table;
  p.table_width = table_width;
  p.read_used = read_used;
  p.n_reads = n_reads;
  p.n_q = n_q;
  p.n_kv = n_kv;
  p.scale_log2 = softmax_scale * 1.4426950408889634f;
  p.out = (uint16_t*)out;
  p.ldo = ldo;
  p.out_q = (uint8_t*)out_q;
  p.ld_out_q = ld_out_q;
  p.out_scales = scales;
  p.ue8m0 = ue8m0;
  p.tile_off = tile_off;
  p.seg_cost = seg_cost;
  if (resident) {
    const int n_hy = n_q / attn::HPW;
    const int per = std::max(1, device_cus() / n_hy);
    dim3 grid((unsigned)(n_hy * per));
    if (fp8) hipLaunchKernelGGL((attn_tree_node_kernel<true>), grid, dim3(512), 0, st, p);
    else hipLaunchKernelGGL((attn_tree_node_kernel<false>), grid, dim3(512), 0, st, p);
    return launch_status("tree attention (node resident)");
  }
  // upper bound on the q-tiles: sum ceil(c/32) <= n_rows/32 + n_seg
  const long max_tiles = (long)n_rows / attn::BQ + n_seg;
  dim3 grid((unsigned)max_tiles, (unsigned)(n_q / attn::HPW));
  if (fp8) hipLaunchKernelGGL((attn_tree_kernel<true>), grid, dim3(256), 0, st, p);
  else hipLaunchKernelGGL((attn_tree_kernel<false>), grid, dim3(256), 0, st, p);
  return launch_status("tree attention");
}

extern "C" int qh_tree_attention(const void* q, long ldq, int n_rows, const void* k_rows,
                                 const void* v_rows, long ld_kv, const int32_t* cu_a,
                                 const int32_t* seg_read, int n_seg, const void* k_pool,
                                 const void* v_pool, int pool_pages, const int32_t* table,
                                 int table_width, const int32_t* read_used, int n_reads,
                                 int page_tokens, int n_q, int n_kv, int d,
                                 float softmax_scale, void* out, long ldo, void* out_q,
                                 long ld_out_q, float* scales, int ue8m0, void* workspace,
                                 size_t workspace_bytes, qh_stream_t stream) {
  return tree_attention_launch(q, ldq, n_rows, k_rows, v_rows, ld_kv, cu_a, seg_read, n_seg,
                               k_pool, v_pool, pool_pages, table, table_width, read_used,
                               n_reads, page_tokens, n_q, n_kv, d, softmax_scale, out, ldo,
                               out_q, ld_out_q, scales, ue8m0, workspace, workspace_bytes,
                               stream, false);
}

extern "C" int qh_tree_attention_resident(
    const void* q, long ldq, int n_rows, const void* k_rows, const void* v_rows, long ld_kv,
    const int32_t* cu_a, const int32_t* seg_read, int n_seg, const void* k_pool,
    const void* v_pool, int pool_pages, const int32_t* table, int table_width,
    const int32_t* read_used, int n_reads, int page_tokens, int n_q, int n_kv, int d,
    float softmax_scale, void* out, long ldo, void* out_q, long ld_out_q, float* scales,
    int ue8m0, void* workspace, size_t workspace_bytes, qh_stream_t stream) {
  return tree_attention_launch(q, ldq, n_rows, k_rows, v_rows, ld_kv, cu_a, seg_read, n_seg,
                               k_pool, v_pool, pool_pages, table, table_width, read_used,
                               n_reads, page_tokens, n_q, n_kv, d, softmax_scale, out, ldo,
                               out_q, ld_out_q, scales, ue8m0, workspace, workspace_bytes,
                               stream, true);
}
