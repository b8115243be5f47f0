// Memory-bound fused kernels of the Qwen3 layer loop: norm + quant, QK norm +
// rotary, SiLU + quant, LSE merge + quant, KV append, gathers, final norm
// and the answer readout. One wave owns one row (or one 128-wide group) so
// every group reduction is a 16-lane shuffle, and all HBM traffic moves in
// 16-byte vectors. Built with -ffp-contract=off: each product and sum rounds
// on its own, as in the reference's op-by-op fp32 expressions.
#include "common.h"

namespace qh {

// ---------------------------------------------------------------------------
// add + RMSNorm + 1x128 group quant (attention.py:325-359 fused path;
// attention.py:143-175 layer-0 path when residual == nullptr).
// One wave per row; lane l's vector v covers columns (v*64 + l)*8 .. +8, so
// lanes 16j..16j+15 of one vector hold one 128-wide group.
// FUSED: residual != nullptr; EXACT: H == VPL * 512 (no per-vector guards).
// Both compile-time, so the kernel body is straight-line code: every load of
// the row is issued first, and each wait leaves the later loads and the
// residual stores in flight. With the loads next to the residual stores and
// these flags tested at run time, a wave made ten dependent HBM round trips
// per row and waited for its own stores (0.31 ms for 102,400 rows of 2560).
template <int VPL, bool FUSED, bool EXACT>
__global__ __launch_bounds__(256) void add_rmsnorm_quant_kernel(
    const uint16_t* __restrict__ x, long ldx, uint16_t* __restrict__ residual,
    long ld_res, const uint16_t* __restrict__ w, float eps, int T, int H,
    uint8_t* __restrict__ out_q, float* __restrict__ scales, int ue8m0) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int nvec = EXACT ? VPL : H >> 9;  // vectors of 8 per lane: H / 512
  bf16x8 xv[VPL], rv[VPL], wv[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    if (i < nvec) {
      const long col = ((long)i * 64 + lane) * 8;
      xv[i] = load8(x + (long)t * ldx + col);
      if (FUSED) rv[i] = load8(residual + (long)t * ld_res + col);
      wv[i] = load8(w + col);
    }
  }
  float v[VPL][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    if (i < nvec) {
      if (FUSED) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float s = xv[i].get(e) + rv[i].get(e);
          v[i][e] = s;
          ss += s * s;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          v[i][e] = xv[i].get(e);
          ss += v[i][e] * v[i][e];
        }
      }
    }
  }
  if (FUSED) {
    // the new residual (x + residual, rounded to bf16)
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      if (i < nvec) {
        const long col = ((long)i * 64 + lane) * 8;
        bf16x8 sum;
#pragma unroll
        for (int e = 0; e < 8; ++e) sum.set(e, f32_to_bf16(v[i][e]));
        store8(residual + (long)t * ld_res + col, sum);
      }
    }
  }
  ss = group_sum<64>(ss);
  const float rstd = 1.0f / sqrtf(ss / (float)H + eps);
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    if (i < nvec) {
      const long col = ((long)i * 64 + lane) * 8;
      float y[8];
      float amax = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (FUSED) {
          y[e] = v[i][e] * rstd * wv[i].get(e);
        } else {
          // vLLM rms_norm: bf16(bf16(x * rstd) * w)
          y[e] = round_bf16(round_bf16(v[i][e] * rstd) * wv[i].get(e));
        }
        amax = fmaxf(amax, fabsf(y[e]));
      }
      amax = group_max<16>(amax);
      const float scale = group_scale(amax, ue8m0 != 0);
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) lo |= quant_e4m3(y[e], scale) << (8 * e);
#pragma unroll
      for (int e = 0; e < 4; ++e) hi |= quant_e4m3(y[e + 4], scale) << (8 * e);
      uint2 packed = make_uint2(lo, hi);
      *reinterpret_cast<uint2*>(out_q + (long)t * H + col) = packed;
      if ((lane & 15) == 0) scales[(long)(col >> 7) * T + t] = scale;
    }
  }
}

// ---------------------------------------------------------------------------
// 1x128 group quant of bf16 rows (vLLM per_token_group_quant_fp8).
// One 16-lane group per 128-wide column group.
__global__ __launch_bounds__(256) void group_quant_kernel(
    const uint16_t* __restrict__ x, long ldx, int T, int W,
    uint8_t* __restrict__ out_q, float* __restrict__ scales, int ue8m0) {
  const int groups = W >> 7;
  const long gid = (long)blockIdx.x * 16 + (threadIdx.x >> 4);
  if (gid >= (long)T * groups) return;
  const int t = (int)(gid / groups), g = (int)(gid % groups);
  const int sub = threadIdx.x & 15;
  const long col = (long)g * 128 + sub * 8;
  bf16x8 xv = load8(x + (long)t * ldx + col);
  float amax = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(xv.get(e)));
  amax = group_max<16>(amax);
  const float scale = group_scale(amax, ue8m0 != 0);
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) lo |= quant_e4m3(xv.get(e), scale) << (8 * e);
#pragma unroll
  for (int e = 0; e < 4; ++e) hi |= quant_e4m3(xv.get(e + 4), scale) << (8 * e);
  *reinterpret_cast<uint2*>(out_q + (long)t * W + col) = make_uint2(lo, hi);
  if (sub == 0) scales[(long)g * T + t] = scale;
}

// ---------------------------------------------------------------------------
// SiLU(gate) * up + group quant (attention.py:300-323).
__global__ __launch_bounds__(256) void silu_mul_quant_kernel(
    const uint16_t* __restrict__ gu, long ld, int T, int I,
    uint8_t* __restrict__ out_q, float* __restrict__ scales, int ue8m0) {
  const int groups = I >> 7;
  const long gid = (long)blockIdx.x * 16 + (threadIdx.x >> 4);
  if (gid >= (long)T * groups) return;
  const int t = (int)(gid / groups), g = (int)(gid % groups);
  const int sub = threadIdx.x & 15;
  const long col = (long)g * 128 + sub * 8;
  bf16x8 gv = load8(gu + (long)t * ld + col);
  bf16x8 uv = load8(gu + (long)t * ld + I + col);
  float y[8];
  float amax = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    y[e] = silu_mul(gv.get(e), uv.get(e));
    amax = fmaxf(amax, fabsf(y[e]));
  }
  amax = group_max<16>(amax);
  const float scale = group_scale(amax, ue8m0 != 0);
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) lo |= quant_e4m3(y[e], scale) << (8 * e);
#pragma unroll
  for (int e = 0; e < 4; ++e) hi |= quant_e4m3(y[e + 4], scale) << (8 * e);
  *reinterpret_cast<uint2*>(out_q + (long)t * I + col) = make_uint2(lo, hi);
  if (sub == 0) scales[(long)g * T + t] = scale;
}

// ---------------------------------------------------------------------------
// Per-head RMSNorm + NeoX rotary for q and k, copy for v (attention.py:361-409).
// A 16-lane group owns one 128-wide head slot; slot s reads qkv columns
// s*128.. (q heads, then k heads, then v heads). Lane j < 8 holds the first
// half's columns 8j..8j+7, lane j >= 8 the matching second-half columns.
// RMSNorm (weight w) + NeoX RoPE of one 128-wide q or k head, for the 16
// threads of a group (j = lane % 16 holds elements 8j .. 8j+7); the partner
// halves (d, d+64) sit in threads j and j^8. Shared by the plain and the
// KV-writing kernels, and summed in the order the qkv GEMM's fused epilogue
// sums (common.h: sumsq4), so all three produce the same bits.
__device__ __forceinline__ bf16x8 norm_rope_head(bf16x8 xv, const uint16_t* __restrict__ wt,
                                                 const uint16_t* __restrict__ cs_row,
                                                 float eps, int j) {
  // the thread's columns 8j.. are the 4-column groups g = 2 (j % 2) and
  // g + 1 of the 16-column block ib = j / 2: reduce each group over ib
  // (lanes j ^ 2, j ^ 4, j ^ 8), then the groups
  float q_lo = sumsq4(xv.get(0), xv.get(1), xv.get(2), xv.get(3));
  float q_hi = sumsq4(xv.get(4), xv.get(5), xv.get(6), xv.get(7));
#pragma unroll
  for (int o = 2; o < 16; o <<= 1) {
    q_lo += __shfl_xor(q_lo, o, kWave);
    q_hi += __shfl_xor(q_hi, o, kWave);
  }
  const float pair = q_lo + q_hi;  // S_0 + S_1 (j even) or S_2 + S_3 (j odd)
  const float total_ss = pair + __shfl_xor(pair, 1, kWave);
  const float rstd = head_rstd(total_ss, eps);
  bf16x8 wv = load8(wt + j * 8);
  float n[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) n[e] = head_norm(xv.get(e), rstd, wv.get(e));
  // partner half
  float p[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) p[e] = __shfl_xor(n[e], 8, kWave);
  const int hc = (j & 7) * 8;
  bf16x8 cv = load8(cs_row + hc);
  bf16x8 sv = load8(cs_row + 64 + hc);
  bf16x8 out;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float c = cv.get(e), s = sv.get(e);
    const float r = j < 8 ? rope_first(n[e], p[e], c, s) : rope_second(n[e], p[e], c, s);
    out.set(e, f32_to_bf16(r));
  }
  return out;
}

__device__ __forceinline__ const uint16_t* cos_sin_row(const uint16_t* __restrict__ cos_sin,
                                                       const int64_t* __restrict__ positions,
                                                       int t, int max_pos) {
  int64_t pos = positions[t];
  pos = pos < 0 ? 0 : (pos >= max_pos ? max_pos - 1 : pos);
  return cos_sin + pos * 128;
}

__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    const uint16_t* __restrict__ qkv, long ld_qkv,
    const int64_t* __restrict__ positions, const uint16_t* __restrict__ cos_sin,
    int max_pos, const uint16_t* __restrict__ qw, const uint16_t* __restrict__ kw,
    float eps, int T, int n_q, int n_kv, uint16_t* __restrict__ q_out,
    uint16_t* __restrict__ k_out, uint16_t* __restrict__ v_out) {
  const int t = blockIdx.x;
  const int slot = blockIdx.y * 16 + (threadIdx.x >> 4);
  const int j = threadIdx.x & 15;
  const int total = n_q + 2 * n_kv;
  if (slot >= total) return;
  const uint16_t* src = qkv + (long)t * ld_qkv + (long)slot * 128 + j * 8;
  bf16x8 xv = load8(src);
  if (slot >= n_q + n_kv) {
    store8(v_out + ((long)t * n_kv + (slot - n_q - n_kv)) * 128 + j * 8, xv);
    return;
  }
  const bool is_q = slot < n_q;
  const bf16x8 out = norm_rope_head(xv, is_q ? qw : kw,
                                    cos_sin_row(cos_sin, positions, t, max_pos), eps, j);
  if (is_q) {
    store8(q_out + ((long)t * n_q + slot) * 128 + j * 8, out);
  } else {
    store8(k_out + ((long)t * n_kv + (slot - n_q)) * 128 + j * 8, out);
  }
}

// qk_norm_rope with k and v written straight into the paged arena: row t's
// k and v go to arena row dst[t] (the unified path writes every chunk row).
// One launch, two kinds of workgroup. The first ceil(T / 4) * slot_blocks
// work as qk_norm_rope_kernel over 4 rows each (16 head slots, the same
// per-head arithmetic), writing q to q_out and k into its K page row; the
// four rows' loads are issued back to back, so that a thread keeps four
// 16-byte reads in flight (one row per workgroup left the kernel short of
// bytes in flight: 4.4 TB/s). The last ceil(T / 16) * n_kv each take one KV
// head's v of 16 rows from qkv, stage it in LDS and write V^T with the row
// index fastest, as kv_scatter_kernel does.
constexpr int kRopeRows = 16;
constexpr int kHeadRows = 4;

__global__ __launch_bounds__(256) void qk_norm_rope_kv_kernel(
    const uint16_t* __restrict__ qkv, long ld_qkv,
    const int64_t* __restrict__ positions, const uint16_t* __restrict__ cos_sin,
    int max_pos, const uint16_t* __restrict__ qw, const uint16_t* __restrict__ kw,
    float eps, int T, int n_q, int n_kv, int slot_blocks, uint16_t* __restrict__ q_out,
    uint16_t* __restrict__ k_pool, uint16_t* __restrict__ v_pool,
    const int64_t* __restrict__ dst, int page) {
  extern __shared__ uint16_t vbuf[];  // [row][128 + 2] of one KV head
  const long head_blocks = (long)((T + kHeadRows - 1) / kHeadRows) * slot_blocks;
  const int j = threadIdx.x & 15;
  if ((long)blockIdx.x < head_blocks) {
    const int t0 = (int)(blockIdx.x / slot_blocks) * kHeadRows;
    const int slot = (int)(blockIdx.x % slot_blocks) * 16 + (threadIdx.x >> 4);
    if (slot >= n_q + n_kv) return;  // v: the row-block workgroups
    const int rows = min(kHeadRows, T - t0);
    bf16x8 xv[kHeadRows];
#pragma unroll
    for (int e = 0; e < kHeadRows; ++e)
      if (e < rows) xv[e] = load8(qkv + (long)(t0 + e) * ld_qkv + (long)slot * 128 + j * 8);
    const bool is_q = slot < n_q;
#pragma unroll
    for (int e = 0; e < kHeadRows; ++e) {
      if (e >= rows) break;
      const int t = t0 + e;
      const bf16x8 out = norm_rope_head(xv[e], is_q ? qw : kw,
                                        cos_sin_row(cos_sin, positions, t, max_pos), eps, j);
      if (is_q) {
        store8(q_out + ((long)t * n_q + slot) * 128 + j * 8, out);
      } else {
        const long r = dst[t];
        const long pg = r / page, sl = r % page;
        store8(k_pool + ((pg * n_kv + (slot - n_q)) * page + sl) * 128 + j * 8, out);
      }
    }
    return;
  }
  // V^T workgroups: 16 rows of one KV head each, so the LDS staging is 4 KiB
  // and does not limit how many head workgroups share a CU
  const long vb = (long)blockIdx.x - head_blocks;
  const int h = (int)(vb % n_kv);
  const int t0 = (int)(vb / n_kv) * kRopeRows;
  const int rows = min(kRopeRows, T - t0);
  constexpr int ld = 128 + 2;
  const uint16_t* vsrc = qkv + (long)(n_q + n_kv + h) * 128;
  for (int c = threadIdx.x; c < rows * 16; c += 256) {
    const int e = c >> 4, hc = c & 15;
    const bf16x8 vv = load8(vsrc + (long)(t0 + e) * ld_qkv + hc * 8);
    uint32_t* vl = reinterpret_cast<uint32_t*>(vbuf + e * ld + hc * 8);
#pragma unroll
    for (int w = 0; w < 4; ++w) vl[w] = vv.w[w];
  }
  __syncthreads();
  // V^T: work item = (d, row), row fastest
  for (int it = threadIdx.x; it < 128 * kRopeRows; it += 256) {
    const int e = it & (kRopeRows - 1);
    if (e >= rows) continue;
    const int d = it >> 4;
    const long r = dst[t0 + e];
    const long pg = r / page, sl = r % page;
    v_pool[((pg * n_kv + h) * 128 + d) * page + sl] = vbuf[e * ld + d];
  }
}

// ---------------------------------------------------------------------------
// KV append into the paged arena. K pages hold [n_kv][page][d]; V pages hold
// [n_kv][d][page]. One wave per row pair; K moves as 16-byte vectors, V as
// 2-byte elements into its transposed page column.
// Chunk rows -> arena rows for the layer's K and V pools (attention.py:411-427
// semantics; the arena layout is the one in quail_hip.h). One workgroup moves
// 16 consecutive entries. K rows are copied as 16-byte chunks. V rows are
// staged in LDS and written as V^T with the entry index fastest across lanes:
// entries that land in consecutive slots of one page give one contiguous
// 32-byte write per (page, head, d) row, wherever the run starts or breaks.
constexpr int kScatterRows = 16;

__global__ __launch_bounds__(256) void kv_scatter_kernel(
    const uint16_t* __restrict__ k_src, const uint16_t* __restrict__ v_src,
    uint16_t* __restrict__ k_pool, uint16_t* __restrict__ v_pool,
    const int64_t* __restrict__ src, const int64_t* __restrict__ dst, int n,
    int n_kv, int page) {
  // V rows of the 16 entries, [entry][n_kv*128] with a 4-byte pad per entry
  // so the transposed reads (entry fastest) fall in distinct banks
  extern __shared__ uint16_t vbuf[];
  const int row_elems = n_kv * 128;
  const int ld = row_elems + 2;
  const int tid = threadIdx.x;
  const int i0 = blockIdx.x * kScatterRows;
  const int rows = min(kScatterRows, n - i0);
  const int chunks = rows * n_kv * 16;  // 16-byte chunks of K (and of V)
  for (int c = tid; c < chunks; c += 256) {
    const int e = c / (n_kv * 16), hc = c % (n_kv * 16);
    const int h = hc >> 4, off = (hc & 15) * 8;
    const long s = src[i0 + e], r = dst[i0 + e];
    const long pg = r / page, slot = r % page;
    store8(k_pool + ((pg * n_kv + h) * page + slot) * 128 + off,
           load8(k_src + (s * n_kv + h) * 128 + off));
    const bf16x8 vv = load8(v_src + (s * n_kv + h) * 128 + off);
    uint32_t* vl = reinterpret_cast<uint32_t*>(vbuf + e * ld + h * 128 + off);
#pragma unroll
    for (int w = 0; w < 4; ++w) vl[w] = vv.w[w];
  }
  __syncthreads();
  // V^T: work item = (head, d, entry), entry fastest
  const int items = row_elems * kScatterRows;
  for (int t = tid; t < items; t += 256) {
    const int e = t & (kScatterRows - 1);
    if (e >= rows) continue;
    const int hd = t >> 4;  // h * 128 + d
    const long r = dst[i0 + e];
    const long pg = r / page, slot = r % page;
    const int h = hd >> 7, d = hd & 127;
    v_pool[((pg * n_kv + h) * 128 + d) * page + slot] = vbuf[e * ld + hd];
  }
}

// Arena row -> arena row copy (the kept partial page of a suffix temporary).
__global__ __launch_bounds__(256) void kv_copy_kernel(
    uint16_t* __restrict__ k_pool, uint16_t* __restrict__ v_pool,
    const int64_t* __restrict__ src, const int64_t* __restrict__ dst, int n,
    int n_kv, int page) {
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= n) return;
  const int lane = threadIdx.x & 63;
  const long rs = src[i], rd = dst[i];
  const long ps = rs / page, ss = rs % page, pd = rd / page, sd = rd % page;
  const int row_vecs = n_kv * 16;
  for (int c = lane; c < row_vecs; c += 64) {
    const int h = c >> 4, off = (c & 15) * 8;
    bf16x8 kv = load8(k_pool + ((ps * n_kv + h) * page + ss) * 128 + off);
    store8(k_pool + ((pd * n_kv + h) * page + sd) * 128 + off, kv);
    const uint16_t* vs = v_pool + ((ps * n_kv + h) * 128 + off) * page + ss;
    uint16_t* vd = v_pool + ((pd * n_kv + h) * 128 + off) * page + sd;
#pragma unroll
    for (int e = 0; e < 8; ++e) vd[(long)e * page] = vs[(long)e * page];
  }
}

// ---------------------------------------------------------------------------
// LSE merge + per-head quant (attention.py:429-473). One 16-lane group per
// (row, head): each head is exactly one 128-wide quant group.
__global__ __launch_bounds__(256) void merge_attn_quant_kernel(
    const uint16_t* __restrict__ a, const float* __restrict__ lse_a,
    long lse_a_stride, const uint16_t* __restrict__ b,
    const float* __restrict__ lse_b, long lse_b_stride,
    const int32_t* __restrict__ source, int T, int n_h,
    uint8_t* __restrict__ out_q, float* __restrict__ scales, int ue8m0) {
  const long gid = (long)blockIdx.x * 16 + (threadIdx.x >> 4);
  if (gid >= (long)T * n_h) return;
  const int t = (int)(gid / n_h), h = (int)(gid % n_h);
  const int sub = threadIdx.x & 15;
  const long col = (long)h * 128 + sub * 8;
  bf16x8 av = load8(a + (long)t * n_h * 128 + col);
  const int src = source[t];
  float y[8];
  if (src >= 0) {
    bf16x8 bv = load8(b + (long)src * n_h * 128 + col);
    const float la = lse_a[(long)h * lse_a_stride + t];
    const float lb = lse_b[(long)h * lse_b_stride + src];
    const float wgt = round_bf16(1.0f / (1.0f + expf(-(lb - la))));
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float av_e = av.get(e);
      y[e] = round_bf16(av_e + (bv.get(e) - av_e) * wgt);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = av.get(e);
  }
  float amax = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(y[e]));
  amax = group_max<16>(amax);
  const float scale = group_scale(amax, ue8m0 != 0);
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) lo |= quant_e4m3(y[e], scale) << (8 * e);
#pragma unroll
  for (int e = 0; e < 4; ++e) hi |= quant_e4m3(y[e + 4], scale) << (8 * e);
  *reinterpret_cast<uint2*>(out_q + (long)t * n_h * 128 + col) = make_uint2(lo, hi);
  if (sub == 0) scales[(long)h * T + t] = scale;
}

// ---------------------------------------------------------------------------
// Row gather of bf16 rows (embedding lookup, index_select).
__global__ __launch_bounds__(256) void gather_rows_kernel(
    const uint16_t* __restrict__ table, long ld_table,
    const int64_t* __restrict__ idx, int n, int W, uint16_t* __restrict__ out) {
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= n) return;
  const int lane = threadIdx.x & 63;
  const long r = idx[i];
  for (int c = lane * 8; c < W; c += 512)
    store8(out + (long)i * W + c, load8(table + r * ld_table + c));
}

// Row gather of an fp8 GEMM input: out_q[i] = q[idx[i]] (W bytes) and its
// 1x128 scales, column-major on both sides: out_s[g][i] = s[g][idx[i]]. One
// wave per row, 16 bytes per lane.
__global__ __launch_bounds__(256) void gather_quant_rows_kernel(
    const uint8_t* __restrict__ q, long ldq, const float* __restrict__ s, int T,
    const int64_t* __restrict__ idx, int n, int W, uint8_t* __restrict__ out_q, long ld_out,
    float* __restrict__ out_s) {
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= n) return;
  const int lane = threadIdx.x & 63;
  const long r = idx[i];
  for (int c = lane * 16; c < W; c += 1024)
    *reinterpret_cast<uint4*>(out_q + (long)i * ld_out + c) =
        *reinterpret_cast<const uint4*>(q + r * ldq + c);
  for (int g = lane; g < W / 128; g += 64) out_s[(long)g * n + i] = s[(long)g * T + r];
}

// ---------------------------------------------------------------------------
// vLLM fused_add_rms_norm: z = bf16(h + r); out = bf16(bf16(z * rstd) * w).
// Row i reads row idx[i] of hidden / residual (row i itself when idx is
// NULL) and writes out row i; res_out, when given, receives z at row i. Each
// lane reads its 8 columns of a row before it writes them, so out and
// res_out may alias hidden and residual (the in-place vLLM form). One wave
// per row.
__global__ __launch_bounds__(256) void final_norm_kernel(
    const uint16_t* hidden, const uint16_t* residual, const int64_t* __restrict__ idx,
    int R, int H, const uint16_t* __restrict__ w, float eps, uint16_t* out,
    uint16_t* res_out) {
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= R) return;
  const int lane = threadIdx.x & 63;
  const long r = idx ? idx[i] : (long)i;
  float ss = 0.f;
  for (int c = lane * 8; c < H; c += 512) {
    bf16x8 hv = load8(hidden + r * H + c);
    bf16x8 rv = load8(residual + r * H + c);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float z = round_bf16(hv.get(e) + rv.get(e));
      ss += z * z;
    }
  }
  ss = group_sum<64>(ss);
  const float rstd = 1.0f / sqrtf(ss / (float)H + eps);
  for (int c = lane * 8; c < H; c += 512) {
    bf16x8 hv = load8(hidden + r * H + c);
    bf16x8 rv = load8(residual + r * H + c);
    bf16x8 wv = load8(w + c);
    bf16x8 o, zr;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float z = round_bf16(hv.get(e) + rv.get(e));
      zr.set(e, f32_to_bf16(z));
      o.set(e, f32_to_bf16(round_bf16(z * rstd) * wv.get(e)));
    }
    if (res_out) store8(res_out + (long)i * H + c, zr);
    store8(out + (long)i * H + c, o);
  }
}

// ---------------------------------------------------------------------------
// Answer readout: per row, bf16 scores against the retained answer rows,
// strict TRUE > FALSE compare (readout.py:45-49, :70-79).
__global__ __launch_bounds__(256) void answer_bits_kernel(
    const uint16_t* __restrict__ normed, int R, int H,
    const uint16_t* __restrict__ w_ans, int n_ans,
    const uint8_t* __restrict__ is_true, uint8_t* __restrict__ bits,
    float* __restrict__ margin, uint16_t* __restrict__ best_true,
    uint16_t* __restrict__ best_false) {
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= R) return;
  const int lane = threadIdx.x & 63;
  float best_t = -INFINITY, best_f = -INFINITY;
  for (int a = 0; a < n_ans; ++a) {
    float acc = 0.f;
    for (int c = lane * 8; c < H; c += 512) {
      bf16x8 nv = load8(normed + (long)i * H + c);
      bf16x8 wv = load8(w_ans + (long)a * H + c);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += nv.get(e) * wv.get(e);
    }
    acc = group_sum<64>(acc);
    const float score = round_bf16(acc);
    if (is_true[a]) best_t = fmaxf(best_t, score);
    else best_f = fmaxf(best_f, score);
  }
  if (lane == 0) {
    if (bits) bits[i] = best_t > best_f ? 1 : 0;
    if (margin) margin[i] = best_t - best_f;
    // the scores are bf16 values already: the top 16 bits are exact
    if (best_true) best_true[i] = (uint16_t)(__float_as_uint(best_t) >> 16);
    if (best_false) best_false[i] = (uint16_t)(__float_as_uint(best_f) >> 16);
  }
}

// The fused epilogues' e4m3 encoder (quant_e4m3_x4, no +-448 clamp) over
// raw fp32 values with scale 1: four values per thread.
__global__ __launch_bounds__(256) void e4m3_encode_kernel(const float* __restrict__ x,
                                                          long n4, uint32_t* __restrict__ out) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  const float4 v = reinterpret_cast<const float4*>(x)[i];
  out[i] = quant_e4m3_x4(v.x, v.y, v.z, v.w, 1.0);
}

}  // namespace qh

// ===========================================================================
// C ABI
// ===========================================================================
using namespace qh;

static inline unsigned blocks_for(long items, int per_block) {
  return (unsigned)((items + per_block - 1) / per_block);
}

extern "C" int qh_add_rmsnorm_quant(const void* x, long ldx, void* residual,
                                    long ld_res, const void* w, float eps,
                                    int T, int H, void* out_q, float* scales,
                                    int ue8m0, qh_stream_t stream) {
  QH_REQUIRE(T >= 0, "add_rmsnorm_quant: T=%d", T);
  QH_REQUIRE(H > 0 && H % 512 == 0 && H <= 8192,
             "add_rmsnorm_quant: H=%d must be a positive multiple of 512 up to 8192", H);
  QH_REQUIRE(ldx >= H && (!residual || ld_res >= H), "add_rmsnorm_quant: row stride");
  QH_REQUIRE(ldx % 8 == 0 && (!residual || ld_res % 8 == 0),
             "add_rmsnorm_quant: row strides must be multiples of 8");
  if (T == 0) return QH_OK;
  QH_REQUIRE(x && w && out_q && scales, "add_rmsnorm_quant: null pointer");
  dim3 grid(blocks_for(T, 4)), block(256);
  const int vpl = H / 512;
  auto args = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, block, 0, (hipStream_t)stream,
                       (const uint16_t*)x, ldx, (uint16_t*)residual, ld_res,
                       (const uint16_t*)w, eps, T, H, (uint8_t*)out_q, scales, ue8m0);
  };
  const bool fused = residual != nullptr;
  if (vpl == 5) fused ? args(add_rmsnorm_quant_kernel<5, true, true>)
                      : args(add_rmsnorm_quant_kernel<5, false, true>);
  else if (vpl == 10) fused ? args(add_rmsnorm_quant_kernel<10, true, true>)
                            : args(add_rmsnorm_quant_kernel<10, false, true>);
  else if (vpl < 10) fused ? args(add_rmsnorm_quant_kernel<10, true, false>)
                           : args(add_rmsnorm_quant_kernel<10, false, false>);
  else fused ? args(add_rmsnorm_quant_kernel<16, true, false>)
             : args(add_rmsnorm_quant_kernel<16, false, false>);
  return launch_status("add_rmsnorm_quant");
}

extern "C" int qh_group_quant(const void* x, long ldx, int T, int W, void* out_q,
                              float* scales, int ue8m0, qh_stream_t stream) {
  QH_REQUIRE(T >= 0 && W > 0 && W % 128 == 0, "group_quant: W=%d must be a multiple of 128", W);
  QH_REQUIRE(ldx >= W && ldx % 8 == 0, "group_quant: row stride %ld", ldx);
  if (T == 0) return QH_OK;
  QH_REQUIRE(x && out_q && scales, "group_quant: null pointer");
  const long groups = (long)T * (W / 128);
  hipLaunchKernelGGL(group_quant_kernel, dim3(blocks_for(groups, 16)), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)x, ldx, T, W,
                     (uint8_t*)out_q, scales, ue8m0);
  return launch_status("group_quant");
}

extern "C" int qh_silu_mul_quant(const void* gate_up, long ld, int T, int I,
                                 void* out_q, float* scales, int ue8m0,
                                 qh_stream_t stream) {
  QH_REQUIRE(T >= 0 && I > 0 && I % 128 == 0, "silu_mul_quant: I=%d must be a multiple of 128", I);
  QH_REQUIRE(ld >= 2L * I && ld % 8 == 0, "silu_mul_quant: row stride %ld", ld);
  if (T == 0) return QH_OK;
  QH_REQUIRE(gate_up && out_q && scales, "silu_mul_quant: null pointer");
  const long groups = (long)T * (I / 128);
  hipLaunchKernelGGL(silu_mul_quant_kernel, dim3(blocks_for(groups, 16)), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)gate_up, ld, T, I,
                     (uint8_t*)out_q, scales, ue8m0);
  return launch_status("silu_mul_quant");
}

extern "C" int qh_qk_norm_rope(const void* qkv, long ld_qkv, const int64_t* positions,
                               const void* cos_sin, int max_pos, const void* qw,
                               const void* kw, float eps, int T, int n_q, int n_kv,
                               int d, void* q_out, void* k_out, void* v_out,
                               qh_stream_t stream) {
  QH_REQUIRE(d == 128, "qk_norm_rope: head_dim %d unsupported (128 only)", d);
  QH_REQUIRE(n_q > 0 && n_kv > 0 && T >= 0 && max_pos > 0, "qk_norm_rope: geometry");
  QH_REQUIRE(ld_qkv >= (long)(n_q + 2 * n_kv) * d && ld_qkv % 8 == 0,
             "qk_norm_rope: row stride %ld", ld_qkv);
  if (T == 0) return QH_OK;
  QH_REQUIRE(qkv && positions && cos_sin && qw && kw && q_out && k_out && v_out,
             "qk_norm_rope: null pointer");
  dim3 grid(T, blocks_for(n_q + 2 * n_kv, 16));
  hipLaunchKernelGGL(qk_norm_rope_kernel, grid, dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)qkv, ld_qkv, positions, (const uint16_t*)cos_sin,
                     max_pos, (const uint16_t*)qw, (const uint16_t*)kw, eps, T, n_q,
                     n_kv, (uint16_t*)q_out, (uint16_t*)k_out, (uint16_t*)v_out);
  return launch_status("qk_norm_rope");
}

extern "C" int qh_qk_norm_rope_kv(const void* qkv, long ld_qkv, const int64_t* positions,
                                  const void* cos_sin, int max_pos, const void* qw,
                                  const void* kw, float eps, int T, int n_q, int n_kv, int d,
                                  void* q_out, void* k_pool, void* v_pool, const int64_t* dst,
                                  int page_tokens, qh_stream_t stream) {
  QH_REQUIRE(d == 128, "qk_norm_rope_kv: head_dim %d unsupported (128 only)", d);
  QH_REQUIRE(n_q > 0 && n_kv > 0 && T >= 0 && max_pos > 0 && page_tokens > 0,
             "qk_norm_rope_kv: geometry");
  QH_REQUIRE(ld_qkv >= (long)(n_q + 2 * n_kv) * d && ld_qkv % 8 == 0,
             "qk_norm_rope_kv: row stride %ld", ld_qkv);
  if (T == 0) return QH_OK;
  QH_REQUIRE(qkv && positions && cos_sin && qw && kw && q_out && k_pool && v_pool && dst,
             "qk_norm_rope_kv: null pointer");
  const size_t smem = (size_t)kRopeRows * (128 + 2) * sizeof(uint16_t);
  const int slot_blocks = blocks_for(n_q + n_kv, 16);
  const long grid =
      (long)blocks_for(T, kHeadRows) * slot_blocks + (long)blocks_for(T, kRopeRows) * n_kv;
  QH_REQUIRE(grid < 0x7fffffffL, "qk_norm_rope_kv: %d rows exceed the grid", T);
  hipLaunchKernelGGL(qk_norm_rope_kv_kernel, dim3((unsigned)grid), dim3(256), smem,
                     (hipStream_t)stream, (const uint16_t*)qkv, ld_qkv, positions,
                     (const uint16_t*)cos_sin, max_pos, (const uint16_t*)qw,
                     (const uint16_t*)kw, eps, T, n_q, n_kv, slot_blocks, (uint16_t*)q_out,
                     (uint16_t*)k_pool, (uint16_t*)v_pool, dst, page_tokens);
  return launch_status("qk_norm_rope_kv");
}

extern "C" int qh_kv_row_scatter(const void* k_src, const void* v_src, void* k_pool,
                                 void* v_pool, const int64_t* src, const int64_t* dst,
                                 int n, int n_kv, int d, int page_tokens,
                                 qh_stream_t stream) {
  QH_REQUIRE(d == 128, "kv_row_scatter: head_dim %d unsupported", d);
  QH_REQUIRE(n >= 0 && n_kv > 0 && page_tokens > 0, "kv_row_scatter: geometry");
  if (n == 0) return QH_OK;
  QH_REQUIRE(k_src && v_src && k_pool && v_pool && src && dst, "kv_row_scatter: null pointer");
  QH_REQUIRE(n_kv <= 15, "kv_row_scatter: n_kv=%d exceeds the 64 KiB staging buffer", n_kv);
  const size_t smem = (size_t)kScatterRows * (n_kv * 128 + 2) * sizeof(uint16_t);
  hipLaunchKernelGGL(kv_scatter_kernel, dim3(blocks_for(n, kScatterRows)), dim3(256), smem,
                     (hipStream_t)stream, (const uint16_t*)k_src, (const uint16_t*)v_src,
                     (uint16_t*)k_pool, (uint16_t*)v_pool, src, dst, n, n_kv, page_tokens);
  return launch_status("kv_row_scatter");
}

extern "C" int qh_kv_row_copy(void* k_pool, void* v_pool, const int64_t* src,
                              const int64_t* dst, int n, int n_kv, int d,
                              int page_tokens, qh_stream_t stream) {
  QH_REQUIRE(d == 128, "kv_row_copy: head_dim %d unsupported", d);
  QH_REQUIRE(n >= 0 && n_kv > 0 && page_tokens > 0, "kv_row_copy: geometry");
  if (n == 0) return QH_OK;
  QH_REQUIRE(k_pool && v_pool && src && dst, "kv_row_copy: null pointer");
  hipLaunchKernelGGL(kv_copy_kernel, dim3(blocks_for(n, 4)), dim3(256), 0,
                     (hipStream_t)stream, (uint16_t*)k_pool, (uint16_t*)v_pool, src, dst,
                     n, n_kv, page_tokens);
  return launch_status("kv_row_copy");
}

extern "C" int qh_merge_attn_quant(const void* out_a, const float* lse_a,
                                   long lse_a_stride, const void* out_b,
                                   const float* lse_b, long lse_b_stride,
                                   const int32_t* source, int T, int n_h, void* out_q,
                                   float* scales, int ue8m0, qh_stream_t stream) {
  QH_REQUIRE(T >= 0 && n_h > 0, "merge_attn_quant: geometry");
  if (T == 0) return QH_OK;
  QH_REQUIRE(out_a && lse_a && source && out_q && scales, "merge_attn_quant: null pointer");
  QH_REQUIRE(out_b && lse_b, "merge_attn_quant: out_b/lse_b null");
  const long groups = (long)T * n_h;
  hipLaunchKernelGGL(merge_attn_quant_kernel, dim3(blocks_for(groups, 16)), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)out_a, lse_a, lse_a_stride,
                     (const uint16_t*)out_b, lse_b, lse_b_stride, source, T, n_h,
                     (uint8_t*)out_q, scales, ue8m0);
  return launch_status("merge_attn_quant");
}

extern "C" int qh_gather_rows(const void* table, long ld_table, const int64_t* idx,
                              int n, int W, void* out, qh_stream_t stream) {
  QH_REQUIRE(n >= 0 && W > 0 && W % 8 == 0 && ld_table >= W && ld_table % 8 == 0,
             "gather_rows: geometry W=%d ld=%ld", W, ld_table);
  if (n == 0) return QH_OK;
  QH_REQUIRE(table && idx && out, "gather_rows: null pointer");
  hipLaunchKernelGGL(gather_rows_kernel, dim3(blocks_for(n, 4)), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)table, ld_table, idx, n, W,
                     (uint16_t*)out);
  return launch_status("gather_rows");
}

extern "C" int qh_gather_quant_rows(const void* q, long ldq, const float* scales, int T,
                                    const int64_t* idx, int n, int W, void* out_q,
                                    long ld_out, float* out_scales, qh_stream_t stream) {
  QH_REQUIRE(T >= 0 && n >= 0 && W > 0 && W % 128 == 0,
             "gather_quant_rows: geometry T=%d n=%d W=%d", T, n, W);
  QH_REQUIRE(ldq >= W && ldq % 16 == 0 && ld_out >= W && ld_out % 16 == 0,
             "gather_quant_rows: row strides %ld, %ld (W=%d, multiples of 16)", ldq, ld_out, W);
  if (n == 0) return QH_OK;
  QH_REQUIRE(T > 0, "gather_quant_rows: rows requested from an empty input");
  QH_REQUIRE(q && scales && idx && out_q && out_scales, "gather_quant_rows: null pointer");
  hipLaunchKernelGGL(gather_quant_rows_kernel, dim3(blocks_for(n, 4)), dim3(256), 0,
                     (hipStream_t)stream, (const uint8_t*)q, ldq, scales, T, idx, n, W,
                     (uint8_t*)out_q, ld_out, out_scales);
  return launch_status("gather_quant_rows");
}

extern "C" int qh_final_norm(const void* hidden, const void* residual,
                             const int64_t* final_idx, int R, int H, const void* w,
                             float eps, void* normed_out, qh_stream_t stream) {
  QH_REQUIRE(R >= 0 && H > 0 && H % 8 == 0, "final_norm: geometry");
  if (R == 0) return QH_OK;
  QH_REQUIRE(hidden && residual && final_idx && w && normed_out, "final_norm: null pointer");
  hipLaunchKernelGGL(final_norm_kernel, dim3(blocks_for(R, 4)), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)hidden,
                     (const uint16_t*)residual, final_idx, R, H, (const uint16_t*)w, eps,
                     (uint16_t*)normed_out, (uint16_t*)nullptr);
  return launch_status("final_norm");
}

extern "C" int qh_fused_add_rms_norm(void* hidden, void* residual, int R, int H,
                                     const void* w, float eps, qh_stream_t stream) {
  QH_REQUIRE(R >= 0 && H > 0 && H % 8 == 0, "fused_add_rms_norm: geometry");
  if (R == 0) return QH_OK;
  QH_REQUIRE(hidden && residual && w, "fused_add_rms_norm: null pointer");
  hipLaunchKernelGGL(final_norm_kernel, dim3(blocks_for(R, 4)), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)hidden,
                     (const uint16_t*)residual, (const int64_t*)nullptr, R, H,
                     (const uint16_t*)w, eps, (uint16_t*)hidden, (uint16_t*)residual);
  return launch_status("fused_add_rms_norm");
}

extern "C" int qh_answer_bits(const void* normed, int R, int H, const void* w_ans,
                              int n_ans, const uint8_t* is_true, uint8_t* bits,
                              float* margin, qh_stream_t stream) {
  QH_REQUIRE(R >= 0 && H > 0 && H % 8 == 0 && n_ans > 0, "answer_bits: geometry");
  if (R == 0) return QH_OK;
  QH_REQUIRE(normed && w_ans && is_true && bits, "answer_bits: null pointer");
  hipLaunchKernelGGL(answer_bits_kernel, dim3(blocks_for(R, 4)), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)normed, R, H,
                     (const uint16_t*)w_ans, n_ans, is_true, bits, margin,
                     (uint16_t*)nullptr, (uint16_t*)nullptr);
  return launch_status("answer_bits");
}

extern "C" int qh_e4m3_encode(const float* x, long n, uint8_t* out, qh_stream_t stream) {
  QH_REQUIRE(n >= 0 && n % 4 == 0, "e4m3_encode: n=%ld must be a multiple of 4", n);
  if (n == 0) return QH_OK;
  QH_REQUIRE(x && out, "e4m3_encode: null pointer");
  QH_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)out & 3) == 0, "e4m3_encode: alignment");
  hipLaunchKernelGGL(e4m3_encode_kernel, dim3(blocks_for(n / 4, 256)), dim3(256), 0,
                     (hipStream_t)stream, x, n / 4, (uint32_t*)out);
  return launch_status("e4m3_encode");
}

extern "C" int qh_answer_logits(const void* normed, int R, int H, const void* w_ans,
                                int n_ans, const uint8_t* is_true, void* best_true,
                                void* best_false, qh_stream_t stream) {
  QH_REQUIRE(R >= 0 && H > 0 && H % 8 == 0 && n_ans > 0, "answer_logits: geometry");
  if (R == 0) return QH_OK;
  QH_REQUIRE(normed && w_ans && is_true && best_true && best_false,
             "answer_logits: null pointer");
  hipLaunchKernelGGL(answer_bits_kernel, dim3(blocks_for(R, 4)), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)normed, R, H,
                     (const uint16_t*)w_ans, n_ans, is_true, (uint8_t*)nullptr,
                     (float*)nullptr, (uint16_t*)best_true, (uint16_t*)best_false);
  return launch_status("answer_logits");
}
