/*
 * quail_hip.h - C ABI of libquail_hip.so, the gfx950 kernels of the Quail
 * executor hot path (Qwen3 fp8 prefill over a paged KV arena).
 *
 * Conventions
 *   - Every entry point returns an int status: QH_OK (0) or a negative
 *     QH_E_* code. qh_last_error() returns a message for the last failure
 *     on the calling host thread.
 *   - Pointers are device pointers unless a comment says otherwise.
 *   - bf16 tensors are passed as void* holding IEEE bfloat16 bit patterns;
 *     e4m3 tensors as void* holding OCP float8_e4m3fn bytes.
 *   - Row strides are in elements of the tensor's own type.
 *   - The last argument is the hipStream_t the work is queued on (the
 *     caller's current torch stream). Nothing blocks the host.
 *   - No entry point allocates or frees memory. Scratch space comes from
 *     the caller through a (workspace, workspace_bytes) pair whose size a
 *     *_workspace_bytes() query returns.
 *   - Activation scales are stored column-major, as the reference stores
 *     them: the scale of (token t, 128-column group g) sits at
 *     scales[g * T + t].
 *
 * KV arena layout (per layer, per pool). The reference's logical arena row
 * of (page p, slot i) is p * page_tokens + i (arena.py:519-523); that
 * numbering is kept bit-exactly. Physically this library stores
 *   K: [n_pages][n_kv][page_tokens][head_dim]   (one 4 KiB block per page
 *                                                and head at 16 x 128 bf16)
 *   V: [n_pages][n_kv][head_dim][page_tokens]   (the same block transposed)
 * so that a page of one KV head is one contiguous block for the paged
 * gather, and V is already key-contiguous for the P.V product.
 */
#ifndef QUAIL_HIP_H
#define QUAIL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* qh_stream_t;

enum {
  QH_OK = 0,
  QH_E_ARGUMENT = -1,     /* bad pointer, size or geometry   -> ValueError   */
  QH_E_UNSUPPORTED = -2,  /* geometry the library has no kernel for       */
  QH_E_WORKSPACE = -3,    /* workspace missing or too small                  */
  QH_E_HIP = -4           /* a HIP runtime call failed       -> RuntimeError */
};

/* Library version, and the message of the last failure on this thread. */
int qh_version(void);
const char* qh_last_error(void);

/*
 * Fused residual add + RMSNorm + per-token 1x128 fp8 group quantization.
 * Replaces Engine.norm_quant (attention.py:763-769): with residual != NULL
 * the Triton add_rms_norm_quant kernel (attention.py:325-359, called at
 * :658-671): residual <- bf16(x + residual); y = (x + residual) * rstd * w
 * in fp32, quantized. With residual == NULL the layer-0 path
 * quant(rms_norm(x)) (attention.py:143-175): y = bf16(bf16(x * rstd) * w),
 * then quantized. scale = max(amax, 1e-10) / 448, or its power-of-two
 * ceiling when ue8m0 != 0; q = e4m3(clamp(y / scale, -448, 448)).
 *   x        [T, H] bf16, row stride ldx
 *   residual [T, H] bf16, row stride ld_res, updated in place, or NULL
 *   w        [H] bf16
 *   out_q    [T, H] e4m3 contiguous; scales [H/128, T] fp32
 * H must be a multiple of 128 and at most 8192.
 */
int qh_add_rmsnorm_quant(const void* x, long ldx, void* residual, long ld_res,
                         const void* w, float eps, int T, int H, void* out_q,
                         float* scales, int ue8m0, qh_stream_t stream);

/*
 * Per-token 1x128 fp8 group quantization of bf16 rows: vLLM's
 * per_token_group_quant_fp8 with column-major scales, as Engine.quant calls
 * it (attention.py:143-151) after unified attention (:798).
 *   x [T, W] bf16 row stride ldx; out_q [T, W] e4m3; scales [W/128, T].
 */
int qh_group_quant(const void* x, long ldx, int T, int W, void* out_q,
                   float* scales, int ue8m0, qh_stream_t stream);

/*
 * FP8 block-scaled GEMM, C = (A * sa) (B * sb)^T, fp32 accumulate, bf16 out.
 * Replaces DeepGEMM fp8_gemm_nt as Engine.gemm calls it
 * (attention.py:129-141; four calls per layer, models/qwen3.py:108-118).
 *   A  [M, K] e4m3 row stride lda;   sa [K/128, M] fp32 (column-major (M, K/128))
 *   B  [N, K] e4m3 row stride ldb;   sb [N/128, K/128] fp32 (row-major)
 *   C  [M, N] bf16 row stride ldc
 *   out[m, n] = sum_kb sa[kb, m] * sb[n/128, kb] * sum_{k in kb} A[m, k] B[n, k]
 * N must be a multiple of 256, K of 128. Any M >= 1.
 */
int qh_fp8_gemm_nt(const void* A, long lda, const float* sa, const void* B,
                   long ldb, const float* sb, void* C, long ldc, int M, int N,
                   int K, qh_stream_t stream);

/*
 * qh_fp8_gemm_nt for UE8M0 scales: every sa and sb value is a power of two
 * (2^-126 .. 2^127), as the reference's scales are when
 * is_deep_gemm_e8m0_used() holds (attention.py:115, :129-141; vLLM then
 * rounds the weight block scales up to powers of two at load time and
 * per_token_group_quant_fp8 runs with use_ue8m0). The MFMA applies the
 * scales through its own E8M0 operands and accumulates the K blocks in
 * place; a scale that is not a power of two is read as its power-of-two
 * exponent alone. Same operands, layouts and limits as qh_fp8_gemm_nt.
 */
int qh_fp8_gemm_nt_ue8m0(const void* A, long lda, const float* sa, const void* B,
                         long ldb, const float* sb, void* C, long ldc, int M, int N,
                         int K, qh_stream_t stream);

/*
 * The gate_up projection fused with the SiLU-gated product and its 1x128 fp8
 * quantization: replaces Engine.gemm(gate_up_proj) followed by
 * Engine.activation_quant (models/qwen3.py:113-116 -> attention.py:129-141,
 * :771-775, :300-323). B holds the gate rows [0, I) then the up rows
 * [I, 2I) (the vLLM merged layout, unchanged). Per output column j:
 *   g = bf16(gemm[m, j]); u = bf16(gemm[m, I + j]); y = g * sigmoid(g) * u
 * in fp32, then quantized per 1x128 group exactly as qh_silu_mul_quant does
 * on the bf16 gate_up tensor, so the result is bit-identical to the
 * unfused pair.
 *   A [M, K] e4m3 (lda); sa [K/128, M];  B [2I, K] e4m3 (ldb); sb [2I/128, K/128]
 *   out_q [M, I] e4m3 row stride ld_out; scales [I/128, M]
 * I must be a multiple of 128, K of 128.
 */
int qh_fp8_gemm_silu_quant(const void* A, long lda, const float* sa,
                           const void* B, long ldb, const float* sb, int M,
                           int I, int K, void* out_q, long ld_out,
                           float* scales, int ue8m0, qh_stream_t stream);

/*
 * qh_fp8_gemm_silu_quant with UE8M0 input scales (as qh_fp8_gemm_nt_ue8m0)
 * and UE8M0 output scales (its ue8m0 = 1): the gate_up projection of the
 * reference's UE8M0 mode (attention.py:115, :300-323).
 */
int qh_fp8_gemm_silu_quant_ue8m0(const void* A, long lda, const float* sa,
                                 const void* B, long ldb, const float* sb, int M,
                                 int I, int K, void* out_q, long ld_out,
                                 float* scales, qh_stream_t stream);

/*
 * The qkv projection with the per-head q/k RMSNorm + NeoX rotary in its
 * epilogue: Engine.gemm of qkv_proj (attention.py:129-141) followed by
 * Engine.qk_norm_rope (attention.py:777-781 -> :361-409) and the v
 * .contiguous() copy of Engine.attention (:793), in one kernel that never
 * writes the qkv rows. Bit-identical to qh_fp8_gemm_nt then qh_qk_norm_rope.
 *   A [M, K] e4m3 (row stride lda bytes), sa [K/128, M]; B [N, K] e4m3 with
 *   N = (n_q + 2 n_kv) * 128 (q rows, then k, then v), sb [N/128, K/128]
 *   positions [M] int64; cos_sin [max_pos, 128] bf16 (cos | sin); q_w, k_w
 *   [128] bf16; q_out [M, ld_q] bf16; k_out, v_out [M, ld_kv] bf16.
 *   n_q and n_kv even; ue8m0_scales as in qh_fp8_gemm_nt_ue8m0.
 */
int qh_fp8_gemm_qkv_rope(const void* A, long lda, const float* sa, const void* B,
                         long ldb, const float* sb, int M, int K, int n_q, int n_kv,
                         const int64_t* positions, const void* cos_sin, int max_pos,
                         const void* q_w, const void* k_w, float eps, void* q_out,
                         long ld_q, void* k_out, void* v_out, long ld_kv, int ue8m0_scales,
                         qh_stream_t stream);

/*
 * qh_fp8_gemm_qkv_rope with k and v written straight into the paged arena:
 * row m's k and v go to arena row row_dst[m] (the unified path's
 * qk_norm_rope + kv_row_scatter, attention.py:361-427, called at
 * :777-781 and :933-934). Bit-identical to qh_fp8_gemm_nt then
 * qh_qk_norm_rope_kv. page_tokens must be 16.
 */
int qh_fp8_gemm_qkv_rope_kv(const void* A, long lda, const float* sa, const void* B,
                            long ldb, const float* sb, int M, int K, int n_q, int n_kv,
                            const int64_t* positions, const void* cos_sin, int max_pos,
                            const void* q_w, const void* k_w, float eps, void* q_out,
                            long ld_q, void* k_pool, void* v_pool, const int64_t* row_dst,
                            int page_tokens, int ue8m0_scales, qh_stream_t stream);

/*
 * Per-head RMSNorm of q and k, then NeoX rotary on the two 64-column halves,
 * plus a contiguous copy of v. Replaces Engine.qk_norm_rope
 * (attention.py:777-781 -> Triton qk_norm_rope :361-409) and the v
 * .contiguous() copy of Engine.attention (:793).
 *   qkv  [T, (n_q + 2 n_kv) * d] bf16, row stride ld_qkv
 *   positions [T] int64; cos_sin [max_pos, d] bf16 (cos | sin halves)
 *   qw, kw [d] bf16
 *   q_out [T, n_q * d], k_out [T, n_kv * d], v_out [T, n_kv * d] bf16
 * d must be 128.
 */
int qh_qk_norm_rope(const void* qkv, long ld_qkv, const int64_t* positions,
                    const void* cos_sin, int max_pos, const void* qw,
                    const void* kw, float eps, int T, int n_q, int n_kv, int d,
                    void* q_out, void* k_out, void* v_out, qh_stream_t stream);

/*
 * qh_qk_norm_rope with k and v written straight into the paged arena instead
 * of k_out/v_out: row t's k and v go to arena row dst[t], for every row
 * (the unified path writes each chunk row once). Fuses Engine.qk_norm_rope
 * (attention.py:777-781 -> :361-409) with the unified call's kv_row_scatter
 * (attention.py:411-427, called at :933-934); q_out, and the arena rows, are
 * bit-identical to qh_qk_norm_rope followed by qh_kv_row_scatter.
 *   dst [T] int64 arena rows; pools in the arena layout above.
 */
int qh_qk_norm_rope_kv(const void* qkv, long ld_qkv, const int64_t* positions,
                       const void* cos_sin, int max_pos, const void* qw,
                       const void* kw, float eps, int T, int n_q, int n_kv, int d,
                       void* q_out, void* k_pool, void* v_pool, const int64_t* dst,
                       int page_tokens, qh_stream_t stream);

/*
 * KV append: arena row dst[i] <- chunk row src[i], for K and V.
 * Replaces Triton kv_row_scatter (attention.py:411-427, called at :725-736,
 * :847-848, :933-934). k_src/v_src are [rows, n_kv, d] bf16 contiguous; the
 * pools use the arena layout above.
 */
int qh_kv_row_scatter(const void* k_src, const void* v_src, void* k_pool,
                      void* v_pool, const int64_t* src, const int64_t* dst,
                      int n, int n_kv, int d, int page_tokens,
                      qh_stream_t stream);

/*
 * Arena-to-arena row copy: pool row dst[i] <- pool row src[i], K and V.
 * The unified path's copy of a kept partial last page into a suffix
 * temporary (attention.py:935-938; tail_src/tail_dst, loop.py:182-191).
 */
int qh_kv_row_copy(void* k_pool, void* v_pool, const int64_t* src,
                   const int64_t* dst, int n, int n_kv, int d, int page_tokens,
                   qh_stream_t stream);

/*
 * Varlen attention over queries and keys, bf16 MFMA, fp32 online softmax.
 * One entry point covers the three FlashAttention calls of the reference:
 *   paged causal     unified path, one call (attention.py:939-943)
 *   paged non-causal tree call B over reader rows (attention.py:858-864)
 *   contiguous causal tree call A over the chunk's own rows (:850-852)
 * Sequence s has queries cu_q[s] .. cu_q[s+1]-1 (of packed query rows, or
 * of q_rows[] when q_rows != NULL) and kv_len[s] keys. With table != NULL
 * key j of s is arena row table[s*table_width + j/page]*page + j%page in
 * (k_pool, v_pool); with table == NULL key j is chunk row cu_k[s] + j of
 * k_rows / v_rows ([rows, n_kv, d] bf16 contiguous). Causal is
 * bottom-right aligned: query i of c attends keys 0 .. kv_len - c + i
 * (tests/kv_checker.py:132-139). GQA: q head h reads KV head h / (n_q/n_kv).
 *   q   [rows, n_q, d] bf16 row stride ldq (elements)
 *   out [n_queries, n_q, d] bf16 row stride ldo; row = packed query index
 *   lse optional fp32, lse[h * lse_stride + row], natural log
 * Requires d == 128, page_tokens == 16 and (n_q / n_kv) % 4 == 0.
 * q_rows_total bounds q row indices; pool_pages bounds table entries and
 * kv_rows_total bounds cu_k rows: out-of-range rows and pages read zeros.
 */
size_t qh_attention_workspace_bytes(int n_seqs);
int qh_attention(const void* q, long ldq, int q_rows_total,
                 const int64_t* q_rows, const void* k_pool,
                 const void* v_pool, int pool_pages, const int32_t* table,
                 int table_width, int page_tokens, const void* k_rows,
                 const void* v_rows, int kv_rows_total, const int32_t* cu_k,
                 const int32_t* cu_q, const int32_t* kv_len, int n_seqs,
                 int n_queries, int max_q, int n_q, int n_kv, int d,
                 float softmax_scale, int causal, void* out, long ldo,
                 float* lse, long lse_stride, void* workspace,
                 size_t workspace_bytes, qh_stream_t stream);

/*
 * The unified path's paged causal call fused with the fp8 quantization that
 * follows it: replaces Engine.attention's _paged + quant (attention.py:939-943
 * then :798). Same inputs as the paged form of qh_attention; instead of bf16
 * out it writes out_q [n_queries, n_q*128] e4m3 (row stride ld_out_q bytes)
 * and scales [n_q, n_queries] fp32, one 1x128 group per (row, head), computed
 * from the bf16-rounded output exactly as qh_group_quant would: bit-identical
 * to qh_attention followed by qh_group_quant.
 */
int qh_attention_fp8(const void* q, long ldq, int q_rows_total,
                     const int64_t* q_rows, const void* k_pool,
                     const void* v_pool, int pool_pages, const int32_t* table,
                     int table_width, int page_tokens, const int32_t* cu_q,
                     const int32_t* kv_len, int n_seqs, int n_queries, int max_q,
                     int n_q, int n_kv, int d, float softmax_scale, int causal,
                     void* out_q, long ld_out_q, float* scales, int ue8m0,
                     void* workspace, size_t workspace_bytes,
                     qh_stream_t stream);

/*
 * qh_attention_fp8 without the workspace argument, allocating nothing. No
 * counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The q-tile scan goes to a static 512 KiB device array per GPU,
 * held until the process ends; its device address is looked up on the
 * first call on each device (the device current at the call must be the
 * stream's). At most 131072 sequences per call (QH_E_ARGUMENT beyond).
 * Calls that overlap on one GPU share that array and race; calls in order
 * on one stream do not. Output bit-identical to qh_attention_fp8.
 */
int qh_attention_fp8_noalloc(const void* q, long ldq, int q_rows_total,
                             const int64_t* q_rows, const void* k_pool,
                             const void* v_pool, int pool_pages, const int32_t* table,
                             int table_width, int page_tokens, const int32_t* cu_q,
                             const int32_t* kv_len, int n_seqs, int n_queries, int max_q,
                             int n_q, int n_kv, int d, float softmax_scale, int causal,
                             void* out_q, long ld_out_q, float* scales, int ue8m0,
                             qh_stream_t stream);

/*
 * The tree path's whole attention in one pass: replaces Engine.
 * attention_tree's call A (varlen causal over the chunk's own segments),
 * call B (non-causal paged read of resident KV) and merge_attn_quant
 * (attention.py:835-870, :738-759, :429-473). Row t of causal segment s
 * (cu_a [n_seg + 1] over the chunk's rows; t counted from the segment
 * start) attends the read_used[r] keys of page-table row r = seg_read[s]
 * (none when r = -1) and its segment's own rows 0..t of k_rows / v_rows
 * [n_rows, n_kv, 128] (row stride ld_kv elements), under one softmax:
 * the exact attention that calls A and B + the LSE merge compose. Output
 * as qh_attention (bf16 out, row stride ldo) or, with out_q non-NULL, as
 * qh_attention_fp8 (e4m3 [n_rows, n_q*128] + scales [n_q, n_rows]).
 * Workspace: qh_attention_workspace_bytes(n_seg).
 */
int qh_tree_attention(const void* q, long ldq, int n_rows, const void* k_rows,
                      const void* v_rows, long ld_kv, const int32_t* cu_a,
                      const int32_t* seg_read, int n_seg, const void* k_pool,
                      const void* v_pool, int pool_pages, const int32_t* table,
                      int table_width, const int32_t* read_used, int n_reads,
                      int page_tokens, int n_q, int n_kv, int d,
                      float softmax_scale, void* out, long ldo, void* out_q,
                      long ld_out_q, float* scales, int ue8m0, void* workspace,
                      size_t workspace_bytes, qh_stream_t stream);

/*
 * qh_tree_attention with each node's K and V^T held in LDS (the shared-
 * prefix staging of attention.py:835-870's call B done once per workgroup
 * for all the q-tiles it takes that read the node, rather than once per
 * q-tile); same arguments, same output bits. Needs every page-table row to
 * fit 256 keys (table_width * page_tokens <= 256). One workgroup per CU
 * (the node takes 128 KiB of LDS), so the streaming qh_tree_attention, at
 * three workgroups per CU, is the faster of the two on the shapes measured.
 */
int qh_tree_attention_resident(const void* q, long ldq, int n_rows, const void* k_rows,
                               const void* v_rows, long ld_kv, const int32_t* cu_a,
                               const int32_t* seg_read, int n_seg, const void* k_pool,
                               const void* v_pool, int pool_pages, const int32_t* table,
                               int table_width, const int32_t* read_used, int n_reads,
                               int page_tokens, int n_q, int n_kv, int d,
                               float softmax_scale, void* out, long ldo, void* out_q,
                               long ld_out_q, float* scales, int ue8m0, void* workspace,
                               size_t workspace_bytes, qh_stream_t stream);

/*
 * LSE merge of the tree path's two attention calls fused with per-head fp8
 * quantization. Replaces Triton merge_attn_quant (attention.py:429-473,
 * :738-759): where source[t] >= 0, w = bf16(sigmoid(lse_b - lse_a)),
 * y = bf16(a + (b - a) w); else y = a. One 128-wide group per head.
 *   out_a [T, n_h, 128] bf16, lse_a[h * lse_a_stride + t]
 *   out_b [R, n_h, 128] bf16, lse_b[h * lse_b_stride + r]
 *   source [T] int32; out_q [T, n_h*128] e4m3; scales [n_h, T]
 */
int qh_merge_attn_quant(const void* out_a, const float* lse_a,
                        long lse_a_stride, const void* out_b,
                        const float* lse_b, long lse_b_stride,
                        const int32_t* source, int T, int n_h, void* out_q,
                        float* scales, int ue8m0, qh_stream_t stream);

/*
 * SiLU-gated product + per-token 1x128 fp8 quantization. Replaces
 * Engine.activation_quant -> Triton silu_mul_quant (attention.py:771-775,
 * :644-656, :300-323): y = g * sigmoid(g) * u in fp32.
 *   gate_up [T, 2I] bf16 row stride ld (gate | up); out_q [T, I] e4m3;
 *   scales [I/128, T]. I must be a multiple of 128.
 */
int qh_silu_mul_quant(const void* gate_up, long ld, int T, int I, void* out_q,
                      float* scales, int ue8m0, qh_stream_t stream);

/*
 * Row gather: out[i] = table[idx[i]] for bf16 rows of width W.
 * The embedding lookup (models/qwen3.py:98) and index_select of the
 * final rows (:120-121).
 */
int qh_gather_rows(const void* table, long ld_table, const int64_t* idx,
                   int n, int W, void* out, qh_stream_t stream);

/*
 * Row gather of an fp8 GEMM input with its 1x128 scales:
 * out_q[i] = q[idx[i]] (W bytes), out_scales[g * n + i] = scales[g * T + idx[i]].
 * The reference's index_select of the answer rows (models/qwen3.py:73-74)
 * moved before the last layer's o_proj: only the answer rows' outputs of
 * that layer are read, so o_proj, the post-attention norm and the MLP of
 * the last layer run on those rows alone (each row's values are the same
 * bits either way).
 *   q [T, ldq] e4m3; scales [W/128, T]; idx [n] int64 in [0, T);
 *   out_q [n, ld_out] e4m3; out_scales [W/128, n]. W a multiple of 128,
 *   ldq and ld_out multiples of 16.
 */
int qh_gather_quant_rows(const void* q, long ldq, const float* scales, int T,
                         const int64_t* idx, int n, int W, void* out_q, long ld_out,
                         float* out_scales, qh_stream_t stream);

/*
 * Final norm of the answer rows: vLLM fused_add_rms_norm on rows gathered
 * by final_idx (models/qwen3.py:119-124; attention.py:177-181):
 * r = bf16(h + res); normed = bf16(bf16(r * rstd) * w).
 *   hidden, residual [T, H] bf16; final_idx [R] int64; out [R, H] bf16.
 */
int qh_final_norm(const void* hidden, const void* residual,
                  const int64_t* final_idx, int R, int H, const void* w,
                  float eps, void* normed_out, qh_stream_t stream);

/*
 * vLLM fused_add_rms_norm in place, as Engine.fused_add_rms_norm calls it
 * (attention.py:177-181, models/qwen3.py:75-76): per row,
 * residual <- bf16(hidden + residual); hidden <- bf16(bf16(residual * rstd) * w).
 *   hidden, residual [R, H] bf16 contiguous, both updated in place.
 */
int qh_fused_add_rms_norm(void* hidden, void* residual, int R, int H,
                          const void* w, float eps, qh_stream_t stream);

/*
 * Answer readout: scores = bf16(normed . W_ans^T) (F.linear in bf16,
 * readout.py:45-49), bit = max over TRUE columns > max over FALSE columns,
 * strict, so a tie reads FALSE (readout.py:70-79).
 *   normed [R, H] bf16; w_ans [n_ans, H] bf16; is_true [n_ans] uint8 (host
 *   memory is not accepted: device array); bits [R] uint8; margin [R] fp32
 *   (max TRUE - max FALSE of the bf16 scores) or NULL.
 */
int qh_answer_bits(const void* normed, int R, int H, const void* w_ans,
                   int n_ans, const uint8_t* is_true, uint8_t* bits,
                   float* margin, qh_stream_t stream);

/*
 * The e4m3 encoder of the fused epilogues (attention, gate_up), which leave
 * out the reference's +-448 clamp (attention.py:318) because their inputs
 * never exceed 448 (1 + 2^-24) in magnitude: x [n] fp32 (16-byte aligned,
 * n a multiple of 4) -> out [n] e4m3 bytes, scale 1. No reference
 * counterpart: it exposes the encoder so its saturation of (448, 464] to
 * +-448 is checked on the device.
 */
int qh_e4m3_encode(const float* x, long n, uint8_t* out, qh_stream_t stream);

/*
 * AnswerRows.logits (readout.py:45-49): per row, the largest bf16 score
 * over the TRUE columns and over the FALSE columns, the same scores
 * qh_answer_bits compares.
 *   best_true, best_false [R] bf16 (device).
 */
int qh_answer_logits(const void* normed, int R, int H, const void* w_ans,
                     int n_ans, const uint8_t* is_true, void* best_true,
                     void* best_false, qh_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QUAIL_HIP_H */
