// Shared helpers for the gfx950 kernels: bf16 / OCP e4m3 conversions, lane
// reductions, status handling. Device code is written for wave64 only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include "../../include/quail_hip.h"

namespace qh {

constexpr int kWave = 64;
constexpr float kFp8Max = 448.0f;     // largest finite OCP e4m3fn magnitude
constexpr float kScaleFloor = 1e-10f;  // amax floor before the scale divide

// ---- host-side status ------------------------------------------------------

void set_error(const char* fmt, ...);

#define QH_REQUIRE(cond, ...)                 \
  do {                                        \
    if (!(cond)) {                            \
      ::qh::set_error(__VA_ARGS__);           \
      return QH_E_ARGUMENT;                   \
    }                                         \
  } while (0)

// Status of the launch just queued; a launch failure becomes QH_E_HIP.
int launch_status(const char* what);

// Compute units of the current device (cached per device; 256 if unknown):
// the persistent kernels size their grids by it.
int device_cus();

// ---- number formats --------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// IEEE round-to-nearest-even to bf16 (NaN stays a quiet NaN), the rounding
// torch applies in .to(torch.bfloat16).
// fp32 -> bf16 bits, round to nearest even, NaN kept quiet: v_cvt_pk_bf16_f32,
// checked bit for bit on gfx950 against the integer formulation
// ((u + 0x7fff + (u >> 16 & 1)) >> 16, NaN -> (u >> 16) | 0x40) over all
// 2^32 fp32 patterns.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ float round_bf16(float f) {
  return bf16_to_f32(f32_to_bf16(f));
}

// OCP float8_e4m3fn encode with round-to-nearest-even for |x| <= 448
// (callers clamp first, as the reference does): v_cvt_pk_fp8_f32, checked
// bit for bit on gfx950 over every fp32 value in [-448, 448] against the
// integer formulation (normal numbers round the fp32 mantissa to 3 bits with
// ties to even; below 2^-6 the value is an integer multiple of 2^-9 rounded
// with rint, whose carry into 8 lands on the smallest normal's code 0x08).
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x, 0.0f, 0, false) & 0xffu;
}

// y / scale correctly rounded to fp32, as a multiply by an fp64 reciprocal
// rinv within 2^-51 (relative) of 1 / scale (computed once per scale;
// loop-invariant for the callers' loops): with the product's rounding the
// result stays within 2^-50 of the quotient, while a quotient of two fp32
// values that is not itself an fp32 value lies at least 2^-49 (relative)
// from every fp32 rounding midpoint and never on one, so the final rounding
// lands where the IEEE division does. Three instructions per value instead
// of the ~12 of the division sequence.
__device__ __forceinline__ float div_exact(float y, double rinv) {
  return (float)((double)y * rinv);
}

// The fp64 reciprocal div_exact takes, without the IEEE division sequence:
// v_rcp_f64 refined by two Newton steps r += r (1 - s r). Each step squares
// the relative error and adds one rounding (2^-53), so from any starting
// error below 2^-13 the result is within 2^-51 of 1 / s; with the product's
// own rounding the quotient stays within 2^-50, inside the 2^-49 that
// div_exact's argument allows. s is a normal fp32 value, so 1 / s is a
// normal fp64 value and no range scaling is needed.
__device__ __forceinline__ double recip_exact(float s) {
  const double d = (double)s;
  double r = __builtin_amdgcn_rcp(d);
  r = __builtin_fma(r, __builtin_fma(-d, r, 1.0), r);
  r = __builtin_fma(r, __builtin_fma(-d, r, 1.0), r);
  return r;
}

// Scale of one 128-wide group from its absolute maximum: max(amax, 1e-10) /
// 448 (correctly rounded, as div_exact by the fp64 1/448), rounded up to a
// power of two in UE8M0 mode (attention.py:313-316).
__device__ __forceinline__ float group_scale(float amax, bool ue8m0) {
  float s = div_exact(fmaxf(amax, kScaleFloor), 1.0 / (double)kFp8Max);
  if (ue8m0) s = exp2f(ceilf(log2f(s)));
  return s;
}

// s_barrier between compiler memory fences. The builtin alone is modelled as
// touching no memory, so the compiler may move LDS reads and writes across
// it; the fences (no instructions) pin them to their side of the barrier.
// The hardware waits (vmcnt / lgkmcnt) a barrier needs stay explicit at each
// call site.
__device__ __forceinline__ void wg_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The kernel's by-value parameter block read through the kernarg segment at
// the point of use. The empty asm makes the pointer opaque, so the compiler
// cannot hoist these scalar loads to the kernel's start: parameters used only
// after a long loop (epilogue outputs) then hold no scalar registers across
// it, which left to the compiler spilled scalars into VGPR lanes.
template <typename P>
__device__ __forceinline__ const __attribute__((address_space(4))) P* late_params() {
  const __attribute__((address_space(4))) uint8_t* ka =
      (const __attribute__((address_space(4))) uint8_t*)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(ka));
  return reinterpret_cast<const __attribute__((address_space(4))) P*>(ka);
}

// Two values rounded to bf16 by one v_cvt_pk_bf16_f32 and widened back to
// fp32: the same bits as round_bf16 on each.
__device__ __forceinline__ void round_bf16_pair(float& a, float& b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  const f32x2_t x = {a, b};
  const uint32_t u = __builtin_bit_cast(uint32_t, __builtin_convertvector(x, bf16x2_t));
  a = __uint_as_float(u << 16);
  b = __uint_as_float(u & 0xffff0000u);
}

// Four values of one group quantized to e4m3 (y * rinv correctly rounded)
// and packed into one word, value r in byte r, by two v_cvt_pk_fp8_f32: the
// same bits as four quant_e4m3 calls with rinv = 1 / (double)scale, for
// finite values no larger in magnitude than the group maximum amax that
// scale = group_scale(amax) came from. quant_e4m3 clamps to +-448 first, as
// the reference does; here |y / scale| <= amax / scale <= 448 (1 + 2^-24),
// whose fp32 rounding is at most 448 + 2^-15, and v_cvt_pk_fp8_f32 rounds
// every value in [448, 464] to 448 (0x7e; checked on gfx950), so the clamp
// changes no byte and is left out.
__device__ __forceinline__ uint32_t quant_e4m3_x4(float y0, float y1, float y2, float y3,
                                                  double rinv) {
  const float q0 = div_exact(y0, rinv);
  const float q1 = div_exact(y1, rinv);
  const float q2 = div_exact(y2, rinv);
  const float q3 = div_exact(y3, rinv);
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(q0, q1, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(q2, q3, w, true);
  return (uint32_t)w;
}

// The maximum and the sum of a value and its partner lane's (lane ^ 32),
// through v_permlane32_swap: the two halves of the wave trade values in one
// VALU op instead of a ds_bpermute round trip through LDS. Both lanes of a
// pair get bit-identical results (max and + are commutative).
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                  false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// The sum of a value and lane l ^ 16's, through v_permlane16_swap (odd
// 16-lane rows of one operand trade places with even rows of the other):
// both lanes of a pair get the same bits.
__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                  false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// The maximum of a value and its partner lane's as IEEE maximum
// (v_maximum_f32): unlike fmaxf's maxNum it needs no quieting of its inputs.
__device__ __forceinline__ float xor32_maximum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                  false, false);
  return __builtin_elementwise_maximum(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                  false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ uint32_t quant_e4m3(float y, float scale) {
  float q = div_exact(y, recip_exact(scale));
  q = fminf(fmaxf(q, -kFp8Max), kFp8Max);
  return f32_to_e4m3(q);
}

// silu(g) * u = g * sigmoid(g) * u in fp32 with sigmoid(g) = 1 / (1 + e^-g)
// from the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32): the same
// formula the reference's Triton kernel evaluates with its fast exp and
// division (attention.py:311). Products are not contracted, so every caller
// gets the same bits.
__device__ __forceinline__ float silu_mul(float g, float u) {
#pragma clang fp contract(off)
  const float e = __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);
  const float sig = __builtin_amdgcn_rcpf(1.0f + e);
  return g * sig * u;
}

// ---- per-head q/k RMSNorm + NeoX rotary (attention.py:361-409) -----------------
// Shared by qk_norm_rope(_kv) and the qkv GEMM's fused epilogue, which hold a
// head's 128 values in different lane layouts; both follow one order of
// operations, so both produce the same bits. Columns d = 16 ib + 4 g + r
// (ib = 0..7, g = 0..3, r = 0..3): q(ib, g) = fma(x3, x3, fma(x2, x2,
// fma(x1, x1, x0 * x0))) over r; S_g = ((q(0,g) + q(1,g)) + (q(2,g) +
// q(3,g))) + ((q(4,g) + q(5,g)) + (q(6,g) + q(7,g))); total = (S_0 + S_1) +
// (S_2 + S_3). The reference's Triton kernel sums with contracted products
// and takes rstd = 1 / sqrt(ms + eps) with its fast square root; here
// rstd = v_rsq_f32(fma(total, 1/128, eps)) (total / 128 is exact, so the
// fma rounds once, as ms + eps does) and the rotation uses one product and
// one fma per output.
__device__ __forceinline__ float sumsq4(float a, float b, float c, float d) {
  return __builtin_fmaf(d, d, __builtin_fmaf(c, c, __builtin_fmaf(b, b, a * a)));
}

__device__ __forceinline__ float head_rstd(float total, float eps) {
  return __builtin_amdgcn_rsqf(__builtin_fmaf(total, 1.0f / 128.0f, eps));
}

// (x * rstd) * w: the normed value, rounded after each product
__device__ __forceinline__ float head_norm(float x, float rstd, float w) {
  const float y = x * rstd;
  return y * w;
}

// NeoX rotation of the pair (a, b) = (d, d + 64): a' = a cos - b sin (first
// half), b' = b cos + a sin (second half)
__device__ __forceinline__ float rope_first(float a, float b, float c, float s) {
  return __builtin_fmaf(a, c, -(b * s));
}
__device__ __forceinline__ float rope_second(float b, float a, float c, float s) {
  return __builtin_fmaf(b, c, a * s);
}

// ---- lane reductions (wave64) -----------------------------------------------

template <int WIDTH>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = 1; o < WIDTH; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = 1; o < WIDTH; o <<= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// 16-byte vector of 8 bf16.
struct alignas(16) bf16x8 {
  uint32_t w[4];
  __device__ __forceinline__ float get(int i) const {
    return bf16_to_f32((w[i >> 1] >> ((i & 1) * 16)) & 0xffffu);
  }
  __device__ __forceinline__ void set(int i, uint32_t bits) {
    uint32_t sh = (i & 1) * 16;
    w[i >> 1] = (w[i >> 1] & ~(0xffffu << sh)) | ((bits & 0xffffu) << sh);
  }
};

__device__ __forceinline__ bf16x8 load8(const void* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}
__device__ __forceinline__ void store8(void* p, const bf16x8& v) {
  *reinterpret_cast<bf16x8*>(p) = v;
}

}  // namespace qh
