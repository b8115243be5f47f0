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

// ---- number formats --------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// IEEE round-to-nearest-even to bf16 (NaN stays a quiet NaN), the rounding
// torch applies in .to(torch.bfloat16).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ float round_bf16(float f) {
  return bf16_to_f32(f32_to_bf16(f));
}

// OCP float8_e4m3fn encode with round-to-nearest-even for |x| <= 448
// (callers clamp first, as the reference does). Normal numbers round the
// fp32 mantissa to 3 bits; below 2^-6 the value is an integer multiple of
// 2^-9 and rounds with rint, whose carry into 8 lands on the smallest
// normal's code 0x08.
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
  uint32_t u = __float_as_uint(x);
  uint32_t sign = (u >> 24) & 0x80u;
  float a = fabsf(x);
  uint32_t code;
  if (a >= 0.015625f) {
    uint32_t m = (u & 0x7fffffffu);
    m += 0x7ffffu + ((m >> 20) & 1u);
    code = (((m >> 23) - 120u) << 3) | ((m >> 20) & 7u);
  } else {
    code = (uint32_t)__builtin_rintf(a * 512.0f);
  }
  return sign | code;
}

// Scale of one 128-wide group from its absolute maximum: max(amax, 1e-10) /
// 448, rounded up to a power of two in UE8M0 mode (attention.py:313-316).
__device__ __forceinline__ float group_scale(float amax, bool ue8m0) {
  float s = fmaxf(amax, kScaleFloor) / kFp8Max;
  if (ue8m0) s = exp2f(ceilf(log2f(s)));
  return s;
}

__device__ __forceinline__ uint32_t quant_e4m3(float y, float scale) {
  float q = y / scale;
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
