// Shared helpers for the gfx950 MoE kernels: error reporting, bf16/fp32
// conversions, the deterministic exp used by the router, and the totalOrder
// key used by top-k.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "hanuman_moe.h"

namespace hmoe {

// ---------------------------------------------------------------- errors --
// Thread-local message of the last failure; set by fail() and read through
// hmoe_last_error().
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

#define HMOE_REQUIRE(cond, ...)            \
  do {                                     \
    if (!(cond)) {                         \
      ::hmoe::set_error(__VA_ARGS__);      \
      return HMOE_ERR_INVALID;             \
    }                                      \
  } while (0)

#define HMOE_REQUIRE_CODE(cond, code, ...) \
  do {                                     \
    if (!(cond)) {                         \
      ::hmoe::set_error(__VA_ARGS__);      \
      return (code);                       \
    }                                      \
  } while (0)

// Checks the launch that was just enqueued.
int check_launch(const char* what);

// ------------------------------------------------------------ vector types --
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// bf16 <-> f32 by bit manipulation: exact widening, round-to-nearest-even
// narrowing (NaN kept quiet).  Matches the oracle's bf16_round.
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16_bits(lo)) |
         (static_cast<uint32_t>(f32_to_bf16_bits(hi)) << 16);
}

// VJP of h = silu(g) * u at one element: dg = dh * u * silu'(g),
// du = dh * silu(g), silu'(g) = s (1 + g (1 - s)), s = 1 / (1 + e^-g) with the
// hardware exponential and reciprocal (v_exp_f32, v_rcp_f32: about 1 ulp each,
// far below the bf16 rounding that follows); float32, contraction off, so that
// every kernel that inlines it gives the same bits.
__device__ __forceinline__ void swiglu_vjp(float d, float g, float u, float& dg, float& du) {
#pragma clang fp contract(off)
  const float s = __builtin_amdgcn_rcpf(1.0f + __expf(-g));
  dg = d * u * (s * (1.0f + g * (1.0f - s)));
  du = d * (g * s);
}

// ------------------------------------------------------- deterministic exp --
// Cody-Waite range reduction (Cody & Waite 1980) and a degree-7 Taylor
// polynomial in Horner form, float32, each step one correctly rounded
// operation (contraction disabled), then an exact ldexp.  x > 88.5 -> +inf,
// x < -87 -> +0, NaN -> NaN.  The oracle's exp_det evaluates the identical
// sequence, so results agree bit for bit.
__device__ __forceinline__ float exp_det(float x) {
#pragma clang fp contract(off)
  if (x != x) return x;
  if (x > 88.5f) return __builtin_inff();
  if (x < -87.0f) return 0.0f;
  // Constants by exact float32 bit pattern (shared with the oracle).
  const float kLog2e = __uint_as_float(0x3fb8aa3bu);
  const float kLn2Hi = __uint_as_float(0x3f317200u);  // low 9 bits zero
  const float kLn2Lo = __uint_as_float(0x35bfbe8eu);
  const float c7 = __uint_as_float(0x39500d01u);      // 1/7!
  const float c6 = __uint_as_float(0x3ab60b61u);      // 1/6!
  const float c5 = __uint_as_float(0x3c088889u);      // 1/5!
  const float c4 = __uint_as_float(0x3d2aaaabu);      // 1/4!
  const float c3 = __uint_as_float(0x3e2aaaabu);      // 1/3!
  float n = __builtin_rintf(x * kLog2e);
  float r = x - n * kLn2Hi;
  r = r - n * kLn2Lo;
  float p = c7;
  p = p * r + c6;
  p = p * r + c5;
  p = p * r + c4;
  p = p * r + c3;
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  return __builtin_ldexpf(p, static_cast<int>(n));
}

__device__ __forceinline__ float sigmoid_det(float x) {
#pragma clang fp contract(off)
  return 1.0f / (1.0f + exp_det(-x));
}

// IEEE-754 totalOrder as a signed 32-bit key (-0 < +0).
__device__ __forceinline__ int32_t total_order_key(float f) {
  int32_t b = __float_as_int(f);
  return b ^ ((b >> 31) & 0x7fffffff);
}

__host__ __device__ __forceinline__ int64_t ceil_div(int64_t a, int64_t b) {
  return (a + b - 1) / b;
}

// Lane `src` of v for the whole wave (src wave-uniform): v_readlane, no LDS
// permute; the result is uniform, so addresses built from it are scalar.
__device__ __forceinline__ int32_t lane_bcast(int32_t v, int src) {
  return __builtin_amdgcn_readlane(v, src);
}
__device__ __forceinline__ float lane_bcast(float v, int src) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}

// fmaxf(v, v of the lane the DPP control CTRL names) in the rows ROW_MASK
// enables (other lanes keep v).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_fmax(float v) {
  const int t = __builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROW_MASK,
                                            0xF, false);
  return fmaxf(v, __int_as_float(t));
}

// Wave-wide fmaxf, returned in every lane, with DPP moves on the VALU: within
// each 16-lane row quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror and
// row_mirror leave the row's maximum in all its lanes; row_bcast15 into rows
// 1 and 3 and row_bcast31 into rows 2 and 3 bring the wave's maximum to lane
// 63, which is read out.
__device__ __forceinline__ float wave_max_f32(float v) {
  v = dpp_fmax<0xB1>(v);
  v = dpp_fmax<0x4E>(v);
  v = dpp_fmax<0x141>(v);
  v = dpp_fmax<0x140>(v);
  v = dpp_fmax<0x142, 0xA>(v);
  v = dpp_fmax<0x143, 0xC>(v);
  return lane_bcast(v, 63);
}

}  // namespace hmoe
