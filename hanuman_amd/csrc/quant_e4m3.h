// Eight-element row chunks and the per-row e4m3 quantisation of a bf16 or
// float32 row (the activation side of the fp8 expert GEMMs), shared by the
// dispatch kernels and the router launch that also quantises x.
#pragma once

#include "hmoe_common.h"

namespace hmoe {

template <typename TI>
struct Chunk8;
template <>
struct Chunk8<uint16_t> {
  u32x4 v;
  __device__ __forceinline__ void load(const uint16_t* p) { v = *reinterpret_cast<const u32x4*>(p); }
  // For data read exactly once (no reuse through the caches).
  __device__ __forceinline__ void load_nt(const uint16_t* p) {
    v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  }
  __device__ __forceinline__ void zero() { v = u32x4{0u, 0u, 0u, 0u}; }
  __device__ __forceinline__ float get(int i) const {
    const uint32_t w = v[i >> 1];
    return __uint_as_float((i & 1) ? (w & 0xffff0000u) : (w << 16));
  }
};
template <>
struct Chunk8<float> {
  f32x4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = *reinterpret_cast<const f32x4*>(p);
    b = *reinterpret_cast<const f32x4*>(p + 4);
  }
  __device__ __forceinline__ void load_nt(const float* p) {
    a = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    b = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p + 4));
  }
  __device__ __forceinline__ void zero() {
    a = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    b = a;
  }
  __device__ __forceinline__ float get(int i) const { return i < 4 ? a[i] : b[i - 4]; }
};

// Per-row rule: amax = max |v| over the row, codes e4m3(clamp(v * (448/amax),
// +-448)) rounded to nearest even by v_cvt_pk_fp8_f32, dequantisation scale
// amax/448 (both divisions correctly rounded); an all-zero row gets scale 1.
constexpr float kE4m3Max = 448.0f;

// Scale and its inverse from the lane-partial amax (reduced over the wave).
__device__ __forceinline__ void scales_from_amax(float amax, float& s, float& inv) {
  amax = wave_max_f32(amax);
  s = amax > 0.0f ? amax / kE4m3Max : 1.0f;
  inv = amax > 0.0f ? kE4m3Max / amax : 1.0f;
}

template <typename TI>
__device__ __forceinline__ void wave_row_scales(const TI* __restrict__ row, int chunks, float& s,
                                                float& inv) {
  const int lane = threadIdx.x & 63;
  float amax = 0.0f;
  for (int c = lane; c < chunks; c += 64) {
    Chunk8<TI> v;
    v.load(row + static_cast<int64_t>(c) * 8);
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v.get(i)));
  }
  scales_from_amax(amax, s, inv);
}

// Rows of up to 64 * kRowRegs 8-element chunks (4096 elements) are read once
// and kept in registers between the amax reduction and the quantisation.
constexpr int kRowRegs = 8;

template <typename TI>
__device__ __forceinline__ void load_row_regs(const TI* __restrict__ row, int chunks,
                                              Chunk8<TI> (&v)[kRowRegs], float& s, float& inv) {
  const int lane = threadIdx.x & 63;
  float amax = 0.0f;
#pragma unroll
  for (int u = 0; u < kRowRegs; ++u) {
    const int c = u * 64 + lane;
    v[u].zero();
    if (c < chunks) v[u].load_nt(row + static_cast<int64_t>(c) * 8);
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[u].get(i)));
  }
  scales_from_amax(amax, s, inv);
}

template <typename TI>
__device__ __forceinline__ uint2 quant8_e4m3(const Chunk8<TI>& v, float inv) {
  float q[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) q[i] = fminf(fmaxf(v.get(i) * inv, -kE4m3Max), kE4m3Max);
  uint2 out;
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
  out.x = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], w, true));
  w = __builtin_amdgcn_cvt_pk_fp8_f32(q[4], q[5], 0, false);
  out.y = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(q[6], q[7], w, true));
  return out;
}

// One row of `cols` values (a multiple of 8) by one wave: codes into q_row,
// the dequantisation scale into *scale.  REGS: the row fits in registers
// (cols <= 64 * kRowRegs * 8) and is read once; otherwise it is read twice.
template <bool REGS>
__device__ __forceinline__ void quant_row_e4m3(const uint16_t* __restrict__ src, int cols,
                                               uint8_t* __restrict__ q_row, float* scale) {
  const int lane = threadIdx.x & 63;
  const int chunks = cols / 8;
  float s, inv;
  if (REGS) {
    Chunk8<uint16_t> v[kRowRegs];
    load_row_regs(src, chunks, v, s, inv);
    if (lane == 0) *scale = s;
#pragma unroll
    for (int u = 0; u < kRowRegs; ++u) {
      const int c = u * 64 + lane;
      if (c < chunks) *reinterpret_cast<uint2*>(q_row + c * 8) = quant8_e4m3(v[u], inv);
    }
    return;
  }
  wave_row_scales(src, chunks, s, inv);
  if (lane == 0) *scale = s;
  for (int c = lane; c < chunks; c += 64) {
    Chunk8<uint16_t> v;
    v.load(src + static_cast<int64_t>(c) * 8);
    *reinterpret_cast<uint2*>(q_row + c * 8) = quant8_e4m3(v, inv);
  }
}

}  // namespace hmoe
