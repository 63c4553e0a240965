// Weighted combine (model/moe.py:80-85): un-permute the expert outputs through
// slot_pos and sum the K slots in float32 with the gates cast to the rows'
// dtype (bf16-rounded for bf16 rows, as they are for float32 rows).
//
// One wave per token.  Lane k < K loads slot k's row index and gate; the wave
// then streams the D columns in 8-element (16-byte bf16) chunks, issuing the
// K row loads of several chunks before accumulating (up to 32 loads in flight
// per lane for bf16 rows).  Rows are read and outputs written exactly once, so
// both use non-temporal accesses (measured 138 -> 120 us at 16384 tokens x 8
// slots x 2048).  Accumulation order is k ascending from +0.0; the
// product of two bf16 values is exact in float32, so a fused multiply-add and
// the oracle's multiply-then-add round identically.
#include "hmoe_common.h"

namespace hmoe {
namespace {

template <typename TY>
struct Row8;
template <>
struct Row8<uint16_t> {
  u32x4 v;
  __device__ __forceinline__ void load(const uint16_t* p) {
    v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  }
  __device__ __forceinline__ float get(int i) const {
    const uint32_t w = v[i >> 1];
    return __uint_as_float((i & 1) ? (w & 0xffff0000u) : (w << 16));
  }
};
template <>
struct Row8<float> {
  f32x4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    b = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p + 4));
  }
  __device__ __forceinline__ float get(int i) const { return i < 4 ? a[i] : b[i - 4]; }
};

template <typename TO>
__device__ __forceinline__ void store_out8(TO* dst, const float (&acc)[8]);
template <>
__device__ __forceinline__ void store_out8<float>(float* dst, const float (&acc)[8]) {
  f32x4 a = {acc[0], acc[1], acc[2], acc[3]};
  f32x4 b = {acc[4], acc[5], acc[6], acc[7]};
  __builtin_nontemporal_store(a, reinterpret_cast<f32x4*>(dst));
  __builtin_nontemporal_store(b, reinterpret_cast<f32x4*>(dst + 4));
}
template <>
__device__ __forceinline__ void store_out8<uint16_t>(uint16_t* dst, const float (&acc)[8]) {
  u32x4 o = {pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]), pack_bf16x2(acc[4], acc[5]),
             pack_bf16x2(acc[6], acc[7])};
  __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(dst));
}

constexpr int kMaxK = 16;

// Chunks whose K row loads are issued together: 32 row loads per lane for
// bf16 rows (4 VGPRs each), 16 for float32 rows (8 VGPRs each).
template <typename TY, int KMAX>
constexpr int chunks_in_flight() {
  constexpr int loads = sizeof(TY) == 2 ? 32 : 16;
  return loads / KMAX < 1 ? 1 : (loads / KMAX > 4 ? 4 : loads / KMAX);
}

// acc + g*y.  For bf16 rows the product is exact in float32, so the fused
// form rounds like the oracle's multiply-then-add; float32 rows need the
// unfused product.
template <typename TY>
__device__ __forceinline__ float madd(float acc, float g, float y);
template <>
__device__ __forceinline__ float madd<uint16_t>(float acc, float g, float y) {
  return __builtin_fmaf(g, y, acc);
}
template <>
__device__ __forceinline__ float madd<float>(float acc, float g, float y) {
#pragma clang fp contract(off)
  const float p = g * y;
  return acc + p;
}

template <typename TY, typename TO, typename TR, int KMAX>
__global__ __launch_bounds__(256) void combine_kernel(const TY* __restrict__ ys,
                                                      const int32_t* __restrict__ slot_pos,
                                                      const float* __restrict__ gates,
                                                      const TR* __restrict__ residual,
                                                      int64_t tokens, int top_k, int d_model,
                                                      TO* __restrict__ out) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= tokens) return;
  int32_t my_pos = -1;
  float my_g = 0.0f;
  if (lane < top_k) {
    my_pos = slot_pos[t * top_k + lane];
    // the gates are cast to the rows' dtype (weights.astype(out.dtype), moe.py:84)
    const float g = gates != nullptr ? gates[t * top_k + lane] : 1.0f;
    my_g = sizeof(TY) == 2 ? bf16_bits_to_f32(f32_to_bf16_bits(g)) : g;
  }
  int32_t pos[KMAX];
  float g[KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    pos[k] = __shfl(my_pos, k, 64);
    g[k] = __shfl(my_g, k, 64);
  }
  constexpr int kChunksInFlight = chunks_in_flight<TY, KMAX>();
  const int chunks = d_model / 8;
  for (int c0 = lane; c0 < chunks; c0 += 64 * kChunksInFlight) {
    Row8<TY> rows[kChunksInFlight][KMAX];
#pragma unroll
    for (int u = 0; u < kChunksInFlight; ++u) {
      const int c = c0 + 64 * u;
#pragma unroll
      for (int k = 0; k < KMAX; ++k)
        if (k < top_k && pos[k] >= 0 && c < chunks)
          rows[u][k].load(ys + static_cast<int64_t>(pos[k]) * d_model + static_cast<int64_t>(c) * 8);
    }
#pragma unroll
    for (int u = 0; u < kChunksInFlight; ++u) {
      const int c = c0 + 64 * u;
      if (c >= chunks) break;
      float acc[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
#pragma unroll
      for (int k = 0; k < KMAX; ++k) {
        if (k < top_k && pos[k] >= 0) {
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[i] = madd<TY>(acc[i], g[k], rows[u][k].get(i));
        }
      }
      if (residual != nullptr) {
        Row8<TR> rr;
        rr.load(residual + t * d_model + static_cast<int64_t>(c) * 8);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = acc[i] + rr.get(i);
      }
      store_out8<TO>(out + t * d_model + static_cast<int64_t>(c) * 8, acc);
    }
  }
}

template <typename TY, typename TO, int KMAX>
void launch_combine3(const void* ys, const int32_t* slot_pos, const float* gates,
                     const void* residual, int residual_dtype, int64_t tokens, int top_k,
                     int d_model, void* out, dim3 grid, hipStream_t s) {
  if (residual_dtype == HMOE_BF16)
    hipLaunchKernelGGL((combine_kernel<TY, TO, uint16_t, KMAX>), grid, dim3(256), 0, s,
                       static_cast<const TY*>(ys), slot_pos, gates,
                       static_cast<const uint16_t*>(residual), tokens, top_k, d_model,
                       static_cast<TO*>(out));
  else
    hipLaunchKernelGGL((combine_kernel<TY, TO, float, KMAX>), grid, dim3(256), 0, s,
                       static_cast<const TY*>(ys), slot_pos, gates,
                       static_cast<const float*>(residual), tokens, top_k, d_model,
                       static_cast<TO*>(out));
}

template <int KMAX>
void launch_combine(const void* ys, int ys_dtype, const int32_t* slot_pos, const float* gates,
                    const void* residual, int residual_dtype, int64_t tokens, int top_k,
                    int d_model, void* out, int out_dtype, dim3 grid, hipStream_t s) {
  if (ys_dtype == HMOE_BF16 && out_dtype == HMOE_F32)
    launch_combine3<uint16_t, float, KMAX>(ys, slot_pos, gates, residual, residual_dtype, tokens, top_k, d_model, out, grid, s);
  else if (ys_dtype == HMOE_BF16 && out_dtype == HMOE_BF16)
    launch_combine3<uint16_t, uint16_t, KMAX>(ys, slot_pos, gates, residual, residual_dtype, tokens, top_k, d_model, out, grid, s);
  else if (ys_dtype == HMOE_F32 && out_dtype == HMOE_F32)
    launch_combine3<float, float, KMAX>(ys, slot_pos, gates, residual, residual_dtype, tokens, top_k, d_model, out, grid, s);
  else
    launch_combine3<float, uint16_t, KMAX>(ys, slot_pos, gates, residual, residual_dtype, tokens, top_k, d_model, out, grid, s);
}

}  // namespace
}  // namespace hmoe

extern "C" int hmoe_combine(const void* ys, int ys_dtype, const int32_t* slot_pos,
                            const float* gates, const void* residual, int residual_dtype,
                            int64_t tokens, int top_k, int d_model, void* out, int out_dtype,
                            hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(tokens >= 0, "combine: tokens must be >= 0");
  HMOE_REQUIRE(top_k >= 1 && top_k <= kMaxK, "combine: top_k must be in [1, %d] (got %d)", kMaxK,
               top_k);
  HMOE_REQUIRE(d_model >= 8 && d_model % 8 == 0, "combine: d_model must be a multiple of 8 (got %d)",
               d_model);
  HMOE_REQUIRE((ys_dtype == HMOE_BF16 || ys_dtype == HMOE_F32) &&
                   (out_dtype == HMOE_BF16 || out_dtype == HMOE_F32),
               "combine: dtypes must be F32 or BF16");
  HMOE_REQUIRE(residual == nullptr || residual_dtype == HMOE_BF16 || residual_dtype == HMOE_F32,
               "combine: residual dtype must be F32 or BF16");
  if (tokens == 0) return HMOE_OK;
  HMOE_REQUIRE(ys && slot_pos && out, "combine: null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(ceil_div(tokens, 4)));
  if (top_k <= 2)
    launch_combine<2>(ys, ys_dtype, slot_pos, gates, residual, residual_dtype, tokens, top_k, d_model, out, out_dtype, grid, s);
  else if (top_k <= 4)
    launch_combine<4>(ys, ys_dtype, slot_pos, gates, residual, residual_dtype, tokens, top_k, d_model, out, out_dtype, grid, s);
  else if (top_k <= 8)
    launch_combine<8>(ys, ys_dtype, slot_pos, gates, residual, residual_dtype, tokens, top_k, d_model, out, out_dtype, grid, s);
  else
    launch_combine<16>(ys, ys_dtype, slot_pos, gates, residual, residual_dtype, tokens, top_k, d_model, out, out_dtype, grid, s);
  return check_launch("hmoe_combine");
}

// The VJP of the row gather xs[j] = x_flat[perm_src[j] / K] (moe.py:56):
// dx[t] = sum_k d_xs[slot_pos[t*K+k]] over kept slots, k ascending in float32
// -- the combine with unit weights; a residual (the shared expert's input
// gradient) is added last.
extern "C" int hmoe_gather_bwd(const void* d_xs, int d_xs_dtype, const int32_t* slot_pos,
                               const void* residual, int residual_dtype, int64_t tokens,
                               int top_k, int d_model, void* dx, int dx_dtype,
                               hmoe_stream_t stream) {
  return hmoe_combine(d_xs, d_xs_dtype, slot_pos, nullptr, residual, residual_dtype, tokens,
                      top_k, d_model, dx, dx_dtype, stream);
}
