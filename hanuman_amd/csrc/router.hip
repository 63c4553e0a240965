// Router: fp32 logits, top-k selection and gate weights (model/moe.py:175-192).
//
// One workgroup of 4 waves handles 32 tokens; each wave owns 8 tokens and a
// lane owns experts lane, lane+64, ... (EPL per lane).  Logits accumulate in
// float64 with d ascending: the products of bf16/fp32 activations and
// fp32/bf16 weights are exact in float64, so the fused multiply-add gives the
// same bits as the oracle's multiply-then-add, and the single rounding to
// float32 at the end makes the logits reproducible bit for bit.  Top-k is K
// rounds of a wave-wide max over a packed (totalOrder key, ~expert) 64-bit
// value, so equal keys resolve to the lower expert index.
#include "hmoe_common.h"

namespace hmoe {
namespace {

constexpr int kWaves = 4;
constexpr int kTokPerWave = 8;
constexpr int kTokPerBlock = kWaves * kTokPerWave;
constexpr int kDChunk = 32;

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    uint64_t o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  return v;
}

__device__ __forceinline__ uint64_t pack_key(float key, int e) {
  const uint32_t u = static_cast<uint32_t>(total_order_key(key)) ^ 0x80000000u;
  return (static_cast<uint64_t>(u) << 32) | static_cast<uint64_t>(0xffffffffu - static_cast<uint32_t>(e));
}

// Selection + gates for one token whose logits are spread over the wave
// (lane owns experts lane + 64*j).  Lane k < K writes slot k.
template <int EPL>
__device__ __forceinline__ void select_and_gate(const float (&logit)[EPL], const float* __restrict__ bias,
                                                int n_experts, int top_k, int mode, float rsf,
                                                int32_t* __restrict__ top_idx_row,
                                                float* __restrict__ gates_row) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  float val[EPL];  // value the gate is built from: sigmoid score or logit
  uint64_t packed[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    float key = logit[j];
    if (mode == HMOE_ROUTE_SIGMOID_BIAS) {
      const float s = sigmoid_det(logit[j]);
      val[j] = s;
      key = s + ((bias != nullptr && e < n_experts) ? bias[e] : 0.0f);
    } else {
      val[j] = logit[j];
    }
    packed[j] = e < n_experts ? pack_key(key, e) : 0ull;
  }
  int my_e = 0;
  for (int k = 0; k < top_k; ++k) {
    uint64_t best = packed[0];
#pragma unroll
    for (int j = 1; j < EPL; ++j) best = packed[j] > best ? packed[j] : best;
    best = wave_max_u64(best);
    const int e_win = static_cast<int>(0xffffffffu - static_cast<uint32_t>(best));
    if (lane == k) my_e = e_win;
#pragma unroll
    for (int j = 0; j < EPL; ++j)
      if (lane + 64 * j == e_win) packed[j] = 0ull;
  }
  // Fetch the selected experts' values from their owner lanes.
  float my_v = 0.0f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const float v = __shfl(val[j], my_e & 63, 64);
    if ((my_e >> 6) == j) my_v = v;
  }
  float w;
  if (mode == HMOE_ROUTE_SIGMOID_BIAS) {
    float denom = 0.0f;
    for (int k = 0; k < top_k; ++k) denom = denom + __shfl(my_v, k, 64);
    denom = denom + 1e-9f;
    w = (my_v / denom) * rsf;
  } else {
    const float m = __shfl(my_v, 0, 64);
    const float ex = exp_det(my_v - m);
    float denom = 0.0f;
    for (int k = 0; k < top_k; ++k) denom = denom + __shfl(ex, k, 64);
    w = ex / denom;
  }
  if (lane < top_k) {
    top_idx_row[lane] = my_e;
    gates_row[lane] = w;
  }
}

template <typename XT>
__device__ __forceinline__ double load_as_f64(const XT* p, int64_t i);
template <>
__device__ __forceinline__ double load_as_f64<float>(const float* p, int64_t i) {
  return static_cast<double>(p[i]);
}
template <>
__device__ __forceinline__ double load_as_f64<uint16_t>(const uint16_t* p, int64_t i) {
  return static_cast<double>(bf16_bits_to_f32(p[i]));
}

template <int EPL, typename XT, typename WT>
__global__ __launch_bounds__(256) void router_kernel(const XT* __restrict__ x, const WT* __restrict__ w,
                                                     const float* __restrict__ bias, int64_t tokens,
                                                     int d_model, int n_experts, int top_k, int mode,
                                                     float rsf, float* __restrict__ logits,
                                                     int32_t* __restrict__ top_idx,
                                                     float* __restrict__ gates) {
  __shared__ double xs_lds[kTokPerBlock][kDChunk + 1];
  __shared__ double w_lds[kDChunk][64 * EPL];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kTokPerBlock;

  double acc[kTokPerWave][EPL];
#pragma unroll
  for (int t = 0; t < kTokPerWave; ++t)
#pragma unroll
    for (int j = 0; j < EPL; ++j) acc[t][j] = 0.0;

  for (int d0 = 0; d0 < d_model; d0 += kDChunk) {
    __syncthreads();
    for (int i = tid; i < kTokPerBlock * kDChunk; i += 256) {
      const int tt = i / kDChunk, dd = i % kDChunk;
      const int64_t t = t0 + tt;
      const int d = d0 + dd;
      xs_lds[tt][dd] = (t < tokens && d < d_model) ? load_as_f64(x, t * d_model + d) : 0.0;
    }
    for (int i = tid; i < kDChunk * 64 * EPL; i += 256) {
      const int dd = i / (64 * EPL), e = i % (64 * EPL);
      const int d = d0 + dd;
      w_lds[dd][e] = (e < n_experts && d < d_model)
                         ? load_as_f64(w, static_cast<int64_t>(d) * n_experts + e)
                         : 0.0;
    }
    __syncthreads();
#pragma unroll 4
    for (int dd = 0; dd < kDChunk; ++dd) {
      double wv[EPL];
#pragma unroll
      for (int j = 0; j < EPL; ++j) wv[j] = w_lds[dd][lane + 64 * j];
#pragma unroll
      for (int t = 0; t < kTokPerWave; ++t) {
        const double xv = xs_lds[wave * kTokPerWave + t][dd];
#pragma unroll
        for (int j = 0; j < EPL; ++j) acc[t][j] = __builtin_fma(xv, wv[j], acc[t][j]);
      }
    }
  }

#pragma unroll 1
  for (int t = 0; t < kTokPerWave; ++t) {
    const int64_t tok = t0 + wave * kTokPerWave + t;
    if (tok >= tokens) break;
    float l[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      l[j] = static_cast<float>(acc[t][j]);
      const int e = lane + 64 * j;
      if (e < n_experts) logits[tok * n_experts + e] = l[j];
    }
    select_and_gate<EPL>(l, bias, n_experts, top_k, mode, rsf, top_idx + tok * top_k,
                         gates + tok * top_k);
  }
}

// One wave per token: selection and gates from given logits.
template <int EPL>
__global__ __launch_bounds__(256) void select_kernel(const float* __restrict__ logits,
                                                     const float* __restrict__ bias, int64_t tokens,
                                                     int n_experts, int top_k, int mode, float rsf,
                                                     int32_t* __restrict__ top_idx,
                                                     float* __restrict__ gates) {
  const int lane = threadIdx.x & 63;
  const int64_t tok = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (tok >= tokens) return;
  float l[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    l[j] = e < n_experts ? logits[tok * n_experts + e] : 0.0f;
  }
  select_and_gate<EPL>(l, bias, n_experts, top_k, mode, rsf, top_idx + tok * top_k,
                       gates + tok * top_k);
}

template <int EPL, typename XT, typename WT>
void launch_router(const void* x, const void* w, const float* bias, int64_t tokens, int d_model,
                   int n_experts, int top_k, int mode, float rsf, float* logits, int32_t* top_idx,
                   float* gates, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(ceil_div(tokens, kTokPerBlock)));
  hipLaunchKernelGGL((router_kernel<EPL, XT, WT>), grid, dim3(256), 0, stream,
                     static_cast<const XT*>(x), static_cast<const WT*>(w), bias, tokens, d_model,
                     n_experts, top_k, mode, rsf, logits, top_idx, gates);
}

template <int EPL>
void dispatch_router(int x_dtype, int w_dtype, const void* x, const void* w, const float* bias,
                     int64_t tokens, int d_model, int n_experts, int top_k, int mode, float rsf,
                     float* logits, int32_t* top_idx, float* gates, hipStream_t s) {
  if (x_dtype == HMOE_BF16 && w_dtype == HMOE_F32)
    launch_router<EPL, uint16_t, float>(x, w, bias, tokens, d_model, n_experts, top_k, mode, rsf, logits, top_idx, gates, s);
  else if (x_dtype == HMOE_F32 && w_dtype == HMOE_F32)
    launch_router<EPL, float, float>(x, w, bias, tokens, d_model, n_experts, top_k, mode, rsf, logits, top_idx, gates, s);
  else if (x_dtype == HMOE_BF16 && w_dtype == HMOE_BF16)
    launch_router<EPL, uint16_t, uint16_t>(x, w, bias, tokens, d_model, n_experts, top_k, mode, rsf, logits, top_idx, gates, s);
  else
    launch_router<EPL, float, uint16_t>(x, w, bias, tokens, d_model, n_experts, top_k, mode, rsf, logits, top_idx, gates, s);
}

int validate_routing(int64_t tokens, int n_experts, int top_k, int mode) {
  HMOE_REQUIRE(tokens >= 0, "router: tokens must be >= 0 (got %lld)", (long long)tokens);
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= 256, "router: n_experts must be in [1, 256] (got %d)",
               n_experts);
  HMOE_REQUIRE(top_k >= 1 && top_k <= n_experts && top_k <= 32,
               "router: top_k must be in [1, min(n_experts, 32)] (got %d, n_experts %d)", top_k,
               n_experts);
  HMOE_REQUIRE(mode == HMOE_ROUTE_SIGMOID_BIAS || mode == HMOE_ROUTE_SOFTMAX,
               "router: unknown routing mode %d", mode);
  return HMOE_OK;
}

}  // namespace
}  // namespace hmoe

extern "C" int hmoe_router(const void* x, int x_dtype, const void* router_w, int w_dtype,
                           const float* bias, int64_t tokens, int d_model, int n_experts,
                           int top_k, int mode, float routed_scaling_factor, float* logits,
                           int32_t* top_idx, float* gates, hmoe_stream_t stream) {
  using namespace hmoe;
  if (int rc = validate_routing(tokens, n_experts, top_k, mode)) return rc;
  HMOE_REQUIRE(d_model >= 1, "router: d_model must be >= 1 (got %d)", d_model);
  HMOE_REQUIRE(x_dtype == HMOE_F32 || x_dtype == HMOE_BF16, "router: x dtype must be F32 or BF16");
  HMOE_REQUIRE(w_dtype == HMOE_F32 || w_dtype == HMOE_BF16, "router: weight dtype must be F32 or BF16");
  if (tokens == 0) return HMOE_OK;
  HMOE_REQUIRE(x && router_w && logits && top_idx && gates, "router: null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (n_experts <= 64)
    dispatch_router<1>(x_dtype, w_dtype, x, router_w, bias, tokens, d_model, n_experts, top_k, mode, routed_scaling_factor, logits, top_idx, gates, s);
  else if (n_experts <= 128)
    dispatch_router<2>(x_dtype, w_dtype, x, router_w, bias, tokens, d_model, n_experts, top_k, mode, routed_scaling_factor, logits, top_idx, gates, s);
  else
    dispatch_router<4>(x_dtype, w_dtype, x, router_w, bias, tokens, d_model, n_experts, top_k, mode, routed_scaling_factor, logits, top_idx, gates, s);
  return check_launch("hmoe_router");
}

extern "C" int hmoe_router_from_logits(const float* logits, const float* bias, int64_t tokens,
                                       int n_experts, int top_k, int mode,
                                       float routed_scaling_factor, int32_t* top_idx,
                                       float* gates, hmoe_stream_t stream) {
  using namespace hmoe;
  if (int rc = validate_routing(tokens, n_experts, top_k, mode)) return rc;
  if (tokens == 0) return HMOE_OK;
  HMOE_REQUIRE(logits && top_idx && gates, "router_from_logits: null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(ceil_div(tokens, 4)));
  if (n_experts <= 64)
    hipLaunchKernelGGL(select_kernel<1>, grid, dim3(256), 0, s, logits, bias, tokens, n_experts, top_k, mode, routed_scaling_factor, top_idx, gates);
  else if (n_experts <= 128)
    hipLaunchKernelGGL(select_kernel<2>, grid, dim3(256), 0, s, logits, bias, tokens, n_experts, top_k, mode, routed_scaling_factor, top_idx, gates);
  else
    hipLaunchKernelGGL(select_kernel<4>, grid, dim3(256), 0, s, logits, bias, tokens, n_experts, top_k, mode, routed_scaling_factor, top_idx, gates);
  return check_launch("hmoe_router_from_logits");
}
