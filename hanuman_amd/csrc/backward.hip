// Data-gradient half of the MoE-layer backward: the VJP of the weighted
// combine (model/moe.py:80-85), of SwiGLU (moe.py:72) and of the router gates
// and logits (moe.py:175-192, and the softmax rule of the measured
// workloads).  The expert GEMMs of the backward run on the grouped GEMM
// (hmoe_grouped_dgrad_*), the gather's VJP on the combine kernel with unit
// weights (hmoe_gather_bwd).
//
// Rounding points follow the forward's dtypes: the cotangent of a bf16
// tensor is rounded to bf16 once, sums over slots and columns accumulate in
// float32 (float64 where a dot product decides a bf16 value).
#include "hmoe_common.h"

namespace hmoe {
namespace {

constexpr int kMaxKBwd = 16;

// ---- combine VJP ------------------------------------------------------------
// One wave per token.  d_ys[pos(t,k)] = bf16(dy[t] * bf16(g[t,k])) (float32
// product, one rounding); d_g[t,k] = bf16(f32(sum_d dy[t,d] * ys[pos,d])) with
// the sum in float64 (every product of a float32 and a bf16 value is exact in
// float64), 0 for dropped slots.  With d_shared, also the cotangent of the
// shared expert's output (moe.py:249-251, each SwiGLU's f32(bf16) result):
// d_shared[t] = bf16(dy[t] / shared_div).
template <int KMAX>
__global__ __launch_bounds__(256) void combine_bwd_kernel(
    const float* __restrict__ dy, const uint16_t* __restrict__ ys,
    const int32_t* __restrict__ slot_pos, const float* __restrict__ gates, int64_t tokens,
    int top_k, int d_model, uint16_t* __restrict__ d_ys, float* __restrict__ d_gates,
    uint16_t* __restrict__ d_shared, float shared_div) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= tokens) return;
  int32_t my_pos = -1;
  float my_g = 0.0f;
  if (lane < top_k) {
    my_pos = slot_pos[t * top_k + lane];
    my_g = bf16_bits_to_f32(f32_to_bf16_bits(gates[t * top_k + lane]));
  }
  int32_t pos[KMAX];
  float g[KMAX];
  double part[KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    pos[k] = __shfl(my_pos, k, 64);
    g[k] = __shfl(my_g, k, 64);
    part[k] = 0.0;
  }
  const int chunks = d_model / 8;
  const float* dy_row = dy + t * d_model;
  // Two chunks per lane per iteration: 2 (K + 2) loads in flight.
  constexpr int kU = KMAX <= 8 ? 2 : 1;
  for (int c0 = lane; c0 < chunks; c0 += 64 * kU) {
    float d[kU][8];
    u32x4 yv[kU][KMAX];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int c = c0 + 64 * u;
      if (c < chunks) {
        const f32x4 a = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(dy_row + c * 8));
        const f32x4 b = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(dy_row + c * 8 + 4));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          d[u][i] = a[i];
          d[u][4 + i] = b[i];
        }
#pragma unroll
        for (int k = 0; k < KMAX; ++k)
          if (k < top_k && pos[k] >= 0)
            yv[u][k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
                ys + static_cast<int64_t>(pos[k]) * d_model + c * 8));
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int c = c0 + 64 * u;
      if (c >= chunks) break;
      if (d_shared != nullptr) {
        u32x4 o;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          o[q] = pack_bf16x2(d[u][2 * q] / shared_div, d[u][2 * q + 1] / shared_div);
        __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(d_shared + t * d_model + c * 8));
      }
#pragma unroll
      for (int k = 0; k < KMAX; ++k) {
        if (k < top_k && pos[k] >= 0) {
          u32x4 o;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            o[q] = pack_bf16x2(d[u][2 * q] * g[k], d[u][2 * q + 1] * g[k]);
            const uint32_t w = yv[u][k][q];
            part[k] += static_cast<double>(d[u][2 * q]) *
                       static_cast<double>(__uint_as_float(w << 16));
            part[k] += static_cast<double>(d[u][2 * q + 1]) *
                       static_cast<double>(__uint_as_float(w & 0xffff0000u));
          }
          __builtin_nontemporal_store(
              o, reinterpret_cast<u32x4*>(d_ys + static_cast<int64_t>(pos[k]) * d_model + c * 8));
        }
      }
    }
  }
  float mine = 0.0f;
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    double v = part[k];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    if (lane == k) mine = bf16_bits_to_f32(f32_to_bf16_bits(static_cast<float>(v)));
  }
  if (lane < top_k) d_gates[t * top_k + lane] = my_pos >= 0 ? mine : 0.0f;
}

// ---- SwiGLU VJP -------------------------------------------------------------
// h = silu(g) * u: dg = dh * u * silu'(g), du = dh * silu(g), silu'(g) =
// s (1 + g (1 - s)), s = 1 / (1 + e^-g), in float32 with one bf16 rounding
// each.  g and u sit in the gate/up GEMM's column order (blocks of 32 gate
// columns then the 32 up columns of the same h columns); dg and du are
// written in the same order.  Rows at or past offsets[n_experts] are skipped.
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const uint16_t* __restrict__ dh,
                                                         const uint16_t* __restrict__ gu,
                                                         const int32_t* __restrict__ offsets,
                                                         int n_experts, int64_t rows, int d_ff,
                                                         uint16_t* __restrict__ dgu) {
  const int64_t kept = offsets != nullptr ? static_cast<int64_t>(offsets[n_experts]) : rows;
  const int64_t n_rows = kept < rows ? kept : rows;
  const int per_row = d_ff / 8;
  const int64_t groups = n_rows * per_row;
  for (int64_t gi = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; gi < groups;
       gi += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t r = gi / per_row;
    const int f0 = static_cast<int>(gi - r * per_row) * 8;
    const int64_t gcol = r * 2 * d_ff + (f0 >> 5) * 64 + (f0 & 31);
    const u32x4 hv = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(dh + r * d_ff + f0));
    const u32x4 gv = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(gu + gcol));
    const u32x4 uv = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(gu + gcol + 32));
    u32x4 og, ou;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float dgq[2], duq[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float d = __uint_as_float(h ? (hv[q] & 0xffff0000u) : (hv[q] << 16));
        const float gg = __uint_as_float(h ? (gv[q] & 0xffff0000u) : (gv[q] << 16));
        const float uu = __uint_as_float(h ? (uv[q] & 0xffff0000u) : (uv[q] << 16));
        swiglu_vjp(d, gg, uu, dgq[h], duq[h]);
      }
      og[q] = pack_bf16x2(dgq[0], dgq[1]);
      ou[q] = pack_bf16x2(duq[0], duq[1]);
    }
    __builtin_nontemporal_store(og, reinterpret_cast<u32x4*>(dgu + gcol));
    __builtin_nontemporal_store(ou, reinterpret_cast<u32x4*>(dgu + gcol + 32));
  }
}

// ---- router VJP -------------------------------------------------------------
// d_logits [T, N] from d_gates [T, K]: zero except the selected experts.
// Softmax rule (g = softmax of the selected logits):
//   dl_k = g_k (dg_k - sum_j g_j dg_j).
// Reference rule (g = rsf s_k / (sum_j s_j + 1e-9), s = sigmoid(l), moe.py:189-192):
//   ds_k = rsf (dg_k / Z - sum_j dg_j s_j / Z^2), dl_k = ds_k s_k (1 - s_k).
// Sums over k run in float32, k ascending.  One wave per token.
__global__ __launch_bounds__(256) void router_bwd_kernel(
    const float* __restrict__ logits, const int32_t* __restrict__ top_idx,
    const float* __restrict__ gates, const float* __restrict__ d_gates, int64_t tokens,
    int n_experts, int top_k, int mode, float rsf, float* __restrict__ d_logits) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= tokens) return;
  int my_e = -1;
  float a = 0.0f, b = 0.0f;  // softmax: (g, dg); reference: (s, dg)
  if (lane < top_k) {
    my_e = top_idx[t * top_k + lane];
    b = d_gates[t * top_k + lane];
    a = mode == HMOE_ROUTE_SOFTMAX ? gates[t * top_k + lane]
                                   : sigmoid_det(logits[t * n_experts + my_e]);
  }
  float s1 = 0.0f, s2 = 0.0f;  // sum_j a_j b_j, sum_j a_j
  for (int j = 0; j < top_k; ++j) {
    const float aj = __shfl(a, j, 64), bj = __shfl(b, j, 64);
    s1 = s1 + aj * bj;
    s2 = s2 + aj;
  }
  float dl = 0.0f;
  if (lane < top_k) {
    if (mode == HMOE_ROUTE_SOFTMAX) {
      dl = a * (b - s1);
    } else {
      const float z = s2 + 1e-9f;
      const float ds = rsf * (b / z - s1 / (z * z));
      dl = ds * a * (1.0f - a);
    }
  }
  for (int n = lane; n < n_experts; n += 64) {
    float v = 0.0f;
    for (int j = 0; j < top_k; ++j) {
      const int ej = __shfl(my_e, j, 64);
      const float dj = __shfl(dl, j, 64);
      if (ej == n) v = dj;
    }
    d_logits[t * n_experts + n] = v;
  }
}

// dx[t, d] (+)= sum_n d_logits[t, n] * W[d, n]  (the VJP of x_f @ router,
// moe.py:178, with respect to x).  Workgroup tile: 128 tokens x 64 columns;
// thread (tg, dg) = (tid / 8, tid % 8) owns tokens tg*4 .. +4 and columns
// dg*8 .. +8 (32 accumulators).  n runs in chunks of 32 through LDS, both
// operands stored n-major there, ascending.
template <typename TW>
__global__ __launch_bounds__(256) void router_dx_kernel(const float* __restrict__ d_logits,
                                                        const TW* __restrict__ w, int64_t tokens,
                                                        int d_model, int n_experts,
                                                        float* __restrict__ dx, int accumulate) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) float sdl[32][128];
  __shared__ __attribute__((aligned(16))) float sw[32][64];
  const int tid = threadIdx.x;
  const int tg = tid >> 3, dg = tid & 7;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * 128;
  const int d0 = blockIdx.y * 64;
  float acc[4][8];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[a][i] = 0.0f;
  for (int n0 = 0; n0 < n_experts; n0 += 32) {
    __syncthreads();
    for (int i = tid; i < 128 * 32; i += 256) {
      const int r = i >> 5, c = i & 31;
      const int64_t t = t0 + r;
      sdl[c][r] = (t < tokens && n0 + c < n_experts) ? d_logits[t * n_experts + n0 + c] : 0.0f;
    }
    for (int i = tid; i < 64 * 32; i += 256) {
      const int dd = i >> 5, c = i & 31;
      float v = 0.0f;
      if (n0 + c < n_experts) {
        const int64_t idx = static_cast<int64_t>(d0 + dd) * n_experts + n0 + c;
        if constexpr (sizeof(TW) == 4) v = w[idx];
        else v = bf16_bits_to_f32(w[idx]);
      }
      sw[c][dd] = v;
    }
    __syncthreads();
    const int nn = n_experts - n0 < 32 ? n_experts - n0 : 32;
    for (int c = 0; c < nn; ++c) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(&sdl[c][tg * 4]);
      const f32x4 w0 = *reinterpret_cast<const f32x4*>(&sw[c][dg * 8]);
      const f32x4 w1 = *reinterpret_cast<const f32x4*>(&sw[c][dg * 8 + 4]);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[r][i] = acc[r][i] + a[r] * w0[i];
          acc[r][4 + i] = acc[r][4 + i] + a[r] * w1[i];
        }
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t t = t0 + tg * 4 + r;
    if (t >= tokens) break;
    float* o = dx + t * d_model + d0 + dg * 8;
    f32x4 r0 = {acc[r][0], acc[r][1], acc[r][2], acc[r][3]};
    f32x4 r1 = {acc[r][4], acc[r][5], acc[r][6], acc[r][7]};
    if (accumulate) {
      const f32x4 p0 = *reinterpret_cast<const f32x4*>(o);
      const f32x4 p1 = *reinterpret_cast<const f32x4*>(o + 4);
      r0 = p0 + r0;
      r1 = p1 + r1;
    }
    *reinterpret_cast<f32x4*>(o) = r0;
    *reinterpret_cast<f32x4*>(o + 4) = r1;
  }
}

// d_router[d, n] = sum_t x[t, d] * d_logits[t, n] (the VJP of x_f @ router,
// moe.py:178, with respect to the router weight), float32, in two passes for
// a fixed summation order: pass 1 sums chunks of kRdwChunk tokens (ascending)
// into partials [chunk][D][N]; pass 2 sums the chunks in order.  Pass 1
// workgroup tile: 64 d x 64 n; thread (dq, nq) = (tid / 16, tid % 16) owns
// d = 4 dq .. +4 and n = 4 nq .. +4, tokens staged 64 at a time in LDS.
constexpr int kRdwChunk = 1024;

template <typename TX>
__global__ __launch_bounds__(256) void router_dw_partial_kernel(const TX* __restrict__ x,
                                                                const float* __restrict__ d_logits,
                                                                int64_t tokens, int d_model,
                                                                int n_experts,
                                                                float* __restrict__ partial) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) float sx[64][64];
  __shared__ __attribute__((aligned(16))) float sl[64][64];
  const int tid = threadIdx.x;
  const int dq = tid >> 4, nq = tid & 15;
  const int d0 = blockIdx.x * 64, n0 = blockIdx.y * 64;
  const int64_t c = blockIdx.z;
  const int64_t t_begin = c * kRdwChunk;
  const int64_t t_end = t_begin + kRdwChunk < tokens ? t_begin + kRdwChunk : tokens;
  float acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = 0.0f;
  for (int64_t t0 = t_begin; t0 < t_end; t0 += 64) {
    __syncthreads();
    for (int i = tid; i < 64 * 64; i += 256) {
      const int r = i >> 6, cc = i & 63;
      const int64_t t = t0 + r;
      float vx = 0.0f, vl = 0.0f;
      if (t < t_end) {
        if constexpr (sizeof(TX) == 4) vx = x[t * d_model + d0 + cc];
        else vx = bf16_bits_to_f32(x[t * d_model + d0 + cc]);
        if (n0 + cc < n_experts) vl = d_logits[t * n_experts + n0 + cc];
      }
      sx[r][cc] = vx;
      sl[r][cc] = vl;
    }
    __syncthreads();
    const int nt = t_end - t0 < 64 ? static_cast<int>(t_end - t0) : 64;
    for (int r = 0; r < nt; ++r) {
      const f32x4 xv = *reinterpret_cast<const f32x4*>(&sx[r][dq * 4]);
      const f32x4 lv = *reinterpret_cast<const f32x4*>(&sl[r][nq * 4]);
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = acc[a][b] + xv[a] * lv[b];
    }
  }
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int d = d0 + dq * 4 + a;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int n = n0 + nq * 4 + b;
      if (n < n_experts) partial[(c * d_model + d) * n_experts + n] = acc[a][b];
    }
  }
}

__global__ __launch_bounds__(256) void router_dw_sum_kernel(const float* __restrict__ partial,
                                                            int chunks, int64_t count,
                                                            float* __restrict__ out) {
#pragma clang fp contract(off)
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < count;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    float v = 0.0f;
    for (int c = 0; c < chunks; ++c) v = v + partial[c * count + i];
    out[i] = v;
  }
}

}  // namespace
}  // namespace hmoe

extern "C" int hmoe_combine_bwd(const float* dy, const void* ys, const int32_t* slot_pos,
                                const float* gates, int64_t tokens, int top_k, int d_model,
                                void* d_ys, float* d_gates, void* d_shared, float shared_div,
                                hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(tokens >= 0, "combine_bwd: tokens must be >= 0");
  HMOE_REQUIRE(top_k >= 1 && top_k <= kMaxKBwd, "combine_bwd: top_k must be in [1, %d] (got %d)",
               kMaxKBwd, top_k);
  HMOE_REQUIRE(d_model >= 8 && d_model % 8 == 0,
               "combine_bwd: d_model must be a multiple of 8 (got %d)", d_model);
  if (tokens == 0) return HMOE_OK;
  HMOE_REQUIRE(dy && ys && slot_pos && gates && d_ys && d_gates, "combine_bwd: null pointer argument");
  HMOE_REQUIRE(d_shared == nullptr || shared_div >= 1.0f,
               "combine_bwd: shared_div must be the number of shared experts (>= 1)");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(ceil_div(tokens, 4)));
  const uint16_t* y = static_cast<const uint16_t*>(ys);
  uint16_t* o = static_cast<uint16_t*>(d_ys);
  uint16_t* sh = static_cast<uint16_t*>(d_shared);
  if (top_k <= 2)
    hipLaunchKernelGGL(combine_bwd_kernel<2>, grid, dim3(256), 0, s, dy, y, slot_pos, gates, tokens, top_k, d_model, o, d_gates, sh, shared_div);
  else if (top_k <= 4)
    hipLaunchKernelGGL(combine_bwd_kernel<4>, grid, dim3(256), 0, s, dy, y, slot_pos, gates, tokens, top_k, d_model, o, d_gates, sh, shared_div);
  else if (top_k <= 8)
    hipLaunchKernelGGL(combine_bwd_kernel<8>, grid, dim3(256), 0, s, dy, y, slot_pos, gates, tokens, top_k, d_model, o, d_gates, sh, shared_div);
  else
    hipLaunchKernelGGL(combine_bwd_kernel<16>, grid, dim3(256), 0, s, dy, y, slot_pos, gates, tokens, top_k, d_model, o, d_gates, sh, shared_div);
  return check_launch("hmoe_combine_bwd");
}

extern "C" int hmoe_swiglu_bwd(const void* dh, const void* gu, const int32_t* offsets,
                               int n_experts, int64_t rows, int d_ff, void* dgu,
                               hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(rows >= 0 && n_experts >= 1, "swiglu_bwd: need rows >= 0 and n_experts >= 1");
  HMOE_REQUIRE(d_ff >= 32 && d_ff % 32 == 0, "swiglu_bwd: d_ff must be a multiple of 32 (got %d)",
               d_ff);
  if (rows == 0) return HMOE_OK;
  HMOE_REQUIRE(dh && gu && dgu, "swiglu_bwd: null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t groups = rows * (d_ff / 8);
  const dim3 grid(static_cast<unsigned>(std::min<int64_t>(ceil_div(groups, 256), 16384)));
  hipLaunchKernelGGL(swiglu_bwd_kernel, grid, dim3(256), 0, s, static_cast<const uint16_t*>(dh),
                     static_cast<const uint16_t*>(gu), offsets, n_experts, rows, d_ff,
                     static_cast<uint16_t*>(dgu));
  return check_launch("hmoe_swiglu_bwd");
}

extern "C" int hmoe_router_bwd(const float* logits, const int32_t* top_idx, const float* gates,
                               const float* d_gates, int64_t tokens, int n_experts, int top_k,
                               int mode, float routed_scaling_factor, float* d_logits,
                               hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(tokens >= 0 && n_experts >= 1 && top_k >= 1 && top_k <= 64 && top_k <= n_experts,
               "router_bwd: need tokens >= 0 and 1 <= top_k <= min(64, n_experts)");
  HMOE_REQUIRE(mode == HMOE_ROUTE_SOFTMAX || mode == HMOE_ROUTE_SIGMOID_BIAS,
               "router_bwd: unknown routing mode %d", mode);
  if (tokens == 0) return HMOE_OK;
  HMOE_REQUIRE(top_idx && d_gates && d_logits, "router_bwd: null pointer argument");
  HMOE_REQUIRE(mode == HMOE_ROUTE_SOFTMAX ? gates != nullptr : logits != nullptr,
               "router_bwd: the softmax rule needs gates, the reference rule logits");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(router_bwd_kernel, dim3(static_cast<unsigned>(ceil_div(tokens, 4))), dim3(256),
                     0, s, logits, top_idx, gates, d_gates, tokens, n_experts, top_k, mode,
                     routed_scaling_factor, d_logits);
  return check_launch("hmoe_router_bwd");
}

extern "C" int hmoe_router_dx(const float* d_logits, const void* router_w, int w_dtype,
                              int64_t tokens, int d_model, int n_experts, float* dx,
                              int accumulate, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(tokens >= 0 && n_experts >= 1, "router_dx: need tokens >= 0 and n_experts >= 1");
  HMOE_REQUIRE(d_model >= 64 && d_model % 64 == 0,
               "router_dx: d_model must be a multiple of 64 (got %d)", d_model);
  HMOE_REQUIRE(w_dtype == HMOE_F32 || w_dtype == HMOE_BF16, "router_dx: W dtype must be F32 or BF16");
  if (tokens == 0) return HMOE_OK;
  HMOE_REQUIRE(d_logits && router_w && dx, "router_dx: null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(ceil_div(tokens, 128)), static_cast<unsigned>(d_model / 64));
  if (w_dtype == HMOE_F32)
    hipLaunchKernelGGL(router_dx_kernel<float>, grid, dim3(256), 0, s, d_logits,
                       static_cast<const float*>(router_w), tokens, d_model, n_experts, dx, accumulate);
  else
    hipLaunchKernelGGL(router_dx_kernel<uint16_t>, grid, dim3(256), 0, s, d_logits,
                       static_cast<const uint16_t*>(router_w), tokens, d_model, n_experts, dx,
                       accumulate);
  return check_launch("hmoe_router_dx");
}

extern "C" size_t hmoe_router_dw_workspace_bytes(int64_t tokens, int d_model, int n_experts) {
  if (tokens <= 0 || d_model <= 0 || n_experts <= 0) return 0;
  return static_cast<size_t>(hmoe::ceil_div(tokens, hmoe::kRdwChunk)) * d_model * n_experts *
         sizeof(float);
}

extern "C" int hmoe_router_dw(const void* x, int x_dtype, const float* d_logits, int64_t tokens,
                              int d_model, int n_experts, float* d_router, void* workspace,
                              size_t workspace_bytes, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(tokens >= 1 && n_experts >= 1, "router_dw: need tokens >= 1 and n_experts >= 1");
  HMOE_REQUIRE(d_model >= 64 && d_model % 64 == 0,
               "router_dw: d_model must be a multiple of 64 (got %d)", d_model);
  HMOE_REQUIRE(x_dtype == HMOE_F32 || x_dtype == HMOE_BF16, "router_dw: x dtype must be F32 or BF16");
  HMOE_REQUIRE(x && d_logits && d_router && workspace, "router_dw: null pointer argument");
  const size_t need = hmoe_router_dw_workspace_bytes(tokens, d_model, n_experts);
  HMOE_REQUIRE_CODE(workspace_bytes >= need, HMOE_ERR_WORKSPACE,
                    "router_dw: workspace of %zu bytes, need %zu", workspace_bytes, need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int chunks = static_cast<int>(ceil_div(tokens, kRdwChunk));
  float* partial = static_cast<float*>(workspace);
  const dim3 grid(static_cast<unsigned>(d_model / 64), static_cast<unsigned>(ceil_div(n_experts, 64)),
                  static_cast<unsigned>(chunks));
  if (x_dtype == HMOE_F32)
    hipLaunchKernelGGL(router_dw_partial_kernel<float>, grid, dim3(256), 0, s,
                       static_cast<const float*>(x), d_logits, tokens, d_model, n_experts, partial);
  else
    hipLaunchKernelGGL(router_dw_partial_kernel<uint16_t>, grid, dim3(256), 0, s,
                       static_cast<const uint16_t*>(x), d_logits, tokens, d_model, n_experts,
                       partial);
  const int64_t count = static_cast<int64_t>(d_model) * n_experts;
  hipLaunchKernelGGL(router_dw_sum_kernel, dim3(static_cast<unsigned>(std::min<int64_t>(ceil_div(count, 256), 4096))),
                     dim3(256), 0, s, partial, chunks, count, d_router);
  return check_launch("hmoe_router_dw");
}
