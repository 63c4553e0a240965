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
// One wave per (token, slot).  d_ys[pos(t,k)] = bf16(dy[t] * bf16(g[t,k]))
// (float32 product, one rounding); d_g[t,k] = bf16(f32(sum_d dy[t,d] *
// ys[pos,d])) with the sum in float64 (every product of a float32 and a bf16
// value is exact in float64): each lane sums its 8-column chunks in column
// order, then the wave adds the lanes in a fixed tree.  Dropped slots get
// d_g = 0 and no row.  The K waves of a token read its dy row from L2 after
// the first; a wave holds few registers, so many waves keep loads in flight.
// The k = 0 wave also writes d_shared[t] = bf16(dy[t] / shared_div), the
// cotangent of the shared expert's output (moe.py:249-251).
__global__ __launch_bounds__(256) void combine_bwd_kernel(
    const float* __restrict__ dy, const uint16_t* __restrict__ ys,
    const int32_t* __restrict__ slot_pos, const float* __restrict__ gates, int64_t tokens,
    int top_k, int d_model, uint16_t* __restrict__ d_ys, float* __restrict__ d_gates,
    uint16_t* __restrict__ d_shared, float shared_div) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (w >= tokens * top_k) return;
  const int64_t t = w / top_k;
  const int k = static_cast<int>(w - t * top_k);
  const int32_t pos = slot_pos[w];
  const bool shared = d_shared != nullptr && k == 0;
  if (pos < 0 && !shared) {
    if (lane == 0) d_gates[w] = 0.0f;
    return;
  }
  const float g = bf16_bits_to_f32(f32_to_bf16_bits(gates[w]));
  const int chunks = d_model / 8;
  const float* dy_row = dy + t * d_model;
  const uint16_t* y_row = ys + static_cast<int64_t>(pos < 0 ? 0 : pos) * d_model;
  uint16_t* o_row = d_ys + static_cast<int64_t>(pos < 0 ? 0 : pos) * d_model;
  double part = 0.0;
  constexpr int kU = 4;  // chunks in flight per lane
  for (int c0 = lane; c0 < chunks; c0 += 64 * kU) {
    f32x4 da[kU], db[kU];
    u32x4 yv[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int c = c0 + 64 * u;
      if (c < chunks) {
        // cached: the token's other slots read the same row
        da[u] = *reinterpret_cast<const f32x4*>(dy_row + c * 8);
        db[u] = *reinterpret_cast<const f32x4*>(dy_row + c * 8 + 4);
        if (pos >= 0) yv[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(y_row + c * 8));
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int c = c0 + 64 * u;
      if (c >= chunks) break;
      float d[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        d[i] = da[u][i];
        d[4 + i] = db[u][i];
      }
      if (shared) {
        u32x4 o;
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = pack_bf16x2(d[2 * q] / shared_div, d[2 * q + 1] / shared_div);
        __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(d_shared + t * d_model + c * 8));
      }
      if (pos >= 0) {
        u32x4 o;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          o[q] = pack_bf16x2(d[2 * q] * g, d[2 * q + 1] * g);
          const uint32_t wv = yv[u][q];
          part += static_cast<double>(d[2 * q]) * static_cast<double>(__uint_as_float(wv << 16));
          part += static_cast<double>(d[2 * q + 1]) *
                  static_cast<double>(__uint_as_float(wv & 0xffff0000u));
        }
        __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(o_row + c * 8));
      }
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) part += __shfl_xor(part, off, 64);
  if (lane == 0) d_gates[w] = pos >= 0 ? bf16_bits_to_f32(f32_to_bf16_bits(static_cast<float>(part))) : 0.0f;
}

// Float32 rows (compute dtype float32): d_ys[pos(t,k)] = dy[t] * g[t,k] and
// d_g[t,k] = f32(sum_d dy[t,d] * ys[pos,d]), the sum in float64 (products of
// two float32 values are exact there), lane partials in column order, then a
// fixed tree; d_shared[t] = dy[t] / shared_div.  Same wave layout as above.
__global__ __launch_bounds__(256) void combine_bwd_f32_kernel(
    const float* __restrict__ dy, const float* __restrict__ ys,
    const int32_t* __restrict__ slot_pos, const float* __restrict__ gates, int64_t tokens,
    int top_k, int d_model, float* __restrict__ d_ys, float* __restrict__ d_gates,
    float* __restrict__ d_shared, float shared_div) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (w >= tokens * top_k) return;
  const int64_t t = w / top_k;
  const int k = static_cast<int>(w - t * top_k);
  const int32_t pos = slot_pos[w];
  const bool shared = d_shared != nullptr && k == 0;
  if (pos < 0 && !shared) {
    if (lane == 0) d_gates[w] = 0.0f;
    return;
  }
  const float g = gates[w];
  const int chunks = d_model / 4;
  const float* dy_row = dy + t * d_model;
  const float* y_row = ys + static_cast<int64_t>(pos < 0 ? 0 : pos) * d_model;
  float* o_row = d_ys + static_cast<int64_t>(pos < 0 ? 0 : pos) * d_model;
  double part = 0.0;
  for (int c = lane; c < chunks; c += 64) {
    const f32x4 d = *reinterpret_cast<const f32x4*>(dy_row + c * 4);
    if (shared) {
      f32x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = d[i] / shared_div;
      *reinterpret_cast<f32x4*>(d_shared + t * d_model + c * 4) = o;
    }
    if (pos >= 0) {
      const f32x4 y = *reinterpret_cast<const f32x4*>(y_row + c * 4);
      f32x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[i] = d[i] * g;
        part += static_cast<double>(d[i]) * static_cast<double>(y[i]);
      }
      *reinterpret_cast<f32x4*>(o_row + c * 4) = o;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) part += __shfl_xor(part, off, 64);
  if (lane == 0) d_gates[w] = pos >= 0 ? static_cast<float>(part) : 0.0f;
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
  // The loop bound is the same for every lane, so every shuffle runs with the
  // whole wave active (a shuffle that reads an inactive lane returns 0).
  for (int n0 = 0; n0 < n_experts; n0 += 64) {
    const int n = n0 + lane;
    float v = 0.0f;
    for (int j = 0; j < top_k; ++j) {
      const int ej = __shfl(my_e, j, 64);
      const float dj = __shfl(dl, j, 64);
      if (ej == n) v = dj;
    }
    if (n < n_experts) d_logits[t * n_experts + n] = v;
  }
}

// The two router products run on the float32 matrix cores,
// v_mfma_f32_32x32x2_f32: D[m][n] += A[m][k] B[k][n] over k = 2 per
// instruction, lane L supplying A[L % 32][L / 32] and B[L / 32][L % 32] and
// holding D[m][L % 32] for m = 8 (r / 4) + 4 (L / 32) + r % 4, r = 0..15.
// Products are exact in float32 and accumulate in float32.  Operands are
// staged in LDS with row strides chosen so that the 64 lanes of an operand
// read hit 64 different banks.
__device__ __forceinline__ f32x16 mfma_f32_32x32x2(float a, float b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// dx[t, d] (+)= sum_n d_logits[t, n] * W[d, n]  (the VJP of x_f @ router,
// moe.py:178, with respect to x).  Workgroup tile: 128 tokens x 64 columns
// of d; wave w owns tokens 32 w .. +32 and both 32-column blocks (A = W rows,
// B = d_logits rows, so a lane holds one token and runs of 4 consecutive d).
// n runs in chunks of 64 (zero padded), both operands [row][n] in LDS.
constexpr int kRdxStride = 66;  // 2 (L % 32) + L / 32 covers the 64 banks

template <typename TW>
__global__ __launch_bounds__(256) void router_dx_kernel(const float* __restrict__ d_logits,
                                                        const TW* __restrict__ w, int64_t tokens,
                                                        int d_model, int n_experts,
                                                        float* __restrict__ dx, int accumulate) {
  __shared__ float sl[128 * kRdxStride];
  __shared__ float sw[64 * kRdxStride];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * 128;
  const int d0 = blockIdx.y * 64;
  f32x16 acc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
  const int c = tid & 63;
  const int64_t t = t0 + wave * 32 + l32;
  float* o = dx + t * d_model + d0 + hi * 4;
  // the rows this lane adds into, fetched before anything waits on memory
  f32x4 prev[2][4];
  if (accumulate && t < tokens) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) prev[j][q] = *reinterpret_cast<const f32x4*>(o + j * 32 + q * 8);
  }
  for (int n0 = 0; n0 < n_experts; n0 += 64) {
    const bool nok = n0 + c < n_experts;
    // every load of the chunk is issued before the first LDS write; loads
    // are unconditional (addresses clamped in range), padding is selected
    // to zero afterwards, so no load waits inside a branch
    const int nc = nok ? n0 + c : n_experts - 1;
    float vl[32], vw[16];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const int64_t tr = t0 + (tid >> 6) + 4 * i;
      vl[i] = d_logits[(tr < tokens ? tr : tokens - 1) * n_experts + nc];
    }
    TW rw[16];
#pragma unroll
    for (int i = 0; i < 16; ++i)
      rw[i] = w[static_cast<int64_t>(d0 + (tid >> 6) + 4 * i) * n_experts + nc];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const int64_t tr = t0 + (tid >> 6) + 4 * i;
      vl[i] = (nok && tr < tokens) ? vl[i] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float v;
      if constexpr (sizeof(TW) == 4) v = rw[i];
      else v = bf16_bits_to_f32(rw[i]);
      vw[i] = nok ? v : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 32; ++i) sl[((tid >> 6) + 4 * i) * kRdxStride + c] = vl[i];
#pragma unroll
    for (int i = 0; i < 16; ++i) sw[((tid >> 6) + 4 * i) * kRdxStride + c] = vw[i];
    __syncthreads();
    const float* pb = sl + (wave * 32 + l32) * kRdxStride + hi;
    const float* pa0 = sw + l32 * kRdxStride + hi;
    const float* pa1 = pa0 + 32 * kRdxStride;
#pragma unroll 8
    for (int kk = 0; kk < 64; kk += 2) {
      const float b = pb[kk];
      acc[0] = mfma_f32_32x32x2(pa0[kk], b, acc[0]);
      acc[1] = mfma_f32_32x32x2(pa1[kk], b, acc[1]);
    }
  }
  if (t >= tokens) return;
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f32x4 v = {acc[j][4 * q], acc[j][4 * q + 1], acc[j][4 * q + 2], acc[j][4 * q + 3]};
      if (accumulate) v = prev[j][q] + v;
      *reinterpret_cast<f32x4*>(o + j * 32 + q * 8) = v;
    }
}

// d_router[d, n] = sum_t x[t, d] * d_logits[t, n] (the VJP of x_f @ router,
// moe.py:178, with respect to the router weight), float32, in two passes for
// a fixed summation order: pass 1 sums chunks of kRdwChunk tokens into
// partials [chunk][D][N]; pass 2 sums the chunks in order.  Pass 1
// workgroup tile: 128 d x 64 n of one chunk; wave w owns d 32 w .. +32 and
// both 32-column n blocks (A = x^T, B = d_logits); tokens staged 64 at a time
// in LDS as [token][d] and [token][n].
constexpr int kRdwChunk = 512;
constexpr int kRdwStrideX = 160;  // row offset 32 banks apart: the two k rows never collide
constexpr int kRdwStrideL = 96;

template <typename TX>
__global__ __launch_bounds__(256) void router_dw_partial_kernel(const TX* __restrict__ x,
                                                                const float* __restrict__ d_logits,
                                                                int64_t tokens, int d_model,
                                                                int n_experts,
                                                                float* __restrict__ partial) {
  __shared__ float sx[64 * kRdwStrideX];
  __shared__ float sl[64 * kRdwStrideL];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int d0 = blockIdx.x * 128, n0 = blockIdx.y * 64;
  const int64_t c = blockIdx.z;
  const int64_t t_begin = c * kRdwChunk;
  const int64_t t_end = t_begin + kRdwChunk < tokens ? t_begin + kRdwChunk : tokens;
  f32x16 acc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
  const int cx = tid & 127, cl = tid & 63;
  const bool nok = n0 + cl < n_experts;
  // 64-token steps, software pipelined: step s+1's operands are loaded into
  // registers while step s's MFMAs run.
  // Loads are unconditional (row and column clamped in range) and the
  // padding is zeroed when the registers go to LDS, so no load waits inside
  // a branch.
  const int nc = nok ? n0 + cl : n_experts - 1;
  TX vx[32];
  float vl[16];
  int64_t fetched = t_begin;
  auto fetch = [&](int64_t tt) __attribute__((always_inline)) {
    fetched = tt;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const int64_t t = tt + (tid >> 7) + 2 * i;
      vx[i] = x[(t < t_end ? t : t_end - 1) * d_model + d0 + cx];
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t t = tt + (tid >> 6) + 4 * i;
      vl[i] = d_logits[(t < t_end ? t : t_end - 1) * n_experts + nc];
    }
  };
  fetch(t_begin);
  for (int64_t tt = t_begin; tt < t_end; tt += 64) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      float v;
      if constexpr (sizeof(TX) == 4) v = vx[i];
      else v = bf16_bits_to_f32(vx[i]);
      sx[((tid >> 7) + 2 * i) * kRdwStrideX + cx] = fetched + (tid >> 7) + 2 * i < t_end ? v : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i)
      sl[((tid >> 6) + 4 * i) * kRdwStrideL + cl] =
          (nok && fetched + (tid >> 6) + 4 * i < t_end) ? vl[i] : 0.0f;
    __syncthreads();
    if (tt + 64 < t_end) fetch(tt + 64);
    const float* pa = sx + hi * kRdwStrideX + wave * 32 + l32;
    const float* pb = sl + hi * kRdwStrideL + l32;
#pragma unroll 8
    for (int kk = 0; kk < 64; kk += 2) {
      const float a = pa[kk * kRdwStrideX];
      acc[0] = mfma_f32_32x32x2(a, pb[kk * kRdwStrideL], acc[0]);
      acc[1] = mfma_f32_32x32x2(a, pb[kk * kRdwStrideL + 32], acc[1]);
    }
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + j * 32 + l32;
    if (n >= n_experts) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = d0 + wave * 32 + (r >> 2) * 8 + hi * 4 + (r & 3);
      partial[(c * d_model + d) * n_experts + n] = acc[j][r];
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
  const dim3 grid(static_cast<unsigned>(ceil_div(tokens * top_k, 4)));
  hipLaunchKernelGGL(combine_bwd_kernel, grid, dim3(256), 0, s, dy,
                     static_cast<const uint16_t*>(ys), slot_pos, gates, tokens, top_k, d_model,
                     static_cast<uint16_t*>(d_ys), d_gates, static_cast<uint16_t*>(d_shared),
                     shared_div);
  return check_launch("hmoe_combine_bwd");
}

extern "C" int hmoe_combine_bwd_f32(const float* dy, const float* ys, const int32_t* slot_pos,
                                    const float* gates, int64_t tokens, int top_k, int d_model,
                                    float* d_ys, float* d_gates, float* d_shared, float shared_div,
                                    hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(tokens >= 0, "combine_bwd_f32: tokens must be >= 0");
  HMOE_REQUIRE(top_k >= 1 && top_k <= kMaxKBwd, "combine_bwd_f32: top_k must be in [1, %d] (got %d)",
               kMaxKBwd, top_k);
  HMOE_REQUIRE(d_model >= 4 && d_model % 4 == 0,
               "combine_bwd_f32: d_model must be a multiple of 4 (got %d)", d_model);
  if (tokens == 0) return HMOE_OK;
  HMOE_REQUIRE(dy && ys && slot_pos && gates && d_ys && d_gates,
               "combine_bwd_f32: null pointer argument");
  HMOE_REQUIRE(d_shared == nullptr || shared_div >= 1.0f,
               "combine_bwd_f32: shared_div must be the number of shared experts (>= 1)");
  const dim3 grid(static_cast<unsigned>(ceil_div(tokens * top_k, 4)));
  hipLaunchKernelGGL(combine_bwd_f32_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     dy, ys, slot_pos, gates, tokens, top_k, d_model, d_ys, d_gates, d_shared,
                     shared_div);
  return check_launch("hmoe_combine_bwd_f32");
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
  HMOE_REQUIRE(d_model >= 128 && d_model % 128 == 0,
               "router_dw: d_model must be a multiple of 128 (got %d)", d_model);
  HMOE_REQUIRE(x_dtype == HMOE_F32 || x_dtype == HMOE_BF16, "router_dw: x dtype must be F32 or BF16");
  HMOE_REQUIRE(x && d_logits && d_router && workspace, "router_dw: null pointer argument");
  const size_t need = hmoe_router_dw_workspace_bytes(tokens, d_model, n_experts);
  HMOE_REQUIRE_CODE(workspace_bytes >= need, HMOE_ERR_WORKSPACE,
                    "router_dw: workspace of %zu bytes, need %zu", workspace_bytes, need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int chunks = static_cast<int>(ceil_div(tokens, kRdwChunk));
  float* partial = static_cast<float*>(workspace);
  const dim3 grid(static_cast<unsigned>(d_model / 128), static_cast<unsigned>(ceil_div(n_experts, 64)),
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
