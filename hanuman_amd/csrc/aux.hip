// Router aux outputs (model/moe.py:253-292): router_z_loss, balance_loss,
// mean_entropy and expert_counts, from the router logits and top-k indices.
//
// Pass 1: one workgroup per 64-token chunk of one sequence; each wave takes
// every fourth token, lanes own experts.  Per token it forms logsumexp,
// sigmoid scores, the normalised routing distribution p and its entropy; it
// accumulates p per expert and lse^2 / entropy per wave, then the four waves
// are summed in a fixed order.  The chunk's per-sequence expert histogram is
// counted in LDS.  Pass 2: one workgroup reduces the chunk partials into the
// four outputs.  Every float reduction has a fixed order, so results are
// identical from run to run.
#include "hmoe_common.h"

namespace hmoe {
namespace {

constexpr int kChunk = 64;
constexpr int kMaxN = 256;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Partial layout per chunk: probs[N], counts[N] (as int), z, ent.
__host__ __device__ inline int64_t part_stride(int n) { return 2 * static_cast<int64_t>(n) + 2; }

template <int EPL>
__global__ __launch_bounds__(256) void aux_chunk_kernel(const float* __restrict__ logits,
                                                        const int32_t* __restrict__ top_idx,
                                                        int seq, int n_experts, int top_k,
                                                        int chunks_per_seq,
                                                        float* __restrict__ parts) {
  __shared__ float wprobs[4][kMaxN];
  __shared__ float wz[4], went[4];
  __shared__ int32_t hist[kMaxN];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int chunk = blockIdx.x;
  const int b = chunk / chunks_per_seq;
  const int c = chunk % chunks_per_seq;
  const int s0 = c * kChunk;
  const int s1 = min(seq, s0 + kChunk);
  const int64_t tok0 = static_cast<int64_t>(b) * seq;
  for (int e = tid; e < n_experts; e += 256) hist[e] = 0;
  __syncthreads();
  for (int i = tid; i < (s1 - s0) * top_k; i += 256) {
    const int e = top_idx[(tok0 + s0) * top_k + i];
    if (static_cast<unsigned>(e) < static_cast<unsigned>(n_experts)) atomicAdd(&hist[e], 1);
  }
  float pacc[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) pacc[j] = 0.0f;
  float zacc = 0.0f, eacc = 0.0f;
  for (int s = s0 + wave; s < s1; s += 4) {
    const float* row = logits + (tok0 + s) * n_experts;
    float l[EPL], sg[EPL];
    float m = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int e = lane + 64 * j;
      l[j] = e < n_experts ? row[e] : -__builtin_inff();
      m = fmaxf(m, l[j]);
    }
    m = wave_max(m);
    float se = 0.0f, ss = 0.0f;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const bool ok = lane + 64 * j < n_experts;
      se += ok ? expf(l[j] - m) : 0.0f;
      sg[j] = ok ? sigmoid_det(l[j]) : 0.0f;
      ss += sg[j];
    }
    se = wave_sum(se);
    ss = wave_sum(ss);
    const float lse = m + logf(se);
    float ent = 0.0f;
    const float inv = 1.0f / (ss + 1e-9f);
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const float p = sg[j] * inv;
      pacc[j] += p;
      if (lane + 64 * j < n_experts) ent -= p * logf(p + 1e-9f);
    }
    ent = wave_sum(ent);
    zacc += lse * lse;
    eacc += ent;
  }
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    if (e < n_experts) wprobs[wave][e] = pacc[j];
  }
  if (lane == 0) {
    wz[wave] = zacc;
    went[wave] = eacc;
  }
  __syncthreads();
  float* out = parts + static_cast<int64_t>(chunk) * part_stride(n_experts);
  for (int e = tid; e < n_experts; e += 256) {
    out[e] = ((wprobs[0][e] + wprobs[1][e]) + wprobs[2][e]) + wprobs[3][e];
    reinterpret_cast<int32_t*>(out)[n_experts + e] = hist[e];
  }
  if (tid == 0) {
    out[2 * n_experts] = ((wz[0] + wz[1]) + wz[2]) + wz[3];
    out[2 * n_experts + 1] = ((went[0] + went[1]) + went[2]) + went[3];
  }
}

// One workgroup of 1024 threads, every loop over the chunk partials spread
// over the threads (the serial version was bound by one dependent load per
// chunk).  z and entropy: thread t sums chunks t, t + 1024, ... in order, then
// the wave sums and the 16 wave totals in order.  Balance: sequences in
// rounds of G, one thread per (sequence, expert) summing that sequence's
// chunks in order; per sequence its expert terms are summed in a fixed order
// and the sequences in order.  Counts are exact integers (LDS atomics).  Every
// float reduction has a fixed order.
constexpr int kFinalThreads = 1024;

__global__ __launch_bounds__(kFinalThreads) void aux_final_kernel(
    const float* __restrict__ parts, int batch, int seq, int n_experts, int top_k,
    int chunks_per_seq, float* __restrict__ losses, float* __restrict__ expert_counts) {
  __shared__ int32_t cnt_e[kMaxN];
  __shared__ float terms[kFinalThreads];
  __shared__ float wtot[2][kFinalThreads / 64];
  __shared__ float bal_round[kFinalThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t stride = part_stride(n_experts);
  const int nchunks = batch * chunks_per_seq;
  for (int e = tid; e < n_experts; e += kFinalThreads) cnt_e[e] = 0;

  float z = 0.0f, ent = 0.0f;
  for (int ch = tid; ch < nchunks; ch += kFinalThreads) {
    z += parts[ch * stride + 2 * n_experts];
    ent += parts[ch * stride + 2 * n_experts + 1];
  }
  z = wave_sum(z);
  ent = wave_sum(ent);
  if (lane == 0) {
    wtot[0][wave] = z;
    wtot[1][wave] = ent;
  }
  __syncthreads();

  // threads per sequence: n_experts rounded up to whole waves
  const int tps = (n_experts + 63) / 64 * 64;
  const int per_round = kFinalThreads / tps;
  const int bl = tid / tps, e = tid % tps;
  float bal = 0.0f;
  for (int b0 = 0; b0 < batch; b0 += per_round) {
    const int b = b0 + bl;
    float term = 0.0f;
    if (bl < per_round && b < batch && e < n_experts) {
      float psum = 0.0f;
      int32_t cnt = 0;
#pragma unroll 8
      for (int c = 0; c < chunks_per_seq; ++c) {
        const float* pp = parts + static_cast<int64_t>(b * chunks_per_seq + c) * stride;
        psum += pp[e];
        cnt += reinterpret_cast<const int32_t*>(pp)[n_experts + e];
      }
      atomicAdd(&cnt_e[e], cnt);
      const float frac = static_cast<float>(cnt) / static_cast<float>(seq * top_k);
      term = frac * (psum / static_cast<float>(seq));
    }
    terms[tid] = term;
    __syncthreads();
    // the first wave of each sequence's group sums its expert terms
    if (bl < per_round && e < 64) {
      float acc = 0.0f;
      for (int k = e; k < tps; k += 64) acc += terms[bl * tps + k];
      acc = wave_sum(acc);
      if (e == 0) bal_round[bl] = static_cast<float>(n_experts) * acc;
    }
    __syncthreads();
    if (tid == 0)
      for (int q = 0; q < per_round && b0 + q < batch; ++q) bal += bal_round[q];
    __syncthreads();
  }
  for (int k = tid; k < n_experts; k += kFinalThreads) expert_counts[k] = static_cast<float>(cnt_e[k]);
  if (tid == 0) {
    float zt = 0.0f, et = 0.0f;
    for (int w = 0; w < kFinalThreads / 64; ++w) {
      zt += wtot[0][w];
      et += wtot[1][w];
    }
    const float tokens = static_cast<float>(batch) * static_cast<float>(seq);
    losses[0] = zt / tokens;
    losses[1] = bal / static_cast<float>(batch);
    losses[2] = et / tokens;
  }
}

// ---- VJP of the aux losses with respect to the logits ------------------------
// The expert counts come from the top-k indices and carry no derivative, so
// the backward needs them only as constants: pass 1 histograms each 64-token
// chunk, pass 2 sums a sequence's chunks into f[b,n] = counts / (S*K), pass 3
// differentiates per token (T = B*S, q = softmax(l), s = sigmoid(l),
// Z = sum s + 1e-9, p = s / Z):
//   z-loss     dl += d_z * 2 lse / T * q
//   balance    dp  = d_bal * N f[b,n] / (B*S)
//   entropy    dp -= d_ent * (log(p + 1e-9) + p / (p + 1e-9)) / T
//   p = s/Z    ds  = dp / Z - sum(dp s) / Z^2,  dl += ds s (1 - s)
// Workspace: chunk counts int32 [B*chunks][N], then f float32 [B][N].

__global__ __launch_bounds__(256) void aux_bwd_count_kernel(const int32_t* __restrict__ top_idx,
                                                            int seq, int n_experts, int top_k,
                                                            int chunks_per_seq,
                                                            int32_t* __restrict__ chunk_counts) {
  __shared__ int32_t hist[kMaxN];
  const int tid = threadIdx.x;
  const int chunk = blockIdx.x;
  const int b = chunk / chunks_per_seq;
  const int s0 = (chunk % chunks_per_seq) * kChunk;
  const int s1 = min(seq, s0 + kChunk);
  const int64_t tok0 = static_cast<int64_t>(b) * seq;
  for (int e = tid; e < n_experts; e += 256) hist[e] = 0;
  __syncthreads();
  for (int i = tid; i < (s1 - s0) * top_k; i += 256) {
    const int e = top_idx[(tok0 + s0) * top_k + i];
    if (static_cast<unsigned>(e) < static_cast<unsigned>(n_experts)) atomicAdd(&hist[e], 1);
  }
  __syncthreads();
  for (int e = tid; e < n_experts; e += 256)
    chunk_counts[static_cast<int64_t>(chunk) * n_experts + e] = hist[e];
}

// One workgroup per sequence.
__global__ __launch_bounds__(256) void aux_bwd_frac_kernel(const int32_t* __restrict__ chunk_counts,
                                                           int seq, int n_experts, int top_k,
                                                           int chunks_per_seq,
                                                           float* __restrict__ frac) {
  const int b = blockIdx.x;
  for (int e = threadIdx.x; e < n_experts; e += 256) {
    int64_t cnt = 0;
    for (int c = 0; c < chunks_per_seq; ++c)
      cnt += chunk_counts[(static_cast<int64_t>(b) * chunks_per_seq + c) * n_experts + e];
    frac[static_cast<int64_t>(b) * n_experts + e] =
        static_cast<float>(cnt) / static_cast<float>(seq * top_k);
  }
}

// One wave per token, lanes own experts (EPL per lane).
template <int EPL>
__global__ __launch_bounds__(256) void aux_bwd_token_kernel(const float* __restrict__ logits,
                                                            const float* __restrict__ frac,
                                                            const float* __restrict__ d_losses,
                                                            int batch, int seq, int n_experts,
                                                            float* __restrict__ d_logits,
                                                            int accumulate) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t tokens = static_cast<int64_t>(batch) * seq;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= tokens) return;
  const int b = static_cast<int>(t / seq);
  const float d_z = d_losses[0], d_bal = d_losses[1], d_ent = d_losses[2];
  const float inv_t = 1.0f / static_cast<float>(tokens);
  const float bal_scale = d_bal * static_cast<float>(n_experts) /
                          (static_cast<float>(batch) * static_cast<float>(seq));
  const float* row = logits + t * n_experts;
  float l[EPL], s[EPL];
  float m = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    l[j] = e < n_experts ? row[e] : -__builtin_inff();
    m = fmaxf(m, l[j]);
  }
  m = wave_max(m);
  float se = 0.0f, ss = 0.0f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const bool ok = lane + 64 * j < n_experts;
    se += ok ? expf(l[j] - m) : 0.0f;
    s[j] = ok ? sigmoid_det(l[j]) : 0.0f;
    ss += s[j];
  }
  se = wave_sum(se);
  ss = wave_sum(ss);
  const float lse = m + logf(se);
  const float z = ss + 1e-9f;
  float dp[EPL];
  float sdps = 0.0f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    dp[j] = 0.0f;
    if (e < n_experts) {
      const float p = s[j] / z;
      dp[j] = bal_scale * frac[static_cast<int64_t>(b) * n_experts + e] -
              d_ent * (logf(p + 1e-9f) + p / (p + 1e-9f)) * inv_t;
      sdps += dp[j] * s[j];
    }
  }
  sdps = wave_sum(sdps);
  const float zscale = d_z * 2.0f * lse * inv_t;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    if (e < n_experts) {
      const float q = expf(l[j] - lse);
      const float ds = dp[j] / z - sdps / (z * z);
      float v = zscale * q + ds * s[j] * (1.0f - s[j]);
      if (accumulate) v = d_logits[t * n_experts + e] + v;
      d_logits[t * n_experts + e] = v;
    }
  }
}

}  // namespace
}  // namespace hmoe

extern "C" size_t hmoe_aux_workspace_bytes(int batch, int seq, int n_experts) {
  if (batch <= 0 || seq <= 0 || n_experts <= 0) return 0;
  const int64_t chunks = static_cast<int64_t>(batch) * hmoe::ceil_div(seq, hmoe::kChunk);
  return static_cast<size_t>(chunks * hmoe::part_stride(n_experts) * sizeof(float));
}

extern "C" int hmoe_router_aux(const float* logits, const int32_t* top_idx, int batch, int seq,
                               int n_experts, int top_k, float* losses, float* expert_counts,
                               void* workspace, size_t workspace_bytes, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(batch >= 1 && batch <= 1024 && seq >= 1,
               "router_aux: need 1 <= batch <= 1024 and seq >= 1 (got %d, %d)", batch, seq);
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= kMaxN, "router_aux: n_experts must be in [1, %d]",
               kMaxN);
  HMOE_REQUIRE(top_k >= 1 && top_k <= n_experts, "router_aux: bad top_k %d", top_k);
  HMOE_REQUIRE(logits && top_idx && losses && expert_counts && workspace,
               "router_aux: null pointer argument");
  const size_t need = hmoe_aux_workspace_bytes(batch, seq, n_experts);
  HMOE_REQUIRE_CODE(workspace_bytes >= need, HMOE_ERR_WORKSPACE,
                    "router_aux: workspace of %zu bytes is smaller than the %zu required",
                    workspace_bytes, need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int cps = static_cast<int>(ceil_div(seq, kChunk));
  const dim3 grid(static_cast<unsigned>(batch * cps));
  float* parts = static_cast<float*>(workspace);
  if (n_experts <= 64)
    hipLaunchKernelGGL(aux_chunk_kernel<1>, grid, dim3(256), 0, s, logits, top_idx, seq, n_experts, top_k, cps, parts);
  else if (n_experts <= 128)
    hipLaunchKernelGGL(aux_chunk_kernel<2>, grid, dim3(256), 0, s, logits, top_idx, seq, n_experts, top_k, cps, parts);
  else
    hipLaunchKernelGGL(aux_chunk_kernel<4>, grid, dim3(256), 0, s, logits, top_idx, seq, n_experts, top_k, cps, parts);
  if (int rc = check_launch("router_aux/chunk")) return rc;
  hipLaunchKernelGGL(aux_final_kernel, dim3(1), dim3(kFinalThreads), 0, s, parts, batch, seq,
                     n_experts, top_k, cps, losses, expert_counts);
  return check_launch("router_aux/final");
}

extern "C" size_t hmoe_aux_bwd_workspace_bytes(int batch, int seq, int n_experts) {
  if (batch <= 0 || seq <= 0 || n_experts <= 0) return 0;
  const int64_t chunks = static_cast<int64_t>(batch) * hmoe::ceil_div(seq, hmoe::kChunk);
  return static_cast<size_t>((chunks + batch) * n_experts * 4);
}

extern "C" int hmoe_router_aux_bwd(const float* logits, const int32_t* top_idx, int batch, int seq,
                                   int n_experts, int top_k, const float* d_losses,
                                   float* d_logits, int accumulate, void* workspace,
                                   size_t workspace_bytes, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(batch >= 1 && seq >= 1, "router_aux_bwd: need batch >= 1 and seq >= 1 (got %d, %d)",
               batch, seq);
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= kMaxN,
               "router_aux_bwd: n_experts must be in [1, %d]", kMaxN);
  HMOE_REQUIRE(top_k >= 1 && top_k <= n_experts, "router_aux_bwd: bad top_k %d", top_k);
  HMOE_REQUIRE(logits && top_idx && d_losses && d_logits && workspace,
               "router_aux_bwd: null pointer argument");
  const size_t need = hmoe_aux_bwd_workspace_bytes(batch, seq, n_experts);
  HMOE_REQUIRE_CODE(workspace_bytes >= need, HMOE_ERR_WORKSPACE,
                    "router_aux_bwd: workspace of %zu bytes is smaller than the %zu required",
                    workspace_bytes, need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int cps = static_cast<int>(ceil_div(seq, kChunk));
  const int64_t chunks = static_cast<int64_t>(batch) * cps;
  int32_t* counts = static_cast<int32_t*>(workspace);
  float* frac = reinterpret_cast<float*>(counts + chunks * n_experts);
  hipLaunchKernelGGL(aux_bwd_count_kernel, dim3(static_cast<unsigned>(chunks)), dim3(256), 0, s,
                     top_idx, seq, n_experts, top_k, cps, counts);
  if (int rc = check_launch("router_aux_bwd/count")) return rc;
  hipLaunchKernelGGL(aux_bwd_frac_kernel, dim3(static_cast<unsigned>(batch)), dim3(256), 0, s,
                     counts, seq, n_experts, top_k, cps, frac);
  if (int rc = check_launch("router_aux_bwd/frac")) return rc;
  const int64_t tokens = static_cast<int64_t>(batch) * seq;
  const dim3 grid(static_cast<unsigned>(ceil_div(tokens, 4)));
  if (n_experts <= 64)
    hipLaunchKernelGGL(aux_bwd_token_kernel<1>, grid, dim3(256), 0, s, logits, frac, d_losses, batch, seq, n_experts, d_logits, accumulate);
  else if (n_experts <= 128)
    hipLaunchKernelGGL(aux_bwd_token_kernel<2>, grid, dim3(256), 0, s, logits, frac, d_losses, batch, seq, n_experts, d_logits, accumulate);
  else
    hipLaunchKernelGGL(aux_bwd_token_kernel<4>, grid, dim3(256), 0, s, logits, frac, d_losses, batch, seq, n_experts, d_logits, accumulate);
  return check_launch("router_aux_bwd/token");
}
