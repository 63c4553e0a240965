// Dispatch plan and row permutation (model/moe.py:54-65, :80, :198).
//
// Plan: three deterministic passes over the R = T*K flat slots i = t*K + k.
//   1. histogram: each block of kSlotsPerBlock slots counts its experts;
//   2. scan: one workgroup turns the [blocks, N] histogram into per-block
//      bases (slots of the same expert in earlier blocks), the totals
//      (= bincount), and kept-row offsets (exclusive scan of min(count, C));
//   3. rank: each wave walks its slots 64 at a time in ascending i; lanes that
//      hold the same expert find each other with one ballot per expert-id bit,
//      so a slot's rank is (base) + (earlier lanes of its expert).  The rank
//      fixes keep (rank < C), slot_pos and perm_src; no atomic decides a value.
// Permutation: one wave per token reads the row once and writes its kept
// slots' rows (token-centric, so x is read exactly once).
#include <mutex>

#include "hmoe_common.h"
#include "quant_e4m3.h"

namespace hmoe {
namespace {

constexpr int kPlanThreads = 256;
constexpr int kSlotsPerWave = 256;
constexpr int kSlotsPerBlock = 4 * kSlotsPerWave;  // 128 blocks at 16384 tokens x top-8
constexpr int kMaxExperts = 1024;

int64_t plan_blocks(int64_t rows) { return ceil_div(rows, kSlotsPerBlock); }

__global__ __launch_bounds__(kPlanThreads) void plan_histogram_kernel(
    const int32_t* __restrict__ top_idx, int64_t rows, int n_experts, int32_t* __restrict__ hist) {
  __shared__ int32_t h[kMaxExperts];
  for (int e = threadIdx.x; e < n_experts; e += kPlanThreads) h[e] = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kSlotsPerBlock;
  for (int i = threadIdx.x; i < kSlotsPerBlock; i += kPlanThreads) {
    const int64_t s = base + i;
    if (s < rows) {
      const int e = top_idx[s];
      if (static_cast<unsigned>(e) < static_cast<unsigned>(n_experts)) atomicAdd(&h[e], 1);
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < n_experts; e += kPlanThreads)
    hist[static_cast<int64_t>(blockIdx.x) * n_experts + e] = h[e];
}

// One workgroup of 1024 threads.  hist is rewritten in place into the
// per-block exclusive bases.  Each expert is served by a group of P lanes
// (P = 1024 / N rounded down to a power of two, at most 64, so a group lies
// inside one wave): lane j of the group sums blocks [j*L, (j+1)*L), the group
// scans those partial sums with shuffles, and each lane then writes its
// blocks' bases.  Totals and kept-row offsets follow as before.
__global__ __launch_bounds__(1024) void plan_scan_kernel(int32_t* __restrict__ hist, int nblk,
                                                          int n_experts, int64_t capacity,
                                                          int32_t* __restrict__ counts,
                                                          int32_t* __restrict__ offsets) {
  __shared__ int32_t kept[kMaxExperts];
  const int tid = threadIdx.x;
  int P = 1;
  while (P < 64 && 2 * P * n_experts <= 1024) P *= 2;
  const int e = tid / P;          // expert of this lane (>= n_experts: idle)
  const int j = tid % P;          // position in the expert's group
  const int L = (nblk + P - 1) / P;
  const int b0 = j * L;
  const int b1 = b0 + L < nblk ? b0 + L : nblk;
  // Eight loads in flight per lane (a long block range otherwise costs one
  // dependent global load per block).
  constexpr int kU = 8;
  int32_t part = 0;
  if (e < n_experts) {
    int b = b0;
    for (; b + kU <= b1; b += kU) {
      int32_t v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) v[u] = hist[static_cast<int64_t>(b + u) * n_experts + e];
#pragma unroll
      for (int u = 0; u < kU; ++u) part += v[u];
    }
    for (; b < b1; ++b) part += hist[static_cast<int64_t>(b) * n_experts + e];
  }
  // Inclusive scan of the partial sums within the group (P lanes, aligned).
  int32_t incl = part;
  for (int off = 1; off < P; off <<= 1) {
    const int32_t v = __shfl_up(incl, off, P);
    if (j >= off) incl += v;
  }
  const int32_t total = __shfl(incl, P - 1, P);
  if (e < n_experts) {
    int32_t run = incl - part;  // exclusive base of block b0
    int b = b0;
    for (; b + kU <= b1; b += kU) {
      int32_t v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) v[u] = hist[static_cast<int64_t>(b + u) * n_experts + e];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        hist[static_cast<int64_t>(b + u) * n_experts + e] = run;
        run += v[u];
      }
    }
    for (; b < b1; ++b) {
      const int64_t idx = static_cast<int64_t>(b) * n_experts + e;
      const int32_t c = hist[idx];
      hist[idx] = run;
      run += c;
    }
    if (j == 0) counts[e] = total;
  }
  if (tid < kMaxExperts) kept[tid] = 0;
  __syncthreads();
  if (e < n_experts && j == 0) kept[e] = static_cast<int32_t>(total < capacity ? total : capacity);
  __syncthreads();
  // Inclusive Hillis-Steele scan over 1024 entries.
  for (int off = 1; off < 1024; off <<= 1) {
    const int32_t v = tid >= off ? kept[tid - off] : 0;
    __syncthreads();
    kept[tid] += v;
    __syncthreads();
  }
  if (tid < n_experts) offsets[tid + 1] = kept[tid];
  if (tid == 0) offsets[0] = 0;
}

// Column scan of the per-block histogram for plans past the fused rank pass,
// one wave per expert over the whole chip (plan_scan_kernel's one workgroup
// walked 128 blocks per lane at 512 blocks x 128 experts: 42 us).  Lane j
// takes blocks [j L, (j + 1) L), L = ceil(nblk / 64), eight loads in flight;
// the wave scans the 64 partial sums, each lane rewrites its blocks' counts
// as exclusive bases, and lane 0 writes the expert's total to counts.  The
// kept-row offsets are formed by every rank workgroup from counts.
constexpr int kScanColWaves = 4;

__global__ __launch_bounds__(64 * kScanColWaves) void plan_scan_cols_kernel(
    int32_t* __restrict__ hist, int nblk, int n_experts, int32_t* __restrict__ counts) {
  const int lane = threadIdx.x & 63;
  const int e = blockIdx.x * kScanColWaves + (threadIdx.x >> 6);
  if (e >= n_experts) return;  // uniform per wave
  const int L = (nblk + 63) / 64;
  const int b0 = lane * L < nblk ? lane * L : nblk;
  const int b1 = b0 + L < nblk ? b0 + L : nblk;
  constexpr int kU = 8;
  int32_t part = 0;
  {
    int b = b0;
    for (; b + kU <= b1; b += kU) {
      int32_t v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) v[u] = hist[static_cast<int64_t>(b + u) * n_experts + e];
#pragma unroll
      for (int u = 0; u < kU; ++u) part += v[u];
    }
    for (; b < b1; ++b) part += hist[static_cast<int64_t>(b) * n_experts + e];
  }
  int32_t incl = part;
  for (int off = 1; off < 64; off <<= 1) {
    const int32_t v = __shfl_up(incl, off, 64);
    if (lane >= off) incl += v;
  }
  const int32_t total = __shfl(incl, 63, 64);
  int32_t run = incl - part;  // exclusive base of block b0
  int b = b0;
  for (; b + kU <= b1; b += kU) {
    int32_t v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) v[u] = hist[static_cast<int64_t>(b + u) * n_experts + e];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      hist[static_cast<int64_t>(b + u) * n_experts + e] = run;
      run += v[u];
    }
  }
  for (; b < b1; ++b) {
    const int64_t idx = static_cast<int64_t>(b) * n_experts + e;
    const int32_t c = hist[idx];
    hist[idx] = run;
    run += c;
  }
  if (lane == 0) counts[e] = total;
}

// Kept-row offsets from the per-expert totals, in LDS: on entry s_off[e]
// holds min(total, capacity) for e < n_experts; on exit the exclusive scan,
// with the kept total in s_off[n_experts].  Each thread scans a run of kPer
// consecutive experts, then a Hillis-Steele scan over the kPlanThreads run
// sums (s_scan).  Ends with a barrier.
__device__ void kept_offsets_lds(int32_t* s_off, int32_t* s_scan, int n_experts) {
  const int tid = threadIdx.x;
  constexpr int kPer = kMaxExperts / kPlanThreads;
  int32_t local[kPer];
  int32_t sum = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = tid * kPer + j;
    local[j] = e < n_experts ? s_off[e] : 0;
    sum += local[j];
  }
  s_scan[tid] = sum;
  __syncthreads();
  for (int off = 1; off < kPlanThreads; off <<= 1) {
    const int32_t v = tid >= off ? s_scan[tid - off] : 0;
    __syncthreads();
    s_scan[tid] += v;
    __syncthreads();
  }
  int32_t run = s_scan[tid] - sum;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = tid * kPer + j;
    if (e < n_experts) s_off[e] = run;
    run += local[j];
  }
  if (tid == kPlanThreads - 1) s_off[n_experts] = s_scan[kPlanThreads - 1];
  __syncthreads();
}

__global__ __launch_bounds__(kPlanThreads) void plan_rank_kernel(
    const int32_t* __restrict__ top_idx, int64_t rows, int n_experts, int64_t capacity,
    const int32_t* __restrict__ bases, const int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ slot_pos, int32_t* __restrict__ perm_src,
    uint8_t* __restrict__ keep, int64_t rows_cap) {
  __shared__ int32_t whist[4][kMaxExperts];
  __shared__ int32_t s_off[kMaxExperts + 1];  // kept-row offsets
  __shared__ int32_t s_scan[kPlanThreads];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t blk_base = static_cast<int64_t>(blockIdx.x) * kSlotsPerBlock;
  const int64_t wave_base = blk_base + static_cast<int64_t>(wave) * kSlotsPerWave;

  for (int i = tid; i < 4 * kMaxExperts; i += kPlanThreads) (&whist[0][0])[i] = 0;
  __syncthreads();
  for (int i = lane; i < kSlotsPerWave; i += 64) {
    const int64_t s = wave_base + i;
    if (s < rows) {
      const int e = top_idx[s];
      if (static_cast<unsigned>(e) < static_cast<unsigned>(n_experts)) atomicAdd(&whist[wave][e], 1);
    }
  }
  __syncthreads();
  for (int e = tid; e < n_experts; e += kPlanThreads) {
    int32_t run = bases[static_cast<int64_t>(blockIdx.x) * n_experts + e];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int32_t c = whist[w][e];
      whist[w][e] = run;
      run += c;
    }
    const int32_t tot = counts[e];
    s_off[e] = static_cast<int32_t>(tot < capacity ? tot : capacity);
  }
  __syncthreads();
  kept_offsets_lds(s_off, s_scan, n_experts);
  if (blockIdx.x == 0)
    for (int e = tid; e <= n_experts; e += kPlanThreads) offsets[e] = s_off[e];

  const int nbits = n_experts > 1 ? 32 - __builtin_clz(static_cast<unsigned>(n_experts - 1)) : 0;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int32_t* my_hist = whist[wave];
  for (int c = 0; c < kSlotsPerWave; c += 64) {
    const int64_t s = wave_base + c + lane;
    int e = s < rows ? top_idx[s] : -1;
    const bool valid = static_cast<unsigned>(e) < static_cast<unsigned>(n_experts);
    if (!valid) e = 0;
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (e >> b) & 1;
      const uint64_t bal = __ballot(bit);
      peers &= bit ? bal : ~bal;
    }
    int32_t base = 0;
    if (valid) base = my_hist[e];
    const int32_t rank = base + __popcll(peers & lt_mask);
    const bool leader = valid && ((peers & lt_mask) == 0);
    if (leader) my_hist[e] = base + __popcll(peers);
    if (s < rows && !valid) {  // out-of-range expert id: never dispatched
      keep[s] = 0;
      slot_pos[s] = -1;
    }
    if (valid) {
      const bool kept = rank < capacity;
      keep[s] = kept ? 1 : 0;
      if (kept) {
        const int32_t pos = s_off[e] + rank;
        slot_pos[s] = pos;
        perm_src[pos] = static_cast<int32_t>(s);
      } else {
        slot_pos[s] = -1;
      }
    }
  }
  // Rows past the kept total hold -1.
  const int64_t total = s_off[n_experts];
  for (int64_t j = total + static_cast<int64_t>(blockIdx.x) * kPlanThreads + tid; j < rows_cap;
       j += static_cast<int64_t>(gridDim.x) * kPlanThreads)
    perm_src[j] = -1;
}

// Rank pass with the scan folded in (plans of at most kFusedScanBlocks
// blocks): every workgroup derives what plan_scan_kernel would have given it
// from the per-block histogram itself -- its block's base per expert (the
// sum over earlier blocks), the totals and the kept-row offsets -- so the
// plan is two launches.  The histogram is nblk * N int32 (32 KB at 16384
// tokens x top-8 x 64 experts), read from L2 by every workgroup; sums run
// in a fixed order, so every workgroup gets the same totals.  Workgroup 0
// writes counts and offsets.
constexpr int kFusedScanBlocks = 256;
// ... and of at most this many histogram entries (nblk * N): every
// workgroup reads the whole histogram, so past this the three-pass plan is
// faster.  Measured on the MI355X (both paths bit-identical): at 32768
// tokens x top-8 (256 blocks) 11.7 / 20.0 / 61.4 us for 64 / 256 / 1024
// experts against 30.3 / 34.8 / 50.0 us in three passes; at 8192 tokens x
// 1024 experts (65536 entries) 22.6 against 22.4 us.
constexpr int64_t kFusedScanEntries = 65536;

__global__ __launch_bounds__(kPlanThreads) void plan_rank_fused_kernel(
    const int32_t* __restrict__ top_idx, int64_t rows, int n_experts, int64_t capacity,
    const int32_t* __restrict__ hist, int nblk, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ slot_pos, int32_t* __restrict__ perm_src,
    uint8_t* __restrict__ keep, int64_t rows_cap) {
  __shared__ int32_t whist[4][kMaxExperts];
  __shared__ int32_t part_pre[kMaxExperts];   // per (group, expert) partial sums
  __shared__ int32_t part_tot[kMaxExperts];
  __shared__ int32_t s_off[kMaxExperts + 1];  // kept-row offsets
  __shared__ int32_t s_scan[kPlanThreads];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int b = blockIdx.x;
  const int64_t blk_base = static_cast<int64_t>(b) * kSlotsPerBlock;
  const int64_t wave_base = blk_base + static_cast<int64_t>(wave) * kSlotsPerWave;

  // This lane's four slots (wave_base + lane + 64 c), loaded once and kept
  // for the rank loop below.
  constexpr int kSlotIters = kSlotsPerWave / 64;
  int ev[kSlotIters];
#pragma unroll
  for (int c = 0; c < kSlotIters; ++c) {
    const int64_t s = wave_base + 64 * c + lane;
    ev[c] = s < rows ? top_idx[s] : -1;
  }
  for (int i = tid; i < 4 * kMaxExperts; i += kPlanThreads) (&whist[0][0])[i] = 0;
  __syncthreads();
#pragma unroll
  for (int c = 0; c < kSlotIters; ++c)
    if (static_cast<unsigned>(ev[c]) < static_cast<unsigned>(n_experts)) atomicAdd(&whist[wave][ev[c]], 1);
  // Histogram sums: G groups of N threads (G = 256 / N; G = 1 with thread
  // tid taking experts tid, tid + 256, ... when N > 256); group g sums the
  // blocks g, g + G, ..., so the 64 lanes of a wave read 64 consecutive
  // experts of one block.
  const int G = n_experts >= kPlanThreads ? 1 : kPlanThreads / n_experts;
  for (int idx = tid; idx < (G > 1 ? G * n_experts : n_experts); idx += kPlanThreads) {
    const int g = G > 1 ? idx / n_experts : 0;
    const int e = G > 1 ? idx - g * n_experts : idx;
    int32_t pre = 0, tot = 0;
    int bb = g;
    // eight loads in flight at a time (the sums are exact integer sums)
    for (; bb + 7 * G < nblk; bb += 8 * G) {
      int32_t c[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) c[u] = hist[static_cast<int64_t>(bb + u * G) * n_experts + e];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        tot += c[u];
        if (bb + u * G < b) pre += c[u];
      }
    }
    for (; bb < nblk; bb += G) {
      const int32_t c = hist[static_cast<int64_t>(bb) * n_experts + e];
      tot += c;
      if (bb < b) pre += c;
    }
    part_pre[idx] = pre;
    part_tot[idx] = tot;
  }
  __syncthreads();
  // Per expert: base of this block, total, kept rows (in part_tot[e]).
  for (int e = tid; e < n_experts; e += kPlanThreads) {
    int32_t pre = 0, tot = 0;
    for (int g = 0; g < G; ++g) {
      pre += part_pre[g * n_experts + e];
      tot += part_tot[g * n_experts + e];
    }
    if (b == 0) counts[e] = tot;
    // per-wave bases of this block's four waves
    int32_t run = pre;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int32_t c = whist[w][e];
      whist[w][e] = run;
      run += c;
    }
    s_off[e] = static_cast<int32_t>(tot < capacity ? tot : capacity);
  }
  __syncthreads();
  kept_offsets_lds(s_off, s_scan, n_experts);
  if (b == 0)
    for (int e = tid; e <= n_experts; e += kPlanThreads) offsets[e] = s_off[e];

  const int nbits = n_experts > 1 ? 32 - __builtin_clz(static_cast<unsigned>(n_experts - 1)) : 0;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int32_t* my_hist = whist[wave];
#pragma unroll
  for (int ci = 0; ci < kSlotIters; ++ci) {
    const int64_t s = wave_base + 64 * ci + lane;
    int e = ev[ci];
    const bool valid = static_cast<unsigned>(e) < static_cast<unsigned>(n_experts);
    if (!valid) e = 0;
    uint64_t peers = __ballot(valid);
    for (int bit = 0; bit < nbits; ++bit) {
      const bool on = (e >> bit) & 1;
      const uint64_t bal = __ballot(on);
      peers &= on ? bal : ~bal;
    }
    int32_t base = 0;
    if (valid) base = my_hist[e];
    const int32_t rank = base + __popcll(peers & lt_mask);
    const bool leader = valid && ((peers & lt_mask) == 0);
    if (leader) my_hist[e] = base + __popcll(peers);
    if (s < rows && !valid) {  // out-of-range expert id: never dispatched
      keep[s] = 0;
      slot_pos[s] = -1;
    }
    if (valid) {
      const bool kept = rank < capacity;
      keep[s] = kept ? 1 : 0;
      if (kept) {
        const int32_t pos = s_off[e] + rank;
        slot_pos[s] = pos;
        perm_src[pos] = static_cast<int32_t>(s);
      } else {
        slot_pos[s] = -1;
      }
    }
  }
  // Rows past the kept total hold -1.
  const int64_t total = s_off[n_experts];
  for (int64_t j = total + static_cast<int64_t>(b) * kPlanThreads + tid; j < rows_cap;
       j += static_cast<int64_t>(gridDim.x) * kPlanThreads)
    perm_src[j] = -1;
}

// ------------------------------------------------------------ permutation --
// The dispatched rows are written once and read later by another kernel, so
// the stores are non-temporal (the full bf16 workload's permutation: 117.5 ->
// 105.4 us measured; non-temporal loads of x on top of that were slower).
template <typename TI, typename TO>
__device__ __forceinline__ void store8(TO* dst, const Chunk8<TI>& c);
template <>
__device__ __forceinline__ void store8<uint16_t, uint16_t>(uint16_t* dst, const Chunk8<uint16_t>& c) {
  __builtin_nontemporal_store(c.v, reinterpret_cast<u32x4*>(dst));
}
template <>
__device__ __forceinline__ void store8<float, uint16_t>(uint16_t* dst, const Chunk8<float>& c) {
  u32x4 o;
  o[0] = pack_bf16x2(c.a[0], c.a[1]);
  o[1] = pack_bf16x2(c.a[2], c.a[3]);
  o[2] = pack_bf16x2(c.b[0], c.b[1]);
  o[3] = pack_bf16x2(c.b[2], c.b[3]);
  __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(dst));
}
template <>
__device__ __forceinline__ void store8<float, float>(float* dst, const Chunk8<float>& c) {
  __builtin_nontemporal_store(c.a, reinterpret_cast<f32x4*>(dst));
  __builtin_nontemporal_store(c.b, reinterpret_cast<f32x4*>(dst + 4));
}
template <>
__device__ __forceinline__ void store8<uint16_t, float>(float* dst, const Chunk8<uint16_t>& c) {
  f32x4 a, b;
  for (int i = 0; i < 4; ++i) {
    a[i] = c.get(i);
    b[i] = c.get(4 + i);
  }
  __builtin_nontemporal_store(a, reinterpret_cast<f32x4*>(dst));
  __builtin_nontemporal_store(b, reinterpret_cast<f32x4*>(dst + 4));
}

constexpr int kPermUnroll = 4;

template <typename TI, typename TO>
__global__ __launch_bounds__(256) void permute_rows_kernel(const TI* __restrict__ x, int64_t tokens,
                                                           int d_model, int top_k,
                                                           const int32_t* __restrict__ slot_pos,
                                                           TO* __restrict__ xs) {
  const int lane = threadIdx.x & 63;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= tokens) return;
  const int32_t my_pos = lane < top_k ? slot_pos[t * top_k + lane] : -1;
  const int chunks = d_model / 8;
  const TI* src = x + t * d_model;
  for (int c0 = 0; c0 < chunks; c0 += 64 * kPermUnroll) {
    Chunk8<TI> v[kPermUnroll];
#pragma unroll
    for (int u = 0; u < kPermUnroll; ++u) {
      const int c = c0 + u * 64 + lane;
      if (c < chunks) v[u].load(src + static_cast<int64_t>(c) * 8);
    }
    for (int k = 0; k < top_k; ++k) {
      const int32_t pos = lane_bcast(my_pos, k);
      if (pos < 0) continue;
      TO* dst = xs + static_cast<int64_t>(pos) * d_model;
#pragma unroll
      for (int u = 0; u < kPermUnroll; ++u) {
        const int c = c0 + u * 64 + lane;
        if (c < chunks) store8<TI, TO>(dst + static_cast<int64_t>(c) * 8, v[u]);
      }
    }
  }
}

// ------------------------------------------------------- e4m3 quantisation --
// One wave per token: quantise the row once and write it to every kept slot.
// REGS: the row fits in registers (d_model <= 64 * kRowRegs * 8) and is read
// once; otherwise it is read twice (amax pass, then quantisation).
template <typename TI, bool REGS>
__global__ __launch_bounds__(256) void permute_rows_fp8_kernel(
    const TI* __restrict__ x, int64_t tokens, int d_model, int top_k,
    const int32_t* __restrict__ slot_pos, uint8_t* __restrict__ xs_q, float* __restrict__ xs_scale) {
  const int lane = threadIdx.x & 63;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= tokens) return;
  const int32_t my_pos = lane < top_k ? slot_pos[t * top_k + lane] : -1;
  const int chunks = d_model / 8;
  const TI* src = x + t * d_model;
  float s, inv;
  if (REGS) {
    Chunk8<TI> v[kRowRegs];
    load_row_regs(src, chunks, v, s, inv);
    if (lane < top_k && my_pos >= 0) xs_scale[my_pos] = s;
#pragma unroll
    for (int u = 0; u < kRowRegs; ++u) {
      if (u * 64 >= chunks) break;  // uniform
      const int c = u * 64 + lane;
      const uint2 q = quant8_e4m3(v[u], inv);
      for (int k = 0; k < top_k; ++k) {
        const int32_t pos = lane_bcast(my_pos, k);
        if (pos >= 0 && c < chunks)
          *reinterpret_cast<uint2*>(xs_q + static_cast<int64_t>(pos) * d_model + c * 8) = q;
      }
    }
    return;
  }
  wave_row_scales(src, chunks, s, inv);
  if (lane < top_k && my_pos >= 0) xs_scale[my_pos] = s;
  // Wave-uniform loop: every lane takes part in the slot broadcasts.
  for (int c0 = 0; c0 < chunks; c0 += 64) {
    const int c = c0 + lane;
    const bool ok = c < chunks;
    Chunk8<TI> v;
    v.load(src + static_cast<int64_t>(ok ? c : 0) * 8);
    const uint2 q = quant8_e4m3(v, inv);
    for (int k = 0; k < top_k; ++k) {
      const int32_t pos = lane_bcast(my_pos, k);
      if (pos >= 0 && ok)
        *reinterpret_cast<uint2*>(xs_q + static_cast<int64_t>(pos) * d_model + c * 8) = q;
    }
  }
}

// One wave per row of a bf16 matrix; rows at or past offsets[n_experts] (when
// given) are skipped.  REGS as for the permutation.
template <bool REGS>
__global__ __launch_bounds__(256) void quantize_rows_fp8_kernel(
    const uint16_t* __restrict__ a, int64_t rows, int cols, const int32_t* __restrict__ offsets,
    int n_experts, uint8_t* __restrict__ q, float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  if (offsets != nullptr && r >= offsets[n_experts]) {  // past the kept rows: not read
    if (lane == 0) scale[r] = 1.0f;
    return;
  }
  quant_row_e4m3<REGS>(a + r * cols, cols, q + r * cols, scale + r);
}

}  // namespace
}  // namespace hmoe

extern "C" int hmoe_permute_rows_fp8(const void* x, int x_dtype, int64_t tokens, int d_model,
                                     int top_k, const int32_t* slot_pos, uint8_t* xs_q,
                                     float* xs_scale, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(tokens >= 0 && top_k >= 1 && top_k <= 64,
               "permute_rows_fp8: need tokens >= 0 and 1 <= top_k <= 64");
  HMOE_REQUIRE(d_model >= 8 && d_model % 8 == 0,
               "permute_rows_fp8: d_model must be a multiple of 8 (got %d)", d_model);
  HMOE_REQUIRE(x_dtype == HMOE_F32 || x_dtype == HMOE_BF16,
               "permute_rows_fp8: x dtype must be F32 or BF16");
  if (tokens == 0) return HMOE_OK;
  HMOE_REQUIRE(x && slot_pos && xs_q && xs_scale, "permute_rows_fp8: null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(ceil_div(tokens, 4)));
  const bool regs = d_model <= 64 * kRowRegs * 8;
#define HMOE_LAUNCH_PERM8(TI, REGS)                                                              \
  hipLaunchKernelGGL((permute_rows_fp8_kernel<TI, REGS>), grid, dim3(256), 0, s,                 \
                     static_cast<const TI*>(x), tokens, d_model, top_k, slot_pos, xs_q, xs_scale)
  if (x_dtype == HMOE_BF16 && regs) HMOE_LAUNCH_PERM8(uint16_t, true);
  else if (x_dtype == HMOE_BF16) HMOE_LAUNCH_PERM8(uint16_t, false);
  else if (regs) HMOE_LAUNCH_PERM8(float, true);
  else HMOE_LAUNCH_PERM8(float, false);
#undef HMOE_LAUNCH_PERM8
  return check_launch("hmoe_permute_rows_fp8");
}

extern "C" int hmoe_quantize_rows_fp8(const void* a, int64_t rows, int cols,
                                      const int32_t* offsets, int n_experts, uint8_t* q,
                                      float* scale, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(rows >= 0, "quantize_rows_fp8: rows must be >= 0");
  HMOE_REQUIRE(cols >= 8 && cols % 8 == 0,
               "quantize_rows_fp8: cols must be a multiple of 8 (got %d)", cols);
  HMOE_REQUIRE(offsets == nullptr || n_experts >= 1,
               "quantize_rows_fp8: n_experts must be >= 1 with offsets");
  if (rows == 0) return HMOE_OK;
  HMOE_REQUIRE(a && q && scale, "quantize_rows_fp8: null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(ceil_div(rows, 4)));
  if (cols <= 64 * kRowRegs * 8)
    hipLaunchKernelGGL(quantize_rows_fp8_kernel<true>, grid, dim3(256), 0, s,
                       static_cast<const uint16_t*>(a), rows, cols, offsets, n_experts, q, scale);
  else
    hipLaunchKernelGGL(quantize_rows_fp8_kernel<false>, grid, dim3(256), 0, s,
                       static_cast<const uint16_t*>(a), rows, cols, offsets, n_experts, q, scale);
  return check_launch("hmoe_quantize_rows_fp8");
}

extern "C" size_t hmoe_plan_workspace_bytes(int64_t tokens, int top_k, int n_experts) {
  if (tokens <= 0 || top_k <= 0 || n_experts <= 0) return 0;
  return static_cast<size_t>(hmoe::plan_blocks(tokens * top_k)) * n_experts * sizeof(int32_t);
}

namespace hmoe {
namespace {

// Argument checks shared by the two plan entry points.
int check_plan_args(const int32_t* top_idx, int64_t tokens, int top_k, int n_experts,
                    int64_t capacity, int32_t* counts, int32_t* offsets, int32_t* slot_pos,
                    int32_t* perm_src, uint8_t* keep, const char* what) {
  HMOE_REQUIRE(tokens >= 0 && top_k >= 1, "%s: need tokens >= 0 and top_k >= 1", what);
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= kMaxExperts,
               "%s: n_experts must be in [1, %d] (got %d)", what, kMaxExperts, n_experts);
  const int64_t rows = tokens * top_k;
  // (no slots: hmoe_capacity gives 0 and the plan is all zeros)
  HMOE_REQUIRE(capacity >= 1 || rows == 0, "%s: capacity must be >= 1 (got %lld)", what,
               (long long)capacity);
  HMOE_REQUIRE(rows < (int64_t(1) << 31), "%s: T*K must fit in int32 (got %lld)", what,
               (long long)rows);
  HMOE_REQUIRE(counts && offsets, "%s: null pointer argument", what);
  HMOE_REQUIRE(rows == 0 || (top_idx && slot_pos && perm_src && keep),
               "%s: null pointer argument", what);
  return HMOE_OK;
}

// The three plan passes on the per-block histogram buffer `hist`
// (plan_blocks(T*K) * N int32, every entry written by the histogram pass
// before it is read, so it needs no clearing).
int launch_plan(const int32_t* top_idx, int64_t tokens, int top_k, int n_experts,
                int64_t capacity, int32_t* counts, int32_t* offsets, int32_t* slot_pos,
                int32_t* perm_src, uint8_t* keep, int32_t* hist, hipStream_t s) {
  const int64_t rows = tokens * top_k;
  const int64_t rows_cap = hmoe_rows_cap(tokens, top_k, n_experts, capacity);
  const int nblk = static_cast<int>(plan_blocks(rows));
  if (rows > 0 && nblk <= kFusedScanBlocks &&
      static_cast<int64_t>(nblk) * n_experts <= kFusedScanEntries) {
    hipLaunchKernelGGL(plan_histogram_kernel, dim3(nblk), dim3(kPlanThreads), 0, s, top_idx, rows,
                       n_experts, hist);
    if (int rc = check_launch("dispatch_plan/histogram")) return rc;
    hipLaunchKernelGGL(plan_rank_fused_kernel, dim3(nblk), dim3(kPlanThreads), 0, s, top_idx, rows,
                       n_experts, capacity, hist, nblk, counts, offsets, slot_pos, perm_src, keep,
                       rows_cap);
    return check_launch("dispatch_plan/rank");
  }
  if (rows > 0) {
    hipLaunchKernelGGL(plan_histogram_kernel, dim3(nblk), dim3(kPlanThreads), 0, s, top_idx, rows,
                       n_experts, hist);
    if (int rc = check_launch("dispatch_plan/histogram")) return rc;
    hipLaunchKernelGGL(plan_scan_cols_kernel, dim3(ceil_div(n_experts, kScanColWaves)),
                       dim3(64 * kScanColWaves), 0, s, hist, nblk, n_experts, counts);
    if (int rc = check_launch("dispatch_plan/scan")) return rc;
    hipLaunchKernelGGL(plan_rank_kernel, dim3(nblk), dim3(kPlanThreads), 0, s, top_idx, rows,
                       n_experts, capacity, hist, counts, offsets, slot_pos, perm_src, keep,
                       rows_cap);
    return check_launch("dispatch_plan/rank");
  }
  // No slots: zero counts and offsets.
  hipLaunchKernelGGL(plan_scan_kernel, dim3(1), dim3(1024), 0, s, static_cast<int32_t*>(nullptr), 0,
                     n_experts, capacity, counts, offsets);
  return check_launch("dispatch_plan/scan");
}

// Plan scratch for hmoe_dispatch_plan_noalloc: the per-block histogram in a
// fixed device array, one copy per GPU for the life of the process.  Host
// code never uses the array's name as an address: each device's copy is
// looked up once (hipGetSymbolAddress, with that device current) and the
// kernels get that pointer.
constexpr size_t kPlanScratchInts = size_t(1) << 18;  // 1 MiB
static __device__ __align__(256) int32_t scratch[kPlanScratchInts];

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
int32_t* g_scratch_ptr[kScratchDevices];

// This device's copy of `scratch` (resolved on its first use).
int plan_scratch(int dev, int32_t** out) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("dispatch_plan_noalloc: cannot resolve the plan scratch on device %d: %s", dev,
                hipGetErrorString(e));
      return HMOE_ERR_HIP;
    }
    g_scratch_ptr[dev] = static_cast<int32_t*>(p);
  }
  *out = g_scratch_ptr[dev];
  return HMOE_OK;
}

}  // namespace
}  // namespace hmoe

extern "C" int hmoe_dispatch_plan(const int32_t* top_idx, int64_t tokens, int top_k,
                                  int n_experts, int64_t capacity, int32_t* counts,
                                  int32_t* offsets, int32_t* slot_pos, int32_t* perm_src,
                                  uint8_t* keep, void* workspace, size_t workspace_bytes,
                                  hmoe_stream_t stream) {
  using namespace hmoe;
  if (int rc = check_plan_args(top_idx, tokens, top_k, n_experts, capacity, counts, offsets,
                               slot_pos, perm_src, keep, "dispatch_plan"))
    return rc;
  const size_t need = hmoe_plan_workspace_bytes(tokens, top_k, n_experts);
  HMOE_REQUIRE_CODE(workspace_bytes >= need, HMOE_ERR_WORKSPACE,
                    "dispatch_plan: workspace of %zu bytes is smaller than the %zu required",
                    workspace_bytes, need);
  HMOE_REQUIRE(tokens * top_k == 0 || workspace, "dispatch_plan: null pointer argument");
  return launch_plan(top_idx, tokens, top_k, n_experts, capacity, counts, offsets, slot_pos,
                     perm_src, keep, static_cast<int32_t*>(workspace),
                     static_cast<hipStream_t>(stream));
}

extern "C" int hmoe_dispatch_plan_noalloc(const int32_t* top_idx, int64_t tokens, int top_k,
                                          int n_experts, int64_t capacity, int32_t* counts,
                                          int32_t* offsets, int32_t* slot_pos, int32_t* perm_src,
                                          uint8_t* keep, hmoe_stream_t stream) {
  using namespace hmoe;
  if (int rc = check_plan_args(top_idx, tokens, top_k, n_experts, capacity, counts, offsets,
                               slot_pos, perm_src, keep, "dispatch_plan_noalloc"))
    return rc;
  const size_t need = hmoe_plan_workspace_bytes(tokens, top_k, n_experts);
  HMOE_REQUIRE_CODE(need <= kPlanScratchInts * sizeof(int32_t), HMOE_ERR_WORKSPACE,
                    "dispatch_plan_noalloc: the plan needs %zu bytes of scratch, more than the "
                    "%zu this entry point holds (ceil(T*K / %d) * N int32); use "
                    "hmoe_dispatch_plan with a workspace",
                    need, kPlanScratchInts * sizeof(int32_t), kSlotsPerBlock);
  hipStream_t s = static_cast<hipStream_t>(stream);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices) {
    set_error("dispatch_plan_noalloc: cannot query the current device (or device id >= %d)",
              kScratchDevices);
    return HMOE_ERR_HIP;
  }
  if (s != nullptr) {
    int sdev = -1;
    if (hipStreamGetDevice(s, &sdev) != hipSuccess || sdev != dev) {
      set_error("dispatch_plan_noalloc: the stream belongs to device %d, the current device is "
                "%d; make the stream's device current", sdev, dev);
      return HMOE_ERR_INVALID;
    }
  }
  int32_t* hist = nullptr;
  if (int rc = plan_scratch(dev, &hist)) return rc;
  return launch_plan(top_idx, tokens, top_k, n_experts, capacity, counts, offsets, slot_pos,
                     perm_src, keep, hist, s);
}

extern "C" int hmoe_permute_rows(const void* x, int x_dtype, int64_t tokens, int d_model,
                                 int top_k, const int32_t* slot_pos, void* xs, int xs_dtype,
                                 hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(tokens >= 0 && top_k >= 1 && top_k <= 64,
               "permute_rows: need tokens >= 0 and 1 <= top_k <= 64");
  HMOE_REQUIRE(d_model >= 8 && d_model % 8 == 0, "permute_rows: d_model must be a multiple of 8 (got %d)",
               d_model);
  HMOE_REQUIRE((x_dtype == HMOE_F32 || x_dtype == HMOE_BF16) &&
                   (xs_dtype == HMOE_F32 || xs_dtype == HMOE_BF16),
               "permute_rows: dtypes must be F32 or BF16");
  if (tokens == 0) return HMOE_OK;
  HMOE_REQUIRE(x && slot_pos && xs, "permute_rows: null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(ceil_div(tokens, 4)));
  if (x_dtype == HMOE_BF16 && xs_dtype == HMOE_BF16)
    hipLaunchKernelGGL((permute_rows_kernel<uint16_t, uint16_t>), grid, dim3(256), 0, s,
                       static_cast<const uint16_t*>(x), tokens, d_model, top_k, slot_pos,
                       static_cast<uint16_t*>(xs));
  else if (x_dtype == HMOE_F32 && xs_dtype == HMOE_BF16)
    hipLaunchKernelGGL((permute_rows_kernel<float, uint16_t>), grid, dim3(256), 0, s,
                       static_cast<const float*>(x), tokens, d_model, top_k, slot_pos,
                       static_cast<uint16_t*>(xs));
  else if (x_dtype == HMOE_F32 && xs_dtype == HMOE_F32)
    hipLaunchKernelGGL((permute_rows_kernel<float, float>), grid, dim3(256), 0, s,
                       static_cast<const float*>(x), tokens, d_model, top_k, slot_pos,
                       static_cast<float*>(xs));
  else
    hipLaunchKernelGGL((permute_rows_kernel<uint16_t, float>), grid, dim3(256), 0, s,
                       static_cast<const uint16_t*>(x), tokens, d_model, top_k, slot_pos,
                       static_cast<float*>(xs));
  return check_launch("hmoe_permute_rows");
}
