// Float32 expert path (compute dtype float32, moe.py:70-74 and the shared
// expert's swiglu, moe.py:23-29) and its backward: grouped GEMMs on the
// float32 matrix cores, v_mfma_f32_32x32x2_f32 (exact float32 products,
// float32 sums), on the masters as they are (w_gate/w_up [N, D, F], w_down
// [N, F, D], row-major float32).
//
// grouped_gemm_f32_kernel: C[r][n] = sum_k A[r][k] * B_e(k, n) over the rows r
// of expert e's segment [offsets[e], offsets[e+1]), A [rows, K] row-major.
// B_e(k, n) is B_e[k][n] (a master [K, ncols]) or, transposed (BT), B_e[n][k]
// (a master [ncols, K] read as its transpose: the data gradients d_ys Wd^T
// and dg Wg^T + du Wu^T).  Epilogues:
//   plain    C = the sums;
//   SwiGLU   the GEMM runs against w_gate and w_up and writes
//            h = silu(g) * u (moe.py:72);
//   dSwiGLU  the same two GEMMs (g, u recomputed) and, with the cotangent dh
//            [rows, F], writes dg to columns [0, F) and du to [F, 2F) of C
//            (the VJP of moe.py:72);
// and, without a second accumulator, a two-phase K: for k >= ksplit the B
// operand is the second matrix at k - ksplit, so that dg Wg^T + du Wu^T is
// one GEMM over [dg | du] (K = 2F).
//
// Tiles of 64 rows x 64 columns, one per workgroup of 4 waves (wave (wm, wn)
// owns a 32 x 32 block); K runs in steps of 16 through LDS.  A single-matrix
// GEMM sums in two interleaved accumulator chains through two LDS stages,
// each step's loads issued two steps ahead; the g/u GEMMs (two chains
// already) load each step at its start through one stage, which keeps more
// workgroups on a CU.  Row tiles are
// numbered per expert segment (ceil(rows / 64) each), found from offsets by
// each workgroup (an LDS scan over the experts); workgroups past the last
// tile exit.  Rows past a segment are never stored.
//
// grouped_wgrad_f32_kernel: the weight gradients, C_e[m][n] = sum over the
// rows r of expert e's segment of A[r][m] * B[r][n] (dWd[e] = h^T d_ys,
// dWg|dWu[e] = xs^T dg|du), one 64 x 64 tile of one expert per workgroup,
// the segment's rows 16 at a time (rows past it load as zero; an empty
// segment writes zeros).  Columns at or past nsplit go to a second output
// (dWu beside dWg).
#include "hmoe_common.h"

namespace hmoe {
namespace {

constexpr int kF32Tile = 64;
constexpr int kF32K = 16;
constexpr int kF32MaxExperts = 1024;

enum F32Epilogue { kEpiPlain = 0, kEpiSwiglu = 1, kEpiDSwiglu = 2 };

__device__ __forceinline__ f32x16 mfma32x2(float a, float b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

template <int EPI, bool BT>
__global__ __launch_bounds__(256) void grouped_gemm_f32_kernel(
    const float* __restrict__ A, const float* __restrict__ B0, const float* __restrict__ B1,
    const int32_t* __restrict__ offsets, int n_experts, int kdim, int ksplit, int ncols,
    const float* __restrict__ dh, float* __restrict__ C, int64_t ldc) {
  constexpr bool kDual = EPI != kEpiPlain;  // two accumulators (g and u)
  __shared__ int32_t mstart[kF32MaxExperts + 1];
  __shared__ int32_t scan[256];
  // A tile [64 rows][16 k] and B tiles [16 k][64 n], +1 float of padding per
  // row so that the operand reads below hit distinct banks; two stages for a
  // single matrix, one for g and u (whose kernels keep more workgroups per CU)
  constexpr int kStages = kDual ? 1 : 2;
  __shared__ float sa[kStages][kF32Tile][kF32K + 1];
  __shared__ float sb0[kStages][kF32K][kF32Tile + 1];
  __shared__ float sb1[1][kDual ? kF32K : 1][kF32Tile + 1];
  const int tid = threadIdx.x;
  // per-expert row-tile starts (exclusive scan of ceil(rows_e / 64))
  const int per = (n_experts + 255) / 256;
  int local = 0;
  for (int j = 0; j < per; ++j) {
    const int e = tid * per + j;
    if (e < n_experts) local += (offsets[e + 1] - offsets[e] + kF32Tile - 1) / kF32Tile;
  }
  scan[tid] = local;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {
    const int v = tid >= off ? scan[tid - off] : 0;
    __syncthreads();
    scan[tid] += v;
    __syncthreads();
  }
  int run = scan[tid] - local;
  for (int j = 0; j < per; ++j) {
    const int e = tid * per + j;
    if (e < n_experts) {
      mstart[e] = run;
      run += (offsets[e + 1] - offsets[e] + kF32Tile - 1) / kF32Tile;
    }
  }
  if (tid == 255) mstart[n_experts] = scan[255];
  __syncthreads();
  const int n_tiles_n = ncols / kF32Tile;
  const int m_tile = blockIdx.x / n_tiles_n;
  const int n0 = (blockIdx.x - m_tile * n_tiles_n) * kF32Tile;
  if (m_tile >= mstart[n_experts]) return;  // uniform per workgroup
  int lo = 0, hi = n_experts;  // largest e with mstart[e] <= m_tile
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (mstart[mid] <= m_tile) lo = mid; else hi = mid;
  }
  const int e = lo;
  const int64_t row0 = offsets[e] + static_cast<int64_t>(m_tile - mstart[e]) * kF32Tile;
  const int64_t row_end = offsets[e + 1];
  // each B matrix is ksplit long along K; expert stride ksplit * ncols
  const int64_t bstride = static_cast<int64_t>(ksplit) * ncols;
  const float* be0 = B0 + e * bstride;
  const float* be1 = B1 != nullptr ? B1 + e * bstride : nullptr;

  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, hi2 = lane >> 5;
  // A single matrix sums in two accumulator chains (the K pairs of a step
  // alternate between them), added before the epilogue.
  f32x16 acc0, acc1, acc0b;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    acc0[r] = 0.0f;
    acc1[r] = 0.0f;
    acc0b[r] = 0.0f;
  }
  // loader: A 64 x 16 = 1024 floats, 4 per thread (row tid / 4, k 4 (tid % 4)
  // .. +4); B 16 x 64, 4 per thread: k tid / 16, n 4 (tid % 16) .. +4, or,
  // transposed, n tid / 4, k 4 (tid % 4) .. +4 (4 consecutive k of a row)
  const int a_r = tid >> 2, a_k = (tid & 3) * 4;
  const int b_k = BT ? (tid & 3) * 4 : tid >> 4;
  const int b_n = BT ? tid >> 2 : (tid & 15) * 4;
  const int64_t ar = row0 + a_r < row_end ? row0 + a_r : row_end - 1;  // rows past: any row
  auto load_b = [&](const float* be, int kk0) __attribute__((always_inline)) {
    return BT ? *reinterpret_cast<const f32x4*>(be + static_cast<int64_t>(n0 + b_n) * ksplit + kk0 + b_k)
              : *reinterpret_cast<const f32x4*>(be + static_cast<int64_t>(kk0 + b_k) * ncols + n0 + b_n);
  };
  f32x4 av, bv0, bv1 = {0.0f, 0.0f, 0.0f, 0.0f};
  auto fetch = [&](int k0) __attribute__((always_inline)) {
    av = *reinterpret_cast<const f32x4*>(A + ar * kdim + k0 + a_k);
    if (kDual) {
      bv0 = load_b(be0, k0);
      bv1 = load_b(be1, k0);
    } else {
      bv0 = k0 < ksplit ? load_b(be0, k0) : load_b(be1, k0 - ksplit);  // uniform branch
    }
  };
  auto park = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      sa[buf][a_r][a_k + q] = av[q];
      if (BT) {
        sb0[buf][b_k + q][b_n] = bv0[q];
        if (kDual) sb1[buf][b_k + q][b_n] = bv1[q];
      } else {
        sb0[buf][b_k][b_n + q] = bv0[q];
        if (kDual) sb1[buf][b_k][b_n + q] = bv1[q];
      }
    }
  };
  const int nsteps = kdim / kF32K;
  if constexpr (kDual) {
    // g and u: one stage, each step's loads at its start; two chains already
    for (int st = 0; st < nsteps; ++st) {
      fetch(st * kF32K);
      __syncthreads();
      park(0);
      __syncthreads();
#pragma unroll
      for (int kk = 0; kk < kF32K; kk += 2) {
        const float x = sa[0][wm * 32 + l32][kk + hi2];
        acc0 = mfma32x2(sb0[0][kk + hi2][wn * 32 + l32], x, acc0);
        acc1 = mfma32x2(sb1[0][kk + hi2][wn * 32 + l32], x, acc1);
      }
    }
  } else {
    // K step s goes global -> registers during step s - 2 and registers ->
    // LDS stage s & 1 at the end of step s - 1.
    fetch(0);
    park(0);
    if (nsteps > 1) fetch(kF32K);
    __syncthreads();
    for (int st = 0; st < nsteps; ++st) {
      const int buf = st & 1;
      // D[m][n] += A[m][k] B[k][n]: lane supplies A[m = l32][k = hi2] (here the
      // weights, so that a lane ends with one token row) and B[k = hi2][n = l32]
#pragma unroll
      for (int kk = 0; kk < kF32K; kk += 4) {
        const float x0 = sa[buf][wm * 32 + l32][kk + hi2];
        const float x1 = sa[buf][wm * 32 + l32][kk + 2 + hi2];
        acc0 = mfma32x2(sb0[buf][kk + hi2][wn * 32 + l32], x0, acc0);
        acc0b = mfma32x2(sb0[buf][kk + 2 + hi2][wn * 32 + l32], x1, acc0b);
      }
      if (st + 1 < nsteps) park(buf ^ 1);
      if (st + 2 < nsteps) fetch((st + 2) * kF32K);
      __syncthreads();
    }
  }
  if (!kDual) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc0[r] += acc0b[r];
  }
  // lane holds row wm*32 + l32 and columns wn*32 + 8 (r/4) + 4 hi2 + r%4
  const int64_t row = row0 + wm * 32 + l32;
  if (row >= row_end) return;
  const int col = n0 + wn * 32 + hi2 * 4;
  float* crow = C + row * ldc + col;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    f32x4 v, w;
    f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
    if (EPI == kEpiDSwiglu) d = *reinterpret_cast<const f32x4*>(dh + row * ncols + col + q * 8);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float g = acc0[4 * q + r];
      if (EPI == kEpiSwiglu) {
        v[r] = (g / (1.0f + expf(-g))) * acc1[4 * q + r];
      } else if (EPI == kEpiDSwiglu) {
#pragma clang fp contract(off)
        const float u = acc1[4 * q + r];
        const float s = 1.0f / (1.0f + expf(-g));
        v[r] = d[r] * u * (s * (1.0f + g * (1.0f - s)));
        w[r] = d[r] * (g * s);
      } else {
        v[r] = g;
      }
    }
    *reinterpret_cast<f32x4*>(crow + q * 8) = v;
    if (EPI == kEpiDSwiglu) *reinterpret_cast<f32x4*>(crow + ncols + q * 8) = w;
  }
}

__global__ __launch_bounds__(256) void grouped_wgrad_f32_kernel(
    const float* __restrict__ A, int64_t lda, const float* __restrict__ B, int64_t ldb,
    const int32_t* __restrict__ offsets, int mdim, int ncols, int nsplit, float* __restrict__ C0,
    float* __restrict__ C1) {
  __shared__ float sa[kF32K][kF32Tile + 1];
  __shared__ float sb[kF32K][kF32Tile + 1];
  const int tid = threadIdx.x;
  const int tm = mdim / kF32Tile, tn = ncols / kF32Tile;
  const int e = static_cast<int>(blockIdx.x / (tm * tn));
  const int rem = static_cast<int>(blockIdx.x - static_cast<int64_t>(e) * tm * tn);
  const int m0 = (rem / tn) * kF32Tile;
  const int n0 = (rem - (rem / tn) * tn) * kF32Tile;
  const int64_t r_lo = offsets[e], r_hi = offsets[e + 1];
  const int lr = tid >> 4, lc = (tid & 15) * 4;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, hi2 = lane >> 5;
  f32x16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
  for (int64_t r0 = r_lo; r0 < r_hi; r0 += kF32K) {
    const int64_t r = r0 + lr;
    f32x4 av = {0.0f, 0.0f, 0.0f, 0.0f}, bv = {0.0f, 0.0f, 0.0f, 0.0f};
    if (r < r_hi) {
      av = *reinterpret_cast<const f32x4*>(A + r * lda + m0 + lc);
      bv = *reinterpret_cast<const f32x4*>(B + r * ldb + n0 + lc);
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      sa[lr][lc + q] = av[q];
      sb[lr][lc + q] = bv[q];
    }
    __syncthreads();
    // D[n][m] += B^T[n][k] A[k][m]: lane supplies B[k = hi2][n = l32] and
    // A[k = hi2][m = l32], so that a lane ends with one output row m
#pragma unroll
    for (int kk = 0; kk < kF32K; kk += 2)
      acc = mfma32x2(sb[kk + hi2][wn * 32 + l32], sa[kk + hi2][wm * 32 + l32], acc);
  }
  // lane holds row m0 + wm*32 + l32 and columns wn*32 + 8 (r/4) + 4 hi2 + r%4
  const int64_t m = m0 + wm * 32 + l32;
  const int col = n0 + wn * 32 + hi2 * 4;
  float* dst;
  if (n0 < nsplit)
    dst = C0 + (static_cast<int64_t>(e) * mdim + m) * nsplit + col;
  else
    dst = C1 + (static_cast<int64_t>(e) * mdim + m) * (ncols - nsplit) + (col - nsplit);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    f32x4 v;
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = acc[4 * q + r];
    *reinterpret_cast<f32x4*>(dst + q * 8) = v;
  }
}

template <int EPI, bool BT>
int launch_f32(const float* A, const float* B0, const float* B1, const int32_t* offsets,
               int n_experts, int64_t rows_cap, int kdim, int ksplit, int ncols, const float* dh,
               float* C, int64_t ldc, hipStream_t s, const char* what) {
  const int64_t m_tiles = ceil_div(rows_cap, kF32Tile) + n_experts;
  const int64_t grid = m_tiles * (ncols / kF32Tile);
  HMOE_REQUIRE(grid < (int64_t(1) << 31), "%s: too many tiles", what);
  hipLaunchKernelGGL((grouped_gemm_f32_kernel<EPI, BT>), dim3(static_cast<unsigned>(grid)), dim3(256),
                     0, s, A, B0, B1, offsets, n_experts, kdim, ksplit, ncols, dh, C, ldc);
  return check_launch(what);
}

int launch_wgrad_f32(const float* A, int64_t lda, const float* B, int64_t ldb,
                     const int32_t* offsets, int n_experts, int mdim, int ncols, int nsplit,
                     float* C0, float* C1, hipStream_t s, const char* what) {
  const int64_t grid = static_cast<int64_t>(n_experts) * (mdim / kF32Tile) * (ncols / kF32Tile);
  HMOE_REQUIRE(grid < (int64_t(1) << 31), "%s: too many tiles", what);
  hipLaunchKernelGGL(grouped_wgrad_f32_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0, s, A,
                     lda, B, ldb, offsets, mdim, ncols, nsplit, C0, C1);
  return check_launch(what);
}

}  // namespace
}  // namespace hmoe

#define HMOE_F32_CHECK_EXPERTS(what)                                                            \
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= kF32MaxExperts,                                   \
               what ": n_experts must be in [1, %d] (got %d)", kF32MaxExperts, n_experts)

extern "C" int hmoe_grouped_gate_up_f32(const float* xs, const int32_t* offsets, int n_experts,
                                        int64_t rows_cap, int d_model, int d_ff,
                                        const float* w_gate, const float* w_up, float* h,
                                        hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_F32_CHECK_EXPERTS("grouped_gate_up_f32");
  HMOE_REQUIRE(rows_cap >= 0, "grouped_gate_up_f32: rows_cap must be >= 0");
  HMOE_REQUIRE_CODE(d_model % kF32K == 0 && d_model > 0 && d_ff % kF32Tile == 0 && d_ff > 0,
                    HMOE_ERR_UNSUPPORTED,
                    "grouped_gate_up_f32: d_model must be a multiple of %d and d_ff of %d "
                    "(got %d, %d)", kF32K, kF32Tile, d_model, d_ff);
  if (rows_cap == 0) return HMOE_OK;
  HMOE_REQUIRE(xs && offsets && w_gate && w_up && h, "grouped_gate_up_f32: null pointer argument");
  return launch_f32<kEpiSwiglu, false>(xs, w_gate, w_up, offsets, n_experts, rows_cap, d_model,
                                       d_model, d_ff, nullptr, h, d_ff,
                                       static_cast<hipStream_t>(stream), "hmoe_grouped_gate_up_f32");
}

extern "C" int hmoe_grouped_down_f32(const float* h, const int32_t* offsets, int n_experts,
                                     int64_t rows_cap, int d_ff, int d_model, const float* w_down,
                                     float* ys, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_F32_CHECK_EXPERTS("grouped_down_f32");
  HMOE_REQUIRE(rows_cap >= 0, "grouped_down_f32: rows_cap must be >= 0");
  HMOE_REQUIRE_CODE(d_ff % kF32K == 0 && d_ff > 0 && d_model % kF32Tile == 0 && d_model > 0,
                    HMOE_ERR_UNSUPPORTED,
                    "grouped_down_f32: d_ff must be a multiple of %d and d_model of %d "
                    "(got %d, %d)", kF32K, kF32Tile, d_ff, d_model);
  if (rows_cap == 0) return HMOE_OK;
  HMOE_REQUIRE(h && offsets && w_down && ys, "grouped_down_f32: null pointer argument");
  return launch_f32<kEpiPlain, false>(h, w_down, nullptr, offsets, n_experts, rows_cap, d_ff, d_ff,
                                      d_model, nullptr, ys, d_model,
                                      static_cast<hipStream_t>(stream), "hmoe_grouped_down_f32");
}

// ---- backward -----------------------------------------------------------------

// Both dims of the backward GEMMs run as K in one of them and as 64-wide
// column tiles in another, so d_model and d_ff are multiples of 64.
#define HMOE_F32_CHECK_DIMS(what)                                                               \
  HMOE_REQUIRE_CODE(d_model % kF32Tile == 0 && d_model > 0 && d_ff % kF32Tile == 0 && d_ff > 0, \
                    HMOE_ERR_UNSUPPORTED,                                                       \
                    what ": d_model and d_ff must be multiples of %d (got %d, %d)", kF32Tile,   \
                    d_model, d_ff)

extern "C" int hmoe_grouped_dgrad_down_f32(const float* d_ys, const int32_t* offsets,
                                           int n_experts, int64_t rows_cap, int d_model, int d_ff,
                                           const float* w_down, float* dh, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_F32_CHECK_EXPERTS("grouped_dgrad_down_f32");
  HMOE_REQUIRE(rows_cap >= 0, "grouped_dgrad_down_f32: rows_cap must be >= 0");
  HMOE_F32_CHECK_DIMS("grouped_dgrad_down_f32");
  if (rows_cap == 0) return HMOE_OK;
  HMOE_REQUIRE(d_ys && offsets && w_down && dh, "grouped_dgrad_down_f32: null pointer argument");
  // dh[r][f] = sum_d d_ys[r][d] Wd[e][f][d]: Wd read transposed
  return launch_f32<kEpiPlain, true>(d_ys, w_down, nullptr, offsets, n_experts, rows_cap, d_model,
                                     d_model, d_ff, nullptr, dh, d_ff,
                                     static_cast<hipStream_t>(stream), "hmoe_grouped_dgrad_down_f32");
}

extern "C" int hmoe_grouped_gate_up_swiglu_bwd_f32(const float* xs, const int32_t* offsets,
                                                   int n_experts, int64_t rows_cap, int d_model,
                                                   int d_ff, const float* w_gate, const float* w_up,
                                                   const float* dh, float* dgu,
                                                   hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_F32_CHECK_EXPERTS("grouped_gate_up_swiglu_bwd_f32");
  HMOE_REQUIRE(rows_cap >= 0, "grouped_gate_up_swiglu_bwd_f32: rows_cap must be >= 0");
  HMOE_F32_CHECK_DIMS("grouped_gate_up_swiglu_bwd_f32");
  if (rows_cap == 0) return HMOE_OK;
  HMOE_REQUIRE(xs && offsets && w_gate && w_up && dh && dgu,
               "grouped_gate_up_swiglu_bwd_f32: null pointer argument");
  return launch_f32<kEpiDSwiglu, false>(xs, w_gate, w_up, offsets, n_experts, rows_cap, d_model,
                                        d_model, d_ff, dh, dgu, 2 * static_cast<int64_t>(d_ff),
                                        static_cast<hipStream_t>(stream),
                                        "hmoe_grouped_gate_up_swiglu_bwd_f32");
}

extern "C" int hmoe_grouped_dgrad_gate_up_f32(const float* dgu, const int32_t* offsets,
                                              int n_experts, int64_t rows_cap, int d_model,
                                              int d_ff, const float* w_gate, const float* w_up,
                                              float* d_xs, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_F32_CHECK_EXPERTS("grouped_dgrad_gate_up_f32");
  HMOE_REQUIRE(rows_cap >= 0, "grouped_dgrad_gate_up_f32: rows_cap must be >= 0");
  HMOE_F32_CHECK_DIMS("grouped_dgrad_gate_up_f32");
  if (rows_cap == 0) return HMOE_OK;
  HMOE_REQUIRE(dgu && offsets && w_gate && w_up && d_xs,
               "grouped_dgrad_gate_up_f32: null pointer argument");
  // d_xs[r][d] = sum_f dg[r][f] Wg[e][d][f] + du[r][f] Wu[e][d][f]: K = 2F in
  // two phases, both masters read transposed
  return launch_f32<kEpiPlain, true>(dgu, w_gate, w_up, offsets, n_experts, rows_cap, 2 * d_ff,
                                     d_ff, d_model, nullptr, d_xs, d_model,
                                     static_cast<hipStream_t>(stream),
                                     "hmoe_grouped_dgrad_gate_up_f32");
}

extern "C" int hmoe_grouped_wgrad_gate_up_f32(const float* xs, const float* dgu,
                                              const int32_t* offsets, int n_experts, int d_model,
                                              int d_ff, float* dw_gate, float* dw_up,
                                              hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_F32_CHECK_EXPERTS("grouped_wgrad_gate_up_f32");
  HMOE_F32_CHECK_DIMS("grouped_wgrad_gate_up_f32");
  HMOE_REQUIRE(xs && dgu && offsets && dw_gate && dw_up,
               "grouped_wgrad_gate_up_f32: null pointer argument");
  return launch_wgrad_f32(xs, d_model, dgu, 2 * static_cast<int64_t>(d_ff), offsets, n_experts,
                          d_model, 2 * d_ff, d_ff, dw_gate, dw_up, static_cast<hipStream_t>(stream),
                          "hmoe_grouped_wgrad_gate_up_f32");
}

extern "C" int hmoe_grouped_wgrad_down_f32(const float* h, const float* d_ys,
                                           const int32_t* offsets, int n_experts, int d_ff,
                                           int d_model, float* dw_down, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_F32_CHECK_EXPERTS("grouped_wgrad_down_f32");
  HMOE_F32_CHECK_DIMS("grouped_wgrad_down_f32");
  HMOE_REQUIRE(h && d_ys && offsets && dw_down, "grouped_wgrad_down_f32: null pointer argument");
  return launch_wgrad_f32(h, d_ff, d_ys, d_model, offsets, n_experts, d_ff, d_model, d_model,
                          dw_down, nullptr, static_cast<hipStream_t>(stream),
                          "hmoe_grouped_wgrad_down_f32");
}
