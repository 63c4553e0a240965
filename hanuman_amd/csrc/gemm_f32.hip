// Float32 expert path (compute dtype float32, moe.py:70-74 and the shared
// expert's swiglu, moe.py:23-29): the grouped GEMM on the float32 matrix
// cores, v_mfma_f32_32x32x2_f32 (exact float32 products, float32 sums).
//
// C[r][n] = sum_k A[r][k] * B_e[k][n] over the rows r of expert e's segment
// [offsets[e], offsets[e+1]); A [rows, K] and B_e [K, ncols] row-major float32
// (the masters as they are: w_gate/w_up [N, D, F], w_down [N, F, D]).  With
// SWIGLU the GEMM runs against both gate and up weights and writes
// h = silu(g) * u in float32.
//
// Tiles of 64 rows x 64 columns, one per workgroup of 4 waves (wave (wm, wn)
// owns a 32 x 32 block); K runs in steps of 16 through LDS.  Row tiles are
// numbered per expert segment (ceil(rows / 64) each), found from offsets by
// each workgroup (an LDS scan over the experts); workgroups past the last
// tile exit.  Rows past a segment are never stored.
#include "hmoe_common.h"

namespace hmoe {
namespace {

constexpr int kF32Tile = 64;
constexpr int kF32K = 16;
constexpr int kF32MaxExperts = 1024;

__device__ __forceinline__ f32x16 mfma32x2(float a, float b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

template <bool SWIGLU>
__global__ __launch_bounds__(256) void grouped_gemm_f32_kernel(
    const float* __restrict__ A, const float* __restrict__ B0, const float* __restrict__ B1,
    const int32_t* __restrict__ offsets, int n_experts, int kdim, int ncols,
    float* __restrict__ C, int64_t ldc) {
  __shared__ int32_t mstart[kF32MaxExperts + 1];
  __shared__ int32_t scan[256];
  // A tile [64 rows][16 k] and B tiles [16 k][64 n], +1 float of padding per
  // row so that the operand reads below hit distinct banks
  __shared__ float sa[kF32Tile][kF32K + 1];
  __shared__ float sb0[kF32K][kF32Tile + 1];
  __shared__ float sb1[SWIGLU ? kF32K : 1][kF32Tile + 1];
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
  const float* be0 = B0 + static_cast<int64_t>(e) * kdim * ncols;
  const float* be1 = SWIGLU ? B1 + static_cast<int64_t>(e) * kdim * ncols : nullptr;

  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, hi2 = lane >> 5;
  f32x16 acc0, acc1;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    acc0[r] = 0.0f;
    acc1[r] = 0.0f;
  }
  // loader: A 64 x 16 = 1024 floats, 4 per thread (rows tid / 4, k 4 (tid % 4)
  // .. +4); B 16 x 64, 4 per thread (k tid / 16, n 4 (tid % 16) .. +4)
  const int a_r = tid >> 2, a_k = (tid & 3) * 4;
  const int b_k = tid >> 4, b_n = (tid & 15) * 4;
  const int64_t ar = row0 + a_r < row_end ? row0 + a_r : row_end - 1;  // rows past: any row
  for (int k0 = 0; k0 < kdim; k0 += kF32K) {
    const f32x4 av = *reinterpret_cast<const f32x4*>(A + ar * kdim + k0 + a_k);
    const f32x4 bv0 =
        *reinterpret_cast<const f32x4*>(be0 + static_cast<int64_t>(k0 + b_k) * ncols + n0 + b_n);
    f32x4 bv1 = {0.0f, 0.0f, 0.0f, 0.0f};
    if (SWIGLU)
      bv1 = *reinterpret_cast<const f32x4*>(be1 + static_cast<int64_t>(k0 + b_k) * ncols + n0 + b_n);
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      sa[a_r][a_k + q] = av[q];
      sb0[b_k][b_n + q] = bv0[q];
      if (SWIGLU) sb1[b_k][b_n + q] = bv1[q];
    }
    __syncthreads();
    // D[m][n] += A[m][k] B[k][n]: lane supplies A[m = l32][k = hi2] (here the
    // weights, so that a lane ends with one token row) and B[k = hi2][n = l32]
#pragma unroll
    for (int kk = 0; kk < kF32K; kk += 2) {
      const float x = sa[wm * 32 + l32][kk + hi2];
      acc0 = mfma32x2(sb0[kk + hi2][wn * 32 + l32], x, acc0);
      if (SWIGLU) acc1 = mfma32x2(sb1[kk + hi2][wn * 32 + l32], x, acc1);
    }
  }
  // lane holds row wm*32 + l32 and columns wn*32 + 8 (r/4) + 4 hi2 + r%4
  const int64_t row = row0 + wm * 32 + l32;
  if (row >= row_end) return;
  float* crow = C + row * ldc + n0 + wn * 32 + hi2 * 4;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    f32x4 v;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float g = acc0[4 * q + r];
      v[r] = SWIGLU ? (g / (1.0f + expf(-g))) * acc1[4 * q + r] : g;
    }
    *reinterpret_cast<f32x4*>(crow + q * 8) = v;
  }
}

int launch_f32(bool swiglu, const float* A, const float* B0, const float* B1,
               const int32_t* offsets, int n_experts, int64_t rows_cap, int kdim, int ncols,
               float* C, hipStream_t s, const char* what) {
  const int64_t m_tiles = ceil_div(rows_cap, kF32Tile) + n_experts;
  const int64_t grid = m_tiles * (ncols / kF32Tile);
  HMOE_REQUIRE(grid < (int64_t(1) << 31), "%s: too many tiles", what);
  if (swiglu)
    hipLaunchKernelGGL(grouped_gemm_f32_kernel<true>, dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                       s, A, B0, B1, offsets, n_experts, kdim, ncols, C, static_cast<int64_t>(ncols));
  else
    hipLaunchKernelGGL(grouped_gemm_f32_kernel<false>, dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                       s, A, B0, B1, offsets, n_experts, kdim, ncols, C, static_cast<int64_t>(ncols));
  return check_launch(what);
}

}  // namespace
}  // namespace hmoe

extern "C" int hmoe_grouped_gate_up_f32(const float* xs, const int32_t* offsets, int n_experts,
                                        int64_t rows_cap, int d_model, int d_ff,
                                        const float* w_gate, const float* w_up, float* h,
                                        hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= kF32MaxExperts,
               "grouped_gate_up_f32: n_experts must be in [1, %d] (got %d)", kF32MaxExperts,
               n_experts);
  HMOE_REQUIRE(rows_cap >= 0, "grouped_gate_up_f32: rows_cap must be >= 0");
  HMOE_REQUIRE_CODE(d_model % kF32K == 0 && d_model > 0 && d_ff % kF32Tile == 0 && d_ff > 0,
                    HMOE_ERR_UNSUPPORTED,
                    "grouped_gate_up_f32: d_model must be a multiple of %d and d_ff of %d "
                    "(got %d, %d)", kF32K, kF32Tile, d_model, d_ff);
  if (rows_cap == 0) return HMOE_OK;
  HMOE_REQUIRE(xs && offsets && w_gate && w_up && h, "grouped_gate_up_f32: null pointer argument");
  return launch_f32(true, xs, w_gate, w_up, offsets, n_experts, rows_cap, d_model, d_ff, h,
                    static_cast<hipStream_t>(stream), "hmoe_grouped_gate_up_f32");
}

extern "C" int hmoe_grouped_down_f32(const float* h, const int32_t* offsets, int n_experts,
                                     int64_t rows_cap, int d_ff, int d_model, const float* w_down,
                                     float* ys, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= kF32MaxExperts,
               "grouped_down_f32: n_experts must be in [1, %d] (got %d)", kF32MaxExperts, n_experts);
  HMOE_REQUIRE(rows_cap >= 0, "grouped_down_f32: rows_cap must be >= 0");
  HMOE_REQUIRE_CODE(d_ff % kF32K == 0 && d_ff > 0 && d_model % kF32Tile == 0 && d_model > 0,
                    HMOE_ERR_UNSUPPORTED,
                    "grouped_down_f32: d_ff must be a multiple of %d and d_model of %d "
                    "(got %d, %d)", kF32K, kF32Tile, d_ff, d_model);
  if (rows_cap == 0) return HMOE_OK;
  HMOE_REQUIRE(h && offsets && w_down && ys, "grouped_down_f32: null pointer argument");
  return launch_f32(false, h, w_down, nullptr, offsets, n_experts, rows_cap, d_ff, d_model, ys,
                    static_cast<hipStream_t>(stream), "hmoe_grouped_down_f32");
}
