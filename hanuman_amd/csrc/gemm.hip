// Ragged grouped GEMM on gfx950 bf16 MFMA (model/moe.py:67-74: the three
// `jax.lax.ragged_dot` calls and the SwiGLU between them).
//
//   C[r, n] = sum_k A[r, k] * B_e[n, k]     for rows r of expert e's segment
//
// A is the dispatched activation buffer (rows grouped by expert, K contiguous)
// and B_e the packed expert weight (one row per output column, K contiguous).
// With SWIGLU the packed columns alternate 32 gate / 32 up columns of the same
// h columns and the epilogue writes h = bf16(silu(gate) * up).
//
// Tiling: one workgroup (4 waves) computes a 256 x 256 output tile; wave
// (wm, wn) owns a 128 x 128 quarter as 4 x 4 blocks of
// v_mfma_f32_32x32x16_bf16.  K advances 64 at a time through two LDS stages
// (rows padded to 72 bf16 = 144 bytes, so the 16-byte fragment reads of eight
// consecutive lanes hit all 32 banks once).  Global loads for the next stage
// are issued before the current stage's MFMAs.  The MFMA takes the weight
// fragment as its first operand, so an accumulator lane holds one token row
// and four consecutive output columns per group, stored as one 8-byte write.
//
// Scheduling: blocks enumerate (m-tile, n-tile) with n fastest; m-tiles are
// numbered expert by expert (ceil(rows_e / 256) each, computed in-kernel from
// `offsets`).  The launch covers the static bound ceil(rows_cap/256) + N
// m-tiles; blocks past the real count return at once.  A rows are read
// through clamped pointers, so buffers need exactly rows_cap rows.  Consecutive logical
// tiles are placed on the same XCD (workgroups are dealt round-robin over the
// 8 XCDs), so tiles sharing an A row block or a B column block share an L2.
#include "hmoe_common.h"

namespace hmoe {
namespace {

constexpr int kBM = HMOE_GEMM_TILE_M;
constexpr int kBN = 256;
constexpr int kBK = 64;
constexpr int kPitch = kBK + 8;
constexpr int kThreads = 256;
constexpr int kStageElems = kBM * kPitch;
constexpr int kMaxExperts = 1024;
constexpr int kNumXcd = 8;

static_assert(kBM == 256, "tile loaders assume 256-row tiles");

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + __expf(-g)); }

template <bool SWIGLU>
__global__ __launch_bounds__(kThreads) void grouped_gemm_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
    const int32_t* __restrict__ offsets, int n_experts, int64_t a_rows, int kdim, int ncols,
    uint16_t* __restrict__ C, int64_t ldc, int n_tiles_n) {
  __shared__ __attribute__((aligned(16))) uint16_t smem[2][2][kStageElems];
  __shared__ int32_t tstart[kMaxExperts + 1];
  __shared__ int32_t scan_tmp[kThreads];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  // ---- tile schedule: m-tiles per expert, exclusive scan ----------------
  {
    int local[4];
    int sum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = tid * 4 + j;
      int tiles = 0;
      if (e < n_experts) {
        const int rows = offsets[e + 1] - offsets[e];
        tiles = (rows + kBM - 1) / kBM;
      }
      local[j] = tiles;
      sum += tiles;
    }
    scan_tmp[tid] = sum;
    __syncthreads();
    for (int off = 1; off < kThreads; off <<= 1) {
      const int v = tid >= off ? scan_tmp[tid - off] : 0;
      __syncthreads();
      scan_tmp[tid] += v;
      __syncthreads();
    }
    int run = scan_tmp[tid] - sum;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = tid * 4 + j;
      if (e < n_experts) tstart[e] = run;
      run += local[j];
    }
    if (tid == kThreads - 1) tstart[n_experts] = scan_tmp[kThreads - 1];
    __syncthreads();
  }

  const int grid = gridDim.x;
  const int pid = blockIdx.x;
  const int logical = (pid % kNumXcd) * (grid / kNumXcd) + pid / kNumXcd;
  const int m_tile = logical / n_tiles_n;
  const int n_tile = logical % n_tiles_n;
  if (m_tile >= tstart[n_experts]) return;  // uniform per workgroup
  int lo = 0, hi = n_experts;  // largest e with tstart[e] <= m_tile
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (tstart[mid] <= m_tile) lo = mid; else hi = mid;
  }
  const int e = lo;
  const int64_t row0 = offsets[e] + static_cast<int64_t>(m_tile - tstart[e]) * kBM;
  const int64_t row_end = offsets[e + 1];
  const int n0 = n_tile * kBN;

  const uint16_t* b_base = B + (static_cast<int64_t>(e) * ncols + n0) * kdim;

  // ---- global -> register staging (8 x 16 B of A and of B per thread) ----
  // A rows past the buffer (the last tile of the last segment) are clamped
  // to its last row; their results are never stored.
  const int ld_row = tid >> 3;
  const int ld_col = (tid & 7) * 8;
  const uint16_t* a_ptr[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int64_t r = row0 + ld_row + 32 * i;
    r = r < a_rows ? r : a_rows - 1;
    a_ptr[i] = A + r * kdim + ld_col;
  }
  u32x4 ra[8], rb[8];
  auto load_stage = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = ld_row + 32 * i;
      ra[i] = *reinterpret_cast<const u32x4*>(a_ptr[i] + k0);
      rb[i] = *reinterpret_cast<const u32x4*>(b_base + static_cast<int64_t>(r) * kdim + k0 + ld_col);
    }
  };
  auto store_stage = [&](int st) {
    uint16_t* sa = smem[st][0];
    uint16_t* sb = smem[st][1];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = ld_row + 32 * i;
      *reinterpret_cast<u32x4*>(sa + r * kPitch + ld_col) = ra[i];
      *reinterpret_cast<u32x4*>(sb + r * kPitch + ld_col) = rb[i];
    }
  };

  const int wm = wave >> 1, wn = wave & 1;
  const int frag_row = lane & 31;
  const int frag_k = (lane >> 5) * 8;
  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int ktiles = kdim / kBK;
  load_stage(0);
  store_stage(0);
  __syncthreads();
  for (int kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < ktiles) load_stage((kt + 1) * kBK);
    const uint16_t* sa = smem[cur][0] + (wm * 128 + frag_row) * kPitch + frag_k;
    const uint16_t* sb = smem[cur][1] + (wn * 128 + frag_row) * kPitch + frag_k;
#pragma unroll
    for (int k16 = 0; k16 < kBK / 16; ++k16) {
      bf16x8 af[4], bfr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        af[i] = *reinterpret_cast<const bf16x8*>(sa + i * 32 * kPitch + k16 * 16);
        bfr[i] = *reinterpret_cast<const bf16x8*>(sb + i * 32 * kPitch + k16 * 16);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < ktiles) store_stage(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue ----------------------------------------------------------
  // acc[i][j] lane L, element r: token row wm*128 + i*32 + (L & 31);
  // column wn*128 + j*32 + (r/4)*8 + (L>>5)*4 + (r&3).
  const int col_lane = (lane >> 5) * 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = row0 + wm * 128 + i * 32 + frag_row;
    if (row >= row_end) continue;
    uint16_t* crow = C + row * ldc;
    if (SWIGLU) {
      const int hbase = (n0 + wn * 128) / 2;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float h[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float gv = acc[i][2 * p][g * 4 + q];
            const float uv = acc[i][2 * p + 1][g * 4 + q];
            h[q] = silu_f32(gv) * uv;
          }
          uint2 pk;
          pk.x = pack_bf16x2(h[0], h[1]);
          pk.y = pack_bf16x2(h[2], h[3]);
          *reinterpret_cast<uint2*>(crow + hbase + p * 32 + g * 8 + col_lane) = pk;
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          uint2 pk;
          pk.x = pack_bf16x2(acc[i][j][g * 4 + 0], acc[i][j][g * 4 + 1]);
          pk.y = pack_bf16x2(acc[i][j][g * 4 + 2], acc[i][j][g * 4 + 3]);
          *reinterpret_cast<uint2*>(crow + n0 + wn * 128 + j * 32 + g * 8 + col_lane) = pk;
        }
      }
    }
  }
}

int launch_grouped(bool swiglu, const void* A, const void* B, const int32_t* offsets,
                   int n_experts, int64_t rows_cap, int kdim, int ncols, void* C, int64_t ldc,
                   hipStream_t s, const char* what) {
  const int n_tiles_n = ncols / kBN;
  const int64_t m_tiles = ceil_div(rows_cap, kBM) + n_experts;
  int64_t blocks = m_tiles * n_tiles_n;
  blocks = ceil_div(blocks, kNumXcd) * kNumXcd;
  HMOE_REQUIRE(blocks < (int64_t(1) << 31), "%s: too many tiles", what);
  if (swiglu)
    hipLaunchKernelGGL(grouped_gemm_kernel<true>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s,
                       static_cast<const uint16_t*>(A), static_cast<const uint16_t*>(B), offsets,
                       n_experts, rows_cap, kdim, ncols, static_cast<uint16_t*>(C), ldc, n_tiles_n);
  else
    hipLaunchKernelGGL(grouped_gemm_kernel<false>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s,
                       static_cast<const uint16_t*>(A), static_cast<const uint16_t*>(B), offsets,
                       n_experts, rows_cap, kdim, ncols, static_cast<uint16_t*>(C), ldc, n_tiles_n);
  return check_launch(what);
}

}  // namespace
}  // namespace hmoe

extern "C" int hmoe_grouped_gate_up(const void* xs, const int32_t* offsets, int n_experts,
                                    int64_t rows_cap, int d_model, int d_ff,
                                    const void* w_gate_up_packed, void* h, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= kMaxExperts,
               "grouped_gate_up: n_experts must be in [1, %d] (got %d)", kMaxExperts, n_experts);
  HMOE_REQUIRE(rows_cap >= 0, "grouped_gate_up: rows_cap must be >= 0");
  HMOE_REQUIRE_CODE(d_model % kBK == 0 && d_model >= kBK, HMOE_ERR_UNSUPPORTED,
                    "grouped_gate_up: d_model must be a multiple of %d (got %d)", kBK, d_model);
  HMOE_REQUIRE_CODE((2 * d_ff) % kBN == 0 && d_ff > 0, HMOE_ERR_UNSUPPORTED,
                    "grouped_gate_up: d_ff must be a multiple of %d (got %d)", kBN / 2, d_ff);
  if (rows_cap == 0) return HMOE_OK;
  HMOE_REQUIRE(xs && offsets && w_gate_up_packed && h, "grouped_gate_up: null pointer argument");
  return launch_grouped(true, xs, w_gate_up_packed, offsets, n_experts, rows_cap, d_model, 2 * d_ff,
                        h, d_ff, static_cast<hipStream_t>(stream), "hmoe_grouped_gate_up");
}

extern "C" int hmoe_grouped_down(const void* h, const int32_t* offsets, int n_experts,
                                 int64_t rows_cap, int d_ff, int d_model,
                                 const void* w_down_packed, void* ys, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= kMaxExperts,
               "grouped_down: n_experts must be in [1, %d] (got %d)", kMaxExperts, n_experts);
  HMOE_REQUIRE(rows_cap >= 0, "grouped_down: rows_cap must be >= 0");
  HMOE_REQUIRE_CODE(d_ff % kBK == 0 && d_ff >= kBK, HMOE_ERR_UNSUPPORTED,
                    "grouped_down: d_ff must be a multiple of %d (got %d)", kBK, d_ff);
  HMOE_REQUIRE_CODE(d_model % kBN == 0 && d_model > 0, HMOE_ERR_UNSUPPORTED,
                    "grouped_down: d_model must be a multiple of %d (got %d)", kBN, d_model);
  if (rows_cap == 0) return HMOE_OK;
  HMOE_REQUIRE(h && offsets && w_down_packed && ys, "grouped_down: null pointer argument");
  return launch_grouped(false, h, w_down_packed, offsets, n_experts, rows_cap, d_ff, d_model, ys,
                        d_model, static_cast<hipStream_t>(stream), "hmoe_grouped_down");
}
