// Expert-weight packing (model/moe.py:204-206 casts the fp32 masters to the
// compute dtype on every call; here the cast happens once, into the layout the
// grouped GEMM reads).
//
// Both packed operands are "K contiguous": one row per output column of the
// GEMM, the reduction dimension innermost, so the GEMM loads A and B tiles the
// same way.  Gate and up weights share one operand whose rows alternate 32
// gate columns and 32 up columns of the same h columns, so one 32x32 MFMA
// output block of gate and the next one of up hold matching h elements in the
// same lanes and the SwiGLU runs in registers.
#include "hmoe_common.h"

namespace hmoe {
namespace {

template <typename TW>
__device__ __forceinline__ float load_w(const TW* p, int64_t i);
template <>
__device__ __forceinline__ float load_w<float>(const float* p, int64_t i) {
  return p[i];
}
template <>
__device__ __forceinline__ float load_w<uint16_t>(const uint16_t* p, int64_t i) {
  return bf16_bits_to_f32(p[i]);
}

// Transposes 64x64 tiles of src[e][r][c] (rows r < R, cols c < Cc) into
// dst[e][c][r] as bf16; `col_of_row` maps a destination row index to the
// source (tensor, column) pair for the interleaved gate/up layout.
template <typename TW, bool GATE_UP>
__global__ __launch_bounds__(256) void pack_transpose_kernel(const TW* __restrict__ src0,
                                                             const TW* __restrict__ src1,
                                                             int rows_r, int cols_c,
                                                             uint16_t* __restrict__ dst) {
  __shared__ float tile[64][65];
  const int e = blockIdx.z;
  const int r0 = blockIdx.y * 64;  // source row (reduction dim)
  const int p0 = blockIdx.x * 64;  // destination row (output column, packed)
  const int dst_rows = GATE_UP ? 2 * cols_c : cols_c;
  const int64_t src_stride_e = static_cast<int64_t>(rows_r) * cols_c;
  const int tid = threadIdx.x;
  // Load: 4 consecutive tile columns per thread (16 threads per source row,
  // 16 rows per pass); the four stay inside one 32-column gate or up block.
  {
    const int q = (tid & 15) * 4;
    const int p = p0 + q;
    const TW* srcp = src0;
    int col = p;
    if (GATE_UP) {
      srcp = ((p & 63) < 32) ? src0 : src1;
      col = (p >> 6) * 32 + (p & 31);
    }
    const bool vec = p + 3 < dst_rows && (cols_c & 3) == 0;  // aligned 4-column groups
#pragma unroll
    for (int pass = 0; pass < 4; ++pass) {
      const int rr = (tid >> 4) + 16 * pass;
      const int r = r0 + rr;
      float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (r < rows_r) {
        const int64_t base = e * src_stride_e + static_cast<int64_t>(r) * cols_c + col;
        if (vec) {
          if constexpr (sizeof(TW) == 4) {
            const f32x4 x = *reinterpret_cast<const f32x4*>(srcp + base);
#pragma unroll
            for (int k = 0; k < 4; ++k) v[k] = x[k];
          } else {
            const uint2 x = *reinterpret_cast<const uint2*>(srcp + base);
            v[0] = __uint_as_float(x.x << 16);
            v[1] = __uint_as_float(x.x & 0xffff0000u);
            v[2] = __uint_as_float(x.y << 16);
            v[3] = __uint_as_float(x.y & 0xffff0000u);
          }
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k)
            if (p + k < dst_rows) v[k] = load_w(srcp, base + k);
        }
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) tile[rr][q + k] = v[k];
    }
  }
  __syncthreads();
  // Store: 8 consecutive reduction-dim values of one destination row per
  // thread as one 16-byte store (8 threads per 128-byte row, 32 rows per
  // pass).
  {
    const int r8 = (tid & 7) * 8;
    const int r = r0 + r8;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      const int pp = (tid >> 3) + 32 * pass;
      const int p = p0 + pp;
      if (p >= dst_rows) continue;
      uint16_t* d = dst + (static_cast<int64_t>(e) * dst_rows + p) * rows_r + r;
      if (r + 7 < rows_r && (rows_r & 7) == 0) {
        u32x4 o;
#pragma unroll
        for (int k = 0; k < 4; ++k)
          o[k] = static_cast<uint32_t>(f32_to_bf16_bits(tile[r8 + 2 * k][pp])) |
                 (static_cast<uint32_t>(f32_to_bf16_bits(tile[r8 + 2 * k + 1][pp])) << 16);
        *reinterpret_cast<u32x4*>(d) = o;
      } else {
        for (int k = 0; k < 8 && r + k < rows_r; ++k) d[k] = f32_to_bf16_bits(tile[r8 + k][pp]);
      }
    }
  }
}

// Operands of the backward's data-gradient GEMMs, which contract over the
// forward's output columns: the masters are already "K contiguous" for them,
// so packing is a bf16 cast row by row.  GATE_UP interleaves row r of w_gate
// and w_up in 32-column blocks (destination column p holds gate column
// (p / 64) * 32 + p % 32 when p % 64 < 32, else that up column), the column
// order of the gate/up GEMM's output.  One thread per 8 destination values.
template <typename TW, bool GATE_UP>
__global__ __launch_bounds__(256) void pack_rows_kernel(const TW* __restrict__ src0,
                                                        const TW* __restrict__ src1,
                                                        int64_t rows, int cols_c,
                                                        uint16_t* __restrict__ dst) {
  const int dst_cols = GATE_UP ? 2 * cols_c : cols_c;
  const int64_t groups = rows * (dst_cols / 8);
  for (int64_t gi = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; gi < groups;
       gi += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t r = gi / (dst_cols / 8);
    const int p0 = static_cast<int>(gi - r * (dst_cols / 8)) * 8;
    const TW* src = src0;
    int c0 = p0;
    if (GATE_UP) {
      src = (p0 & 63) < 32 ? src0 : src1;
      c0 = (p0 >> 6) * 32 + (p0 & 31);
    }
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      w[q] = pack_bf16x2(load_w(src, r * cols_c + c0 + 2 * q), load_w(src, r * cols_c + c0 + 2 * q + 1));
    *reinterpret_cast<u32x4*>(dst + r * dst_cols + p0) = u32x4{w[0], w[1], w[2], w[3]};
  }
}

// ----------------------------------------------------------- e4m3 packing --
// Per-output-channel e4m3 codes (same rule as the activations: codes
// e4m3(clamp(w * (448/amax), +-448)), scale amax/448, amax over the reduction
// dimension of the column).  Three passes: column amax into `scales` (packed
// order), the transpose-quantise, then amax -> amax/448 in place.

// amax over rows_r of column c of src[e] (rows_r x cols_c), written to
// out[e * out_stride + packed_row(c)].  Block (64, 4): 64 columns, 4 row groups.
template <typename TW, bool GATE_UP>
__global__ __launch_bounds__(256) void colmax_kernel(const TW* __restrict__ src, int rows_r,
                                                     int cols_c, int up_half, float* __restrict__ out,
                                                     int out_stride) {
  __shared__ float part[4][64];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int e = blockIdx.y;
  const int c = blockIdx.x * 64 + tx;
  float m = 0.0f;
  if (c < cols_c) {
    const TW* col = src + static_cast<int64_t>(e) * rows_r * cols_c + c;
    for (int r = ty; r < rows_r; r += 4) m = fmaxf(m, fabsf(load_w(col, static_cast<int64_t>(r) * cols_c)));
  }
  part[ty][tx] = m;
  __syncthreads();
  if (ty == 0 && c < cols_c) {
    m = fmaxf(fmaxf(part[0][tx], part[1][tx]), fmaxf(part[2][tx], part[3][tx]));
    // Packed row of column c: gate/up interleave 32 columns of each per 64 rows.
    const int p = GATE_UP ? (c >> 5) * 64 + up_half * 32 + (c & 31) : c;
    out[static_cast<int64_t>(e) * out_stride + p] = m;
  }
}

__device__ __forceinline__ uint8_t e4m3_code(float v) {
  v = fminf(fmaxf(v, -448.0f), 448.0f);
  return static_cast<uint8_t>(__builtin_amdgcn_cvt_pk_fp8_f32(v, 0.0f, 0, false) & 0xff);
}

// Transposes 64x64 tiles of src[e][r][c] into e4m3 dst[e][p][r] like
// pack_transpose_kernel, scaling each packed row p by 448/amax[e][p].
template <typename TW, bool GATE_UP>
__global__ __launch_bounds__(256) void pack_fp8_kernel(const TW* __restrict__ src0,
                                                       const TW* __restrict__ src1, int rows_r,
                                                       int cols_c, const float* __restrict__ amax,
                                                       uint8_t* __restrict__ dst) {
  __shared__ float tile[64][65];
  const int e = blockIdx.z;
  const int r0 = blockIdx.y * 64;
  const int p0 = blockIdx.x * 64;
  const int dst_rows = GATE_UP ? 2 * cols_c : cols_c;
  const int64_t src_stride_e = static_cast<int64_t>(rows_r) * cols_c;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int rr = ty; rr < 64; rr += 4) {
    const int r = r0 + rr;
    const int p = p0 + tx;
    float v = 0.0f;
    if (r < rows_r && p < dst_rows) {
      const TW* s = src0;
      int col = p;
      if (GATE_UP) {
        s = ((p & 63) < 32) ? src0 : src1;
        col = (p >> 6) * 32 + (p & 31);
      }
      v = load_w(s, e * src_stride_e + static_cast<int64_t>(r) * cols_c + col);
    }
    tile[rr][tx] = v;
  }
  __syncthreads();
  for (int pp = ty; pp < 64; pp += 4) {
    const int p = p0 + pp;
    const int r = r0 + tx;
    if (p < dst_rows && r < rows_r) {
      const float m = amax[static_cast<int64_t>(e) * dst_rows + p];
      const float inv = m > 0.0f ? 448.0f / m : 1.0f;
      dst[(static_cast<int64_t>(e) * dst_rows + p) * rows_r + r] = e4m3_code(tile[tx][pp] * inv);
    }
  }
}

__global__ __launch_bounds__(256) void amax_to_scale_kernel(float* __restrict__ v, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) v[i] = v[i] > 0.0f ? v[i] / 448.0f : 1.0f;
}

}  // namespace
}  // namespace hmoe

extern "C" size_t hmoe_packed_fp8_gate_up_bytes(int n_experts, int d_model, int d_ff) {
  if (n_experts <= 0 || d_model <= 0 || d_ff <= 0) return 0;
  return static_cast<size_t>(n_experts) * 2 * d_ff * d_model;
}

extern "C" size_t hmoe_packed_fp8_down_bytes(int n_experts, int d_ff, int d_model) {
  if (n_experts <= 0 || d_model <= 0 || d_ff <= 0) return 0;
  return static_cast<size_t>(n_experts) * d_ff * d_model;
}

extern "C" int hmoe_pack_fp8_gate_up(const void* w_gate, const void* w_up, int w_dtype,
                                     int n_experts, int d_model, int d_ff, uint8_t* packed,
                                     float* scales, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(n_experts >= 1 && d_model >= 1 && d_ff >= 1, "pack_fp8_gate_up: sizes must be >= 1");
  HMOE_REQUIRE(d_ff % 32 == 0, "pack_fp8_gate_up: d_ff must be a multiple of 32 (got %d)", d_ff);
  HMOE_REQUIRE(w_dtype == HMOE_F32 || w_dtype == HMOE_BF16,
               "pack_fp8_gate_up: dtype must be F32 or BF16");
  HMOE_REQUIRE(w_gate && w_up && packed && scales, "pack_fp8_gate_up: null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 cgrid(static_cast<unsigned>(ceil_div(d_ff, 64)), static_cast<unsigned>(n_experts));
  const dim3 tgrid(static_cast<unsigned>(ceil_div(2 * d_ff, 64)),
                   static_cast<unsigned>(ceil_div(d_model, 64)), static_cast<unsigned>(n_experts));
  if (w_dtype == HMOE_F32) {
    const float* g = static_cast<const float*>(w_gate);
    const float* u = static_cast<const float*>(w_up);
    hipLaunchKernelGGL((colmax_kernel<float, true>), cgrid, dim3(256), 0, s, g, d_model, d_ff, 0, scales, 2 * d_ff);
    hipLaunchKernelGGL((colmax_kernel<float, true>), cgrid, dim3(256), 0, s, u, d_model, d_ff, 1, scales, 2 * d_ff);
    hipLaunchKernelGGL((pack_fp8_kernel<float, true>), tgrid, dim3(256), 0, s, g, u, d_model, d_ff, scales, packed);
  } else {
    const uint16_t* g = static_cast<const uint16_t*>(w_gate);
    const uint16_t* u = static_cast<const uint16_t*>(w_up);
    hipLaunchKernelGGL((colmax_kernel<uint16_t, true>), cgrid, dim3(256), 0, s, g, d_model, d_ff, 0, scales, 2 * d_ff);
    hipLaunchKernelGGL((colmax_kernel<uint16_t, true>), cgrid, dim3(256), 0, s, u, d_model, d_ff, 1, scales, 2 * d_ff);
    hipLaunchKernelGGL((pack_fp8_kernel<uint16_t, true>), tgrid, dim3(256), 0, s, g, u, d_model, d_ff, scales, packed);
  }
  const int64_t n = static_cast<int64_t>(n_experts) * 2 * d_ff;
  hipLaunchKernelGGL(amax_to_scale_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0, s,
                     scales, n);
  return check_launch("hmoe_pack_fp8_gate_up");
}

extern "C" int hmoe_pack_fp8_down(const void* w_down, int w_dtype, int n_experts, int d_ff,
                                  int d_model, uint8_t* packed, float* scales,
                                  hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(n_experts >= 1 && d_model >= 1 && d_ff >= 1, "pack_fp8_down: sizes must be >= 1");
  HMOE_REQUIRE(w_dtype == HMOE_F32 || w_dtype == HMOE_BF16, "pack_fp8_down: dtype must be F32 or BF16");
  HMOE_REQUIRE(w_down && packed && scales, "pack_fp8_down: null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 cgrid(static_cast<unsigned>(ceil_div(d_model, 64)), static_cast<unsigned>(n_experts));
  const dim3 tgrid(static_cast<unsigned>(ceil_div(d_model, 64)), static_cast<unsigned>(ceil_div(d_ff, 64)),
                   static_cast<unsigned>(n_experts));
  if (w_dtype == HMOE_F32) {
    const float* w = static_cast<const float*>(w_down);
    hipLaunchKernelGGL((colmax_kernel<float, false>), cgrid, dim3(256), 0, s, w, d_ff, d_model, 0, scales, d_model);
    hipLaunchKernelGGL((pack_fp8_kernel<float, false>), tgrid, dim3(256), 0, s, w, static_cast<const float*>(nullptr), d_ff, d_model, scales, packed);
  } else {
    const uint16_t* w = static_cast<const uint16_t*>(w_down);
    hipLaunchKernelGGL((colmax_kernel<uint16_t, false>), cgrid, dim3(256), 0, s, w, d_ff, d_model, 0, scales, d_model);
    hipLaunchKernelGGL((pack_fp8_kernel<uint16_t, false>), tgrid, dim3(256), 0, s, w, static_cast<const uint16_t*>(nullptr), d_ff, d_model, scales, packed);
  }
  const int64_t n = static_cast<int64_t>(n_experts) * d_model;
  hipLaunchKernelGGL(amax_to_scale_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0, s,
                     scales, n);
  return check_launch("hmoe_pack_fp8_down");
}

extern "C" size_t hmoe_packed_gate_up_bytes(int n_experts, int d_model, int d_ff) {
  if (n_experts <= 0 || d_model <= 0 || d_ff <= 0) return 0;
  return static_cast<size_t>(n_experts) * 2 * d_ff * d_model * sizeof(uint16_t);
}

extern "C" size_t hmoe_packed_down_bytes(int n_experts, int d_ff, int d_model) {
  if (n_experts <= 0 || d_model <= 0 || d_ff <= 0) return 0;
  return static_cast<size_t>(n_experts) * d_ff * d_model * sizeof(uint16_t);
}

extern "C" int hmoe_pack_gate_up(const void* w_gate, const void* w_up, int w_dtype,
                                 int n_experts, int d_model, int d_ff, void* packed,
                                 hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(n_experts >= 1 && d_model >= 1 && d_ff >= 1, "pack_gate_up: sizes must be >= 1");
  HMOE_REQUIRE(d_ff % 32 == 0, "pack_gate_up: d_ff must be a multiple of 32 (got %d)", d_ff);
  HMOE_REQUIRE(w_dtype == HMOE_F32 || w_dtype == HMOE_BF16, "pack_gate_up: dtype must be F32 or BF16");
  HMOE_REQUIRE(w_gate && w_up && packed, "pack_gate_up: null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(ceil_div(2 * d_ff, 64)), static_cast<unsigned>(ceil_div(d_model, 64)),
                  static_cast<unsigned>(n_experts));
  if (w_dtype == HMOE_F32)
    hipLaunchKernelGGL((pack_transpose_kernel<float, true>), grid, dim3(256), 0, s,
                       static_cast<const float*>(w_gate), static_cast<const float*>(w_up), d_model,
                       d_ff, static_cast<uint16_t*>(packed));
  else
    hipLaunchKernelGGL((pack_transpose_kernel<uint16_t, true>), grid, dim3(256), 0, s,
                       static_cast<const uint16_t*>(w_gate), static_cast<const uint16_t*>(w_up),
                       d_model, d_ff, static_cast<uint16_t*>(packed));
  return check_launch("hmoe_pack_gate_up");
}

extern "C" int hmoe_pack_down(const void* w_down, int w_dtype, int n_experts, int d_ff,
                              int d_model, void* packed, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(n_experts >= 1 && d_model >= 1 && d_ff >= 1, "pack_down: sizes must be >= 1");
  HMOE_REQUIRE(w_dtype == HMOE_F32 || w_dtype == HMOE_BF16, "pack_down: dtype must be F32 or BF16");
  HMOE_REQUIRE(w_down && packed, "pack_down: null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(ceil_div(d_model, 64)), static_cast<unsigned>(ceil_div(d_ff, 64)),
                  static_cast<unsigned>(n_experts));
  if (w_dtype == HMOE_F32)
    hipLaunchKernelGGL((pack_transpose_kernel<float, false>), grid, dim3(256), 0, s,
                       static_cast<const float*>(w_down), static_cast<const float*>(nullptr), d_ff,
                       d_model, static_cast<uint16_t*>(packed));
  else
    hipLaunchKernelGGL((pack_transpose_kernel<uint16_t, false>), grid, dim3(256), 0, s,
                       static_cast<const uint16_t*>(w_down), static_cast<const uint16_t*>(nullptr),
                       d_ff, d_model, static_cast<uint16_t*>(packed));
  return check_launch("hmoe_pack_down");
}

// ---- backward operands --------------------------------------------------------

extern "C" int hmoe_pack_down_dgrad(const void* w_down, int w_dtype, int n_experts, int d_ff,
                                    int d_model, void* packed, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(n_experts >= 1 && d_model >= 1 && d_ff >= 1, "pack_down_dgrad: sizes must be >= 1");
  HMOE_REQUIRE(d_model % 8 == 0, "pack_down_dgrad: d_model must be a multiple of 8 (got %d)", d_model);
  HMOE_REQUIRE(w_dtype == HMOE_F32 || w_dtype == HMOE_BF16, "pack_down_dgrad: dtype must be F32 or BF16");
  HMOE_REQUIRE(w_down && packed, "pack_down_dgrad: null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t rows = static_cast<int64_t>(n_experts) * d_ff;
  const dim3 grid(static_cast<unsigned>(std::min<int64_t>(ceil_div(rows * (d_model / 8), 256), 65536)));
  if (w_dtype == HMOE_F32)
    hipLaunchKernelGGL((pack_rows_kernel<float, false>), grid, dim3(256), 0, s,
                       static_cast<const float*>(w_down), static_cast<const float*>(nullptr), rows,
                       d_model, static_cast<uint16_t*>(packed));
  else
    hipLaunchKernelGGL((pack_rows_kernel<uint16_t, false>), grid, dim3(256), 0, s,
                       static_cast<const uint16_t*>(w_down), static_cast<const uint16_t*>(nullptr),
                       rows, d_model, static_cast<uint16_t*>(packed));
  return check_launch("hmoe_pack_down_dgrad");
}

extern "C" int hmoe_pack_gate_up_dgrad(const void* w_gate, const void* w_up, int w_dtype,
                                       int n_experts, int d_model, int d_ff, void* packed,
                                       hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(n_experts >= 1 && d_model >= 1 && d_ff >= 1, "pack_gate_up_dgrad: sizes must be >= 1");
  HMOE_REQUIRE(d_ff % 32 == 0, "pack_gate_up_dgrad: d_ff must be a multiple of 32 (got %d)", d_ff);
  HMOE_REQUIRE(w_dtype == HMOE_F32 || w_dtype == HMOE_BF16,
               "pack_gate_up_dgrad: dtype must be F32 or BF16");
  HMOE_REQUIRE(w_gate && w_up && packed, "pack_gate_up_dgrad: null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t rows = static_cast<int64_t>(n_experts) * d_model;
  const dim3 grid(static_cast<unsigned>(std::min<int64_t>(ceil_div(rows * (2 * d_ff / 8), 256), 65536)));
  if (w_dtype == HMOE_F32)
    hipLaunchKernelGGL((pack_rows_kernel<float, true>), grid, dim3(256), 0, s,
                       static_cast<const float*>(w_gate), static_cast<const float*>(w_up), rows,
                       d_ff, static_cast<uint16_t*>(packed));
  else
    hipLaunchKernelGGL((pack_rows_kernel<uint16_t, true>), grid, dim3(256), 0, s,
                       static_cast<const uint16_t*>(w_gate), static_cast<const uint16_t*>(w_up), rows,
                       d_ff, static_cast<uint16_t*>(packed));
  return check_launch("hmoe_pack_gate_up_dgrad");
}
