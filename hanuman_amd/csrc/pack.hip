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
    if (p < dst_rows && r < rows_r)
      dst[(static_cast<int64_t>(e) * dst_rows + p) * rows_r + r] = f32_to_bf16_bits(tile[tx][pp]);
  }
}

}  // namespace
}  // namespace hmoe

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
