// Ragged grouped GEMM on gfx950 MFMA (model/moe.py:67-74: the three
// `jax.lax.ragged_dot` calls and the SwiGLU between them).
//
//   C[r, n] = sum_k A[r, k] * B_e[n, k]     for rows r of expert e's segment
//
// A is the dispatched activation buffer (rows grouped by expert, K contiguous)
// or, for the gathered gate/up GEMM, the token matrix x read through the
// dispatch plan's perm_src (row r = x[perm_src[r] / K]); B_e is the packed
// expert weight (one row per output column, K contiguous).  With SWIGLU the
// packed columns alternate 32 gate / 32 up columns of the same h columns and
// the epilogue writes h = bf16(silu(gate) * up).
//
// Persistent kernels: one workgroup per CU loops over 256 x 256 output
// tiles.  Tiles are numbered expert by expert (ceil(rows_e / 256) m-tiles
// each, n fastest); every workgroup computes the numbering from `offsets`,
// so the launch never depends on the routing.  The tile range is split
// evenly over the 8 XCDs (workgroup i runs on XCD i % 8) and the workgroups
// of an XCD stride through their range together, so at any moment an XCD
// works on a few consecutive m-tiles of one expert and shares their A rows
// and B columns in its L2.  The load side runs on into the next tile, so the
// pipeline does not drain between tiles.
//   * bf16 (grouped_gemm_regs, 4 waves, each a 128 x 128 quarter of the
//     tile): a K step is 64 values = 128 bytes of every A and B row, 4 x 16
//     v_mfma_f32_32x32x16_bf16 per wave from the current LDS stage; two
//     stages alternate.  An LDS row holds 128 bytes as eight 16-byte chunks;
//     chunk c of row r is stored at position c ^ lds_swz(r) (conflict-free
//     fragment reads over the 64 LDS banks).  Global loads run two K steps
//     ahead into two register slots (2 x 64 KB per workgroup in flight) and
//     each slot is written into the other stage during the step before it is
//     used; the loads, LDS writes and fragment reads of each sub-step are
//     interleaved between its MFMAs, and a step ends with one barrier that
//     never waits for global memory.
//   * e4m3 (grouped_gemm_w8_fp8, 8 waves = 2 per SIMD, each a 128 x 64 block):
//     a K step is 64 values = 64 bytes per row, one 32x32x64 fp8 MFMA per
//     fragment pair; the tiles go straight from global memory into a ring of
//     four LDS stages (buffer_load ... lds, three steps ahead), because the
//     32-byte fp8 fragments leave no registers for load staging.
#include <atomic>

#include "hmoe_common.h"

namespace hmoe {
namespace {


constexpr int kBM = HMOE_GEMM_TILE_M;
constexpr int kBN = 256;
constexpr int kBK = 64;
constexpr int kThreads = 256;
constexpr int kStageBytes = 65536;  // A 32 KB | B 32 KB
constexpr int kMaxExperts = 1024;
constexpr int kNumXcd = 8;
// Word 3 of a raw buffer resource on gfx9 (32-bit data format, no swizzle).
constexpr int kBufferWord3 = 0x00020000;

static_assert(kBM == 256, "tile loaders assume 256-row tiles");

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2_rne(float lo, float hi) {
  f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// silu(g) = g / (1 + e^-g) with the hardware reciprocal (v_rcp_f32, 1 ulp)
// in place of the correctly rounded division sequence; the result is
// rounded to bf16 right after.
__device__ __forceinline__ float silu_f32(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

// h = bf16(silu(g) * u) at moe.py:70-72's rounding points: g and u are the
// bf16 outputs of the two ragged_dot calls (their dtype is the input dtype),
// so both are rounded to bf16 first; silu and the product run in float32
// and h is rounded once more by the caller.  The backward's recompute rounds
// at the same points, so its VJP is the VJP of this forward.
__device__ __forceinline__ float swiglu_bf16_points(float g, float u) {
  const uint32_t gu = pack_bf16x2_rne(g, u);
  return silu_f32(__uint_as_float(gu << 16)) * __uint_as_float(gu & 0xffff0000u);
}

// Byte offset of gathered token row tk: tk * row_bytes + add, as a 24-bit
// multiply-add (the hosts bound tk * row_bytes below 2^31 and row_bytes below
// 2^23).  Written as a plain 32-bit expression it compiled to a 64-bit
// multiply-add whose unused high addend half the register allocator placed on
// the destination of a gather-source load still in flight; the wait-count
// pass then waited for that load, which (loads complete in order) drained
// every operand load of the pipeline at each tile switch.
__device__ __forceinline__ uint32_t gather_offset(int tk, int row_bytes, int add) {
  return __umul24(static_cast<uint32_t>(tk), static_cast<uint32_t>(row_bytes)) +
         static_cast<uint32_t>(add);
}

// Exclusive scan of per-expert m-tile counts into tstart[0..n_experts];
// returns the total.  NT threads, each taking kMaxExperts / NT experts.
template <int NT = kThreads>
__device__ __forceinline__ int scan_tiles(const int32_t* __restrict__ offsets, int n_experts,
                                          int32_t* tstart, int32_t* scan_tmp) {
  constexpr int kPer = kMaxExperts / NT;
  const int tid = threadIdx.x;
  int local[kPer];
  int sum = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = tid * kPer + j;
    int tiles = 0;
    if (e < n_experts) tiles = (offsets[e + 1] - offsets[e] + kBM - 1) / kBM;
    local[j] = tiles;
    sum += tiles;
  }
  scan_tmp[tid] = sum;
  __syncthreads();
  for (int off = 1; off < NT; off <<= 1) {
    const int v = tid >= off ? scan_tmp[tid - off] : 0;
    __syncthreads();
    scan_tmp[tid] += v;
    __syncthreads();
  }
  int run = scan_tmp[tid] - sum;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = tid * kPer + j;
    if (e < n_experts) tstart[e] = run;
    run += local[j];
  }
  if (tid == NT - 1) tstart[n_experts] = scan_tmp[NT - 1];
  __syncthreads();
  return tstart[n_experts];
}

// Expert, first row, segment end and first column of logical tile t.
__device__ __forceinline__ void decode_tile(int t, int n_tiles_n, const int32_t* tstart,
                                            const int32_t* __restrict__ offsets, int n_experts,
                                            int& e, int64_t& row0, int64_t& row_end, int& n0) {
  const int m_tile = t / n_tiles_n;
  const int n_tile = t - m_tile * n_tiles_n;
  int lo = 0, hi = n_experts;  // largest e with tstart[e] <= m_tile (it has >= 1 tile)
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (tstart[mid] <= m_tile) lo = mid; else hi = mid;
  }
  e = lo;
  row0 = offsets[e] + static_cast<int64_t>(m_tile - tstart[e]) * kBM;
  row_end = offsets[e + 1];
  n0 = n_tile * kBN;
}

// Tile order of the persistent grouped GEMMs: an expert's tiles are taken in
// groups of G row tiles, each group swept column tile by column tile (row
// tile fastest), so that the ~32 consecutive tiles one XCD's workgroups hold
// at a time share G A row-blocks and 32 / G B column-blocks instead of 2
// row-blocks and every column block: less traffic past the XCD's L2.  The
// set of tiles and their results are those of decode_tile.  Measured (one
// process, A/B over G = 1, 2, 4, 8): the bf16 kernels are best at 4 (down
// 553 us against 562-567 at 8), the e4m3 ones at 8 (down 333-335 against
// 342 at 4; gate/up 557-560 at 4 and 8, 590-597 at 1).
constexpr int kTileGroupBf16 = 4;
constexpr int kTileGroupFp8 = 8;

template <int G>
__device__ __forceinline__ void decode_tile_grouped(int t, int n_tiles_n, const int32_t* tstart,
                                                    const int32_t* __restrict__ offsets,
                                                    int n_experts, int& e, int64_t& row0,
                                                    int64_t& row_end, int& n0) {
  const int m_any = t / n_tiles_n;  // some row tile of t's expert
  int lo = 0, hi = n_experts;       // largest e with tstart[e] <= m_any (it has >= 1 tile)
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (tstart[mid] <= m_any) lo = mid; else hi = mid;
  }
  e = lo;
  const int u = t - tstart[e] * n_tiles_n;  // tile within the expert
  const int me = tstart[e + 1] - tstart[e];
  const int g = u / (G * n_tiles_n);
  const int gm = me - g * G < G ? me - g * G : G;
  const int v = u - g * G * n_tiles_n;
  const int n_tile = v / gm;
  row0 = offsets[e] + static_cast<int64_t>(g * G + (v - n_tile * gm)) * kBM;
  row_end = offsets[e + 1];
  n0 = n_tile * kBN;
}

// Position of the 16-byte chunks of LDS row r: chunk c sits at c ^ lds_swz(r).
// A fragment read has lanes 0..31 on 32 consecutive rows (128 bytes apart)
// at the same chunk; the LDS serves 16 lanes of a 16-byte read per pass from
// 64 four-byte banks, i.e. one 256-byte span, which rows r and r + 1 already
// fill.  So the eight rows of one parity among 16 consecutive rows must take
// eight different positions: r & 7 alone repeats every 8 rows (rows r and
// r + 8 would collide); flipping the low bit with bit 3 separates them.
// Rows of one 8-row group still take eight different positions, so reads in
// passes of 8 lanes over 32 banks stay conflict-free as well.
__device__ __forceinline__ int lds_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

typedef int i32x8 __attribute__((ext_vector_type(8)));

// Element-type traits: bf16 (32x32x16 MFMA, 64 elements = 128 bytes per LDS
// row per K step, 4 sub-steps) or OCP e4m3 (32x32x64 MFMA at unit block
// scales; its fragments are read by grouped_gemm_w8_fp8 itself).
template <bool FP8>
struct GemmElem;
template <>
struct GemmElem<false> {
  static constexpr int kBytes = 2;
  static constexpr int kSub = 4;
  typedef bf16x8 frag_t;
  // Lane L, sub-step s: row L&31, 16-byte chunk 2s + L/32.
  __device__ static frag_t read(const uint8_t* base, int row_byte, int row, int s, int half) {
    return *reinterpret_cast<const bf16x8*>(base + row_byte + (((2 * s + half) ^ lds_swz(row)) * 16));
  }
  __device__ static f32x16 mfma(const frag_t& b, const frag_t& a, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, a, c, 0, 0, 0);
  }
};
template <>
struct GemmElem<true> {
  typedef i32x8 frag_t;
  __device__ static f32x16 mfma(const frag_t& b, const frag_t& a, const f32x16& c) {
    // Format 0 = e4m3 for both operands; E8M0 block scales 127 = 1.0.
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, a, c, 0, 0, 0, 127, 0, 127);
  }
};

// Workgroup barrier that waits for this wave's LDS operations only.  Global
// loads in flight stay in flight: their results land in registers, and the
// compiler waits for each one before its register is read.
__device__ __forceinline__ void barrier_lds() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left at their maximum
  __builtin_amdgcn_s_barrier();
}

// Epilogues of the register-staged kernel, both through the idle 64 KB LDS
// stage: the waves write their bf16 results to LDS, then every thread stores
// whole 16-byte chunks, so that each store instruction writes complete row
// segments.  The stores are raw-buffer stores whose range ends at the expert
// segment's last row: rows past it are dropped by the hardware range check
// rather than by a branch.  The barriers wait for LDS operations only: the
// stores stay in flight while the next tile starts.

// Without SwiGLU (the down GEMM): 512-byte rows, so the 256 x 256 tile goes in
// two passes of 128 rows (rows i = 2q, 2q+1 of every wave in pass q).
__device__ __forceinline__ void store_tile_lds(const f32x16 (&acc)[4][4], uint8_t* lds,
                                               uint16_t* __restrict__ C, int64_t ldc, int64_t row0,
                                               int64_t row_end, int n0, int wm, int wn, int lane,
                                               int tid) {
  const int frow = lane & 31;
  const int half = lane >> 5;
  const int64_t nrows = row_end - row0 < kBM ? row_end - row0 : kBM;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      C + row0 * ldc, 0, static_cast<int>(nrows * ldc * 2), kBufferWord3);
  const int row_bytes = static_cast<int>(ldc * 2);
  // LDS row l (0..127) of pass q holds tile row (l >> 6) * 128 + q * 64 + (l & 63):
  // 32 chunks of 8 values; chunk c of row l at position c ^ (l & 31).
  const int c = tid & 31;
  const int voff = ((tid >> 5) * static_cast<int>(ldc) + n0 + c * 8) * 2;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      const int i = 2 * q + ii;
      const int l = wm * 64 + ii * 32 + frow;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = acc[i][j][g * 4 + r];
          uint2 pk;
          pk.x = pack_bf16x2_rne(v[0], v[1]);
          pk.y = pack_bf16x2_rne(v[2], v[3]);
          const int cc = wn * 16 + j * 4 + g;
          *reinterpret_cast<uint2*>(lds + l * 512 + ((cc ^ (l & 31)) * 16) + half * 8) = pk;
        }
      __builtin_amdgcn_sched_barrier(0);
    }
    barrier_lds();
    // Thread tid: chunk tid & 31 of LDS rows (tid >> 5) + 8 m.
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const int l = m * 8 + (tid >> 5);
      const u32x4 v = *reinterpret_cast<const u32x4*>(lds + l * 512 + ((c ^ (l & 31)) * 16));
      const int trow0 = (m >> 3) * 128 + q * 64 + (m & 7) * 8;  // tile row of l, less tid >> 5
      __builtin_amdgcn_raw_buffer_store_b128(v, rsrc, voff, __builtin_amdgcn_readfirstlane(trow0 * row_bytes), 0);
    }
    barrier_lds();
  }
}

// With SwiGLU (the gate/up GEMM): h = bf16(silu(g) * u) from the interleaved
// gate/up column blocks is half the tile's columns, 256-byte rows, so the
// whole tile fits the stage in one pass.  LDS row l = tile row l, 16 chunks of
// 8 h values; chunk c of row l at position c ^ (l & 15).
__device__ __forceinline__ void store_tile_lds_swiglu(const f32x16 (&acc)[4][4], uint8_t* lds,
                                                      uint16_t* __restrict__ C, int64_t ldc,
                                                      int64_t row0, int64_t row_end, int n0, int wm,
                                                      int wn, int lane, int tid) {
  const int frow = lane & 31;
  const int half = lane >> 5;
  const int64_t nrows = row_end - row0 < kBM ? row_end - row0 : kBM;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      C + row0 * ldc, 0, static_cast<int>(nrows * ldc * 2), kBufferWord3);
  const int row_bytes = static_cast<int>(ldc * 2);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int l = wm * 128 + i * 32 + frow;
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float h[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          h[q] = swiglu_bf16_points(acc[i][2 * p][g * 4 + q], acc[i][2 * p + 1][g * 4 + q]);
        uint2 pk;
        pk.x = pack_bf16x2_rne(h[0], h[1]);
        pk.y = pack_bf16x2_rne(h[2], h[3]);
        const int cc = wn * 8 + p * 4 + g;
        *reinterpret_cast<uint2*>(lds + l * 256 + ((cc ^ (l & 15)) * 16) + half * 8) = pk;
      }
    __builtin_amdgcn_sched_barrier(0);
  }
  barrier_lds();
  // Thread tid: chunk tid & 15 of LDS rows (tid >> 4) + 16 m.
  const int c = tid & 15;
  const int voff = ((tid >> 4) * static_cast<int>(ldc) + n0 / 2 + c * 8) * 2;
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    const int l = m * 16 + (tid >> 4);
    const u32x4 v = *reinterpret_cast<const u32x4*>(lds + l * 256 + ((c ^ (l & 15)) * 16));
    __builtin_amdgcn_raw_buffer_store_b128(v, rsrc, voff, m * 16 * row_bytes, 0);
  }
  barrier_lds();
}

// The recompute of the backward with the SwiGLU VJP fused (C = dgu, ldc = 2F):
// the accumulators are g and u, rounded to bf16 as the forward's outputs are,
// the tile's dh [256 rows][128 h columns] comes from global memory straight
// into registers (each lane the 4 h columns of its accumulator groups, 8-byte
// range-checked buffer loads issued before any arithmetic; rows past the
// segment read zeros), and dg, du (swiglu_vjp) go out in g and u's places
// through the same two 128-row LDS passes as store_tile_lds.
__device__ __forceinline__ void store_tile_lds_dswiglu(const f32x16 (&acc)[4][4], uint8_t* lds,
                                                       uint16_t* __restrict__ C, int64_t ldc,
                                                       const uint16_t* __restrict__ dh,
                                                       int64_t row0, int64_t row_end, int n0,
                                                       int wm, int wn, int lane, int tid) {
  const int frow = lane & 31;
  const int half = lane >> 5;
  const int64_t nrows = row_end - row0 < kBM ? row_end - row0 : kBM;
  const int f = static_cast<int>(ldc / 2);
  const __amdgpu_buffer_rsrc_t dh_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(dh + row0 * f), 0, static_cast<int>(nrows * f * 2), kBufferWord3);
  const int hc = (n0 + wn * 128) / 2 + half * 4;
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  // dh of pass q's accumulator rows (i = 2q, 2q+1); pass 1's loads go out
  // right after pass 0's LDS writes, so they fly while pass 0 is stored.
  u32x2_t dv[2][2][4];
  auto load_dh = [&](int q) __attribute__((always_inline)) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii)
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          dv[ii][p][g] = __builtin_bit_cast(
              u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(
                           dh_rsrc, ((wm * 128 + (2 * q + ii) * 32 + frow) * f + hc + p * 32 + g * 8) * 2,
                           0, 0));
  };
  load_dh(0);
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      C + row0 * ldc, 0, static_cast<int>(nrows * ldc * 2), kBufferWord3);
  const int row_bytes = static_cast<int>(ldc * 2);
  const int c = tid & 31;
  const int voff = ((tid >> 5) * static_cast<int>(ldc) + n0 + c * 8) * 2;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      const int i = 2 * q + ii;
      const int l = wm * 64 + ii * 32 + frow;
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float dg[4], du[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint32_t w = dv[ii][p][g][r >> 1];
            const float d = __uint_as_float((r & 1) ? (w & 0xffff0000u) : (w << 16));
            const uint32_t gu = pack_bf16x2_rne(acc[i][2 * p][g * 4 + r], acc[i][2 * p + 1][g * 4 + r]);
            swiglu_vjp(d, __uint_as_float(gu << 16), __uint_as_float(gu & 0xffff0000u), dg[r], du[r]);
          }
          uint2 pg, pu;
          pg.x = pack_bf16x2_rne(dg[0], dg[1]);
          pg.y = pack_bf16x2_rne(dg[2], dg[3]);
          pu.x = pack_bf16x2_rne(du[0], du[1]);
          pu.y = pack_bf16x2_rne(du[2], du[3]);
          const int cg = wn * 16 + 2 * p * 4 + g;
          const int cu = cg + 4;
          *reinterpret_cast<uint2*>(lds + l * 512 + ((cg ^ (l & 31)) * 16) + half * 8) = pg;
          *reinterpret_cast<uint2*>(lds + l * 512 + ((cu ^ (l & 31)) * 16) + half * 8) = pu;
        }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (q == 0) load_dh(1);
    barrier_lds();
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const int l = m * 8 + (tid >> 5);
      const u32x4 v = *reinterpret_cast<const u32x4*>(lds + l * 512 + ((c ^ (l & 31)) * 16));
      const int trow0 = (m >> 3) * 128 + q * 64 + (m & 7) * 8;
      __builtin_amdgcn_raw_buffer_store_b128(v, rsrc, voff, __builtin_amdgcn_readfirstlane(trow0 * row_bytes), 0);
    }
    barrier_lds();
  }
}

template <int V>
struct IntC {
  static constexpr int value = V;
};

// ---- eight-wave e4m3 kernel ------------------------------------------------------
// The e4m3 grouped GEMM with two waves per SIMD.  One workgroup of 8 waves
// per CU loops over 256 x 256 tiles as grouped_gemm_regs does, each wave
// owning a 128 x 64 block (4 x 2 fragments, 128 accumulator registers), so
// that while one wave of a SIMD waits on LDS or a barrier the other keeps the
// matrix core busy: with one wave per SIMD a CU draws ~67 B/clk of fragments
// from LDS, with two ~170 B/clk, and the 256 x 256 tile's MFMAs need ~100.
// A K step is 64 bytes of every A and B row (64 e4m3 values: one
// v_mfma_scale_f32_32x32x64_f8f6f4 per fragment pair).  Four LDS stages of
// 32 KB hold steps g .. g+3; the tiles go straight from global memory into
// the stage of step g + 3 (buffer_load ... lds), the fragments of step g + 1
// are read during step g (its stage completed at the previous barrier), and
// the step ends with one barrier after which step g + 2 is complete.  The
// tile's 256 row and 256 column scales are staged in LDS for the epilogue,
// which dequantises (acc * s_row * s_col) and stores straight from the
// accumulators.  GATHER: A is the per-token e4m3 matrix of x and row r of
// the dispatched operand is its token perm_src[r] / top_k, whose scale is
// the row scale (rows without a source read token 0).
constexpr int kW8Threads = 512;
constexpr int kW8StepBytes = 64;
constexpr int kW8Stages = 4;
constexpr int kW8StageBytes = 2 * kBM * kW8StepBytes;  // A 16 KB | B 16 KB
constexpr int kW8Lds = kW8Stages * kW8StageBytes;       // 128 KB
constexpr int kW8MxLds = kW8Lds + 2 * 2048;              // + exponents of A
static_assert(kW8Lds <= 2 * kStageBytes, "allow_dynamic_lds grants 2 * kStageBytes");

// 64-byte LDS rows: chunk c of row r sits at c ^ swz64(r), so the 16 lanes
// of a fragment read served together (rows r .. r + 15) cover the 16
// different 16-byte bank groups of the 256-byte bank space.
__device__ __forceinline__ int swz64(int r) { return (r >> 2) & 3; }

// s_waitcnt vmcnt(N) lgkmcnt(0), expcnt left alone (gfx9 encoding: vmcnt bits
// 0..3 and 14..15).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit count");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0070);
}

template <bool SWIGLU, bool GATHER, bool MX = false>
__global__ __launch_bounds__(kW8Threads) void grouped_gemm_w8_fp8(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ B,
    const float* __restrict__ a_scale, const float* __restrict__ b_scale,
    const int32_t* __restrict__ offsets, int n_experts, int64_t a_rows, int kdim, int ncols,
    uint16_t* __restrict__ C, int64_t ldc, int n_tiles_n, const int32_t* __restrict__ gather_src,
    int gather_k, int gather_rows, uint8_t* __restrict__ mx_exp) {
  // MX with SWIGLU: h leaves as block-scaled e4m3 (codes into C, ldc bytes a
  // row; biased exponents into mx_exp, ldc / 32 bytes a row).  MX without
  // SWIGLU: A is block-scaled (a_scale unused; A's exponents in mx_exp,
  // kdim / 32 bytes a row) and the MFMA applies them.
  constexpr bool kQuantH = MX && SWIGLU;
  constexpr bool kScaledA = MX && !SWIGLU;
  static_assert(!(kScaledA && GATHER), "the block-scaled A operand is not gathered");
  typedef GemmElem<true> E;
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int32_t tstart[kMaxExperts + 1];
  __shared__ int32_t scan_tmp[kW8Threads];
  __shared__ __attribute__((aligned(16))) float sscale[2 * kBM];  // rows | columns

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  const int total = __builtin_amdgcn_readfirstlane(
      scan_tiles<kW8Threads>(offsets, n_experts, tstart, scan_tmp) * n_tiles_n);
  const int xcd = blockIdx.x % kNumXcd;
  const int per_xcd = gridDim.x / kNumXcd;
  const int slot = blockIdx.x / kNumXcd;
  const int lo = static_cast<int>((static_cast<int64_t>(total) * xcd) / kNumXcd);
  const int hi = static_cast<int>((static_cast<int64_t>(total) * (xcd + 1)) / kNumXcd);
  const int first = lo + slot;
  if (first >= hi) return;  // uniform per workgroup
  const int row_bytes = kdim;  // one byte per value
  const int ks = row_bytes / kW8StepBytes;  // even: kdim % 128 == 0
  const int n_my = (hi - first + per_xcd - 1) / per_xcd;
  const int iters = n_my * ks;

  // ---- global -> LDS (DMA) ---------------------------------------------------
  // Instruction j (0, 1) of wave w fills rows 32 w + 16 j + lane / 4 of the A
  // and of the B stage (1 KB of contiguous LDS each); lane position lane & 3
  // receives chunk (lane & 3) ^ swz64(row) = (lane & 3) ^ ((lane >> 4) & 3).
  const int dma_row = wave * 32 + (lane >> 2);  // + 16 j
  const int dma_byte = ((lane & 3) ^ ((lane >> 4) & 3)) * 16;
  const int tile_bytes = kBM * row_bytes;
  __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(A), 0, GATHER ? gather_rows * row_bytes : tile_bytes, kBufferWord3);
  __amdgpu_buffer_rsrc_t b_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(B), 0, tile_bytes, kBufferWord3);
  const uint32_t b_voff0 = static_cast<uint32_t>(dma_row * row_bytes + dma_byte);
  uint32_t a_voff[2];
  const int ex_row_bytes = kdim / 32;  // kScaledA: exponent bytes per row of A
  __amdgpu_buffer_rsrc_t e_rsrc = b_rsrc;
  uint32_t e_voff = 0;
  int ld_kb = 0, ld_g = 0, ld_t = first;
  int32_t pf_src[2];  // GATHER: sources of this lane's rows in the next tile
  auto fetch_src = [&](int t) __attribute__((always_inline)) {
    int e, n0;
    int64_t row0, row_end;
    decode_tile_grouped<kTileGroupFp8>(t, n_tiles_n, tstart, offsets, n_experts, e, row0, row_end, n0);
    const int r0 = __builtin_amdgcn_readfirstlane(static_cast<int>(row0));
    const int64_t lim = row_end - 1 - r0;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      int rr = dma_row + 16 * j;
      rr = rr < lim ? rr : static_cast<int>(lim);
      pf_src[j] = gather_src[r0 + rr];
    }
  };
  auto set_load_tile = [&](int t) __attribute__((always_inline)) {
    int e, n0;
    int64_t row0, row_end;
    decode_tile_grouped<kTileGroupFp8>(t, n_tiles_n, tstart, offsets, n_experts, e, row0, row_end, n0);
    e = __builtin_amdgcn_readfirstlane(e);
    n0 = __builtin_amdgcn_readfirstlane(n0);
    const int r0 = __builtin_amdgcn_readfirstlane(static_cast<int>(row0));
    b_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(B + (static_cast<int64_t>(e) * ncols + n0) * row_bytes), 0,
        tile_bytes, kBufferWord3);
    if (GATHER) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        int tk = pf_src[j] >= 0 ? pf_src[j] / gather_k : 0;
        tk = tk < gather_rows ? tk : gather_rows - 1;
        a_voff[j] = gather_offset(tk, row_bytes, dma_byte);
      }
      if (t + per_xcd < hi) fetch_src(t + per_xcd);
    } else {
      // rows past the segment repeat its last row; their results are never stored
      a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint8_t*>(A + static_cast<int64_t>(r0) * row_bytes), 0, tile_bytes,
          kBufferWord3);
      const int64_t lim = row_end - 1 - r0;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        int rr = dma_row + 16 * j;
        rr = rr < lim ? rr : static_cast<int>(lim);
        a_voff[j] = static_cast<uint32_t>(rr * row_bytes + dma_byte);
      }
      if (kScaledA) {
        e_rsrc = __builtin_amdgcn_make_buffer_rsrc(
            mx_exp + static_cast<int64_t>(r0) * ex_row_bytes, 0, kBM * ex_row_bytes, kBufferWord3);
        int rr = wave * 32 + (lane & 31);
        rr = rr < lim ? rr : static_cast<int>(lim);
        e_voff = static_cast<uint32_t>(rr * ex_row_bytes);
      }
    }
  };
  auto issue_dma = [&](int stage, int j) __attribute__((always_inline)) {
    uint8_t* base = smem + stage * kW8StageBytes + (2 * wave + j) * 1024;
    const int koff = ld_kb * kW8StepBytes;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (lds_ptr_t)base, 16, a_voff[j], koff, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(b_rsrc, (lds_ptr_t)(base + kBM * kW8StepBytes), 16,
                                             b_voff0 + static_cast<uint32_t>(16 * j * row_bytes),
                                             koff, 0, 0);
  };
  // kScaledA: A's exponents for two K steps (4 bytes of a row: blocks
  // 2 kb .. 2 kb + 3) go into one of two 2 KB LDS regions past the stages,
  // by one 4-byte DMA per wave issued with the data of an even step: wave w
  // lane L fills bytes 4 L of the wave's 256 (row 32 w + L % 32 of the tile;
  // lanes 32..63 repeat lanes 0..31 into bytes 128..255, which nothing reads).
  // Issued before that step's data DMA, it is covered by the same waits.
  auto issue_exp_dma = [&]() __attribute__((always_inline)) {
    uint8_t* base = smem + kW8Lds + ((ld_g >> 1) & 1) * 2048 + wave * 256;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(e_rsrc, (lds_ptr_t)base, 4, e_voff, ld_kb * 2, 0, 0);
  };
  // Once every step is loaded the load side repeats the last one (into a
  // stage nothing reads), so every step issues the same DMA count.  The load
  // side runs three steps ahead and ks is even, so it crosses into the next
  // tile only in the advance of an even step (and of the prologue's second
  // step): with the tile switch (WRAP) only there, the compiler's wait for
  // the next tile's gather sources no longer lands mid-step on a path with a
  // few DMAs since their issue (it drained the DMA ring once per tile).
  auto advance = [&](auto Wc) __attribute__((always_inline)) {
    if (ld_g + 1 < iters) {
      ++ld_g;
      ++ld_kb;
      if constexpr (decltype(Wc)::value) {
        if (ld_kb == ks) {
          ld_kb = 0;
          ld_t += per_xcd;
          set_load_tile(ld_t);
        }
      }
    }
  };

  // ---- MFMA fragments ------------------------------------------------------
  // Wave w: rows 128 (w & 1) .. +128, columns 64 (w >> 1) .. +64 of the tile.
  // Lane L: row L & 31 of each 32-row fragment; VGPRs 0..3 hold 16-byte
  // chunk L / 32 of the step and VGPRs 4..7 chunk 2 + L / 32.  The MFMA takes
  // VGPR half v of lane group g as K values 32 v + 16 g .. + 16 (measured:
  // with per-block operand scales only this assignment reproduces exact
  // float64 sums), so its 32-value scale block v is bytes 32 v .. + 32 of the
  // step, and lane L's operand scale is that of block L / 32.
  const int wm = wave & 1, wn = wave >> 1;
  const int frow = lane & 31;
  const int fhalf = lane >> 5;
  const int fsw = swz64(frow);
  const int p0 = (fhalf ^ fsw) * 16, p1 = ((2 + fhalf) ^ fsw) * 16;
  const int fa_off = (wm * 128 + frow) * kW8StepBytes;
  const int fb_off = kBM * kW8StepBytes + (wn * 64 + frow) * kW8StepBytes;
  E::frag_t fa[2][4], fb[2][2];
  // kScaledA: fragment i's exponent word (blocks 2 kb .. 2 kb + 3 of row
  // 128 wm + 32 i + L % 32), shifted right by 8 (L / 32) so that byte 0 is
  // the lane's block of the even step and byte 2 that of the odd step.
  uint32_t ex_cur[4], ex_nxt[4];
  auto read_frag = [&](const uint8_t* row) __attribute__((always_inline)) {
    const u32x4 lo4 = *reinterpret_cast<const u32x4*>(row + p0);
    const u32x4 hi4 = *reinterpret_cast<const u32x4*>(row + p1);
    E::frag_t f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f[q] = static_cast<int>(lo4[q]);
      f[4 + q] = static_cast<int>(hi4[q]);
    }
    return f;
  };
  auto read_frags = [&](auto Bc, int stage, int s) __attribute__((always_inline)) {
    constexpr int b = decltype(Bc)::value;
    const uint8_t* base = smem + stage * kW8StageBytes;
    // B's two fragments first: the MFMAs run row fragment by row fragment
    // (i outer), so fragment (i, j) needs B's j early and A's i only from
    // MFMA 2 i on, and the last read issued is needed two MFMAs from the end
    // (measured: gate/up 2.2 % and down 1 % faster than A first; the bf16
    // kernel, four B fragments per sub-step, was 1 % slower with it)
#pragma unroll
    for (int j = 0; j < 2; ++j) fb[b][j] = read_frag(base + fb_off + j * 32 * kW8StepBytes);
#pragma unroll
    for (int i = 0; i < 4; ++i) fa[b][i] = read_frag(base + fa_off + i * 32 * kW8StepBytes);
    if (kScaledA && b == 0) {
      const uint8_t* ex = smem + kW8Lds + ((s >> 1) & 1) * 2048 + wm * 1024 + frow * 4;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        ex_nxt[i] = *reinterpret_cast<const uint32_t*>(ex + i * 256) >> (8 * fhalf);
    }
  };
  f32x16 acc[4][2];

  // Step g on fragment buffer B = g & 1: DMA of step g + 3, fragments of step
  // g + 1 into buffer B ^ 1, the MFMAs of step g, one barrier.
  auto step = [&](auto Bc, int g, auto Wc) __attribute__((always_inline)) {
    constexpr int b = decltype(Bc)::value;
    // odd g: the load side is at an even step (or, done, repeats an odd one)
    if (kScaledA && b == 1 && (ld_kb & 1) == 0) issue_exp_dma();
#pragma unroll
    for (int j = 0; j < 2; ++j) issue_dma((g + 3) & 3, j);
    advance(IntC<b == 0>{});
    read_frags(IntC<b ^ 1>{}, (g + 1) & 3, g + 1);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (kScaledA)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
              fb[b][j], fa[b][i], acc[i][j], 0, 0, 0, 127, 2 * b, static_cast<int>(ex_cur[i]));
        else
          acc[i][j] = E::mfma(fb[b][j], fa[b][i], acc[i][j]);
      }
    // The accumulators are used here, before the step's barrier: otherwise
    // the compiler sinks this step's MFMAs into the next step (past the
    // barrier), and every other step leaves the matrix cores idle.
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) asm volatile("" ::"v"(acc[i][j]));
    // per MFMA: a DMA or fragment reads
    constexpr int kReads = (kScaledA && b == 1) ? 4 : 3;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // DMA
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, kReads, 0);  // LDS read
    }
    __builtin_amdgcn_sched_barrier(0);
    // this wave's DMA of step g + 2 landed (step g + 3's four may still fly);
    // after the barrier every wave's has
    wait_vm_lgkm0<decltype(Wc)::value>();
    __builtin_amdgcn_s_barrier();
  };

  // GATHER: the source of tile row tid (tid < 256) of the current tile,
  // loaded one tile ahead so that the scale lookup never waits on it
  auto row_src = [&](int t) __attribute__((always_inline)) {
    int e, n0;
    int64_t row0, row_end;
    decode_tile_grouped<kTileGroupFp8>(t, n_tiles_n, tstart, offsets, n_experts, e, row0, row_end, n0);
    return gather_src[row0 + tid < row_end ? row0 + tid : row_end - 1];
  };
  // (loaded before the prologue's DMAs, so that its use at the first tile's
  // start finds them between its issue and its use, as at every later tile)
  int32_t my_src = 0;
  if (GATHER && tid < kBM) my_src = row_src(first);
  // Prologue: steps 0, 1, 2 into stages 0, 1, 2; steps 0 and 1 complete.
  if (GATHER) fetch_src(first);
  set_load_tile(first);
  auto prologue_step = [&](int st, auto Wc) __attribute__((always_inline)) {
    if (kScaledA && (ld_kb & 1) == 0) issue_exp_dma();
#pragma unroll
    for (int j = 0; j < 2; ++j) issue_dma(st, j);
    advance(Wc);
  };
  prologue_step(0, IntC<0>{});
  prologue_step(1, IntC<1>{});
  prologue_step(2, IntC<0>{});
  wait_vm_lgkm0<4>();
  __builtin_amdgcn_s_barrier();
  read_frags(IntC<0>{}, 0, 0);


  int g = 0;
  for (int t = first; t < hi; t += per_xcd) {
    int e, n0;
    int64_t row0, row_end;
    decode_tile_grouped<kTileGroupFp8>(t, n_tiles_n, tstart, offsets, n_experts, e, row0, row_end, n0);
    // this thread's row scale (tid < 256) or column scale (tid >= 256) of the
    // tile, loaded now and staged in LDS after the K loop
    float my_scale;
    if (kScaledA && tid < kBM) {
      my_scale = 1.0f;  // the row scales are in the MFMA's block exponents
    } else if (tid < kBM) {
      if (GATHER) {
        int tk = my_src >= 0 ? my_src / gather_k : 0;
        tk = tk < gather_rows ? tk : gather_rows - 1;
        my_scale = a_scale[tk];
        if (t + per_xcd < hi) my_src = row_src(t + per_xcd);
      } else {
        my_scale = a_scale[row0 + tid < row_end ? row0 + tid : row_end - 1];
      }
    } else {
      my_scale = b_scale[static_cast<int64_t>(e) * ncols + n0 + tid - kBM];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    // ks >= 2: a do-while, so that no path skips the K loop between a load
    // issued at the tile's start and its use in the epilogue (the
    // compiler's wait counts then need not drain the DMA ring there)
    int kb = 0;
    do {
      if (kScaledA) {
#pragma unroll
        for (int i = 0; i < 4; ++i) ex_cur[i] = ex_nxt[i];
      }
      step(IntC<0>{}, g, IntC<4>{});
      step(IntC<1>{}, g + 1, IntC<4>{});
      kb += 2;
      g += 2;
    } while (kb < ks);
    // the previous tile's epilogue read sscale before this tile's barriers
    sscale[tid] = my_scale;
    barrier_lds();
    // Epilogue: lane L of acc[i][j] holds tile row 128 wm + 32 i + L % 32 and
    // columns 64 wn + 32 j + 8 q + 4 (L / 32) + 0..3 (q = 0..3).  Each 32-column
    // block is packed to bf16 (d[2q], d[2q + 1] = the 4 values of group q) and
    // lanes L and L + 32 trade groups (v_permlane32_swap: lanes 32..63 of the
    // first operand with lanes 0..31 of the second), after which lane L < 32
    // holds columns 0..7 and 16..23 and lane L + 32 columns 8..15 and 24..31
    // of its row: two 16-byte stores per block, each writing 32 contiguous
    // bytes of every row.
    const int64_t nrows = row_end - row0 < kBM ? row_end - row0 : kBM;
    constexpr int kOutBytes = kQuantH ? 1 : 2;
    const __amdgpu_buffer_rsrc_t c_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<uint8_t*>(C) + row0 * ldc * kOutBytes, 0,
        static_cast<int>(nrows * ldc * kOutBytes), kBufferWord3);
    __amdgpu_buffer_rsrc_t e_out = c_rsrc;
    if (kQuantH)
      e_out = __builtin_amdgcn_make_buffer_rsrc(mx_exp + row0 * (ldc / 32), 0,
                                                static_cast<int>(nrows * (ldc / 32)), kBufferWord3);
    auto store_block = [&](uint32_t (&d)[8], int r, int col) __attribute__((always_inline)) {
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        const auto p01 = __builtin_amdgcn_permlane32_swap(d[w], d[2 + w], false, false);
        d[w] = p01[0];
        d[2 + w] = p01[1];
        const auto p23 = __builtin_amdgcn_permlane32_swap(d[4 + w], d[6 + w], false, false);
        d[4 + w] = p23[0];
        d[6 + w] = p23[1];
      }
      const int off = static_cast<int>((r * ldc + col + fhalf * 8) * 2);
      const u32x4 lo4 = {d[0], d[1], d[2], d[3]};
      const u32x4 hi4 = {d[4], d[5], d[6], d[7]};
      __builtin_amdgcn_raw_buffer_store_b128(lo4, c_rsrc, off, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(hi4, c_rsrc, off + 32, 0, 0);
    };
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = wm * 128 + i * 32 + frow;
      const float sa = sscale[r];
      if (kQuantH) {
        // h of this row's 32 columns n0 / 2 + 32 wn .. + 32 (one scale block):
        // lane L holds columns 8 q + 4 (L / 32) + k.  Block maximum over
        // lanes L and L + 32, exponent e = the smallest with max <= 448 * 2^e
        // (at least -127), codes e4m3(h * 2^-e), an exact scaling.
        float hv[16];
        float amax = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 sg = *reinterpret_cast<const f32x4*>(sscale + kBM + wn * 64 + q * 8 + fhalf * 4);
          const f32x4 su =
              *reinterpret_cast<const f32x4*>(sscale + kBM + wn * 64 + 32 + q * 8 + fhalf * 4);
#pragma unroll
          for (int k = 0; k < 4; k += 2) {
            const uint32_t pk = pack_bf16x2_rne(
                swiglu_bf16_points(acc[i][0][q * 4 + k] * sa * sg[k], acc[i][1][q * 4 + k] * sa * su[k]),
                swiglu_bf16_points(acc[i][0][q * 4 + k + 1] * sa * sg[k + 1],
                                   acc[i][1][q * 4 + k + 1] * sa * su[k + 1]));
            hv[q * 4 + k] = __uint_as_float(pk << 16);
            hv[q * 4 + k + 1] = __uint_as_float(pk & 0xffff0000u);
            amax = fmaxf(amax, fmaxf(fabsf(hv[q * 4 + k]), fabsf(hv[q * 4 + k + 1])));
          }
        }
        const uint32_t abits = __float_as_uint(amax);
        const auto pa = __builtin_amdgcn_permlane32_swap(abits, abits, false, false);
        const uint32_t bmax = __float_as_uint(fmaxf(__uint_as_float(pa[0]), __uint_as_float(pa[1])));
        int ex = static_cast<int>(bmax >> 23) - 135 + ((bmax & 0x7FFFFFu) > 0x600000u ? 1 : 0);
        ex = ex > -127 ? ex : -127;
        const float inv = __uint_as_float(static_cast<uint32_t>(127 - ex) << 23);
        uint32_t d[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float v[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) v[k] = fminf(fmaxf(hv[q * 4 + k] * inv, -448.0f), 448.0f);
          const int w = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], 0, false);
          d[q] = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], w, true));
        }
        // lanes L < 32 take columns 0..15 (their groups 0, 2 and the partner's),
        // lanes L + 32 columns 16..31: one 16-byte store each
        const auto p02 = __builtin_amdgcn_permlane32_swap(d[0], d[2], false, false);
        const auto p13 = __builtin_amdgcn_permlane32_swap(d[1], d[3], false, false);
        const u32x4 codes = {p02[0], p02[1], p13[0], p13[1]};
        const int col = n0 / 2 + wn * 32;
        __builtin_amdgcn_raw_buffer_store_b128(codes, c_rsrc, static_cast<int>(r * ldc + col + 16 * fhalf),
                                               0, 0);
        if (fhalf == 0)
          __builtin_amdgcn_raw_buffer_store_b8(static_cast<uint8_t>(ex + 127), e_out,
                                               static_cast<int>(r * (ldc / 32) + col / 32), 0, 0);
      } else if (SWIGLU) {
        // gate columns in acc[i][0], the up columns of the same h columns in acc[i][1]
        uint32_t d[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 sg = *reinterpret_cast<const f32x4*>(sscale + kBM + wn * 64 + q * 8 + fhalf * 4);
          const f32x4 su =
              *reinterpret_cast<const f32x4*>(sscale + kBM + wn * 64 + 32 + q * 8 + fhalf * 4);
          float h[4];
#pragma unroll
          for (int k = 0; k < 4; ++k)
            h[k] = swiglu_bf16_points(acc[i][0][q * 4 + k] * sa * sg[k],
                                      acc[i][1][q * 4 + k] * sa * su[k]);
          d[2 * q] = pack_bf16x2_rne(h[0], h[1]);
          d[2 * q + 1] = pack_bf16x2_rne(h[2], h[3]);
        }
        store_block(d, r, n0 / 2 + wn * 32);
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          uint32_t d[8];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x4 sb =
                *reinterpret_cast<const f32x4*>(sscale + kBM + wn * 64 + j * 32 + q * 8 + fhalf * 4);
            d[2 * q] = pack_bf16x2_rne(acc[i][j][q * 4] * sa * sb[0], acc[i][j][q * 4 + 1] * sa * sb[1]);
            d[2 * q + 1] =
                pack_bf16x2_rne(acc[i][j][q * 4 + 2] * sa * sb[2], acc[i][j][q * 4 + 3] * sa * sb[3]);
          }
          store_block(d, r, n0 + wn * 64 + j * 32);
        }
      }
    }
  }
  // nothing may still be writing into LDS when the workgroup ends
  __builtin_amdgcn_s_waitcnt(0);
}

// Main loop with register-staged loads (bf16): global loads run two K steps
// ahead of the MFMAs.  ODD: the K dimension has an odd number of 64-element
// steps; every tile then runs one more step whose LDS stage is filled with
// zeros, so tiles always start on an even step and the two register slots
// alternate statically.  GATHER: A is the token matrix x and row r of the
// dispatched operand is x[gather_src[r] / gather_k] (gather_src = perm_src,
// -1 past the kept rows), so the row permutation is done by the GEMM's own
// loads and the dispatched copy of x is never written.  DSWIGLU (backward,
// without SWIGLU): the epilogue is store_tile_lds_dswiglu with dh.
template <bool SWIGLU, bool ODD, bool GATHER, bool DSWIGLU = false>
__global__ __launch_bounds__(kThreads) void grouped_gemm_regs(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ B,
    const int32_t* __restrict__ offsets, int n_experts, int64_t a_rows, int kdim, int ncols,
    uint16_t* __restrict__ C, int64_t ldc, int n_tiles_n,
    const int32_t* __restrict__ gather_src, int gather_k, int gather_rows,
    const uint16_t* __restrict__ dh) {
  static_assert(!(SWIGLU && DSWIGLU), "the SwiGLU VJP epilogue takes the raw g, u tile");
  typedef GemmElem<false> E;
  constexpr int kParts = 4 / E::kSub;  // load parts per MFMA sub-step
  // The two stages live in dynamic LDS: stage g & 1 holds global K step g.
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int32_t tstart[kMaxExperts + 1];
  __shared__ int32_t scan_tmp[kThreads];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  const int total =
      __builtin_amdgcn_readfirstlane(scan_tiles(offsets, n_experts, tstart, scan_tmp) * n_tiles_n);
  const int xcd = blockIdx.x % kNumXcd;
  const int per_xcd = gridDim.x / kNumXcd;
  const int slot = blockIdx.x / kNumXcd;
  const int lo = static_cast<int>((static_cast<int64_t>(total) * xcd) / kNumXcd);
  const int hi = static_cast<int>((static_cast<int64_t>(total) * (xcd + 1)) / kNumXcd);
  const int first = lo + slot;
  if (first >= hi) return;  // uniform per workgroup
  const int row_bytes = kdim * E::kBytes;
  const int ksteps = row_bytes / 128;
  const int kpad = ODD ? ksteps + 1 : ksteps;  // steps per tile, even
  const int n_my = (hi - first + per_xcd - 1) / per_xcd;
  const int iters = n_my * kpad;  // K steps this workgroup runs, over all its tiles

  // ---- global -> registers -> LDS --------------------------------------------
  // Round i (0..7) of a K step: this thread loads 16-byte chunk ld_c of A row
  // and B row i*32 + ld_r (eight threads cover a row's 128 bytes) and stores it
  // at position ld_c ^ lds_swz(row) of the LDS row.  Loads run two K steps ahead
  // of the MFMAs in two register slots; a slot is written to the idle LDS
  // stage one step ahead, so the barrier at the end of a step never waits for
  // global memory.
  const int ld_r = tid >> 3;
  const int ld_c = tid & 7;
  const int st_pos = (ld_c ^ lds_swz(ld_r)) * 16;
  const uint32_t b_off0 = static_cast<uint32_t>(ld_r * row_bytes + ld_c * 16);
  uint32_t a_off[8];
  const uint8_t* a_tile = A;
  // B goes through buffer loads on the tile's 256 weight rows: the per-thread
  // offset b_off0 stays in one VGPR and the step and round offsets are
  // uniform (soffset), so no 64-bit address is formed per load.
  const int b_tile_bytes = 256 * row_bytes;
  __amdgpu_buffer_rsrc_t b_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(B), 0, b_tile_bytes, kBufferWord3);
  int ld_t = first, ld_kb = 0, ld_g = 0;  // load side: tile, K step in it, global step
  // GATHER: perm_src of the 8 rows this thread loads in the next tile the load
  // side enters.
  int32_t pf_src[8];
  auto fetch_src = [&](int t) __attribute__((always_inline)) {
    int e, n0;
    int64_t row0, row_end;
    decode_tile_grouped<kTileGroupBf16>(t, n_tiles_n, tstart, offsets, n_experts, e, row0, row_end, n0);
    const int r0 = __builtin_amdgcn_readfirstlane(static_cast<int>(row0));
    // rows past the segment repeat its last row (its token row stays cached)
    const int64_t lim = row_end - 1 - r0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int rr = i * 32 + ld_r;
      rr = rr < lim ? rr : static_cast<int>(lim);
      pf_src[i] = gather_src[r0 + rr];
    }
  };
  auto set_load_tile = [&](int t) __attribute__((always_inline)) {
    int e, n0;
    int64_t row0, row_end;
    decode_tile_grouped<kTileGroupBf16>(t, n_tiles_n, tstart, offsets, n_experts, e, row0, row_end, n0);
    e = __builtin_amdgcn_readfirstlane(e);
    n0 = __builtin_amdgcn_readfirstlane(n0);
    const int r0 = __builtin_amdgcn_readfirstlane(static_cast<int>(row0));
    b_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(B + (static_cast<int64_t>(e) * ncols + n0) * row_bytes), 0,
        b_tile_bytes, kBufferWord3);
    // Rows past the expert's segment are clamped to its last row (repeated
    // loads of one row hit the caches); their results are never stored.
    const int64_t lim = row_end - 1 - r0;
    if (GATHER) {
      // Row offsets into x from the sources prefetched one tile earlier; rows
      // without a source (-1) read token 0, and a source past the token count
      // is clamped (x is never read out of range).  Then prefetch the sources
      // of this workgroup's next tile, so that their load latency is hidden.
      a_tile = A;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        int tk = pf_src[i] >= 0 ? pf_src[i] / gather_k : 0;
        tk = tk < gather_rows ? tk : gather_rows - 1;
        a_off[i] = gather_offset(tk, row_bytes, ld_c * 16);
      }
      if (t + per_xcd < hi) fetch_src(t + per_xcd);
    } else {
      a_tile = A + static_cast<int64_t>(r0) * row_bytes;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        int rr = i * 32 + ld_r;
        rr = rr < lim ? rr : static_cast<int>(lim);
        a_off[i] = static_cast<uint32_t>(rr * row_bytes + ld_c * 16);
      }
    }
  };
  // Part p (0..3): rounds 2p and 2p+1 of A and of B of load step ld_g.
  auto issue_part = [&](u32x4* ra, u32x4* rb, int p) __attribute__((always_inline)) {
    const int kb = ODD && ld_kb == ksteps ? ksteps - 1 : ld_kb;  // the zero step reloads a real one
    const uint8_t* ab = a_tile + kb * 128;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int i = 2 * p + q;
      ra[i] = *reinterpret_cast<const u32x4*>(ab + a_off[i]);
      rb[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            b_rsrc, b_off0, kb * 128 + i * 32 * row_bytes, 0));
    }
  };
  // Once every step is loaded the load side repeats the last one, so every
  // K step issues the same loads.  The load side runs two steps ahead and
  // kpad is even, so it crosses into the next tile only in the advance that
  // follows an odd step's loads (WRAP): the even steps' advance has no tile
  // switch on its path, and the compiler's wait counts for the next tile's
  // gather sources then see a whole step of loads between their issue and
  // their use.  The gate/up kernels use it (with the gather offset below
  // it took the gathered gate/up GEMM 1.0-1.6 % faster, bit-identical); the
  // others keep the switch check in every step, which measured 0.3-0.6 %
  // faster for the down GEMM.
  auto advance = [&](auto Wc) __attribute__((always_inline)) {
    if (ld_g + 1 < iters) {
      ++ld_g;
      ++ld_kb;
      if constexpr (decltype(Wc)::value) {
        if (ld_kb == kpad) {
          ld_kb = 0;
          ld_t += per_xcd;
          set_load_tile(ld_t);
        }
      }
    }
  };
  auto park_part = [&](const u32x4* ra, const u32x4* rb, int stage, int p, uint32_t keep)
      __attribute__((always_inline)) {
    uint8_t* base = smem + stage * kStageBytes;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int i = 2 * p + q;
      const int row = i * 32 + ld_r;
      u32x4 va = ra[i], vb = rb[i];
      if (ODD) {
        va &= keep;
        vb &= keep;
      }
      *reinterpret_cast<u32x4*>(base + row * 128 + st_pos) = va;
      *reinterpret_cast<u32x4*>(base + 32768 + row * 128 + st_pos) = vb;
    }
  };
  u32x4 ra0[8], rb0[8], ra1[8], rb1[8];

  // ---- MFMA fragments -------------------------------------------------------
  // The weight fragment is the first MFMA operand, so an accumulator lane
  // holds one token row and groups of four consecutive output columns.
  // Fragment i of the wave's 128 rows is 32 rows (4096 bytes) further down.
  const int wm = wave >> 1, wn = wave & 1;
  const int frow = lane & 31;
  const int fhalf = lane >> 5;
  const int fa_row = wm * 128 + frow;
  const int fb_row = wn * 128 + frow;
  typename E::frag_t fa[2][4], fb[2][4];
  auto read_frags = [&](int buf, int stage, int s) __attribute__((always_inline)) {
    const uint8_t* base = smem + stage * kStageBytes;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fa[buf][i] = E::read(base, (fa_row + 32 * i) * 128, fa_row, s, fhalf);
      fb[buf][i] = E::read(base + 32768, (fb_row + 32 * i) * 128, fb_row, s, fhalf);
    }
  };
  f32x16 acc[4][4];

  // With the SwiGLU epilogue (gate/up) the last sub-step's 16 MFMAs run after
  // the step's barrier (tail_mfma), beside the next step's first fragment
  // reads, which otherwise leave the matrix core idle until they land
  // (measured 1.1 % on the gathered gate/up GEMM at both bf16 workloads,
  // bit-identical; the down GEMM was unchanged or 0.7 % slower, so it keeps
  // every MFMA before the barrier).
  constexpr bool kTailAfterBarrier = SWIGLU;
  auto tail_mfma = [&]() __attribute__((always_inline)) {
    if constexpr (kTailAfterBarrier) {
      constexpr int b = (E::kSub - 1) & 1;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = E::mfma(fb[b][j], fa[b][i], acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // K step kb of a tile on stage P (= parity of the global step g; fragments
  // for sub-step 0 are already in buffer 0).  Each sub-step issues a quarter
  // of step g+2's loads into the free register slot, writes a quarter of step
  // g+1's slot into stage P^1 (zeros if g+1 is a tile's padding step), reads
  // the next sub-step's fragments and runs 16 MFMAs; the memory operations
  // are spread between the MFMAs.
  auto step = [&](auto Pc, int kb) __attribute__((always_inline)) {
    constexpr int P = decltype(Pc)::value;
    const uint32_t keep = ODD && kb + 1 == ksteps ? 0u : ~0u;
    u32x4* ld_a = P == 0 ? ra0 : ra1;
    u32x4* ld_b = P == 0 ? rb0 : rb1;
    const u32x4* pk_a = P == 0 ? ra1 : ra0;
    const u32x4* pk_b = P == 0 ? rb1 : rb0;
#pragma unroll
    for (int s = 0; s < E::kSub; ++s) {
#pragma unroll
      for (int pp = 0; pp < kParts; ++pp) issue_part(ld_a, ld_b, s * kParts + pp);
#pragma unroll
      for (int pp = 0; pp < kParts; ++pp) park_part(pk_a, pk_b, P ^ 1, s * kParts + pp, keep);
      if (s + 1 < E::kSub) read_frags((s + 1) & 1, P, s + 1);
      if (!kTailAfterBarrier || s + 1 < E::kSub) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = E::mfma(fb[s & 1][j], fa[s & 1][i], acc[i][j]);
      }
      // Per 4 MFMAs: kParts global loads, kParts LDS writes, 2 * kParts LDS reads.
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);           // MFMA
        __builtin_amdgcn_sched_group_barrier(0x020, kParts, 0);      // global load
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x200, kParts, 0);      // LDS write
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * kParts, 0);  // LDS read
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    advance(IntC<SWIGLU ? P : 1>{});
    barrier_lds();
  };

  if (GATHER) fetch_src(first);
  set_load_tile(first);
#pragma unroll
  for (int p = 0; p < 4; ++p) issue_part(ra0, rb0, p);
  advance(IntC<SWIGLU ? 0 : 1>{});
#pragma unroll
  for (int p = 0; p < 4; ++p) issue_part(ra1, rb1, p);
  advance(IntC<1>{});
#pragma unroll
  for (int p = 0; p < 4; ++p) park_part(ra0, rb0, 0, p, ODD && ksteps == 0 ? 0u : ~0u);
  __syncthreads();
  read_frags(0, 0, 0);

  int g = 0;
  for (int t = first; t < hi; t += per_xcd) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    for (int kb = 0; kb < kpad; kb += 2) {
      step(IntC<0>{}, kb);
      read_frags(0, 1, 0);
      tail_mfma();
      step(IntC<1>{}, kb + 1);
      if (kb + 2 < kpad) read_frags(0, 0, 0);
      tail_mfma();
    }
    g += kpad;

    int e, n0;
    int64_t row0, row_end;
    decode_tile_grouped<kTileGroupBf16>(t, n_tiles_n, tstart, offsets, n_experts, e, row0, row_end, n0);
    // stage 1 is idle here: the tile's last step (odd) read it, step 0 of the
    // next tile writes it only after the epilogue's last barrier
    if constexpr (DSWIGLU)
      store_tile_lds_dswiglu(acc, smem + kStageBytes, C, ldc, dh, row0, row_end, n0, wm, wn, lane,
                             tid);
    else if constexpr (SWIGLU)
      store_tile_lds_swiglu(acc, smem + kStageBytes, C, ldc, row0, row_end, n0, wm, wn, lane, tid);
    else
      store_tile_lds(acc, smem + kStageBytes, C, ldc, row0, row_end, n0, wm, wn, lane, tid);
    if (g < iters) read_frags(0, 0, 0);
  }
}

// ---- weight gradients: ragged-K grouped GEMM -----------------------------------
// C_e[m][n] = sum over the rows r of expert e's segment [offsets[e],
// offsets[e+1]) of A[r][m] * B[r][n]: dWd[e] = h^T d_ys and dWg|dWu[e] =
// xs^T dg|du (the VJPs of moe.py:70-73 with respect to the expert weights).
// Both operands are row-major with the reduction index as the row, so a K
// step stages 64 rows x 256 columns of A and of B in LDS as they lie in
// memory ([k][col], 512-byte rows, 32-byte segment s of row k at s ^ 2(k&3))
// and the MFMA fragments come out of LDS through the transposing read
// ds_read_b64_tr_b16: in a group of 16 lanes, lane j receives element j % 4 of
// the 8 bytes addressed by lanes j/4 + 4q, q = 0..3.  Lane s of group G
// addresses row k0 + s/4, columns c0 + 16 (G % 2) + 4 (s % 4), so lane L
// receives rows k0 .. k0+3 of column c0 + L % 32; two such reads (k0 and
// k0 + 4, k0 = 8 (L / 32) of the sub-step) give the 8 consecutive K values of
// the 32x32x16 operand.  Tiles: every expert (an empty one too, whose
// gradient is zero) x (M / 256) x (N / 256), persistent as in the forward.
// Rows past the segment read zeros: the loads are raw buffer loads whose
// resource ends at the segment's last row (the row offset is in the
// range-checked VGPR offset; a segment of 2 GiB or more rebases its
// resources at every K step), so a tile runs max(2, ceil(rows / 64)) steps,
// rounded up to even, with no masking, and no buffer size limits it.  The output is float32; SPLIT: B's
// columns are in the gate/up order (blocks of 32 gate columns, then the 32 up
// columns of the same h columns) and C goes to out0 (gate) and out1 (up) as
// [e][m][F].
template <bool SPLIT, bool BIG>
__global__ __launch_bounds__(kThreads) void grouped_gemm_wgrad(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
    const int32_t* __restrict__ offsets, int n_experts, int M, int N, float* __restrict__ out0,
    float* __restrict__ out1) {
  typedef GemmElem<false> E;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int tm = M / kBM, tn = N / kBN;
  const int per_e = tm * tn;
  const int total = n_experts * per_e;
  const int xcd = blockIdx.x % kNumXcd;
  const int per_xcd = gridDim.x / kNumXcd;
  const int slot = blockIdx.x / kNumXcd;
  const int lo = static_cast<int>((static_cast<int64_t>(total) * xcd) / kNumXcd);
  const int hi = static_cast<int>((static_cast<int64_t>(total) * (xcd + 1)) / kNumXcd);
  const int first = lo + slot;
  if (first >= hi) return;  // uniform per workgroup
  const int a_row_bytes = M * 2, b_row_bytes = N * 2;

  struct Tile {
    int e, m0, n0, kpad;
    int64_t seg0;
    int rows;
  };
  auto decode = [&](int t) __attribute__((always_inline)) {
    Tile r;
    r.e = __builtin_amdgcn_readfirstlane(t / per_e);
    const int l = t - r.e * per_e;
    r.m0 = (l / tn) * kBM;
    r.n0 = (l - (l / tn) * tn) * kBN;
    const int s0 = __builtin_amdgcn_readfirstlane(offsets[r.e]);
    const int s1 = __builtin_amdgcn_readfirstlane(offsets[r.e + 1]);
    r.seg0 = s0;
    r.rows = s1 - s0;
    const int ks = (r.rows + 63) / 64;
    r.kpad = ks < 2 ? 2 : ks + (ks & 1);
    return r;
  };

  // ---- global -> registers -> LDS ------------------------------------------
  // Round i (0..7): this thread loads 16-byte chunk ld_c of row 8i + ld_r of
  // the A and B tiles (32 chunks per 512-byte row).
  const int ld_r = tid >> 5;
  const int ld_c = tid & 31;
  auto swz = [](int k, int byte) __attribute__((always_inline)) {
    return (((byte >> 5) ^ (2 * (k & 3))) << 5) | (byte & 31);
  };
  // A tile's buffer resources start at its segment's first row and end at
  // its last (the row offset k * row_bytes is in the range-checked VGPR
  // offset), which holds while the segment is below 2 GiB, whatever the size
  // of the whole buffer.  BIG (chosen by the host when the buffer could hold
  // a segment of 2 GiB or more): a tile whose segment is that large rebases
  // both resources at every K step instead, so its offsets stay within 64
  // rows.  (The two loaders are separate instantiations: the BIG one's extra
  // bookkeeping costs the common case about a third of its speed.)
  __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(A), 0, 0, kBufferWord3);
  __amdgpu_buffer_rsrc_t b_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(B), 0, 0, kBufferWord3);
  Tile lt = decode(first);
  int ld_t = first, ld_kb = 0;
  bool ld_more = true;
  int ld_koff = 0;      // BIG: row of the current K step relative to the resources' base
  bool ld_big = false;  // BIG: the load tile's segment is rebased per K step
  const int max_row_bytes = a_row_bytes > b_row_bytes ? a_row_bytes : b_row_bytes;
  auto set_rsrc = [&](int row_from) __attribute__((always_inline)) {
    const int64_t r0 = lt.seg0 + row_from;
    int left = lt.rows - row_from;
    left = left < 0 ? 0 : left;
    if (ld_big) left = left > 64 ? 64 : left;
    a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(A + r0 * M + lt.m0), 0,
        static_cast<int>(static_cast<uint32_t>(left) * a_row_bytes), kBufferWord3);
    b_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(B + r0 * N + lt.n0), 0,
        static_cast<int>(static_cast<uint32_t>(left) * b_row_bytes), kBufferWord3);
  };
  auto set_load_tile = [&](int t) __attribute__((always_inline)) {
    lt = decode(t);
    if constexpr (BIG) {
      ld_big = static_cast<int64_t>(lt.kpad) * 64 * max_row_bytes >= (int64_t(1) << 31);
      ld_koff = 0;
      set_rsrc(0);
    } else {
      const uint32_t nr = static_cast<uint32_t>(lt.rows);
      a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t*>(A + lt.seg0 * M + lt.m0), 0, static_cast<int>(nr * a_row_bytes), kBufferWord3);
      b_rsrc = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t*>(B + lt.seg0 * N + lt.n0), 0, static_cast<int>(nr * b_row_bytes), kBufferWord3);
    }
  };
  auto issue_part = [&](u32x4* ra, u32x4* rb, int p) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int i = 2 * p + q;
      const int k = (BIG ? ld_koff : ld_kb * 64) + 8 * i + ld_r;
      ra[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            a_rsrc, k * a_row_bytes + ld_c * 16, 0, 0));
      rb[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            b_rsrc, k * b_row_bytes + ld_c * 16, 0, 0));
    }
  };
  auto advance = [&]() __attribute__((always_inline)) {
    if (ld_more && ++ld_kb == lt.kpad) {
      if (ld_t + per_xcd < hi) {
        ld_t += per_xcd;
        ld_kb = 0;
        set_load_tile(ld_t);
      } else {
        ld_kb = lt.kpad - 1;
        ld_more = false;
      }
    } else if (BIG && ld_more) {
      if (ld_big)
        set_rsrc(ld_kb * 64);
      else
        ld_koff = ld_kb * 64;
    }
  };
  auto park_part = [&](const u32x4* ra, const u32x4* rb, int stage, int p) __attribute__((always_inline)) {
    uint8_t* base = smem + stage * kStageBytes;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int i = 2 * p + q;
      const int k = 8 * i + ld_r;
      const int off = k * 512 + swz(k, ld_c * 16);
      *reinterpret_cast<u32x4*>(base + off) = ra[i];
      *reinterpret_cast<u32x4*>(base + 32768 + off) = rb[i];
    }
  };
  u32x4 ra[8], rb[8];

  // ---- MFMA fragments (transposing LDS reads) --------------------------------
  const int wm = wave >> 1, wn = wave & 1;
  const int grp = lane >> 4, j16 = lane & 15;
  const int fr_k = 8 * (grp >> 1) + (j16 >> 2);                  // + 16 s (+ 4)
  const int fr_c = 16 * (grp & 1) + 4 * (j16 & 3);               // + 32-column block
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  auto tr_read = [&](const uint8_t* base, int k, int col) __attribute__((always_inline)) {
    const int off = k * 512 + swz(k, col * 2);
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4i16*)(
            (__attribute__((address_space(3))) uint8_t*)(base) + off));
  };
  typename E::frag_t fa[2][4], fb[2][4];
  auto read_frags = [&](int buf, int stage, int s) __attribute__((always_inline)) {
    const uint8_t* base = smem + stage * kStageBytes;
    const int k = 16 * s + fr_k;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ca = wm * 128 + 32 * i + fr_c;
      const int cb = wn * 128 + 32 * i + fr_c;
      const v4i16 a0 = tr_read(base, k, ca), a1 = tr_read(base, k + 4, ca);
      const v4i16 b0 = tr_read(base + 32768, k, cb), b1 = tr_read(base + 32768, k + 4, cb);
      fa[buf][i] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7));
      fb[buf][i] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7));
    }
  };
  f32x16 acc[4][4];

  auto step = [&](auto Pc) __attribute__((always_inline)) {
    constexpr int P = decltype(Pc)::value;
#pragma unroll
    for (int s = 0; s < E::kSub; ++s) {
      park_part(ra, rb, P ^ 1, s);
      issue_part(ra, rb, s);
      if (s + 1 < E::kSub) read_frags((s + 1) & 1, P, s + 1);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = E::mfma(fb[s & 1][j], fa[s & 1][i], acc[i][j]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global load
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // LDS read
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    advance();
    barrier_lds();
  };

  set_load_tile(first);
#pragma unroll
  for (int p = 0; p < 4; ++p) issue_part(ra, rb, p);
  advance();
#pragma unroll
  for (int p = 0; p < 4; ++p) park_part(ra, rb, 0, p);
#pragma unroll
  for (int p = 0; p < 4; ++p) issue_part(ra, rb, p);
  advance();
  __syncthreads();

  for (int t = first; t < hi; t += per_xcd) {
    const Tile ct = decode(t);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    read_frags(0, 0, 0);
    for (int kb = 0; kb < ct.kpad; kb += 2) {
      step(IntC<0>{});
      read_frags(0, 1, 0);
      step(IntC<1>{});
      if (kb + 2 < ct.kpad) read_frags(0, 0, 0);
    }
    // Epilogue: acc[i][j] lane L element r is C[m][n] with m = wm*128 + 32i +
    // L%32, n = wn*128 + 32j + (r/4)*8 + (L/32)*4 + r%4 (tile-relative).
    const int frow = lane & 31;
    const int col_lane = (lane >> 5) * 4;
    const int F = N / 2;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t m = ct.m0 + wm * 128 + 32 * i + frow;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = ct.n0 + wn * 128 + 32 * j + g * 8 + col_lane;
          const f32x4 v = {acc[i][j][g * 4], acc[i][j][g * 4 + 1], acc[i][j][g * 4 + 2],
                           acc[i][j][g * 4 + 3]};
          float* dst;
          if (SPLIT) {
            const int f = (n >> 6) * 32 + (n & 31);
            dst = ((n & 63) < 32 ? out0 : out1) + (static_cast<int64_t>(ct.e) * M + m) * F + f;
          } else {
            dst = out0 + (static_cast<int64_t>(ct.e) * M + m) * N + n;
          }
          __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(dst));
        }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// ---- gate/up and down in one persistent launch -----------------------------------
// The layer's two bf16 GEMMs (moe.py:70-74) as one launch: neither leaves a
// partial last round of tiles, there is one launch gap instead of two, and
// the store-heavy down tiles run beside other CUs' load-heavy gate/up tiles.
// The m-tiles (256-row blocks of the experts' segments) are split evenly
// over the XCDs, and each XCD keeps one work list: the gate/up tiles of its
// m-tiles (m-major, n fastest), then their down tiles.  The XCD of a
// workgroup is the hardware XCC id of the CU it runs on, not its block
// index, so the h rows a down tile reads were written by gate/up tiles of
// the same XCD, into that XCD's L2 (whose lines for h rows are only ever
// written or read by this XCD during the launch): no L2 write-back or
// invalidation is needed between them.  Workgroups claim list positions one
// at a time from the XCD's counter, three tiles ahead of the tile they
// compute (so the load pipeline and the gather's source prefetch can look
// ahead), and compute their claims in order.  A down tile of m-tile m waits
// until ready[m] counts every gate/up tile of m: a gate/up tile adds one
// once all its waves' stores have completed (s_waitcnt vmcnt(0) and a
// barrier, in the first K step of the workgroup's next tile, or at the end
// of its gate/up tiles).  No deadlock: a workgroup claims a down tile only
// after every gate/up position of its XCD has been claimed, by workgroups
// that are running and never wait inside a gate/up tile.  The wait is
// bounded by a wall-clock limit: a wait that gives up sets status bit 0 and
// its tile is computed from whatever h holds (every access stays in bounds),
// so every workgroup always exits.
// Sync words of the workspace.  The launch leaves every counter at zero when
// it ends (the last workgroup to finish clears them), so a workspace that
// was zero before its first call needs no clearing between calls.
constexpr int kFusedStatus = 8;   // status of the last completed call (bit 0: a wait gave up)
constexpr int kFusedError = 9;    // status bits of the running call
constexpr int kFusedDone = 10;    // workgroups finished in the running call
// The claim ring lives in LDS; volatile, so that every read after a barrier
// sees what thread 0 wrote before it.
typedef __attribute__((address_space(3))) volatile int32_t lds_ring_t;
constexpr int kFusedReady = 16;   // sync words from here: ready count per m-tile
                                  // (words 0..7: claim counter per XCD)

// HW_REG_XCC_ID (hardware register 20), bits 3:0: the XCD this wave runs on.
__device__ __forceinline__ int hw_xcc_id() {
  return static_cast<int>(__builtin_amdgcn_s_getreg((3 << 11) | 20) & (kNumXcd - 1));
}

// One XCD's work list.  Position p < n_gu is gate/up tile (m_lo + p / nt_gu,
// p % nt_gu); n_gu <= p < total is down tile (m_lo + q / nt_dn, q % nt_dn),
// q = p - n_gu; -1 is no tile.
struct FusedList {
  int m_lo, n_gu, total, nt_gu, nt_dn;
  __device__ bool gate_up(int p) const { return p >= 0 && p < n_gu; }
  __device__ bool down(int p) const { return p >= n_gu; }
  __device__ int mtile(int p) const {
    return p < n_gu ? m_lo + p / nt_gu : m_lo + (p - n_gu) / nt_dn;
  }
  // Logical tile index of decode_tile (m * n_tiles + n).
  __device__ int tile(int p) const {
    if (p < n_gu) return (m_lo + p / nt_gu) * nt_gu + p % nt_gu;
    const int q = p - n_gu;
    return (m_lo + q / nt_dn) * nt_dn + q % nt_dn;
  }
};

// Waits (thread 0 only) until ready[m] >= need or the wall clock has run
// wait_ticks past the first failed look; v is a value already loaded.
__device__ __forceinline__ void fused_wait_ready(uint32_t v, const uint32_t* ready, int m,
                                                 uint32_t need, uint64_t wait_ticks,
                                                 uint32_t* status) {
  if (v >= need) return;
  const uint64_t t0 = static_cast<uint64_t>(wall_clock64());
  for (;;) {
    __builtin_amdgcn_s_sleep(2);
    v = __hip_atomic_load(ready + m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (v >= need) return;
    if (static_cast<uint64_t>(wall_clock64()) - t0 > wait_ticks) {
      __hip_atomic_fetch_or(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
  }
}

// The tiles of one phase of the fused launch (GATE_UP: gate/up with the
// gather and the SwiGLU epilogue; else down), the claims ring[k], ring[k+1],
// ... of this workgroup while they belong to the phase.  The pipeline is the
// one of grouped_gemm_regs (even number of K steps, at least 4).
template <bool GATE_UP>
__device__ __forceinline__ void fused_phase(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ B, int kdim, int ncols,
    uint16_t* __restrict__ C, int64_t ldc, const int32_t* __restrict__ gather_src, int gather_k,
    int gather_rows, const int32_t* __restrict__ offsets, int n_experts, const int32_t* tstart,
    uint8_t* smem, lds_ring_t* ring, int& k, const FusedList& L,
    uint32_t* __restrict__ claim_ctr, uint32_t* __restrict__ status, uint32_t* __restrict__ ready,
    uint32_t need, uint64_t wait_ticks) {
  constexpr bool GATHER = GATE_UP;
  typedef GemmElem<false> E;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n_tiles_n = GATE_UP ? L.nt_gu : L.nt_dn;
  auto ring_at = [&](int j) __attribute__((always_inline)) {
    return __builtin_amdgcn_readfirstlane(ring[j & 3]);
  };
  auto mine = [&](int p) __attribute__((always_inline)) {
    return GATE_UP ? L.gate_up(p) : L.down(p);
  };
  if (!mine(ring_at(k))) return;  // uniform
  auto decode = [&](int p, int& e, int64_t& row0, int64_t& row_end, int& n0)
      __attribute__((always_inline)) {
    decode_tile(L.tile(p), n_tiles_n, tstart, offsets, n_experts, e, row0, row_end, n0);
  };

  if (!GATE_UP) {
    // The first down tile: nothing of it is loaded before its m-tile is ready.
    const int p0 = ring_at(k);
    if (tid == 0)
      fused_wait_ready(__hip_atomic_load(ready + L.mtile(p0), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT),
                       ready, L.mtile(p0), need, wait_ticks, status);
    __syncthreads();
  }

  const int row_bytes = kdim * E::kBytes;
  const int kpad = row_bytes / 128;
  const int ld_r = tid >> 3;
  const int ld_c = tid & 7;
  const int st_pos = (ld_c ^ lds_swz(ld_r)) * 16;
  const uint32_t b_off0 = static_cast<uint32_t>(ld_r * row_bytes + ld_c * 16);
  uint32_t a_off[8];
  const uint8_t* a_tile = A;
  const int b_tile_bytes = 256 * row_bytes;
  __amdgpu_buffer_rsrc_t b_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(B), 0, b_tile_bytes, kBufferWord3);
  int ld_k = k, ld_kb = 0;
  bool ld_done = false;
  int32_t pf_src[8];
  auto fetch_src = [&](int p) __attribute__((always_inline)) {
    int e, n0;
    int64_t row0, row_end;
    decode(p, e, row0, row_end, n0);
    const int r0 = __builtin_amdgcn_readfirstlane(static_cast<int>(row0));
    const int64_t lim = row_end - 1 - r0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int rr = i * 32 + ld_r;
      rr = rr < lim ? rr : static_cast<int>(lim);
      pf_src[i] = gather_src[r0 + rr];
    }
  };
  // The load side enters tile p; p_next is the claim after it (prefetched
  // gather sources when it belongs to the phase).
  auto set_load_tile = [&](int p, int p_next) __attribute__((always_inline)) {
    int e, n0;
    int64_t row0, row_end;
    decode(p, e, row0, row_end, n0);
    e = __builtin_amdgcn_readfirstlane(e);
    n0 = __builtin_amdgcn_readfirstlane(n0);
    const int r0 = __builtin_amdgcn_readfirstlane(static_cast<int>(row0));
    b_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(B + (static_cast<int64_t>(e) * ncols + n0) * row_bytes), 0,
        b_tile_bytes, kBufferWord3);
    const int64_t lim = row_end - 1 - r0;
    if (GATHER) {
      a_tile = A;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        int tk = pf_src[i] >= 0 ? pf_src[i] / gather_k : 0;
        tk = tk < gather_rows ? tk : gather_rows - 1;
        a_off[i] = gather_offset(tk, row_bytes, ld_c * 16);
      }
      if (mine(p_next)) fetch_src(p_next);
    } else {
      a_tile = A + static_cast<int64_t>(r0) * row_bytes;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        int rr = i * 32 + ld_r;
        rr = rr < lim ? rr : static_cast<int>(lim);
        a_off[i] = static_cast<uint32_t>(rr * row_bytes + ld_c * 16);
      }
    }
  };
  auto issue_part = [&](u32x4* ra, u32x4* rb, int p) __attribute__((always_inline)) {
    const uint8_t* ab = a_tile + ld_kb * 128;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int i = 2 * p + q;
      ra[i] = *reinterpret_cast<const u32x4*>(ab + a_off[i]);
      rb[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            b_rsrc, b_off0, ld_kb * 128 + i * 32 * row_bytes, 0));
    }
  };
  // After the phase's last claimed tile the load side repeats its last step.
  auto advance = [&]() __attribute__((always_inline)) {
    if (ld_done) return;
    if (++ld_kb == kpad) {
      const int np = ring_at(ld_k + 1);
      if (!mine(np)) {
        ld_done = true;
        ld_kb = kpad - 1;
        return;
      }
      ld_kb = 0;
      ++ld_k;
      set_load_tile(np, ring_at(ld_k + 1));
    }
  };
  auto park_part = [&](const u32x4* ra, const u32x4* rb, int stage, int p)
      __attribute__((always_inline)) {
    uint8_t* base = smem + stage * kStageBytes;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int i = 2 * p + q;
      const int row = i * 32 + ld_r;
      *reinterpret_cast<u32x4*>(base + row * 128 + st_pos) = ra[i];
      *reinterpret_cast<u32x4*>(base + 32768 + row * 128 + st_pos) = rb[i];
    }
  };
  u32x4 ra0[8], rb0[8], ra1[8], rb1[8];

  const int wm = wave >> 1, wn = wave & 1;
  const int frow = lane & 31;
  const int fhalf = lane >> 5;
  const int fa_row = wm * 128 + frow;
  const int fb_row = wn * 128 + frow;
  typename E::frag_t fa[2][4], fb[2][4];
  auto read_frags = [&](int buf, int stage, int s) __attribute__((always_inline)) {
    const uint8_t* base = smem + stage * kStageBytes;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fa[buf][i] = E::read(base, (fa_row + 32 * i) * 128, fa_row, s, fhalf);
      fb[buf][i] = E::read(base + 32768, (fb_row + 32 * i) * 128, fb_row, s, fhalf);
    }
  };
  f32x16 acc[4][4];

  // Per tile: thread 0 claims the position of tile k + 3 when the tile
  // starts and publishes it in the ring at the end of K step hook_step; in
  // the down phase it also resolves the readiness of tile k + 1 there, before
  // the barrier, and the load side enters tile k + 1 only after that barrier
  // (at the end of step kpad - 3 > hook_step).  In the gate/up phase the
  // previous tile's stores are waited for (vmcnt(0)) before that barrier and
  // counted in ready[] right after it.
  int m_pending = -1;
  uint32_t claimed = 0;
  // K step (even) whose end runs the hook: the third when the tile has at
  // least six, so the claim and the probe have two more steps to return
  // (under the operand stream's load an atomic can outlast one K step, and
  // the barrier would wait for it); the first otherwise.
  const int hook_step = kpad >= 6 ? 2 : 0;
  uint32_t probe = 0;
  int probe_m = 0;
  auto first_step_hook = [&]() __attribute__((always_inline)) {
    if (GATE_UP && m_pending >= 0) wait_vm_lgkm0<0>();
    if (tid == 0) {
      // The empty asm pins the first read of the claim (and of the probe)
      // here: the compiler would otherwise hoist the comparisons to the tile
      // start, and with them the wait for the atomics' results.
      uint32_t c = claimed;
      asm volatile("" : "+v"(c));
      ring[(k + 3) & 3] = c < static_cast<uint32_t>(L.total) ? static_cast<int>(c) : -1;
      if (!GATE_UP && probe_m >= 0) {
        uint32_t v = probe;
        asm volatile("" : "+v"(v));
        fused_wait_ready(v, ready, probe_m, need, wait_ticks, status);
      }
    }
  };
  auto step = [&](auto Pc, bool first) __attribute__((always_inline)) {
    constexpr int P = decltype(Pc)::value;
    u32x4* ld_a = P == 0 ? ra0 : ra1;
    u32x4* ld_b = P == 0 ? rb0 : rb1;
    const u32x4* pk_a = P == 0 ? ra1 : ra0;
    const u32x4* pk_b = P == 0 ? rb1 : rb0;
#pragma unroll
    for (int s = 0; s < E::kSub; ++s) {
      issue_part(ld_a, ld_b, s);
      park_part(pk_a, pk_b, P ^ 1, s);
      if (s + 1 < E::kSub) read_frags((s + 1) & 1, P, s + 1);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = E::mfma(fb[s & 1][j], fa[s & 1][i], acc[i][j]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global load
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // LDS read
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    advance();
    if (first) first_step_hook();
    barrier_lds();
  };

  if (GATHER) fetch_src(ring_at(k));
  set_load_tile(ring_at(k), ring_at(k + 1));
#pragma unroll
  for (int p = 0; p < 4; ++p) issue_part(ra0, rb0, p);
  advance();
#pragma unroll
  for (int p = 0; p < 4; ++p) issue_part(ra1, rb1, p);
  advance();
#pragma unroll
  for (int p = 0; p < 4; ++p) park_part(ra0, rb0, 0, p);
  __syncthreads();
  read_frags(0, 0, 0);

  for (;;) {
    const int p = ring_at(k);
    if (tid == 0) {
      // the result is first read in the first K step's hook, so the wait for
      // it does not hold up the step's loads
      claimed = __hip_atomic_fetch_add(claim_ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      probe_m = -1;
      if (!GATE_UP) {
        const int pn = ring_at(k + 1);
        if (L.down(pn)) {
          probe_m = L.mtile(pn);
          probe = __hip_atomic_load(ready + probe_m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    for (int kb = 0; kb < kpad; kb += 2) {
      step(IntC<0>{}, kb == hook_step);
      if (GATE_UP && kb == hook_step && m_pending >= 0) {
        if (tid == 0)
          __hip_atomic_fetch_add(ready + m_pending, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        m_pending = -1;
      }
      read_frags(0, 1, 0);
      step(IntC<1>{}, false);
      if (kb + 2 < kpad) read_frags(0, 0, 0);
    }

    int e, n0;
    int64_t row0, row_end;
    decode(p, e, row0, row_end, n0);
    if constexpr (GATE_UP)
      store_tile_lds_swiglu(acc, smem + kStageBytes, C, ldc, row0, row_end, n0, wm, wn, lane, tid);
    else
      store_tile_lds(acc, smem + kStageBytes, C, ldc, row0, row_end, n0, wm, wn, lane, tid);
    if (GATE_UP) m_pending = L.mtile(p);
    const bool more = mine(ring_at(k + 1));
    ++k;
    if (!more) break;
    read_frags(0, 0, 0);
  }
  if (GATE_UP && m_pending >= 0) {
    wait_vm_lgkm0<0>();
    barrier_lds();
    if (tid == 0)
      __hip_atomic_fetch_add(ready + m_pending, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

__global__ __launch_bounds__(kThreads) void grouped_swiglu_fused(
    const uint8_t* __restrict__ x, const uint8_t* __restrict__ w_gu,
    const uint8_t* __restrict__ w_dn, const int32_t* __restrict__ offsets, int n_experts,
    int d_model, int d_ff, uint16_t* __restrict__ h, uint16_t* __restrict__ ys,
    const int32_t* __restrict__ perm_src, int top_k, int tokens, uint32_t* __restrict__ sync,
    uint32_t need, uint64_t wait_ticks) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int32_t tstart[kMaxExperts + 1];
  __shared__ int32_t scan_tmp[kThreads];
  __shared__ int32_t ring_s[4];
  lds_ring_t* ring = (lds_ring_t*)ring_s;
  const int tid = threadIdx.x;
  const int m_total = __builtin_amdgcn_readfirstlane(scan_tiles(offsets, n_experts, tstart, scan_tmp));
  const int xcc = __builtin_amdgcn_readfirstlane(hw_xcc_id());
  FusedList L;
  L.nt_gu = 2 * d_ff / kBN;
  L.nt_dn = d_model / kBN;
  L.m_lo = static_cast<int>((static_cast<int64_t>(m_total) * xcc) / kNumXcd);
  const int m_hi = static_cast<int>((static_cast<int64_t>(m_total) * (xcc + 1)) / kNumXcd);
  L.n_gu = (m_hi - L.m_lo) * L.nt_gu;
  L.total = L.n_gu + (m_hi - L.m_lo) * L.nt_dn;
  uint32_t* claim_ctr = sync + xcc;
  uint32_t* error = sync + kFusedError;
  uint32_t* ready = sync + kFusedReady;
  if (tid == 0) {
    // three claims in flight together; their results are read after all
    // three are issued
    uint32_t c[3];
#pragma unroll
    for (int j = 0; j < 3; ++j)
      c[j] = __hip_atomic_fetch_add(claim_ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int j = 0; j < 3; ++j) ring[j] = c[j] < static_cast<uint32_t>(L.total) ? static_cast<int>(c[j]) : -1;
  }
  __syncthreads();
  int k = 0;
  fused_phase<true>(x, w_gu, d_model, 2 * d_ff, h, d_ff, perm_src, top_k, tokens, offsets,
                    n_experts, tstart, smem, ring, k, L, claim_ctr, error, ready, need, wait_ticks);
  fused_phase<false>(reinterpret_cast<const uint8_t*>(h), w_dn, d_ff, d_model, ys, d_model,
                     nullptr, 1, 1, offsets, n_experts, tstart, smem, ring, k, L, claim_ctr,
                     error, ready, need, wait_ticks);
  // The last workgroup to finish publishes the status and clears every
  // counter for the next call.  Thread 0 waits for its own atomics first
  // (vmcnt(0)), so no count of this workgroup can land after the clearing.
  wait_vm_lgkm0<0>();
  __syncthreads();
  if (tid == 0) {
    const uint32_t d =
        __hip_atomic_fetch_add(sync + kFusedDone, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ring[0] = d == gridDim.x - 1 ? 1 : 0;
  }
  __syncthreads();
  if (ring[0]) {
    for (int i = tid; i < m_total; i += kThreads) ready[i] = 0u;
    if (tid < kNumXcd) sync[tid] = 0u;
    if (tid == 0) {
      sync[kFusedStatus] =
          __hip_atomic_exchange(error, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sync[kFusedDone] = 0u;
    }
  }
}

// Workgroups per launch: one per CU, a multiple of the XCD count.
int persistent_grid(hipStream_t s, int* grid, int* dev_out) {
  int dev = 0;
  if (hipStreamGetDevice(s, &dev) != hipSuccess) {
    if (hipGetDevice(&dev) != hipSuccess) {
      set_error("grouped GEMM: cannot query the current device");
      return HMOE_ERR_HIP;
    }
  }
  static std::atomic<int> cached[64];
  int cus = dev >= 0 && dev < 64 ? cached[dev].load(std::memory_order_relaxed) : 0;
  if (cus == 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0) {
      set_error("grouped GEMM: cannot query the CU count of device %d", dev);
      return HMOE_ERR_HIP;
    }
    if (dev >= 0 && dev < 64) cached[dev].store(cus, std::memory_order_relaxed);
  }
  int g = (cus / kNumXcd) * kNumXcd;
  *grid = g > 0 ? g : kNumXcd;
  *dev_out = dev;
  return HMOE_OK;
}

bool set_lds_limit(const void* kernel, int bytes) {
  return hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) == hipSuccess;
}

// Allows 2 * kStageBytes of dynamic LDS for every kernel variant, once per device.
int allow_dynamic_lds(int dev) {
  static std::atomic<bool> done[64];
  if (dev >= 0 && dev < 64 && done[dev].load(std::memory_order_acquire)) return HMOE_OK;
  const int bytes = 2 * kStageBytes;
  const void* kernels[] = {
      reinterpret_cast<const void*>(grouped_gemm_regs<true, false, false>),
      reinterpret_cast<const void*>(grouped_gemm_regs<true, true, false>),
      reinterpret_cast<const void*>(grouped_gemm_regs<false, false, false>),
      reinterpret_cast<const void*>(grouped_gemm_regs<false, true, false>),
      reinterpret_cast<const void*>(grouped_gemm_regs<true, false, true>),
      reinterpret_cast<const void*>(grouped_gemm_regs<true, true, true>),
      reinterpret_cast<const void*>(grouped_gemm_regs<false, false, true>),
      reinterpret_cast<const void*>(grouped_gemm_regs<false, true, true>),
      reinterpret_cast<const void*>(grouped_gemm_regs<false, false, false, true>),
      reinterpret_cast<const void*>(grouped_gemm_regs<false, true, false, true>),
      reinterpret_cast<const void*>(grouped_gemm_regs<false, false, true, true>),
      reinterpret_cast<const void*>(grouped_gemm_regs<false, true, true, true>),
      reinterpret_cast<const void*>(grouped_gemm_wgrad<false, false>),
      reinterpret_cast<const void*>(grouped_gemm_wgrad<true, false>),
      reinterpret_cast<const void*>(grouped_gemm_wgrad<false, true>),
      reinterpret_cast<const void*>(grouped_gemm_wgrad<true, true>),
      reinterpret_cast<const void*>(grouped_gemm_w8_fp8<true, false>),
      reinterpret_cast<const void*>(grouped_gemm_w8_fp8<true, true>),
      reinterpret_cast<const void*>(grouped_gemm_w8_fp8<false, false>),
      reinterpret_cast<const void*>(grouped_gemm_w8_fp8<true, false, true>),
      reinterpret_cast<const void*>(grouped_gemm_w8_fp8<true, true, true>),
      reinterpret_cast<const void*>(grouped_swiglu_fused),
  };
  bool ok = true;
  for (const void* k : kernels) ok = ok && set_lds_limit(k, bytes);
  // the block-scaled down GEMM: two 2 KB exponent regions past the stages
  ok = ok && set_lds_limit(reinterpret_cast<const void*>(grouped_gemm_w8_fp8<false, false, true>),
                           kW8MxLds);
  if (!ok) {
    set_error("grouped GEMM: cannot allow %d bytes of dynamic LDS on device %d", bytes, dev);
    return HMOE_ERR_HIP;
  }
  if (dev >= 0 && dev < 64) done[dev].store(true, std::memory_order_release);
  return HMOE_OK;
}

int launch_grouped(bool swiglu, bool fp8, const void* A, const void* B, const float* a_scale,
                   const float* b_scale, const int32_t* offsets, int n_experts, int64_t rows_cap,
                   int kdim, int ncols, void* C, int64_t ldc, hipStream_t s, const char* what,
                   const int32_t* gather_src = nullptr, int gather_k = 1, int gather_rows = 1,
                   const uint16_t* dswiglu_dh = nullptr, uint8_t* mx_exp = nullptr) {
  const int n_tiles_n = ncols / kBN;
  HMOE_REQUIRE(mx_exp == nullptr || fp8, "%s: block exponents belong to the e4m3 GEMM", what);
  HMOE_REQUIRE(dswiglu_dh == nullptr || (!swiglu && !fp8), "%s: SwiGLU VJP epilogue needs the raw bf16 GEMM", what);
  const int64_t max_tiles = (ceil_div(rows_cap, kBM) + n_experts) * n_tiles_n;
  HMOE_REQUIRE(max_tiles < (int64_t(1) << 31), "%s: too many tiles", what);
  HMOE_REQUIRE(rows_cap < (int64_t(1) << 31), "%s: rows_cap must fit in int32", what);
  HMOE_REQUIRE(static_cast<int64_t>(kBM) * kdim * (fp8 ? 1 : 2) < (int64_t(1) << 31),
               "%s: reduction dimension too large", what);
  HMOE_REQUIRE(static_cast<int64_t>(kBM) * ldc * 2 < (int64_t(1) << 31), "%s: output rows too wide", what);
  int dev = 0;
  int grid = 0;
  if (int rc = persistent_grid(s, &grid, &dev)) return rc;
  if (int rc = allow_dynamic_lds(dev)) return rc;
  const size_t lds = 2 * kStageBytes;
  const uint8_t* a = static_cast<const uint8_t*>(A);
  const uint8_t* b = static_cast<const uint8_t*>(B);
  uint16_t* c = static_cast<uint16_t*>(C);
  const bool odd = ((static_cast<int64_t>(kdim) * (fp8 ? 1 : 2) / 128) & 1) != 0;
  if (fp8) {
    HMOE_REQUIRE(kdim % (2 * kW8StepBytes) == 0,
                 "%s: reduction dimension must be a multiple of %d", what, 2 * kW8StepBytes);
    HMOE_REQUIRE(static_cast<int64_t>(gather_rows) * kdim < (int64_t(1) << 31),
                 "%s: gathered matrix too large", what);
#define HMOE_LAUNCH_W8(SW, GA, MX, LDS)                                                           \
  hipLaunchKernelGGL((grouped_gemm_w8_fp8<SW, GA, MX>), dim3(grid), dim3(kW8Threads), LDS, s, a, \
                     b, a_scale, b_scale, offsets, n_experts, rows_cap, kdim, ncols, c, ldc,        \
                     n_tiles_n, gather_src, gather_k, gather_rows, mx_exp)
    HMOE_REQUIRE(swiglu || gather_src == nullptr, "%s: the fp8 down GEMM does not gather", what);
    if (mx_exp != nullptr) {
      if (swiglu && gather_src != nullptr) HMOE_LAUNCH_W8(true, true, true, kW8Lds);
      else if (swiglu) HMOE_LAUNCH_W8(true, false, true, kW8Lds);
      else HMOE_LAUNCH_W8(false, false, true, kW8MxLds);
    } else if (swiglu && gather_src != nullptr) HMOE_LAUNCH_W8(true, true, false, kW8Lds);
    else if (swiglu) HMOE_LAUNCH_W8(true, false, false, kW8Lds);
    else HMOE_LAUNCH_W8(false, false, false, kW8Lds);
#undef HMOE_LAUNCH_W8
  } else {
#define HMOE_LAUNCH_REGS(SW, OD, GA, ...)                                                         \
  hipLaunchKernelGGL((grouped_gemm_regs<SW, OD, GA, ##__VA_ARGS__>), dim3(grid), dim3(kThreads),   \
                     lds, s, a, b, offsets, n_experts, rows_cap, kdim, ncols, c, ldc, n_tiles_n,  \
                     gather_src, gather_k, gather_rows, dswiglu_dh)
    if (dswiglu_dh != nullptr) {
      if (gather_src != nullptr && odd) HMOE_LAUNCH_REGS(false, true, true, true);
      else if (gather_src != nullptr) HMOE_LAUNCH_REGS(false, false, true, true);
      else if (odd) HMOE_LAUNCH_REGS(false, true, false, true);
      else HMOE_LAUNCH_REGS(false, false, false, true);
    } else if (gather_src != nullptr) {
      if (swiglu && odd) HMOE_LAUNCH_REGS(true, true, true);
      else if (swiglu) HMOE_LAUNCH_REGS(true, false, true);
      else if (odd) HMOE_LAUNCH_REGS(false, true, true);
      else HMOE_LAUNCH_REGS(false, false, true);
    } else if (swiglu && odd) HMOE_LAUNCH_REGS(true, true, false);
    else if (swiglu) HMOE_LAUNCH_REGS(true, false, false);
    else if (odd) HMOE_LAUNCH_REGS(false, true, false);
    else HMOE_LAUNCH_REGS(false, false, false);
#undef HMOE_LAUNCH_REGS
  }
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
  return launch_grouped(true, false, xs, w_gate_up_packed, nullptr, nullptr, offsets, n_experts,
                        rows_cap, d_model, 2 * d_ff, h, d_ff, static_cast<hipStream_t>(stream),
                        "hmoe_grouped_gate_up");
}

extern "C" int hmoe_grouped_gate_up_gather(const void* x, int64_t tokens, int top_k,
                                           const int32_t* perm_src, const int32_t* offsets,
                                           int n_experts, int64_t rows_cap, int d_model, int d_ff,
                                           const void* w_gate_up_packed, void* h,
                                           hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= kMaxExperts,
               "grouped_gate_up_gather: n_experts must be in [1, %d] (got %d)", kMaxExperts,
               n_experts);
  HMOE_REQUIRE(rows_cap >= 0 && tokens >= 0 && top_k >= 1 && (tokens >= 1 || rows_cap == 0),
               "grouped_gate_up_gather: need rows_cap >= 0, tokens >= 0, top_k >= 1 (tokens >= 1 with rows)");
  HMOE_REQUIRE_CODE(d_model % kBK == 0 && d_model >= kBK, HMOE_ERR_UNSUPPORTED,
                    "grouped_gate_up_gather: d_model must be a multiple of %d (got %d)", kBK,
                    d_model);
  HMOE_REQUIRE_CODE((2 * d_ff) % kBN == 0 && d_ff > 0, HMOE_ERR_UNSUPPORTED,
                    "grouped_gate_up_gather: d_ff must be a multiple of %d (got %d)", kBN / 2,
                    d_ff);
  HMOE_REQUIRE(tokens * d_model * 2 < (int64_t(1) << 31),
               "grouped_gate_up_gather: x must be smaller than 2 GiB");
  if (rows_cap == 0) return HMOE_OK;
  HMOE_REQUIRE(x && perm_src && offsets && w_gate_up_packed && h,
               "grouped_gate_up_gather: null pointer argument");
  return launch_grouped(true, false, x, w_gate_up_packed, nullptr, nullptr, offsets, n_experts,
                        rows_cap, d_model, 2 * d_ff, h, d_ff, static_cast<hipStream_t>(stream),
                        "hmoe_grouped_gate_up_gather", perm_src, top_k, static_cast<int>(tokens));
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
  return launch_grouped(false, false, h, w_down_packed, nullptr, nullptr, offsets, n_experts,
                        rows_cap, d_ff, d_model, ys, d_model, static_cast<hipStream_t>(stream),
                        "hmoe_grouped_down");
}

namespace hmoe {
namespace {
// Ticks of the wall clock (s_memrealtime) per microsecond, once per device.
int wall_ticks_per_us(int dev, int64_t* out) {
  static std::atomic<int64_t> cached[64];
  int64_t v = dev >= 0 && dev < 64 ? cached[dev].load(std::memory_order_relaxed) : 0;
  if (v == 0) {
    int khz = 0;
    if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || khz <= 0) {
      set_error("grouped_swiglu_fused: cannot query the wall clock rate of device %d", dev);
      return HMOE_ERR_HIP;
    }
    v = (khz + 999) / 1000;
    if (dev >= 0 && dev < 64) cached[dev].store(v, std::memory_order_relaxed);
  }
  *out = v;
  return HMOE_OK;
}
}  // namespace
}  // namespace hmoe

namespace hmoe {
namespace {
__global__ void zero_fill_kernel(uint32_t* __restrict__ p, int64_t words) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < words;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = 0u;
}
}  // namespace
}  // namespace hmoe

extern "C" int hmoe_zero_fill(void* buffer, size_t bytes, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(bytes % 4 == 0, "zero_fill: byte count must be a multiple of 4 (got %zu)", bytes);
  if (bytes == 0) return HMOE_OK;
  HMOE_REQUIRE(buffer != nullptr, "zero_fill: null buffer");
  const int64_t words = static_cast<int64_t>(bytes / 4);
  const int blocks = static_cast<int>(ceil_div(words, 256) < 1024 ? ceil_div(words, 256) : 1024);
  hipLaunchKernelGGL(zero_fill_kernel, dim3(blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<uint32_t*>(buffer), words);
  return check_launch("hmoe_zero_fill");
}

extern "C" size_t hmoe_grouped_swiglu_fused_workspace_bytes(int64_t rows_cap, int n_experts) {
  using namespace hmoe;
  if (rows_cap < 0 || n_experts < 1) return 0;
  return static_cast<size_t>(kFusedReady + ceil_div(rows_cap, kBM) + n_experts) * sizeof(uint32_t);
}

extern "C" int hmoe_grouped_swiglu_fused(const void* x, int64_t tokens, int top_k,
                                         const int32_t* perm_src, const int32_t* offsets,
                                         int n_experts, int64_t rows_cap, int d_model, int d_ff,
                                         const void* w_gate_up_packed, const void* w_down_packed,
                                         void* h, void* ys, void* workspace,
                                         size_t workspace_bytes, int64_t wait_timeout_us,
                                         int extra_ready_needed, hmoe_stream_t stream) {
  using namespace hmoe;
  const char* what = "hmoe_grouped_swiglu_fused";
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= kMaxExperts,
               "%s: n_experts must be in [1, %d] (got %d)", what, kMaxExperts, n_experts);
  HMOE_REQUIRE(rows_cap >= 0 && tokens >= 0 && top_k >= 1 && (tokens >= 1 || rows_cap == 0),
               "%s: need rows_cap >= 0, tokens >= 0, top_k >= 1 (tokens >= 1 with rows)", what);
  HMOE_REQUIRE_CODE(d_model % kBN == 0 && d_model >= kBN, HMOE_ERR_UNSUPPORTED,
                    "%s: d_model must be a multiple of %d (got %d)", what, kBN, d_model);
  HMOE_REQUIRE_CODE((2 * d_ff) % kBN == 0 && d_ff >= kBN,
                    HMOE_ERR_UNSUPPORTED,
                    "%s: d_ff must be a multiple of %d and at least %d (got %d)", what, kBN / 2,
                    kBN, d_ff);
  HMOE_REQUIRE(extra_ready_needed >= 0, "%s: extra_ready_needed must be >= 0", what);
  HMOE_REQUIRE(tokens * d_model * 2 < (int64_t(1) << 31), "%s: x must be smaller than 2 GiB", what);
  HMOE_REQUIRE(rows_cap < (int64_t(1) << 31), "%s: rows_cap must fit in int32", what);
  HMOE_REQUIRE(static_cast<int64_t>(kBM) * d_model * 2 < (int64_t(1) << 31),
               "%s: output rows too wide", what);
  if (rows_cap == 0) return HMOE_OK;
  HMOE_REQUIRE(x && perm_src && offsets && w_gate_up_packed && w_down_packed && h && ys && workspace,
               "%s: null pointer argument", what);
  const size_t need_ws = hmoe_grouped_swiglu_fused_workspace_bytes(rows_cap, n_experts);
  HMOE_REQUIRE_CODE(workspace_bytes >= need_ws, HMOE_ERR_WORKSPACE,
                    "%s: workspace of %zu bytes, %zu needed", what, workspace_bytes, need_ws);
  hipStream_t s = static_cast<hipStream_t>(stream);
  int dev = 0, grid = 0;
  if (int rc = persistent_grid(s, &grid, &dev)) return rc;
  if (int rc = allow_dynamic_lds(dev)) return rc;
  int64_t tpu = 0;
  if (int rc = wall_ticks_per_us(dev, &tpu)) return rc;
  const int64_t us = wait_timeout_us > 0 ? wait_timeout_us : 200000;  // default 0.2 s
  const uint64_t ticks = static_cast<uint64_t>(us) * static_cast<uint64_t>(tpu);
  uint32_t* sync = static_cast<uint32_t*>(workspace);
  const uint32_t need = static_cast<uint32_t>(2 * d_ff / kBN + extra_ready_needed);
  hipLaunchKernelGGL(grouped_swiglu_fused, dim3(grid), dim3(kThreads), 2 * kStageBytes, s,
                     static_cast<const uint8_t*>(x), static_cast<const uint8_t*>(w_gate_up_packed),
                     static_cast<const uint8_t*>(w_down_packed), offsets, n_experts, d_model, d_ff,
                     static_cast<uint16_t*>(h), static_cast<uint16_t*>(ys), perm_src, top_k,
                     static_cast<int>(tokens), sync, need, ticks);
  return check_launch(what);
}

// ---- backward (the VJP of moe.py:70-74) -------------------------------------

extern "C" int hmoe_grouped_gate_up_raw_gather(const void* x, int64_t tokens, int top_k,
                                               const int32_t* perm_src, const int32_t* offsets,
                                               int n_experts, int64_t rows_cap, int d_model,
                                               int d_ff, const void* w_gate_up_packed, void* gu,
                                               hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= kMaxExperts,
               "grouped_gate_up_raw_gather: n_experts must be in [1, %d] (got %d)", kMaxExperts,
               n_experts);
  HMOE_REQUIRE(rows_cap >= 0 && tokens >= 0 && top_k >= 1 && (tokens >= 1 || rows_cap == 0),
               "grouped_gate_up_raw_gather: need rows_cap >= 0, tokens >= 0, top_k >= 1 (tokens >= 1 with rows)");
  HMOE_REQUIRE_CODE(d_model % kBK == 0 && d_model >= kBK, HMOE_ERR_UNSUPPORTED,
                    "grouped_gate_up_raw_gather: d_model must be a multiple of %d (got %d)", kBK,
                    d_model);
  HMOE_REQUIRE_CODE((2 * d_ff) % kBN == 0 && d_ff > 0, HMOE_ERR_UNSUPPORTED,
                    "grouped_gate_up_raw_gather: d_ff must be a multiple of %d (got %d)", kBN / 2,
                    d_ff);
  HMOE_REQUIRE(tokens * d_model * 2 < (int64_t(1) << 31),
               "grouped_gate_up_raw_gather: x must be smaller than 2 GiB");
  if (rows_cap == 0) return HMOE_OK;
  HMOE_REQUIRE(x && perm_src && offsets && w_gate_up_packed && gu,
               "grouped_gate_up_raw_gather: null pointer argument");
  return launch_grouped(false, false, x, w_gate_up_packed, nullptr, nullptr, offsets, n_experts,
                        rows_cap, d_model, 2 * d_ff, gu, 2 * d_ff, static_cast<hipStream_t>(stream),
                        "hmoe_grouped_gate_up_raw_gather", perm_src, top_k,
                        static_cast<int>(tokens));
}

extern "C" int hmoe_grouped_gate_up_raw(const void* xs, const int32_t* offsets, int n_experts,
                                        int64_t rows_cap, int d_model, int d_ff,
                                        const void* w_gate_up_packed, void* gu,
                                        hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= kMaxExperts,
               "grouped_gate_up_raw: n_experts must be in [1, %d] (got %d)", kMaxExperts, n_experts);
  HMOE_REQUIRE(rows_cap >= 0, "grouped_gate_up_raw: rows_cap must be >= 0");
  HMOE_REQUIRE_CODE(d_model % kBK == 0 && d_model >= kBK, HMOE_ERR_UNSUPPORTED,
                    "grouped_gate_up_raw: d_model must be a multiple of %d (got %d)", kBK, d_model);
  HMOE_REQUIRE_CODE((2 * d_ff) % kBN == 0 && d_ff > 0, HMOE_ERR_UNSUPPORTED,
                    "grouped_gate_up_raw: d_ff must be a multiple of %d (got %d)", kBN / 2, d_ff);
  if (rows_cap == 0) return HMOE_OK;
  HMOE_REQUIRE(xs && offsets && w_gate_up_packed && gu, "grouped_gate_up_raw: null pointer argument");
  return launch_grouped(false, false, xs, w_gate_up_packed, nullptr, nullptr, offsets, n_experts,
                        rows_cap, d_model, 2 * d_ff, gu, 2 * d_ff, static_cast<hipStream_t>(stream),
                        "hmoe_grouped_gate_up_raw");
}

extern "C" int hmoe_grouped_gate_up_swiglu_bwd_gather(
    const void* x, int64_t tokens, int top_k, const int32_t* perm_src, const int32_t* offsets,
    int n_experts, int64_t rows_cap, int d_model, int d_ff, const void* w_gate_up_packed,
    const void* dh, void* dgu, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= kMaxExperts,
               "grouped_gate_up_swiglu_bwd_gather: n_experts must be in [1, %d] (got %d)",
               kMaxExperts, n_experts);
  HMOE_REQUIRE(rows_cap >= 0 && tokens >= 0 && top_k >= 1 && (tokens >= 1 || rows_cap == 0),
               "grouped_gate_up_swiglu_bwd_gather: need rows_cap >= 0, tokens >= 0, top_k >= 1 (tokens >= 1 with rows)");
  HMOE_REQUIRE_CODE(d_model % kBK == 0 && d_model >= kBK, HMOE_ERR_UNSUPPORTED,
                    "grouped_gate_up_swiglu_bwd_gather: d_model must be a multiple of %d (got %d)",
                    kBK, d_model);
  HMOE_REQUIRE_CODE((2 * d_ff) % kBN == 0 && d_ff > 0, HMOE_ERR_UNSUPPORTED,
                    "grouped_gate_up_swiglu_bwd_gather: d_ff must be a multiple of %d (got %d)",
                    kBN / 2, d_ff);
  HMOE_REQUIRE(tokens * d_model * 2 < (int64_t(1) << 31),
               "grouped_gate_up_swiglu_bwd_gather: x must be smaller than 2 GiB");
  if (rows_cap == 0) return HMOE_OK;
  HMOE_REQUIRE(x && perm_src && offsets && w_gate_up_packed && dh && dgu,
               "grouped_gate_up_swiglu_bwd_gather: null pointer argument");
  return launch_grouped(false, false, x, w_gate_up_packed, nullptr, nullptr, offsets, n_experts,
                        rows_cap, d_model, 2 * d_ff, dgu, 2 * d_ff, static_cast<hipStream_t>(stream),
                        "hmoe_grouped_gate_up_swiglu_bwd_gather", perm_src, top_k,
                        static_cast<int>(tokens), static_cast<const uint16_t*>(dh));
}

extern "C" int hmoe_grouped_gate_up_swiglu_bwd(const void* xs, const int32_t* offsets,
                                               int n_experts, int64_t rows_cap, int d_model,
                                               int d_ff, const void* w_gate_up_packed,
                                               const void* dh, void* dgu, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= kMaxExperts,
               "grouped_gate_up_swiglu_bwd: n_experts must be in [1, %d] (got %d)", kMaxExperts,
               n_experts);
  HMOE_REQUIRE(rows_cap >= 0, "grouped_gate_up_swiglu_bwd: rows_cap must be >= 0");
  HMOE_REQUIRE_CODE(d_model % kBK == 0 && d_model >= kBK, HMOE_ERR_UNSUPPORTED,
                    "grouped_gate_up_swiglu_bwd: d_model must be a multiple of %d (got %d)", kBK,
                    d_model);
  HMOE_REQUIRE_CODE((2 * d_ff) % kBN == 0 && d_ff > 0, HMOE_ERR_UNSUPPORTED,
                    "grouped_gate_up_swiglu_bwd: d_ff must be a multiple of %d (got %d)", kBN / 2,
                    d_ff);
  if (rows_cap == 0) return HMOE_OK;
  HMOE_REQUIRE(xs && offsets && w_gate_up_packed && dh && dgu,
               "grouped_gate_up_swiglu_bwd: null pointer argument");
  return launch_grouped(false, false, xs, w_gate_up_packed, nullptr, nullptr, offsets, n_experts,
                        rows_cap, d_model, 2 * d_ff, dgu, 2 * d_ff, static_cast<hipStream_t>(stream),
                        "hmoe_grouped_gate_up_swiglu_bwd", nullptr, 1, 1,
                        static_cast<const uint16_t*>(dh));
}

extern "C" int hmoe_grouped_dgrad_down(const void* d_ys, const int32_t* offsets, int n_experts,
                                       int64_t rows_cap, int d_model, int d_ff,
                                       const void* w_down_dgrad, void* dh, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= kMaxExperts,
               "grouped_dgrad_down: n_experts must be in [1, %d] (got %d)", kMaxExperts, n_experts);
  HMOE_REQUIRE(rows_cap >= 0, "grouped_dgrad_down: rows_cap must be >= 0");
  HMOE_REQUIRE_CODE(d_model % kBK == 0 && d_model >= kBK, HMOE_ERR_UNSUPPORTED,
                    "grouped_dgrad_down: d_model must be a multiple of %d (got %d)", kBK, d_model);
  HMOE_REQUIRE_CODE(d_ff % kBN == 0 && d_ff > 0, HMOE_ERR_UNSUPPORTED,
                    "grouped_dgrad_down: d_ff must be a multiple of %d (got %d)", kBN, d_ff);
  if (rows_cap == 0) return HMOE_OK;
  HMOE_REQUIRE(d_ys && offsets && w_down_dgrad && dh, "grouped_dgrad_down: null pointer argument");
  return launch_grouped(false, false, d_ys, w_down_dgrad, nullptr, nullptr, offsets, n_experts,
                        rows_cap, d_model, d_ff, dh, d_ff, static_cast<hipStream_t>(stream),
                        "hmoe_grouped_dgrad_down");
}

extern "C" int hmoe_grouped_dgrad_gate_up(const void* dgu, const int32_t* offsets, int n_experts,
                                          int64_t rows_cap, int d_model, int d_ff,
                                          const void* w_gate_up_dgrad, void* d_xs,
                                          hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= kMaxExperts,
               "grouped_dgrad_gate_up: n_experts must be in [1, %d] (got %d)", kMaxExperts,
               n_experts);
  HMOE_REQUIRE(rows_cap >= 0, "grouped_dgrad_gate_up: rows_cap must be >= 0");
  HMOE_REQUIRE_CODE(d_ff % (kBK / 2) == 0 && d_ff > 0, HMOE_ERR_UNSUPPORTED,
                    "grouped_dgrad_gate_up: d_ff must be a multiple of %d (got %d)", kBK / 2, d_ff);
  HMOE_REQUIRE_CODE(d_model % kBN == 0 && d_model > 0, HMOE_ERR_UNSUPPORTED,
                    "grouped_dgrad_gate_up: d_model must be a multiple of %d (got %d)", kBN,
                    d_model);
  if (rows_cap == 0) return HMOE_OK;
  HMOE_REQUIRE(dgu && offsets && w_gate_up_dgrad && d_xs,
               "grouped_dgrad_gate_up: null pointer argument");
  return launch_grouped(false, false, dgu, w_gate_up_dgrad, nullptr, nullptr, offsets, n_experts,
                        rows_cap, 2 * d_ff, d_model, d_xs, d_model,
                        static_cast<hipStream_t>(stream), "hmoe_grouped_dgrad_gate_up");
}

namespace hmoe {
namespace {

// The e4m3 gate/up GEMM, plain (perm_src null: A holds the dispatched rows)
// or gathering (A holds per-token rows, row r is token perm_src[r] / top_k),
// with bf16 h (h_exp null) or block-scaled e4m3 h (codes into h, exponents
// into h_exp).
int gate_up_fp8(const char* what, const uint8_t* x_q, const float* x_scale, int64_t tokens,
                int top_k, const int32_t* perm_src, const int32_t* offsets, int n_experts,
                int64_t rows_cap, int d_model, int d_ff, const uint8_t* w_packed,
                const float* w_scales, void* h, uint8_t* h_exp, hipStream_t stream) {
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= kMaxExperts,
               "%s: n_experts must be in [1, %d] (got %d)", what, kMaxExperts, n_experts);
  HMOE_REQUIRE(rows_cap >= 0, "%s: rows_cap must be >= 0", what);
  if (perm_src != nullptr || tokens >= 0)
    HMOE_REQUIRE(tokens >= 0 && top_k >= 1 && (tokens >= 1 || rows_cap == 0),
                 "%s: need rows_cap >= 0, tokens >= 0, top_k >= 1 (tokens >= 1 with rows)", what);
  HMOE_REQUIRE_CODE(d_model % 128 == 0 && d_model >= 128, HMOE_ERR_UNSUPPORTED,
                    "%s: d_model must be a multiple of 128 (got %d)", what, d_model);
  HMOE_REQUIRE_CODE((2 * d_ff) % kBN == 0 && d_ff > 0, HMOE_ERR_UNSUPPORTED,
                    "%s: d_ff must be a multiple of %d (got %d)", what, kBN / 2, d_ff);
  if (tokens >= 0)
    HMOE_REQUIRE(tokens * d_model < (int64_t(1) << 31), "%s: x_q must be smaller than 2 GiB", what);
  if (rows_cap == 0) return HMOE_OK;
  HMOE_REQUIRE(x_q && x_scale && offsets && w_packed && w_scales && h, "%s: null pointer argument",
               what);
  HMOE_REQUIRE(tokens < 0 || perm_src != nullptr, "%s: null pointer argument", what);
  return launch_grouped(true, true, x_q, w_packed, x_scale, w_scales, offsets, n_experts, rows_cap,
                        d_model, 2 * d_ff, h, d_ff, stream, what, perm_src, top_k,
                        tokens >= 0 ? static_cast<int>(tokens) : 1, nullptr, h_exp);
}

// The e4m3 down GEMM on h with one float32 scale per row (h_scale) or one
// power-of-two scale per 32 columns (h_exp, biased exponents).
int down_fp8(const char* what, const uint8_t* h_q, const float* h_scale, const uint8_t* h_exp,
             const int32_t* offsets, int n_experts, int64_t rows_cap, int d_ff, int d_model,
             const uint8_t* w_packed, const float* w_scales, void* ys, hipStream_t stream) {
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= kMaxExperts,
               "%s: n_experts must be in [1, %d] (got %d)", what, kMaxExperts, n_experts);
  HMOE_REQUIRE(rows_cap >= 0, "%s: rows_cap must be >= 0", what);
  HMOE_REQUIRE_CODE(d_ff % 128 == 0 && d_ff >= 128, HMOE_ERR_UNSUPPORTED,
                    "%s: d_ff must be a multiple of 128 (got %d)", what, d_ff);
  HMOE_REQUIRE_CODE(d_model % kBN == 0 && d_model > 0, HMOE_ERR_UNSUPPORTED,
                    "%s: d_model must be a multiple of %d (got %d)", what, kBN, d_model);
  if (rows_cap == 0) return HMOE_OK;
  HMOE_REQUIRE(h_q && (h_scale || h_exp) && offsets && w_packed && w_scales && ys,
               "%s: null pointer argument", what);
  return launch_grouped(false, true, h_q, w_packed, h_scale, w_scales, offsets, n_experts, rows_cap,
                        d_ff, d_model, ys, d_model, stream, what, nullptr, 1, 1, nullptr,
                        const_cast<uint8_t*>(h_exp));
}

}  // namespace
}  // namespace hmoe

extern "C" int hmoe_grouped_gate_up_fp8(const uint8_t* xs_q, const float* xs_scale,
                                        const int32_t* offsets, int n_experts, int64_t rows_cap,
                                        int d_model, int d_ff, const uint8_t* w_packed,
                                        const float* w_scales, void* h, hmoe_stream_t stream) {
  return hmoe::gate_up_fp8("grouped_gate_up_fp8", xs_q, xs_scale, -1, 1, nullptr, offsets,
                           n_experts, rows_cap, d_model, d_ff, w_packed, w_scales, h, nullptr,
                           static_cast<hipStream_t>(stream));
}

extern "C" int hmoe_grouped_gate_up_fp8_gather(const uint8_t* x_q, const float* x_scale,
                                               int64_t tokens, int top_k, const int32_t* perm_src,
                                               const int32_t* offsets, int n_experts,
                                               int64_t rows_cap, int d_model, int d_ff,
                                               const uint8_t* w_packed, const float* w_scales,
                                               void* h, hmoe_stream_t stream) {
  if (tokens < 0) {
    hmoe::set_error("grouped_gate_up_fp8_gather: tokens must be >= 0 (got %lld)",
                    static_cast<long long>(tokens));
    return HMOE_ERR_INVALID;
  }
  return hmoe::gate_up_fp8("grouped_gate_up_fp8_gather", x_q, x_scale, tokens, top_k, perm_src,
                           offsets, n_experts, rows_cap, d_model, d_ff, w_packed, w_scales, h,
                           nullptr, static_cast<hipStream_t>(stream));
}

extern "C" int hmoe_grouped_gate_up_fp8_qh(const uint8_t* xs_q, const float* xs_scale,
                                           const int32_t* offsets, int n_experts, int64_t rows_cap,
                                           int d_model, int d_ff, const uint8_t* w_packed,
                                           const float* w_scales, uint8_t* h_q, uint8_t* h_exp,
                                           hmoe_stream_t stream) {
  if (rows_cap > 0 && h_exp == nullptr) {
    hmoe::set_error("grouped_gate_up_fp8_qh: null pointer argument");
    return HMOE_ERR_INVALID;
  }
  return hmoe::gate_up_fp8("grouped_gate_up_fp8_qh", xs_q, xs_scale, -1, 1, nullptr, offsets,
                           n_experts, rows_cap, d_model, d_ff, w_packed, w_scales, h_q, h_exp,
                           static_cast<hipStream_t>(stream));
}

extern "C" int hmoe_grouped_gate_up_fp8_gather_qh(const uint8_t* x_q, const float* x_scale,
                                                  int64_t tokens, int top_k,
                                                  const int32_t* perm_src, const int32_t* offsets,
                                                  int n_experts, int64_t rows_cap, int d_model,
                                                  int d_ff, const uint8_t* w_packed,
                                                  const float* w_scales, uint8_t* h_q,
                                                  uint8_t* h_exp, hmoe_stream_t stream) {
  if (tokens < 0 || (rows_cap > 0 && h_exp == nullptr)) {
    hmoe::set_error("grouped_gate_up_fp8_gather_qh: need tokens >= 0 and a non-null h_exp");
    return HMOE_ERR_INVALID;
  }
  return hmoe::gate_up_fp8("grouped_gate_up_fp8_gather_qh", x_q, x_scale, tokens, top_k, perm_src,
                           offsets, n_experts, rows_cap, d_model, d_ff, w_packed, w_scales, h_q,
                           h_exp, static_cast<hipStream_t>(stream));
}

extern "C" int hmoe_grouped_down_fp8(const uint8_t* h_q, const float* h_scale,
                                     const int32_t* offsets, int n_experts, int64_t rows_cap,
                                     int d_ff, int d_model, const uint8_t* w_packed,
                                     const float* w_scales, void* ys, hmoe_stream_t stream) {
  if (rows_cap > 0 && h_scale == nullptr) {
    hmoe::set_error("grouped_down_fp8: null pointer argument");
    return HMOE_ERR_INVALID;
  }
  return hmoe::down_fp8("grouped_down_fp8", h_q, h_scale, nullptr, offsets, n_experts, rows_cap,
                        d_ff, d_model, w_packed, w_scales, ys, static_cast<hipStream_t>(stream));
}

extern "C" int hmoe_grouped_down_fp8_mx(const uint8_t* h_q, const uint8_t* h_exp,
                                        const int32_t* offsets, int n_experts, int64_t rows_cap,
                                        int d_ff, int d_model, const uint8_t* w_packed,
                                        const float* w_scales, void* ys, hmoe_stream_t stream) {
  if (rows_cap > 0 && h_exp == nullptr) {
    hmoe::set_error("grouped_down_fp8_mx: null pointer argument");
    return HMOE_ERR_INVALID;
  }
  return hmoe::down_fp8("grouped_down_fp8_mx", h_q, nullptr, h_exp, offsets, n_experts, rows_cap,
                        d_ff, d_model, w_packed, w_scales, ys, static_cast<hipStream_t>(stream));
}

// ---- backward weight gradients (the VJP of moe.py:70-73 w.r.t. the weights) --

namespace hmoe {
namespace {
int launch_wgrad(bool split, const void* A, const void* B, const int32_t* offsets, int n_experts,
                 int64_t rows_cap, int M, int N, float* out0, float* out1, hipStream_t s,
                 const char* what) {
  HMOE_REQUIRE(static_cast<int64_t>(64) * (M > N ? M : N) * 2 < (int64_t(1) << 31),
               "%s: rows too wide", what);
  HMOE_REQUIRE(static_cast<int64_t>(n_experts) * (M / kBM) * (N / kBN) < (int64_t(1) << 31),
               "%s: too many tiles", what);
  int dev = 0;
  int grid = 0;
  if (int rc = persistent_grid(s, &grid, &dev)) return rc;
  if (int rc = allow_dynamic_lds(dev)) return rc;
  const size_t lds = 2 * kStageBytes;
  const uint16_t* a = static_cast<const uint16_t*>(A);
  const uint16_t* b = static_cast<const uint16_t*>(B);
  // A segment holds at most rows_cap rows and a tile reads up to 127 rows past
  // it (its padding steps); below 2 GiB for that the per-tile resources hold.
  const int64_t max_row_bytes = 2 * static_cast<int64_t>(M > N ? M : N);
  const bool big = (rows_cap + 128) * max_row_bytes >= (int64_t(1) << 31);
#define HMOE_LAUNCH_WGRAD(SP, BG)                                                               \
  hipLaunchKernelGGL((grouped_gemm_wgrad<SP, BG>), dim3(grid), dim3(kThreads), lds, s, a, b,     \
                     offsets, n_experts, M, N, out0, out1)
  if (split && big) HMOE_LAUNCH_WGRAD(true, true);
  else if (split) HMOE_LAUNCH_WGRAD(true, false);
  else if (big) HMOE_LAUNCH_WGRAD(false, true);
  else HMOE_LAUNCH_WGRAD(false, false);
#undef HMOE_LAUNCH_WGRAD
  return check_launch(what);
}
}  // namespace
}  // namespace hmoe

extern "C" int hmoe_grouped_wgrad_down(const void* h, const void* d_ys, const int32_t* offsets,
                                       int n_experts, int64_t rows_cap, int d_ff, int d_model,
                                       float* dw_down, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= kMaxExperts,
               "grouped_wgrad_down: n_experts must be in [1, %d] (got %d)", kMaxExperts, n_experts);
  HMOE_REQUIRE_CODE(d_ff % kBM == 0 && d_ff > 0 && d_model % kBN == 0 && d_model > 0,
                    HMOE_ERR_UNSUPPORTED,
                    "grouped_wgrad_down: d_ff and d_model must be multiples of 256 (got %d, %d)",
                    d_ff, d_model);
  HMOE_REQUIRE(rows_cap >= 0 && rows_cap < (int64_t(1) << 31),
               "grouped_wgrad_down: rows_cap must fit in int32");
  HMOE_REQUIRE(h && d_ys && offsets && dw_down, "grouped_wgrad_down: null pointer argument");
  return launch_wgrad(false, h, d_ys, offsets, n_experts, rows_cap, d_ff, d_model, dw_down,
                      nullptr, static_cast<hipStream_t>(stream), "hmoe_grouped_wgrad_down");
}

extern "C" int hmoe_grouped_wgrad_gate_up(const void* xs, const void* dgu, const int32_t* offsets,
                                          int n_experts, int64_t rows_cap, int d_model, int d_ff,
                                          float* dw_gate, float* dw_up, hmoe_stream_t stream) {
  using namespace hmoe;
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= kMaxExperts,
               "grouped_wgrad_gate_up: n_experts must be in [1, %d] (got %d)", kMaxExperts,
               n_experts);
  HMOE_REQUIRE_CODE(d_model % kBM == 0 && d_model > 0 && (2 * d_ff) % kBN == 0 && d_ff > 0,
                    HMOE_ERR_UNSUPPORTED,
                    "grouped_wgrad_gate_up: d_model must be a multiple of 256 and d_ff of 128 "
                    "(got %d, %d)", d_model, d_ff);
  HMOE_REQUIRE(rows_cap >= 0 && rows_cap < (int64_t(1) << 31),
               "grouped_wgrad_gate_up: rows_cap must fit in int32");
  HMOE_REQUIRE(xs && dgu && offsets && dw_gate && dw_up,
               "grouped_wgrad_gate_up: null pointer argument");
  return launch_wgrad(true, xs, dgu, offsets, n_experts, rows_cap, d_model, 2 * d_ff, dw_gate,
                      dw_up, static_cast<hipStream_t>(stream), "hmoe_grouped_wgrad_gate_up");
}
