// Router: fp32 logits, top-k selection and gate weights (model/moe.py:175-192).
//
// Logits are float32 roundings of float64 sums taken in ascending d from +0.0
// (see router_kernel for how the float64 matrix cores keep that order).
// Top-k is K rounds of a max over the totalOrder keys that resolves equal
// keys to the lower expert index: up to 64 experts eight tokens per wave (8
// lanes per token, 64-bit (key, expert) composites, select_group8); beyond,
// one token per wave (a wave-wide max, then a ballot of the lanes at the
// maximum whose lowest expert wins, select_and_gate).
#include <atomic>

#include "hmoe_common.h"
#include "quant_e4m3.h"

namespace hmoe {
namespace {

typedef double f64x4 __attribute__((ext_vector_type(4)));

// max(v, v of the lane DPP control CTRL names), in the rows ROW_MASK enables
// (other lanes keep v).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ int32_t dpp_max_i32(int32_t v) {
  const int32_t t = ROW_MASK == 0xF ? __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false)
                                    : __builtin_amdgcn_update_dpp(v, v, CTRL, ROW_MASK, 0xF, false);
  return t > v ? t : v;
}

// Wave-wide maxima of NTOK independent values, returned in every lane, on
// the VALU (data-parallel-primitive moves instead of LDS permutes): within
// each row of 16 lanes quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror
// and row_mirror leave the row's maximum in all its lanes; row_bcast15 into
// rows 1 and 3 and row_bcast31 into rows 2 and 3 bring the wave's maximum to
// lane 63, which is read out.
template <int NTOK>
__device__ __forceinline__ void wave_max_i32(int32_t (&v)[NTOK]) {
#pragma unroll
  for (int q = 0; q < NTOK; ++q) v[q] = dpp_max_i32<0xB1>(v[q]);
#pragma unroll
  for (int q = 0; q < NTOK; ++q) v[q] = dpp_max_i32<0x4E>(v[q]);
#pragma unroll
  for (int q = 0; q < NTOK; ++q) v[q] = dpp_max_i32<0x141>(v[q]);
#pragma unroll
  for (int q = 0; q < NTOK; ++q) v[q] = dpp_max_i32<0x140>(v[q]);
#pragma unroll
  for (int q = 0; q < NTOK; ++q) v[q] = dpp_max_i32<0x142, 0xA>(v[q]);
#pragma unroll
  for (int q = 0; q < NTOK; ++q) v[q] = dpp_max_i32<0x143, 0xC>(v[q]);
#pragma unroll
  for (int q = 0; q < NTOK; ++q) v[q] = __builtin_amdgcn_readlane(v[q], 63);
}

// Selection + gates for NTOK tokens whose logits are spread over the wave
// (lane owns experts lane + 64*j); the tokens' reduction chains interleave.
// Round k takes the wave maximum of the live totalOrder keys, then the
// lowest expert holding it: the first j (ascending) whose ballot of live
// entries at the maximum is non-empty, and that ballot's lowest lane -- the
// lower-index tie-break of lax.top_k.  The winner's value is read from its
// lane, and the gate denominators are summed from those values in k order.
// Lane k < K writes slot k of every token q with store[q].
template <int EPL, int NTOK>
__device__ __forceinline__ void select_and_gate(const float (&logit)[NTOK][EPL],
                                                const bool (&store)[NTOK],
                                                const float* __restrict__ bias, int n_experts,
                                                int top_k, int mode, float rsf,
                                                int32_t* const (&top_idx_row)[NTOK],
                                                float* const (&gates_row)[NTOK]) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  constexpr int32_t kDead = INT32_MIN;
  float val[NTOK][EPL];  // value the gate is built from: sigmoid score or logit
  int32_t key[NTOK][EPL];
  uint64_t dead[NTOK][EPL];  // lanes whose entry j is retired or past n_experts (uniform)
#pragma unroll
  for (int q = 0; q < NTOK; ++q)
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int e = lane + 64 * j;
      float kf = logit[q][j];
      if (mode == HMOE_ROUTE_SIGMOID_BIAS) {
        const float sg = sigmoid_det(logit[q][j]);
        val[q][j] = sg;
        kf = sg + ((bias != nullptr && e < n_experts) ? bias[e] : 0.0f);
      } else {
        val[q][j] = logit[q][j];
      }
      key[q][j] = e < n_experts ? total_order_key(kf) : kDead;
      dead[q][j] = __builtin_amdgcn_ballot_w64(e >= n_experts);
    }
  int my_e[NTOK];
  float my_v[NTOK], denom[NTOK], vmax[NTOK];
#pragma unroll
  for (int q = 0; q < NTOK; ++q) {
    my_e[q] = 0;
    my_v[q] = 0.0f;
    denom[q] = 0.0f;
    vmax[q] = 0.0f;
  }
  for (int k = 0; k < top_k; ++k) {
    int32_t best[NTOK];
#pragma unroll
    for (int q = 0; q < NTOK; ++q) {
      best[q] = key[q][0];
#pragma unroll
      for (int j = 1; j < EPL; ++j) best[q] = key[q][j] > best[q] ? key[q][j] : best[q];
    }
    wave_max_i32<NTOK>(best);
#pragma unroll
    for (int q = 0; q < NTOK; ++q) {
      uint64_t mask = 0;
      int jw = 0;
#pragma unroll
      for (int j = 0; j < EPL; ++j) {
        const uint64_t mj = __builtin_amdgcn_ballot_w64(key[q][j] == best[q]) & ~dead[q][j];
        if (mask == 0 && mj != 0) {
          mask = mj;
          jw = j;
        }
      }
      // mask is non-empty: top_k <= n_experts keeps a live entry at the maximum
      const int lw = __builtin_ctzll(mask);
      float v_win = 0.0f;
#pragma unroll
      for (int j = 0; j < EPL; ++j) {
        if (j == jw) {
          v_win = lane_bcast(val[q][j], lw);
          if (lane == lw) key[q][j] = kDead;
          dead[q][j] |= 1ull << lw;
        }
      }
      if (lane == k) {
        my_e[q] = lw + 64 * jw;
        my_v[q] = v_win;
      }
      if (mode == HMOE_ROUTE_SIGMOID_BIAS) denom[q] = denom[q] + v_win;
      else if (k == 0) vmax[q] = v_win;
    }
  }
#pragma unroll
  for (int q = 0; q < NTOK; ++q) {
    float w;
    if (mode == HMOE_ROUTE_SIGMOID_BIAS) {
      w = (my_v[q] / (denom[q] + 1e-9f)) * rsf;
    } else {
      // exp of each slot in its lane, summed in k order
      const float ex = exp_det(my_v[q] - vmax[q]);
      for (int k = 0; k < top_k; ++k) denom[q] = denom[q] + lane_bcast(ex, k);
      w = ex / denom[q];
    }
    if (store[q] && lane < top_k) {
      top_idx_row[q][lane] = my_e[q];
      gates_row[q][lane] = w;
    }
  }
}

// One stage of a max over each aligned group of 8 lanes of a (64-bit key,
// value) pair: the pair of the lane the DPP control CTRL names replaces this
// lane's if its key is larger.  quad_perm [1,0,3,2], then [2,3,0,1], then
// row_half_mirror leave the group's largest pair in all 8 lanes.
template <int CTRL>
__device__ __forceinline__ void dpp_max_kv(int64_t& k, float& v) {
  const int32_t lo = __builtin_amdgcn_mov_dpp(static_cast<int32_t>(k), CTRL, 0xF, 0xF, false);
  const int32_t hi = __builtin_amdgcn_mov_dpp(static_cast<int32_t>(k >> 32), CTRL, 0xF, 0xF, false);
  const int32_t vv = __builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false);
  const int64_t t = static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                                         static_cast<uint32_t>(lo));
  if (t > k) {
    k = t;
    v = __int_as_float(vv);
  }
}

// Selection + gates for 8 tokens per wave: lane group g = lane / 8 takes one
// token, lane p = lane % 8 of the group its experts p*E .. p*E + E - 1.  Every
// entry is a 64-bit composite, the totalOrder key in the high bits above
// 0xFFFF - expert, so the larger composite is the larger key and on equal
// keys the lower expert (the lax.top_k order); retired entries and those past
// n_experts hold INT64_MIN, below every live one.  Round k: each lane's
// largest entry, then the group's largest (three DPP stages, carrying the
// entry's value); the lane that holds it retires it.  Lane p records slots
// p, p + 8, p + 16, p + 24; the gate denominators are summed in k order.
template <int E>
__device__ __forceinline__ void select_group8(const float (&logit)[E], bool store,
                                              const float* __restrict__ bias, int n_experts,
                                              int top_k, int mode, float rsf,
                                              int32_t* __restrict__ top_idx_row,
                                              float* __restrict__ gates_row) {
#pragma clang fp contract(off)
  const int p = threadIdx.x & 7;
  constexpr int64_t kGone = INT64_MIN;
  int64_t ck[E];
  float val[E];  // value the gate is built from: sigmoid score or logit
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const int e = p * E + j;
    float kf = logit[j];
    if (mode == HMOE_ROUTE_SIGMOID_BIAS) {
      const float sg = sigmoid_det(logit[j]);
      val[j] = sg;
      kf = sg + ((bias != nullptr && e < n_experts) ? bias[e] : 0.0f);
    } else {
      val[j] = logit[j];
    }
    const uint64_t key = static_cast<uint64_t>(static_cast<int64_t>(total_order_key(kf)));
    ck[j] = e < n_experts ? static_cast<int64_t>((key << 16) | static_cast<uint64_t>(0xFFFF - e)) : kGone;
  }
  int my_e[4] = {0, 0, 0, 0};
  float my_v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  float denom = 0.0f, vmax = 0.0f;
  for (int k = 0; k < top_k; ++k) {
    int64_t best = ck[0];
    float bv = val[0];
    int barg = 0;
#pragma unroll
    for (int j = 1; j < E; ++j) {
      if (ck[j] > best) {
        best = ck[j];
        bv = val[j];
        barg = j;
      }
    }
    int64_t gb = best;
    float gv = bv;
    dpp_max_kv<0xB1>(gb, gv);
    dpp_max_kv<0x4E>(gb, gv);
    dpp_max_kv<0x141>(gb, gv);
    // composites are unique, so exactly one lane of the group holds gb
    const bool owner = gb == best;
#pragma unroll
    for (int j = 0; j < E; ++j)
      if (owner && barg == j) ck[j] = kGone;
    const int w = 0xFFFF - static_cast<int>(gb & 0xFFFF);
    float rec = gv;
    if (mode == HMOE_ROUTE_SIGMOID_BIAS) {
      denom = denom + gv;
    } else {
      if (k == 0) vmax = gv;
      rec = exp_det(gv - vmax);
      denom = denom + rec;
    }
    if ((k & 7) == p) {
      const int r = k >> 3;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (q == r) {
          my_e[q] = w;
          my_v[q] = rec;
        }
    }
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int k = 8 * q + p;
    if (store && k < top_k) {
      top_idx_row[k] = my_e[q];
      gates_row[k] = mode == HMOE_ROUTE_SIGMOID_BIAS ? (my_v[q] / (denom + 1e-9f)) * rsf
                                                     : my_v[q] / denom;
    }
  }
}

// Eight consecutive activations as raw bits (one or two 16-byte loads; the
// address must be 16-byte aligned), widened to float32 later.
template <typename XT>
struct X8;
template <>
struct X8<float> {
  f32x4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = *reinterpret_cast<const f32x4*>(p);
    b = *reinterpret_cast<const f32x4*>(p + 4);
  }
  __device__ __forceinline__ float get(int i) const { return i < 4 ? a[i] : b[i - 4]; }
};
template <>
struct X8<uint16_t> {
  u32x4 v;
  __device__ __forceinline__ void load(const uint16_t* p) { v = *reinterpret_cast<const u32x4*>(p); }
  __device__ __forceinline__ float get(int i) const {
    const uint32_t u = v[i >> 1];
    return __uint_as_float((i & 1) ? (u & 0xffff0000u) : (u << 16));
  }
};
template <typename WT>
__device__ __forceinline__ float load_w_f32(const WT* p, int64_t i);
template <>
__device__ __forceinline__ float load_w_f32<float>(const float* p, int64_t i) {
  return p[i];
}
template <>
__device__ __forceinline__ float load_w_f32<uint16_t>(const uint16_t* p, int64_t i) {
  return bf16_bits_to_f32(p[i]);
}

// Logits on the float64 matrix cores.  v_mfma_f64_16x16x4f64 computes
// D = C + A[:,0]B[0,:] + ... + A[:,3]B[3,:] with the additions done one after
// another in k order, each rounded to float64 (C first); the products of
// bf16/fp32 activations and fp32/bf16 weights are exact in float64.  Walking d
// upwards four at a time from C = +0.0 therefore reproduces the sequential
// d-ascending float64 sum bit for bit.  Operand layout: A[i][k] in lane
// i + 16k, B[k][j] in lane j + 16k; D[i][j] in lane j + 16*(i%4), register i/4.
//
// A workgroup of 4 waves takes 64 tokens; each wave 16 tokens against all
// experts (NT tiles of 16 experts, zero-padded past n_experts).  x and W are
// staged in LDS as float32, a chunk of d at a time (router_dc), double-buffered through registers
// (the next chunk's global loads are issued before the current chunk's
// MFMAs).  The float32-rounded logits go through LDS to the wave-per-token
// selection.
template <int V>
struct IntC {
  static constexpr int value = V;
};

constexpr int kRTokWave = 16;
// d per LDS chunk (one barrier per chunk): as many as keep the staging
// within one 8-wave workgroup per CU (up to 64 experts: 128 d, 141 KB) or two
// 4-wave ones (up to 32 experts: 128 d; up to 64: 64 d), 32 beyond.  Halving
// the barriers took 1.5-2 us off 62-93 us.  The scalar W staging (WV false)
// keeps 64 d, whose registers 128 d would spill.
constexpr int router_dc(int nt, int nw, bool wv) {
  return wv && (nt <= 2 || (nt <= 4 && nw == 8)) ? 128 : (nt <= 4 ? 64 : 32);
}

// ES waves share a group of 16 tokens and split its expert tiles, so a
// workgroup of NW waves takes 16 NW / ES tokens.  With ES = 2 two waves run
// on every SIMD and each keeps NT/2 independent accumulator chains.
template <int NT, int ES, int NW, bool WV = true>
struct alignas(16) RouterLds {
  static constexpr int kNP = 16 * NT;
  static constexpr int kWPitch = kNP + 8;
  static constexpr int kTB = 16 * NW / ES;
  static constexpr int kDc = router_dc(NT, NW, WV);
  static constexpr int kXPitch = kDc + 4;  // 16-byte aligned rows
  float x[2][kTB][kXPitch];
  float w[2][kDc][kWPitch];
};

// WV: n_experts is a multiple of the W elements in 16 bytes, so a chunk of W
// (kRDc consecutive rows of n_experts values, contiguous in memory) is staged
// with 16-byte loads and LDS writes.
//
// QX: the launch also quantises x to e4m3 per token (the rule and code of
// hmoe_quantize_rows_fp8): workgroups past the first router_blocks take NW
// rows of x each, one wave per row.  They start once the router's workgroups
// are placed and run beside them, whose float64 MFMA chains leave the memory
// system and most of the VALU issue idle.
template <int NT, int ES, int NW, typename XT, typename WT, bool WV, bool QX = false>
__global__ __launch_bounds__(64 * NW) void router_kernel(const XT* __restrict__ x, const WT* __restrict__ w,
                                                     const float* __restrict__ bias, int64_t tokens,
                                                     int d_model, int n_experts, int top_k, int mode,
                                                     float rsf, float* __restrict__ logits,
                                                     int32_t* __restrict__ top_idx,
                                                     float* __restrict__ gates,
                                                     uint8_t* __restrict__ x_q,
                                                     float* __restrict__ x_scale, int router_blocks) {
  static_assert(NT % ES == 0, "expert tiles must split evenly");
  static_assert(!QX || sizeof(XT) == 2, "x is quantised from bf16");
  if constexpr (QX) {
    if (static_cast<int>(blockIdx.x) >= router_blocks) {
      const int64_t r = static_cast<int64_t>(static_cast<int>(blockIdx.x) - router_blocks) * NW +
                        (threadIdx.x >> 6);
      if (r < tokens) {
        const uint16_t* xr = reinterpret_cast<const uint16_t*>(x) + r * d_model;
        if (d_model <= 64 * kRowRegs * 8)
          quant_row_e4m3<true>(xr, d_model, x_q + r * d_model, x_scale + r);
        else
          quant_row_e4m3<false>(xr, d_model, x_q + r * d_model, x_scale + r);
      }
      return;
    }
  }
  constexpr int kThr = 64 * NW;
  constexpr int kNP = RouterLds<NT, ES, NW, WV>::kNP;
  constexpr int kTB = RouterLds<NT, ES, NW, WV>::kTB;
  constexpr int kRDc = RouterLds<NT, ES, NW, WV>::kDc;
  constexpr int kTG = kTB / kRTokWave;                // token groups per workgroup
  constexpr int kNTW = NT / ES;                       // expert tiles per wave
  constexpr int kEPL = (kNP + 63) / 64;
  constexpr int kWPer = (kRDc * kNP + kThr - 1) / kThr;  // w elements per thread per chunk
  constexpr int kE16 = 16 / static_cast<int>(sizeof(WT));  // W elements per 16-byte load
  constexpr int kWV = (kRDc * kNP / kE16 + kThr - 1) / kThr;  // 16-byte W loads per thread per chunk
  __shared__ RouterLds<NT, ES, NW, WV> lds;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int tg = wave % kTG;
  const int ep = wave / kTG;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kTB;

  // Staging assignment: x elements (tt, dd..dd+7) = (g / kXT, (g % kXT) * 8) for
  // the groups g = tid + kThr r < kXT*kTB (kXT = kRDc / 8 groups per token
  // row).  d_model is a multiple of 8, so a group of 8 is wholly inside or
  // outside the row.  Every load is unconditional from an
  // in-range address (clamped token row, d or expert 0) and masked
  // afterwards, so the loads of a chunk stay in flight together until they
  // are parked in LDS.
  constexpr int kXT = kRDc / 8;
  constexpr int kXR = (kXT * kTB + kThr - 1) / kThr;  // x groups per thread
  int xs_tt[kXR], xs_dd[kXR];
  bool x_thread[kXR];
  int64_t xs_row[kXR];
#pragma unroll
  for (int r = 0; r < kXR; ++r) {
    const int g = tid + kThr * r;
    xs_tt[r] = g / kXT;
    x_thread[r] = xs_tt[r] < kTB;
    xs_dd[r] = (g % kXT) * 8;
    const int64_t tok = t0 + (x_thread[r] ? xs_tt[r] : 0);
    xs_row[r] = (tok < tokens ? tok : tokens - 1) * static_cast<int64_t>(d_model);
  }
  // Two register sets: the loads of chunk c + 2 are issued at the start of
  // chunk c, so a load has two chunks of MFMAs to arrive before it is parked.
  X8<XT> xr0[kXR], xr1[kXR];
  // W staging registers: kWPer scalars, or kWV 16-byte vectors (WV).
  constexpr int kWRegs = WV ? 4 * kWV : kWPer;
  uint32_t wr0[kWRegs], wr1[kWRegs];
  auto w_ok = [&](int q, int d0) __attribute__((always_inline)) {
    const int idx = q * kThr + tid;
    return idx < kRDc * kNP && idx % kNP < n_experts && d0 + idx / kNP < d_model;
  };
  // WV: vector q covers elements idx .. idx + kE16 - 1 (idx = (q*kThr + tid) *
  // kE16) of the chunk, i.e. row idx / n_experts, experts idx % n_experts ...
  auto wv_idx = [&](int q) __attribute__((always_inline)) { return (q * kThr + tid) * kE16; };
  auto fetch = [&](X8<XT>* xr, uint32_t* wr, int d0) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < kXR; ++r) {
      const int dx = d0 + xs_dd[r];
      xr[r].load(x + xs_row[r] + (dx < d_model ? dx : 0));
    }
    if (WV) {
#pragma unroll
      for (int q = 0; q < kWV; ++q) {
        const int idx = wv_idx(q);
        const bool ok = idx < kRDc * n_experts && d0 + idx / n_experts < d_model;
        const u32x4 v = *reinterpret_cast<const u32x4*>(
            w + (ok ? static_cast<int64_t>(d0) * n_experts + idx : 0));
#pragma unroll
        for (int j = 0; j < 4; ++j) wr[4 * q + j] = v[j];
      }
    } else {
#pragma unroll
      for (int q = 0; q < kWPer; ++q) {
        const int idx = q * kThr + tid;
        const int64_t off = static_cast<int64_t>(d0 + idx / kNP) * n_experts + idx % kNP;
        wr[q] = __float_as_uint(load_w_f32(w, w_ok(q, d0) ? off : 0));
      }
    }
    // Keep the loads ahead of the MFMAs; the masking happens in park().
    __builtin_amdgcn_sched_barrier(0);
  };
  auto park = [&](const X8<XT>* xr, const uint32_t* wr, int buf, int d0) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < kXR; ++r) {
      if (x_thread[r]) {
        const bool x_ok = d0 + xs_dd[r] < d_model;
        f32x4 lo, hi;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          lo[q] = x_ok ? xr[r].get(q) : 0.0f;
          hi[q] = x_ok ? xr[r].get(4 + q) : 0.0f;
        }
        *reinterpret_cast<f32x4*>(&lds.x[buf][xs_tt[r]][xs_dd[r]]) = lo;
        *reinterpret_cast<f32x4*>(&lds.x[buf][xs_tt[r]][xs_dd[r] + 4]) = hi;
      }
    }
    if (WV) {
#pragma unroll
      for (int q = 0; q < kWV; ++q) {
        const int idx = wv_idx(q);
        if (idx < kRDc * n_experts) {
          const int d = idx / n_experts;
          const int n = idx - d * n_experts;
          const bool ok = d0 + d < d_model;
          float* dst = &lds.w[buf][d][n];
          if (sizeof(WT) == 4) {
            f32x4 v;
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = ok ? __uint_as_float(wr[4 * q + j]) : 0.0f;
            *reinterpret_cast<f32x4*>(dst) = v;
          } else {
            f32x4 lo, hi;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              const uint32_t a = wr[4 * q + j], b = wr[4 * q + 2 + j];
              lo[2 * j] = ok ? __uint_as_float(a << 16) : 0.0f;
              lo[2 * j + 1] = ok ? __uint_as_float(a & 0xffff0000u) : 0.0f;
              hi[2 * j] = ok ? __uint_as_float(b << 16) : 0.0f;
              hi[2 * j + 1] = ok ? __uint_as_float(b & 0xffff0000u) : 0.0f;
            }
            *reinterpret_cast<f32x4*>(dst) = lo;
            *reinterpret_cast<f32x4*>(dst + 4) = hi;
          }
        }
      }
    } else {
#pragma unroll
      for (int q = 0; q < kWPer; ++q) {
        const int idx = q * kThr + tid;
        if (idx < kRDc * kNP) lds.w[buf][idx / kNP][idx % kNP] = w_ok(q, d0) ? __uint_as_float(wr[q]) : 0.0f;
      }
    }
  };
  if (WV && n_experts < kNP) {
    // Expert columns past n_experts are never written by the vector staging:
    // zero them once in both buffers.
    for (int i = tid; i < 2 * kRDc * kNP; i += kThr) {
      const int n = i % kNP;
      if (n >= n_experts) lds.w[i / (kRDc * kNP)][(i / kNP) % kRDc][n] = 0.0f;
    }
  }

  f64x4 acc[kNTW];
#pragma unroll
  for (int t = 0; t < kNTW; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[t][r] = 0.0;

  const int a_row = tg * kRTokWave + (lane & 15);
  const int k_of_lane = lane >> 4;
  const int col0 = ep * kNTW * 16 + (lane & 15);
  const int nchunks = (d_model + kRDc - 1) / kRDc;
  // Chunk c (S = c % 2): prefetch chunk c + 2 into register set S, run the
  // MFMAs on LDS buffer S, park chunk c + 1 (register set S ^ 1) into buffer
  // S ^ 1.
  auto chunk = [&](auto Sc, int c) __attribute__((always_inline)) {
    constexpr int S = decltype(Sc)::value;
    X8<XT>* xs_ld = S == 0 ? xr0 : xr1;
    uint32_t* ws_ld = S == 0 ? wr0 : wr1;
    const X8<XT>* xs_pk = S == 0 ? xr1 : xr0;
    const uint32_t* ws_pk = S == 0 ? wr1 : wr0;
    if (c + 2 < nchunks) fetch(xs_ld, ws_ld, (c + 2) * kRDc);
#pragma unroll
    for (int s = 0; s < kRDc / 4; ++s) {
      const double a = static_cast<double>(lds.x[S][a_row][4 * s + k_of_lane]);
#pragma unroll
      for (int t = 0; t < kNTW; ++t) {
        const double b = static_cast<double>(lds.w[S][4 * s + k_of_lane][col0 + t * 16]);
        acc[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, acc[t], 0, 0, 0);
      }
    }
    if (c + 1 < nchunks) park(xs_pk, ws_pk, S ^ 1, (c + 1) * kRDc);
    __syncthreads();
  };
  fetch(xr0, wr0, 0);
  if (nchunks > 1) fetch(xr1, wr1, kRDc);
  park(xr0, wr0, 0, 0);
  __syncthreads();
  for (int c = 0; c < nchunks; c += 2) {
    chunk(IntC<0>{}, c);
    if (c + 1 < nchunks) chunk(IntC<1>{}, c + 1);
  }

  // float32 logits into LDS, row = token of the workgroup, col = expert.
  float* lg = &lds.w[0][0][0];
  static_assert(sizeof(float) * kTB * kNP <= sizeof(lds.w), "logit staging does not fit");
#pragma unroll
  for (int t = 0; t < kNTW; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      lg[(tg * kRTokWave + (lane >> 4) + 4 * r) * kNP + col0 - (lane & 15) + t * 16 + (lane & 15)] =
          static_cast<float>(acc[t][r]);
  __syncthreads();

  if constexpr (NT <= 4) {
    // Selection: wave w takes tokens w*kTB/NW .. (w+1)*kTB/NW - 1 of the
    // workgroup, eight at a time (lane group lane / 8 one token).
    constexpr int kSel = kTB / NW;
    static_assert(kSel % 8 == 0, "selection takes tokens in groups of eight");
    constexpr int kE8 = kNP / 8;
    const int p8 = lane & 7;
#pragma unroll 1
    for (int i = 0; i < kSel; i += 8) {
      if (t0 + wave * kSel + i >= tokens) break;
      const int row = wave * kSel + i + (lane >> 3);
      const int64_t tok = t0 + row;
      const bool st = tok < tokens;
      const int64_t tq = st ? tok : tokens - 1;
      float l[kE8];
#pragma unroll
      for (int j = 0; j < kE8; ++j) {
        const int e = p8 * kE8 + j;
        l[j] = lg[row * kNP + e];
        if (st && e < n_experts) logits[tq * n_experts + e] = l[j];
      }
      select_group8<kE8>(l, st, bias, n_experts, top_k, mode, rsf, top_idx + tq * top_k,
                         gates + tq * top_k);
    }
  } else {
    // Selection: wave w takes tokens w*kTB/NW .. (w+1)*kTB/NW - 1 of the workgroup.
    constexpr int kSel = kTB / NW;
    static_assert(kSel % 2 == 0, "selection takes tokens in pairs");
#pragma unroll 1
    for (int i = 0; i < kSel; i += 2) {
      const int row = wave * kSel + i;
      const int64_t tok = t0 + row;
      if (tok >= tokens) break;
      float l[2][kEPL];
      bool st[2];
      int32_t* ti[2];
      float* gt[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        st[q] = tok + q < tokens;
        const int64_t tq = st[q] ? tok + q : tok;
        ti[q] = top_idx + tq * top_k;
        gt[q] = gates + tq * top_k;
#pragma unroll
        for (int j = 0; j < kEPL; ++j) {
          const int e = lane + 64 * j;
          l[q][j] = e < kNP ? lg[(row + q) * kNP + e] : 0.0f;
          if (st[q] && e < n_experts) logits[tq * n_experts + e] = l[q][j];
        }
      }
      select_and_gate<kEPL, 2>(l, st, bias, n_experts, top_k, mode, rsf, ti, gt);
    }
  }
}

// One wave per token: selection and gates from given logits.
// Tokens per wave (their reduction chains would interleave); one measured
// fastest once the reductions moved off the LDS permutes (4: 24.5 against
// 22.8 us at 32768 tokens, 64 experts, top-8).
constexpr int kSelTok = 1;

template <int EPL>
__global__ __launch_bounds__(256) void select_kernel(const float* __restrict__ logits,
                                                     const float* __restrict__ bias, int64_t tokens,
                                                     int n_experts, int top_k, int mode, float rsf,
                                                     int32_t* __restrict__ top_idx,
                                                     float* __restrict__ gates) {
  const int lane = threadIdx.x & 63;
  const int64_t tok0 = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * kSelTok;
  if (tok0 >= tokens) return;
  float l[kSelTok][EPL];
  bool st[kSelTok];
  int32_t* ti[kSelTok];
  float* gt[kSelTok];
#pragma unroll
  for (int q = 0; q < kSelTok; ++q) {
    st[q] = tok0 + q < tokens;
    const int64_t tq = st[q] ? tok0 + q : tok0;  // a token past the end repeats the first
    ti[q] = top_idx + tq * top_k;
    gt[q] = gates + tq * top_k;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int e = lane + 64 * j;
      l[q][j] = e < n_experts ? logits[tq * n_experts + e] : 0.0f;
    }
  }
  select_and_gate<EPL, kSelTok>(l, st, bias, n_experts, top_k, mode, rsf, ti, gt);
}

// Selection and gates from given logits for up to 64 experts, eight tokens
// per wave (lane group lane / 8 one token, lane p its experts 8p .. 8p + 7).
__global__ __launch_bounds__(256) void select_kernel_g8(const float* __restrict__ logits,
                                                        const float* __restrict__ bias,
                                                        int64_t tokens, int n_experts, int top_k,
                                                        int mode, float rsf,
                                                        int32_t* __restrict__ top_idx,
                                                        float* __restrict__ gates) {
  const int lane = threadIdx.x & 63;
  const int p = lane & 7;
  const int64_t tok0 = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * 8;
  if (tok0 >= tokens) return;  // uniform per wave
  const int64_t tok = tok0 + (lane >> 3);
  const bool st = tok < tokens;
  const int64_t tq = st ? tok : tokens - 1;
  float l[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int e = p * 8 + j;
    l[j] = e < n_experts ? logits[tq * n_experts + e] : 0.0f;
  }
  select_group8<8>(l, st, bias, n_experts, top_k, mode, rsf, top_idx + tq * top_k,
                   gates + tq * top_k);
}

// CU count of the stream's device (0 if it cannot be queried), cached per device.
int stream_cus(hipStream_t s) {
  int dev = 0;
  if (hipStreamGetDevice(s, &dev) != hipSuccess && hipGetDevice(&dev) != hipSuccess) return 0;
  static std::atomic<int> cached[64];
  int cus = dev >= 0 && dev < 64 ? cached[dev].load(std::memory_order_relaxed) : 0;
  if (cus == 0 && hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
      cus > 0 && dev >= 0 && dev < 64)
    cached[dev].store(cus, std::memory_order_relaxed);
  return cus > 0 ? cus : 0;
}

// Optional e4m3 quantisation of x in the router's launch (router_kernel QX).
struct XQuant {
  uint8_t* q = nullptr;
  float* scale = nullptr;
};

template <int NT, int NW, typename XT, typename WT>
void launch_router_nw(const void* x, const void* w, const float* bias, int64_t tokens,
                      int d_model, int n_experts, int top_k, int mode, float rsf, float* logits,
                      int32_t* top_idx, float* gates, hipStream_t stream, XQuant xq) {
  constexpr int ES = NT >= 2 ? 2 : 1;
  const int rblocks = static_cast<int>(ceil_div(tokens, RouterLds<NT, ES, NW>::kTB));
  const bool wv = n_experts % (16 / static_cast<int>(sizeof(WT))) == 0 &&
                  reinterpret_cast<uintptr_t>(w) % 16 == 0;
  if constexpr (sizeof(XT) == 2) {
    if (xq.q != nullptr) {
      const dim3 grid(static_cast<unsigned>(rblocks + ceil_div(tokens, NW)));
      if (wv)
        hipLaunchKernelGGL((router_kernel<NT, ES, NW, XT, WT, true, true>), grid, dim3(64 * NW), 0,
                           stream, static_cast<const XT*>(x), static_cast<const WT*>(w), bias,
                           tokens, d_model, n_experts, top_k, mode, rsf, logits, top_idx, gates,
                           xq.q, xq.scale, rblocks);
      else
        hipLaunchKernelGGL((router_kernel<NT, ES, NW, XT, WT, false, true>), grid, dim3(64 * NW), 0,
                           stream, static_cast<const XT*>(x), static_cast<const WT*>(w), bias,
                           tokens, d_model, n_experts, top_k, mode, rsf, logits, top_idx, gates,
                           xq.q, xq.scale, rblocks);
      return;
    }
  }
  const dim3 grid(static_cast<unsigned>(rblocks));
  if (wv)
    hipLaunchKernelGGL((router_kernel<NT, ES, NW, XT, WT, true>), grid, dim3(64 * NW), 0, stream,
                       static_cast<const XT*>(x), static_cast<const WT*>(w), bias, tokens, d_model,
                       n_experts, top_k, mode, rsf, logits, top_idx, gates, nullptr, nullptr,
                       rblocks);
  else
    hipLaunchKernelGGL((router_kernel<NT, ES, NW, XT, WT, false>), grid, dim3(64 * NW), 0, stream,
                       static_cast<const XT*>(x), static_cast<const WT*>(w), bias, tokens, d_model,
                       n_experts, top_k, mode, rsf, logits, top_idx, gates, nullptr, nullptr,
                       rblocks);
}

// From 64 experts up, workgroups of 8 waves (64 tokens) when they still give
// every CU one: they stage each chunk of W once for twice the tokens.
// Measured at 16384 tokens, d_model 2048, 64 experts: 112 -> 106 us; 65536
// tokens, 128 experts: 703 -> 637 us; at 8192 tokens (half the CUs) 8 waves
// were slower (72 -> 104 us), hence the token-count switch.
template <int NT, typename XT, typename WT>
void launch_router(const void* x, const void* w, const float* bias, int64_t tokens, int d_model,
                   int n_experts, int top_k, int mode, float rsf, float* logits, int32_t* top_idx,
                   float* gates, hipStream_t stream, XQuant xq) {
  if constexpr (NT >= 4) {
    const int cus = stream_cus(stream);
    if (cus > 0 && ceil_div(tokens, RouterLds<NT, 2, 8>::kTB) >= cus) {
      launch_router_nw<NT, 8, XT, WT>(x, w, bias, tokens, d_model, n_experts, top_k, mode, rsf,
                                      logits, top_idx, gates, stream, xq);
      return;
    }
  }
  launch_router_nw<NT, 4, XT, WT>(x, w, bias, tokens, d_model, n_experts, top_k, mode, rsf, logits,
                                  top_idx, gates, stream, xq);
}

template <int NT>
void dispatch_router(int x_dtype, int w_dtype, const void* x, const void* w, const float* bias,
                     int64_t tokens, int d_model, int n_experts, int top_k, int mode, float rsf,
                     float* logits, int32_t* top_idx, float* gates, hipStream_t s,
                     XQuant xq = XQuant()) {
  if (x_dtype == HMOE_BF16 && w_dtype == HMOE_F32)
    launch_router<NT, uint16_t, float>(x, w, bias, tokens, d_model, n_experts, top_k, mode, rsf, logits, top_idx, gates, s, xq);
  else if (x_dtype == HMOE_F32 && w_dtype == HMOE_F32)
    launch_router<NT, float, float>(x, w, bias, tokens, d_model, n_experts, top_k, mode, rsf, logits, top_idx, gates, s, xq);
  else if (x_dtype == HMOE_BF16 && w_dtype == HMOE_BF16)
    launch_router<NT, uint16_t, uint16_t>(x, w, bias, tokens, d_model, n_experts, top_k, mode, rsf, logits, top_idx, gates, s, xq);
  else
    launch_router<NT, float, uint16_t>(x, w, bias, tokens, d_model, n_experts, top_k, mode, rsf, logits, top_idx, gates, s, xq);
}

int validate_routing(int64_t tokens, int n_experts, int top_k, int mode) {
  HMOE_REQUIRE(tokens >= 0, "router: tokens must be >= 0 (got %lld)", (long long)tokens);
  HMOE_REQUIRE(n_experts >= 1 && n_experts <= 256, "router: n_experts must be in [1, 256] (got %d)",
               n_experts);
  HMOE_REQUIRE(top_k >= 1 && top_k <= n_experts && top_k <= 32,
               "router: top_k must be in [1, min(n_experts, 32)] (got %d, n_experts %d)", top_k,
               n_experts);
  HMOE_REQUIRE(mode == HMOE_ROUTE_SIGMOID_BIAS || mode == HMOE_ROUTE_SOFTMAX,
               "router: unknown routing mode %d", mode);
  return HMOE_OK;
}

}  // namespace
}  // namespace hmoe

extern "C" int hmoe_router(const void* x, int x_dtype, const void* router_w, int w_dtype,
                           const float* bias, int64_t tokens, int d_model, int n_experts,
                           int top_k, int mode, float routed_scaling_factor, float* logits,
                           int32_t* top_idx, float* gates, hmoe_stream_t stream) {
  using namespace hmoe;
  if (int rc = validate_routing(tokens, n_experts, top_k, mode)) return rc;
  HMOE_REQUIRE(d_model >= 8 && d_model % 8 == 0,
               "router: d_model must be a positive multiple of 8 (got %d)", d_model);
  HMOE_REQUIRE(x_dtype == HMOE_F32 || x_dtype == HMOE_BF16, "router: x dtype must be F32 or BF16");
  HMOE_REQUIRE(w_dtype == HMOE_F32 || w_dtype == HMOE_BF16, "router: weight dtype must be F32 or BF16");
  if (tokens == 0) return HMOE_OK;
  HMOE_REQUIRE(x && router_w && logits && top_idx && gates, "router: null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const float rsf = routed_scaling_factor;
  if (n_experts <= 16)
    dispatch_router<1>(x_dtype, w_dtype, x, router_w, bias, tokens, d_model, n_experts, top_k, mode, rsf, logits, top_idx, gates, s);
  else if (n_experts <= 32)
    dispatch_router<2>(x_dtype, w_dtype, x, router_w, bias, tokens, d_model, n_experts, top_k, mode, rsf, logits, top_idx, gates, s);
  else if (n_experts <= 64)
    dispatch_router<4>(x_dtype, w_dtype, x, router_w, bias, tokens, d_model, n_experts, top_k, mode, rsf, logits, top_idx, gates, s);
  else if (n_experts <= 128)
    dispatch_router<8>(x_dtype, w_dtype, x, router_w, bias, tokens, d_model, n_experts, top_k, mode, rsf, logits, top_idx, gates, s);
  else
    dispatch_router<16>(x_dtype, w_dtype, x, router_w, bias, tokens, d_model, n_experts, top_k, mode, rsf, logits, top_idx, gates, s);
  return check_launch("hmoe_router");
}

extern "C" int hmoe_router_quant_fp8(const void* x, int x_dtype, const void* router_w, int w_dtype,
                                     const float* bias, int64_t tokens, int d_model, int n_experts,
                                     int top_k, int mode, float routed_scaling_factor,
                                     float* logits, int32_t* top_idx, float* gates, uint8_t* x_q,
                                     float* x_scale, hmoe_stream_t stream) {
  using namespace hmoe;
  if (int rc = validate_routing(tokens, n_experts, top_k, mode)) return rc;
  HMOE_REQUIRE(d_model >= 8 && d_model % 8 == 0,
               "router_quant_fp8: d_model must be a positive multiple of 8 (got %d)", d_model);
  HMOE_REQUIRE(x_dtype == HMOE_BF16, "router_quant_fp8: x dtype must be BF16");
  HMOE_REQUIRE(w_dtype == HMOE_F32 || w_dtype == HMOE_BF16,
               "router_quant_fp8: weight dtype must be F32 or BF16");
  if (tokens == 0) return HMOE_OK;
  HMOE_REQUIRE(x && router_w && logits && top_idx && gates && x_q && x_scale,
               "router_quant_fp8: null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const float rsf = routed_scaling_factor;
  XQuant xq;
  xq.q = x_q;
  xq.scale = x_scale;
  if (n_experts <= 16)
    dispatch_router<1>(x_dtype, w_dtype, x, router_w, bias, tokens, d_model, n_experts, top_k, mode, rsf, logits, top_idx, gates, s, xq);
  else if (n_experts <= 32)
    dispatch_router<2>(x_dtype, w_dtype, x, router_w, bias, tokens, d_model, n_experts, top_k, mode, rsf, logits, top_idx, gates, s, xq);
  else if (n_experts <= 64)
    dispatch_router<4>(x_dtype, w_dtype, x, router_w, bias, tokens, d_model, n_experts, top_k, mode, rsf, logits, top_idx, gates, s, xq);
  else if (n_experts <= 128)
    dispatch_router<8>(x_dtype, w_dtype, x, router_w, bias, tokens, d_model, n_experts, top_k, mode, rsf, logits, top_idx, gates, s, xq);
  else
    dispatch_router<16>(x_dtype, w_dtype, x, router_w, bias, tokens, d_model, n_experts, top_k, mode, rsf, logits, top_idx, gates, s, xq);
  return check_launch("hmoe_router_quant_fp8");
}

extern "C" int hmoe_router_from_logits(const float* logits, const float* bias, int64_t tokens,
                                       int n_experts, int top_k, int mode,
                                       float routed_scaling_factor, int32_t* top_idx,
                                       float* gates, hmoe_stream_t stream) {
  using namespace hmoe;
  if (int rc = validate_routing(tokens, n_experts, top_k, mode)) return rc;
  if (tokens == 0) return HMOE_OK;
  HMOE_REQUIRE(logits && top_idx && gates, "router_from_logits: null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(ceil_div(tokens, 4 * kSelTok)));
  if (n_experts <= 64)
    hipLaunchKernelGGL(select_kernel_g8, dim3(static_cast<unsigned>(ceil_div(tokens, 32))), dim3(256), 0, s,
                       logits, bias, tokens, n_experts, top_k, mode, routed_scaling_factor, top_idx, gates);
  else if (n_experts <= 128)
    hipLaunchKernelGGL(select_kernel<2>, grid, dim3(256), 0, s, logits, bias, tokens, n_experts, top_k, mode, routed_scaling_factor, top_idx, gates);
  else
    hipLaunchKernelGGL(select_kernel<4>, grid, dim3(256), 0, s, logits, bias, tokens, n_experts, top_k, mode, routed_scaling_factor, top_idx, gates);
  return check_launch("hmoe_router_from_logits");
}
