/*
 * hanuman_moe.h -- C ABI of the MI355X (gfx950) MoE-layer forward.
 *
 * The reference layer is `MoE.__call__` in model/moe.py:170-294 of
 * theorionic/hanuman (JAX).  Its stages map onto the entry points below; each
 * declaration cites the reference lines it replaces.  A jax.ffi handler (or a
 * ctypes binding) forwards XLA/torch-owned device buffers to these calls.
 *
 * Conventions
 *   - Every pointer is a device pointer unless noted.  The library never
 *     allocates device memory: callers pass outputs and workspace.
 *   - Every call enqueues work on `stream` (a hipStream_t; NULL = the legacy
 *     default stream) and returns without synchronising.
 *   - Return value: HMOE_OK (0) or an HMOE_ERR_* code; hmoe_last_error()
 *     gives a message for the calling thread.  No call aborts the process.
 *   - T tokens, D d_model, N experts, K top-k, F d_ff, C capacity per expert,
 *     R = T*K (token, slot) pairs; flat slot index i = t*K + k.
 *   - Results are deterministic: no atomics decide any output value.
 */
#ifndef HANUMAN_MOE_H
#define HANUMAN_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* hmoe_stream_t; /* hipStream_t */

enum {
  HMOE_OK = 0,
  HMOE_ERR_INVALID = 1,     /* bad argument (shape, dtype, null pointer)   */
  HMOE_ERR_UNSUPPORTED = 2, /* valid but not supported by this build       */
  HMOE_ERR_HIP = 3,         /* HIP runtime error (launch, attribute)       */
  HMOE_ERR_WORKSPACE = 4    /* workspace too small                         */
};

enum { HMOE_F32 = 0, HMOE_BF16 = 1, HMOE_FP8_E4M3 = 2 };

enum {
  HMOE_ROUTE_SIGMOID_BIAS = 0, /* moe.py:179-192: top-k of sigmoid(l)+bias,
                                  gates sel/(sum sel + 1e-9) * rsf          */
  HMOE_ROUTE_SOFTMAX = 1       /* top-k of softmax(l), gates renormalised   */
};

/* Row tile of the grouped GEMM (a tile's reads past the buffer are clamped to
 * its last row, so dispatched buffers hold exactly rows_cap rows). */
#define HMOE_GEMM_TILE_M 256

/* ---- library --------------------------------------------------------- */

/* Message of the last failed call on this thread ("" if none). */
const char* hmoe_last_error(void);
/* ABI version of this header (bumped on incompatible change). */
int hmoe_abi_version(void);

/* ---- sizes ------------------------------------------------------------ */

/* Capacity per expert: ceil(capacity_factor * T * K / N); a factor <= 0 means
 * dropless (C = T*K, the reference's behaviour, moe.py:54-65). */
int64_t hmoe_capacity(int64_t tokens, int top_k, int n_experts, double capacity_factor);
/* Static bound on kept rows: min(T*K, N*C) (moe.py:59-65 pads to a multiple
 * of 128 instead; rows past the kept total are never read). */
int64_t hmoe_rows_cap(int64_t tokens, int top_k, int n_experts, int64_t capacity);
/* Workspace bytes needed by hmoe_dispatch_plan. */
size_t hmoe_plan_workspace_bytes(int64_t tokens, int top_k, int n_experts);

/* ---- router: moe.py:175-192 (replaces `x_f @ router`, `sigmoid`, `+bias`,
 *      `lax.top_k`, `take_along_axis`, the gate normalisation) ------------ */

/* x [T,D] (HMOE_F32 or HMOE_BF16), router_w [D,N] (HMOE_F32 or HMOE_BF16),
 * bias [N] f32 (may be NULL = zeros; used by HMOE_ROUTE_SIGMOID_BIAS only).
 * Outputs: logits [T,N] f32 (fp32 rounding of a float64 d-ascending sum),
 * top_idx [T,K] int32 (descending key, lower index first on ties), gates
 * [T,K] f32.  N <= 256, K <= min(N, 32), D % 8 == 0. */
int hmoe_router(const void* x, int x_dtype, const void* router_w, int w_dtype,
                const float* bias, int64_t tokens, int d_model, int n_experts,
                int top_k, int mode, float routed_scaling_factor, float* logits,
                int32_t* top_idx, float* gates, hmoe_stream_t stream);

/* Same selection and gates from precomputed logits [T,N] f32 (moe.py:179-192
 * applied to given `gate_logits`). */
int hmoe_router_from_logits(const float* logits, const float* bias, int64_t tokens,
                            int n_experts, int top_k, int mode,
                            float routed_scaling_factor, int32_t* top_idx,
                            float* gates, hmoe_stream_t stream);

/* ---- dispatch plan: moe.py:54-57,80 (replaces `argsort(slot_expert)`,
 *      `bincount`, `argsort(order)`) plus the capacity drop --------------- */

/* top_idx [T,K] int32 in [0,N).  Outputs:
 *   counts   [N]        rows routed to each expert before drops (bincount)
 *   offsets  [N+1]      exclusive scan of min(counts, C): kept-row segments
 *   slot_pos [T*K]      dispatched row of slot i, or -1 if dropped (= inv)
 *   perm_src [rows_cap] slot i of dispatched row j (= order), -1 past the end
 *   keep     [T*K]      1 if slot i is kept (rank within its expert < C)
 * Stable: within an expert, rows keep ascending i. */
int hmoe_dispatch_plan(const int32_t* top_idx, int64_t tokens, int top_k,
                       int n_experts, int64_t capacity, int32_t* counts,
                       int32_t* offsets, int32_t* slot_pos, int32_t* perm_src,
                       uint8_t* keep, void* workspace, size_t workspace_bytes,
                       hmoe_stream_t stream);

/* The same plan without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops).  No counterpart in the reference.  The per-block histogram lives
 * in a fixed 1 MiB device array of the library, one per GPU for the life of
 * the process, so ceil(T*K / 1024) * N <= 262144 (e.g. T*K up to 4M slots
 * at N = 64); larger plans return HMOE_ERR_WORKSPACE.  The stream's device
 * must be the current device.  Calls on one GPU share the array: two calls
 * that overlap in time on the same GPU (different streams) race; calls
 * ordered on one stream do not.  Allocates nothing. */
int hmoe_dispatch_plan_noalloc(const int32_t* top_idx, int64_t tokens, int top_k,
                               int n_experts, int64_t capacity, int32_t* counts,
                               int32_t* offsets, int32_t* slot_pos, int32_t* perm_src,
                               uint8_t* keep, hmoe_stream_t stream);

/* ---- row permutation: moe.py:56,198 (replaces `x.astype(dtype)` and
 *      `x_flat[order // K]`) ------------------------------------------------ */

/* xs[slot_pos[t*K+k]] = cast(x[t]) for kept slots; each token row is read
 * once.  x [T,D] (F32/BF16), xs [rows_cap, D] (F32/BF16). D % 8 == 0. */
int hmoe_permute_rows(const void* x, int x_dtype, int64_t tokens, int d_model,
                      int top_k, const int32_t* slot_pos, void* xs, int xs_dtype,
                      hmoe_stream_t stream);

/* ---- fp8 dispatch (workload rule, no reference code): the row permutation
 *      above with per-token e4m3 quantisation fused in ---------------------- */

/* xs_q[slot_pos[t*K+k]] = e4m3 codes of x[t] for kept slots, xs_scale[...] =
 * that token's scale.  Per row: amax = max|x|, codes
 * e4m3(clamp(x * (448/amax), +-448)) (round to nearest even), scale amax/448;
 * an all-zero row gets scale 1.  x [T,D] (F32/BF16), xs_q [rows_cap, D]
 * uint8, xs_scale [rows_cap] f32.  D % 8 == 0. */
int hmoe_permute_rows_fp8(const void* x, int x_dtype, int64_t tokens, int d_model,
                          int top_k, const int32_t* slot_pos, uint8_t* xs_q,
                          float* xs_scale, hmoe_stream_t stream);

/* Same per-row rule for a bf16 matrix a [rows, cols] (the SwiGLU output h
 * before the fp8 down GEMM).  With offsets != NULL, rows at or past
 * offsets[n_experts] are not read: their codes are left untouched and their
 * scale is set to 1.  cols % 8 == 0. */
int hmoe_quantize_rows_fp8(const void* a, int64_t rows, int cols, const int32_t* offsets,
                           int n_experts, uint8_t* q, float* scale, hmoe_stream_t stream);

/* hmoe_router (moe.py:175-192) and hmoe_quantize_rows_fp8(x, T, D, NULL, 0,
 * x_q, x_scale) in one launch, for the fp8 experts on bf16 tokens: the
 * quantisation runs in workgroups beside the router's, whose float64 matrix
 * chains leave the memory system idle.  Outputs are bit-identical to the two
 * calls.  x [T,D] HMOE_BF16 only; x_q [T,D] uint8, x_scale [T] f32; the
 * router's arguments and limits as for hmoe_router. */
int hmoe_router_quant_fp8(const void* x, int x_dtype, const void* router_w, int w_dtype,
                          const float* bias, int64_t tokens, int d_model, int n_experts,
                          int top_k, int mode, float routed_scaling_factor, float* logits,
                          int32_t* top_idx, float* gates, uint8_t* x_q, float* x_scale,
                          hmoe_stream_t stream);

/* ---- expert weights: moe.py:204-206 (replaces the per-call `.astype(dtype)`
 *      of the stacked fp32 masters) ---------------------------------------- */

/* Packs expert_w_gate/expert_w_up [N,D,F] (F32/BF16) into the bf16 gate/up
 * operand [N][2F][D]: packed row p holds column h = (p/64)*32 + p%32 of the
 * gate (p%64 < 32) or up (p%64 >= 32) weight, D contiguous.  F % 128 == 0. */
size_t hmoe_packed_gate_up_bytes(int n_experts, int d_model, int d_ff);
int hmoe_pack_gate_up(const void* w_gate, const void* w_up, int w_dtype,
                      int n_experts, int d_model, int d_ff, void* packed,
                      hmoe_stream_t stream);
/* Packs expert_w_down [N,F,D] into bf16 [N][D][F] (F contiguous). */
size_t hmoe_packed_down_bytes(int n_experts, int d_ff, int d_model);
int hmoe_pack_down(const void* w_down, int w_dtype, int n_experts, int d_ff,
                   int d_model, void* packed, hmoe_stream_t stream);

/* e4m3 versions of the two packed operands (same layouts, one byte per
 * weight) with per-output-channel scales in packed-row order: gate/up scales
 * [N][2F], down scales [N][D].  Rule as hmoe_permute_rows_fp8, amax over the
 * reduction dimension of each output column. */
size_t hmoe_packed_fp8_gate_up_bytes(int n_experts, int d_model, int d_ff);
int hmoe_pack_fp8_gate_up(const void* w_gate, const void* w_up, int w_dtype, int n_experts,
                          int d_model, int d_ff, uint8_t* packed, float* scales,
                          hmoe_stream_t stream);
size_t hmoe_packed_fp8_down_bytes(int n_experts, int d_ff, int d_model);
int hmoe_pack_fp8_down(const void* w_down, int w_dtype, int n_experts, int d_ff, int d_model,
                       uint8_t* packed, float* scales, hmoe_stream_t stream);

/* ---- grouped expert GEMMs: moe.py:67-74 (replaces the three
 *      `jax.lax.ragged_dot` calls and the SwiGLU between them) ------------- */

/* h[r, :] = bf16( silu(g) * u ) for rows r of expert e's segment
 * [offsets[e], offsets[e+1]), with g = bf16(xs[r]·Wg[e]) and
 * u = bf16(xs[r]·Wu[e]) (fp32 accumulation, rounded to bf16 as the
 * `ragged_dot` outputs of moe.py:70-71 are; silu and the product in fp32,
 * moe.py:72).  xs [rows_cap, D] bf16, packed gate/up from hmoe_pack_gate_up,
 * h [rows_cap, F] bf16.  D % 64 == 0, F % 128 == 0, N <= 1024. */
int hmoe_grouped_gate_up(const void* xs, const int32_t* offsets, int n_experts,
                         int64_t rows_cap, int d_model, int d_ff,
                         const void* w_gate_up_packed, void* h, hmoe_stream_t stream);

/* The same h with the row permutation (moe.py:56, `x_flat[order // K]`) done
 * by the GEMM's own loads: row r of the dispatched operand is
 * x[perm_src[r] / top_k], so the dispatched copy of x is never written (a
 * fusion of hmoe_permute_rows and hmoe_grouped_gate_up; bit-identical h).
 * x [tokens, D] bf16, perm_src [rows_cap] from hmoe_dispatch_plan (rows with
 * -1 are computed from token 0 and not meaningful, as past the kept rows
 * above).  tokens * D * 2 < 2^31. */
int hmoe_grouped_gate_up_gather(const void* x, int64_t tokens, int top_k,
                                const int32_t* perm_src, const int32_t* offsets,
                                int n_experts, int64_t rows_cap, int d_model, int d_ff,
                                const void* w_gate_up_packed, void* h,
                                hmoe_stream_t stream);

/* ys[r, :] = bf16( h[r]·Wd[e] ) per expert segment.  h [rows_cap, F] bf16,
 * packed down from hmoe_pack_down, ys [rows_cap, D] bf16.  F % 64 == 0,
 * D % 256 == 0. */
int hmoe_grouped_down(const void* h, const int32_t* offsets, int n_experts,
                      int64_t rows_cap, int d_ff, int d_model,
                      const void* w_down_packed, void* ys, hmoe_stream_t stream);

/* The layer's whole expert FFN in one persistent launch (moe.py:56,70-74:
 * the gathered gate/up GEMM with the SwiGLU, then the down GEMM): h and ys
 * are bit-identical to hmoe_grouped_gate_up_gather followed by
 * hmoe_grouped_down.  Each XCD of the GPU takes an even share of the 256-row
 * m-tiles and runs their gate/up tiles, then their down tiles; a down tile
 * starts once the gate/up tiles of its m-tile are stored (per-m-tile counts
 * in the workspace).  A wait that runs past wait_timeout_us (<= 0: 200 ms)
 * gives up and sets bit 0 of the workspace's uint32 word 8 (status; 0 when
 * every wait was met), and that tile's ys is not meaningful; every launch
 * exits.  extra_ready_needed > 0 raises the count a down tile waits for
 * past what the gate/up tiles can reach, so that every wait gives up (it
 * exists to test that path; pass 0).  Workspace: at least
 * hmoe_grouped_swiglu_fused_workspace_bytes(rows_cap, n_experts) bytes,
 * zero-filled before its first call; every call leaves its counters at zero
 * again (and word 8 holding its status), so no clearing is needed between
 * calls.  Calls that overlap in time must not share one.  D % 256 == 0,
 * F % 128 == 0 and F >= 256, tokens * D * 2 < 2^31. */
size_t hmoe_grouped_swiglu_fused_workspace_bytes(int64_t rows_cap, int n_experts);
/* Sets `bytes` (a multiple of 4) of device memory to zero with a kernel
 * (graph-capturable, unlike a memset node): the first-use clearing of a
 * fused workspace that a caller allocates afresh per call (an XLA result
 * buffer).  No counterpart in the reference. */
int hmoe_zero_fill(void* buffer, size_t bytes, hmoe_stream_t stream);
int hmoe_grouped_swiglu_fused(const void* x, int64_t tokens, int top_k,
                              const int32_t* perm_src, const int32_t* offsets, int n_experts,
                              int64_t rows_cap, int d_model, int d_ff,
                              const void* w_gate_up_packed, const void* w_down_packed, void* h,
                              void* ys, void* workspace, size_t workspace_bytes,
                              int64_t wait_timeout_us, int extra_ready_needed,
                              hmoe_stream_t stream);

/* fp8 expert GEMMs (workload rule): e4m3 operands on the CDNA4 32x32x64
 * fp8 MFMA with float32 accumulation; the accumulators are dequantised with
 * the row scale times the column scale, then (gate/up) g and u are rounded to
 * bf16 and the SwiGLU is applied as in hmoe_grouped_gate_up.
 * h and ys are bf16.  gate/up: D % 128 == 0, F % 128 == 0; down: F % 128 == 0,
 * D % 256 == 0. */
int hmoe_grouped_gate_up_fp8(const uint8_t* xs_q, const float* xs_scale, const int32_t* offsets,
                             int n_experts, int64_t rows_cap, int d_model, int d_ff,
                             const uint8_t* w_packed, const float* w_scales, void* h,
                             hmoe_stream_t stream);
/* The fp8 h with the row permutation done by the GEMM's loads, as
 * hmoe_grouped_gate_up_gather does for bf16: x_q [tokens, D] and x_scale
 * [tokens] are the per-token codes and scales of x (hmoe_quantize_rows_fp8
 * of x, whose rule is hmoe_permute_rows_fp8's, so h is bit-identical to the
 * permuted path) and row r of the dispatched operand is token
 * perm_src[r] / top_k.  tokens * D < 2^31. */
int hmoe_grouped_gate_up_fp8_gather(const uint8_t* x_q, const float* x_scale, int64_t tokens,
                                    int top_k, const int32_t* perm_src, const int32_t* offsets,
                                    int n_experts, int64_t rows_cap, int d_model, int d_ff,
                                    const uint8_t* w_packed, const float* w_scales, void* h,
                                    hmoe_stream_t stream);
int hmoe_grouped_down_fp8(const uint8_t* h_q, const float* h_scale, const int32_t* offsets,
                          int n_experts, int64_t rows_cap, int d_ff, int d_model,
                          const uint8_t* w_packed, const float* w_scales, void* ys,
                          hmoe_stream_t stream);
/* Block-scaled h (the fp8 workload's rule for the down GEMM's operand, the
 * re-quantisation the reference's bf16 path has no counterpart of; it
 * replaces hmoe_quantize_rows_fp8 of h between the two GEMMs of
 * moe.py:70-72).  The gate/up GEMM's epilogue computes h as the _fp8 entries
 * do (bf16-rounded), then every 32 consecutive h columns of a row share a
 * power-of-two scale 2^e, e the smallest integer with max|h| <= 448 * 2^e
 * over the block (at least -127), and the codes are e4m3(h * 2^-e) rounded
 * to nearest even: h_q [rows_cap, F] uint8 and h_exp [rows_cap, F / 32]
 * uint8 biased exponents e + 127 (E8M0).  Rows past offsets[N] are not
 * written.  The down GEMM feeds h_exp to the MFMA's per-32-value operand
 * scales and dequantises the accumulators by the column scales only.
 * Shape rules as for the _fp8 entries. */
int hmoe_grouped_gate_up_fp8_qh(const uint8_t* xs_q, const float* xs_scale,
                                const int32_t* offsets, int n_experts, int64_t rows_cap,
                                int d_model, int d_ff, const uint8_t* w_packed,
                                const float* w_scales, uint8_t* h_q, uint8_t* h_exp,
                                hmoe_stream_t stream);
int hmoe_grouped_gate_up_fp8_gather_qh(const uint8_t* x_q, const float* x_scale, int64_t tokens,
                                       int top_k, const int32_t* perm_src,
                                       const int32_t* offsets, int n_experts, int64_t rows_cap,
                                       int d_model, int d_ff, const uint8_t* w_packed,
                                       const float* w_scales, uint8_t* h_q, uint8_t* h_exp,
                                       hmoe_stream_t stream);
int hmoe_grouped_down_fp8_mx(const uint8_t* h_q, const uint8_t* h_exp, const int32_t* offsets,
                             int n_experts, int64_t rows_cap, int d_ff, int d_model,
                             const uint8_t* w_packed, const float* w_scales, void* ys,
                             hmoe_stream_t stream);

/* Float32 compute dtype (moe.py:70-74 with dtype = float32): the grouped
 * GEMMs on the float32 matrix cores with the masters as they are.
 * gate/up: h [rows_cap, F] = silu(xs W_gate[e]) * (xs W_up[e]) in float32,
 * xs [rows_cap, D] f32, w_gate / w_up [N, D, F] f32; D % 16 == 0,
 * F % 64 == 0.  down: ys [rows_cap, D] = h W_down[e], w_down [N, F, D] f32;
 * F % 16 == 0, D % 64 == 0.  Rows past offsets[N] are not written. */
int hmoe_grouped_gate_up_f32(const float* xs, const int32_t* offsets, int n_experts,
                             int64_t rows_cap, int d_model, int d_ff, const float* w_gate,
                             const float* w_up, float* h, hmoe_stream_t stream);
int hmoe_grouped_down_f32(const float* h, const int32_t* offsets, int n_experts,
                          int64_t rows_cap, int d_ff, int d_model, const float* w_down, float* ys,
                          hmoe_stream_t stream);

/* Backward of the float32 compute dtype (the VJP of moe.py:70-85 with
 * dtype = float32, routing held fixed; replaces what jax.value_and_grad,
 * train.py:266, derives for these lines), on the masters as they are.
 * d_model and d_ff are multiples of 64 in all of them.
 *
 * combine_bwd_f32: the VJP of hmoe_combine for float32 rows:
 *   d_ys[pos(t,k)] = dy[t] * g[t,k], d_gates[t,k] = sum_d dy[t,d] *
 *   ys[pos(t,k),d] (float64 sum, rounded once), 0 for a dropped slot;
 *   d_shared [T, D] (or NULL) = dy / shared_div.  d_model % 4 == 0.
 * dgrad_down_f32: dh [rows_cap, F] = d_ys W_down[e]^T per segment.
 * gate_up_swiglu_bwd_f32: g = xs W_gate[e], u = xs W_up[e] recomputed and
 *   dgu [rows_cap, 2F] = [dg | du] (columns [0, F) and [F, 2F)) for the
 *   cotangent dh [rows_cap, F] of h = silu(g) * u.
 * dgrad_gate_up_f32: d_xs [rows_cap, D] = dg W_gate[e]^T + du W_up[e]^T.
 * wgrad_gate_up_f32: dw_gate, dw_up [N, D, F] = xs^T dg, xs^T du over each
 *   segment (an empty segment gives zeros).
 * wgrad_down_f32: dw_down [N, F, D] = h^T d_ys over each segment.
 * Rows past offsets[N] are neither read by the weight gradients nor
 * written by the others. */
int hmoe_combine_bwd_f32(const float* dy, const float* ys, const int32_t* slot_pos,
                         const float* gates, int64_t tokens, int top_k, int d_model, float* d_ys,
                         float* d_gates, float* d_shared, float shared_div, hmoe_stream_t stream);
int hmoe_grouped_dgrad_down_f32(const float* d_ys, const int32_t* offsets, int n_experts,
                                int64_t rows_cap, int d_model, int d_ff, const float* w_down,
                                float* dh, hmoe_stream_t stream);
int hmoe_grouped_gate_up_swiglu_bwd_f32(const float* xs, const int32_t* offsets, int n_experts,
                                        int64_t rows_cap, int d_model, int d_ff,
                                        const float* w_gate, const float* w_up, const float* dh,
                                        float* dgu, hmoe_stream_t stream);
int hmoe_grouped_dgrad_gate_up_f32(const float* dgu, const int32_t* offsets, int n_experts,
                                   int64_t rows_cap, int d_model, int d_ff, const float* w_gate,
                                   const float* w_up, float* d_xs, hmoe_stream_t stream);
int hmoe_grouped_wgrad_gate_up_f32(const float* xs, const float* dgu, const int32_t* offsets,
                                   int n_experts, int d_model, int d_ff, float* dw_gate,
                                   float* dw_up, hmoe_stream_t stream);
int hmoe_grouped_wgrad_down_f32(const float* h, const float* d_ys, const int32_t* offsets,
                                int n_experts, int d_ff, int d_model, float* dw_down,
                                hmoe_stream_t stream);

/* ---- combine: moe.py:80-85 (replaces `ys[inv]` and the weighted einsum) - */

/* out[t] = sum_k g'[t,k] * ys[slot_pos[t*K+k]] (+ residual[t]), g' the gates
 * cast to ys's dtype (bf16(gates) for BF16 rows, gates for F32 rows:
 * weights.astype(out.dtype), moe.py:84), float32 accumulation over k
 * ascending, dropped slots skipped.
 * ys [rows, D] (BF16/F32); gates [T,K] f32, or NULL for unit weights;
 * residual [T,D] (F32/BF16) or NULL: the shared expert's output, added last
 * (moe.py:249-251); out [T,D] (F32/BF16). */
int hmoe_combine(const void* ys, int ys_dtype, const int32_t* slot_pos,
                 const float* gates, const void* residual, int residual_dtype,
                 int64_t tokens, int top_k, int d_model, void* out, int out_dtype,
                 hmoe_stream_t stream);

/* ---- aux outputs: moe.py:253-292 (replaces logsumexp, the per-sequence
 *      bincount, the balance loss, the entropy diagnostic) ---------------- */

/* logits [B*S, N] f32 and top_idx [B*S, K] of B sequences of S tokens.
 * losses[3] = {router_z_loss, balance_loss, mean_entropy}; expert_counts [N]
 * f32 (integer valued, = counts of hmoe_dispatch_plan).  N <= 256,
 * B <= 1024.  Scores are the router's sigmoid (moe.py:179). */
size_t hmoe_aux_workspace_bytes(int batch, int seq, int n_experts);
int hmoe_router_aux(const float* logits, const int32_t* top_idx, int batch, int seq,
                    int n_experts, int top_k, float* losses, float* expert_counts,
                    void* workspace, size_t workspace_bytes, hmoe_stream_t stream);

/* ---- backward: the VJP that jax.value_and_grad (train.py:266) takes of
 *      MoE.__call__ (moe.py:170-294) for the loss of train.py:191-200.
 *      Routing decisions (top-k, drops, the plan, the expert counts) are
 *      held fixed: integer valued. --------------------------------------- */

/* VJP of the weighted combine (moe.py:80-85) for dy = d out [T,D] f32:
 * d_ys[slot_pos[t*K+k]] = bf16(dy[t] * bf16(gates[t,k])) (float32 product)
 * for kept slots (other rows of d_ys are not written), d_gates[t,k] =
 * bf16(f32(sum_d dy[t,d] * ys[pos,d])) with the sum in float64, 0 for dropped
 * slots.  ys and d_ys [rows, D] bf16, d_gates [T,K] f32.  D % 8 == 0,
 * K <= 16.  d_shared (NULL: not written) [T,D] bf16 = bf16(dy / shared_div):
 * the cotangent of each shared expert's output (moe.py:161-168, 249-251),
 * shared_div = n_shared_experts. */
int hmoe_combine_bwd(const float* dy, const void* ys, const int32_t* slot_pos,
                     const float* gates, int64_t tokens, int top_k, int d_model, void* d_ys,
                     float* d_gates, void* d_shared, float shared_div, hmoe_stream_t stream);

/* Recomputes the gate/up GEMM outputs g and u (moe.py:70-71) on the
 * dispatched rows of x, as bf16 [rows_cap, 2F] in the packed operand's
 * column order (blocks of 32 gate columns, then the 32 up columns of the
 * same h columns), no SwiGLU.  Same operands and limits as
 * hmoe_grouped_gate_up_gather. */
int hmoe_grouped_gate_up_raw_gather(const void* x, int64_t tokens, int top_k,
                                    const int32_t* perm_src, const int32_t* offsets,
                                    int n_experts, int64_t rows_cap, int d_model, int d_ff,
                                    const void* w_gate_up_packed, void* gu,
                                    hmoe_stream_t stream);
/* The same on rows given in order (xs [rows_cap, D] bf16, as
 * hmoe_grouped_gate_up): the shared expert's g and u (moe.py:23-29). */
int hmoe_grouped_gate_up_raw(const void* xs, const int32_t* offsets, int n_experts,
                             int64_t rows_cap, int d_model, int d_ff,
                             const void* w_gate_up_packed, void* gu, hmoe_stream_t stream);

/* The recompute with the SwiGLU VJP in the GEMM's epilogue: g and u are
 * rounded to bf16 in registers and dgu = hmoe_swiglu_bwd(dh, g, u) is written
 * directly (bit-identical to the raw recompute followed by hmoe_swiglu_bwd;
 * g and u never reach memory).  dh [rows_cap, F] bf16, dgu [rows_cap, 2F]
 * bf16; operands and limits as the raw entries above. */
int hmoe_grouped_gate_up_swiglu_bwd_gather(const void* x, int64_t tokens, int top_k,
                                           const int32_t* perm_src, const int32_t* offsets,
                                           int n_experts, int64_t rows_cap, int d_model, int d_ff,
                                           const void* w_gate_up_packed, const void* dh, void* dgu,
                                           hmoe_stream_t stream);
int hmoe_grouped_gate_up_swiglu_bwd(const void* xs, const int32_t* offsets, int n_experts,
                                    int64_t rows_cap, int d_model, int d_ff,
                                    const void* w_gate_up_packed, const void* dh, void* dgu,
                                    hmoe_stream_t stream);

/* VJP of h = silu(g) * u (moe.py:72): dg = dh * u * silu'(g), du = dh *
 * silu(g), float32 arithmetic, one bf16 rounding each.  dh [rows, F], gu and
 * dgu [rows, 2F] bf16 in the column order of hmoe_grouped_gate_up_raw_gather.
 * Rows at or past offsets[n_experts] are not touched (offsets may be NULL:
 * all rows).  F % 32 == 0. */
int hmoe_swiglu_bwd(const void* dh, const void* gu, const int32_t* offsets, int n_experts,
                    int64_t rows, int d_ff, void* dgu, hmoe_stream_t stream);

/* Backward operands of the expert GEMMs, packed once from the fp32/bf16
 * masters: w_down [N,F,D] -> bf16 [N,F,D] (rows = h columns, D contiguous);
 * w_gate, w_up [N,D,F] -> bf16 [N,D,2F] (rows = d, columns in the gate/up
 * column order). */
int hmoe_pack_down_dgrad(const void* w_down, int w_dtype, int n_experts, int d_ff,
                         int d_model, void* packed, hmoe_stream_t stream);
int hmoe_pack_gate_up_dgrad(const void* w_gate, const void* w_up, int w_dtype, int n_experts,
                            int d_model, int d_ff, void* packed, hmoe_stream_t stream);

/* dh = bf16(d_ys Wd[e]^T) per expert segment (the VJP of moe.py:73 with
 * respect to h): d_ys [rows_cap, D], dh [rows_cap, F] bf16, w_down_dgrad
 * from hmoe_pack_down_dgrad.  D % 64 == 0, F % 256 == 0. */
int hmoe_grouped_dgrad_down(const void* d_ys, const int32_t* offsets, int n_experts,
                            int64_t rows_cap, int d_model, int d_ff, const void* w_down_dgrad,
                            void* dh, hmoe_stream_t stream);

/* d_xs = bf16(dg Wg[e]^T + du Wu[e]^T) per expert segment, one float32
 * accumulation over the 2F columns (the VJP of moe.py:70-71 with respect to
 * xs): dgu [rows_cap, 2F] (hmoe_swiglu_bwd), d_xs [rows_cap, D] bf16,
 * w_gate_up_dgrad from hmoe_pack_gate_up_dgrad.  F % 32 == 0, D % 256 == 0. */
int hmoe_grouped_dgrad_gate_up(const void* dgu, const int32_t* offsets, int n_experts,
                               int64_t rows_cap, int d_model, int d_ff,
                               const void* w_gate_up_dgrad, void* d_xs, hmoe_stream_t stream);

/* VJP of the row gather (moe.py:56): dx[t] = sum_k d_xs[slot_pos[t*K+k]]
 * over kept slots, float32, k ascending (hmoe_combine with unit weights),
 * then + residual[t] (NULL: none; F32/BF16 [T,D]: the shared expert's input
 * gradient). */
int hmoe_gather_bwd(const void* d_xs, int d_xs_dtype, const int32_t* slot_pos,
                    const void* residual, int residual_dtype, int64_t tokens, int top_k,
                    int d_model, void* dx, int dx_dtype, hmoe_stream_t stream);

/* VJP of the gates with respect to the logits (moe.py:179-192; mode as in
 * hmoe_router): d_logits [T,N] f32, zero off the selected experts.
 * HMOE_ROUTE_SOFTMAX: dl_k = g_k (dg_k - sum_j g_j dg_j) (needs gates);
 * HMOE_ROUTE_SIGMOID_BIAS: with s = sigmoid(l), Z = sum_j s_j + 1e-9,
 * dl_k = rsf (dg_k/Z - sum_j dg_j s_j/Z^2) s_k (1 - s_k) (needs logits).
 * Sums over k in float32, k ascending. */
int hmoe_router_bwd(const float* logits, const int32_t* top_idx, const float* gates,
                    const float* d_gates, int64_t tokens, int n_experts, int top_k, int mode,
                    float routed_scaling_factor, float* d_logits, hmoe_stream_t stream);

/* VJP of the aux losses (moe.py:253-283) with respect to the logits, for
 * d_losses[3] = cotangents of {router_z_loss, balance_loss, mean_entropy}
 * (device memory; train.py:198-200 weighs the first two): d_logits [B*S, N]
 * f32 (+)= (accumulate != 0) d_z * 2 lse/T * softmax(l) + the balance and
 * entropy terms through p = sigmoid(l) / (sum sigmoid(l) + 1e-9), with the
 * per-sequence counts of top_idx held fixed.  N <= 256.
 * workspace >= hmoe_aux_bwd_workspace_bytes. */
size_t hmoe_aux_bwd_workspace_bytes(int batch, int seq, int n_experts);
int hmoe_router_aux_bwd(const float* logits, const int32_t* top_idx, int batch, int seq,
                        int n_experts, int top_k, const float* d_losses, float* d_logits,
                        int accumulate, void* workspace, size_t workspace_bytes,
                        hmoe_stream_t stream);

/* dx [T,D] f32 (+)= d_logits [T,N] @ router_w^T (router_w [D,N] F32/BF16):
 * the VJP of l = f32(x) @ router (moe.py:175,178) with respect to x, on the
 * float32 matrix cores.  accumulate != 0 adds into dx.  D % 64 == 0. */
int hmoe_router_dx(const float* d_logits, const void* router_w, int w_dtype, int64_t tokens,
                   int d_model, int n_experts, float* dx, int accumulate, hmoe_stream_t stream);

/* Expert weight gradients, float32, per expert e over its segment rows
 * [offsets[e], offsets[e+1]) (an empty expert gets zeros):
 *   dw_down [N,F,D] = h^T d_ys            (VJP of moe.py:73)
 *   dw_gate, dw_up [N,D,F] = xs^T dg, xs^T du  (VJP of moe.py:70-71)
 * h [rows_cap, F], d_ys [rows_cap, D], xs [rows_cap, D] (the dispatched rows,
 * hmoe_permute_rows) and dgu [rows_cap, 2F] (hmoe_swiglu_bwd's column order)
 * bf16.  Summation order over the rows is fixed (64-row steps, float32
 * accumulation in the matrix cores).  F % 256 and D % 256 == 0 for
 * dw_down; D % 256 and F % 128 == 0 for dw_gate/up. */
int hmoe_grouped_wgrad_down(const void* h, const void* d_ys, const int32_t* offsets,
                            int n_experts, int64_t rows_cap, int d_ff, int d_model,
                            float* dw_down, hmoe_stream_t stream);
int hmoe_grouped_wgrad_gate_up(const void* xs, const void* dgu, const int32_t* offsets,
                               int n_experts, int64_t rows_cap, int d_model, int d_ff,
                               float* dw_gate, float* dw_up, hmoe_stream_t stream);

/* d_router [D,N] f32 = x^T d_logits (the VJP of moe.py:178 with respect to
 * the router weight), x [T,D] F32/BF16, d_logits [T,N] f32; float32 sums
 * over chunks of 512 tokens (float32 matrix cores), then over the chunks in
 * order.  workspace >= hmoe_router_dw_workspace_bytes.  D % 128 == 0. */
size_t hmoe_router_dw_workspace_bytes(int64_t tokens, int d_model, int n_experts);
int hmoe_router_dw(const void* x, int x_dtype, const float* d_logits, int64_t tokens,
                   int d_model, int n_experts, float* d_router, void* workspace,
                   size_t workspace_bytes, hmoe_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* HANUMAN_MOE_H */
