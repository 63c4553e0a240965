// XLA FFI handlers for the entry points of libhanuman_moe.so (forward and backward).
//
// The reference layer is JAX (model/moe.py).  A maintainer keeps its Python
// and replaces the router lines (moe.py:175-192) and the body of
// ragged_dispatch (moe.py:37-85) with custom calls to these handlers.  Each
// handler forwards XLA-owned device buffers and XLA's stream to one hmoe_*
// entry point of include/hanuman_moe.h and turns a non-zero status into an
// ffi::Error; none allocates, synchronises or keeps a pointer past the call.
//
// Build (needs JAX's FFI headers, jax.ffi.include_dir(); hanuman_amd/build.py
// build_xla_ffi() runs it when jax is importable):
//   hipcc --offload-arch=gfx950 -O2 -std=c++17 -fPIC -shared \
//     -I<jax.ffi.include_dir()> -I include hanuman_amd/xla_ffi/hmoe_xla_ffi.cc \
//     -L hanuman_amd -lhanuman_moe -Wl,-rpath,'$ORIGIN/..' \
//     -o hanuman_amd/xla_ffi/libhanuman_moe_xla.so
// Registration (Python), once per process:
//   lib = ctypes.cdll.LoadLibrary(".../libhanuman_moe_xla.so")
//   jax.ffi.register_ffi_target("hmoe_router", jax.ffi.pycapsule(lib.HmoeRouter),
//                               platform="ROCM")
// and likewise for every XLA_FFI_DEFINE_HANDLER_SYMBOL below (symbol name =
// the target name in CamelCase).  Output shapes are static: rows_cap =
// hmoe_rows_cap(T, K, N, C), workspaces from hmoe_plan_workspace_bytes and
// hmoe_aux_workspace_bytes, packed weights from hmoe_packed_*_bytes.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "hanuman_moe.h"
#include "xla/ffi/api/ffi.h"

namespace ffi = xla::ffi;

namespace {

ffi::Error Status(int rc) {
  if (rc == HMOE_OK) return ffi::Error::Success();
  const ffi::ErrorCode code = rc == HMOE_ERR_HIP           ? ffi::ErrorCode::kInternal
                              : rc == HMOE_ERR_UNSUPPORTED ? ffi::ErrorCode::kUnimplemented
                                                           : ffi::ErrorCode::kInvalidArgument;
  return ffi::Error(code, hmoe_last_error());
}

// hmoe dtype code of a float buffer (F32 or BF16); -1 otherwise.
int DtypeCode(ffi::DataType t) {
  switch (t) {
    case ffi::DataType::F32: return HMOE_F32;
    case ffi::DataType::BF16: return HMOE_BF16;
    default: return -1;
  }
}

ffi::Error BadDtype(const char* what) {
  return ffi::Error(ffi::ErrorCode::kInvalidArgument,
                    std::string(what) + ": expected a float32 or bfloat16 buffer");
}

hmoe_stream_t S(hipStream_t s) { return static_cast<hmoe_stream_t>(s); }

// Leading dimension (rows) and trailing dimension of a rank-2 buffer.
template <typename B>
int64_t Rows(const B& b) { return b.dimensions()[0]; }
template <typename B>
int64_t Cols(const B& b) { return b.dimensions()[b.dimensions().size() - 1]; }

}  // namespace

// ---- router: moe.py:175-192 -------------------------------------------------
// x [T, D] (f32/bf16), router_w [D, N] (f32/bf16), bias [N] f32 ->
// logits [T, N] f32, top_idx [T, K] s32, gates [T, K] f32.
static ffi::Error RouterImpl(hipStream_t stream, ffi::AnyBuffer x, ffi::AnyBuffer w,
                             ffi::Buffer<ffi::F32> bias, int64_t mode, float rsf,
                             ffi::ResultBuffer<ffi::F32> logits,
                             ffi::ResultBuffer<ffi::S32> top_idx,
                             ffi::ResultBuffer<ffi::F32> gates) {
  const int xd = DtypeCode(x.element_type()), wd = DtypeCode(w.element_type());
  if (xd < 0) return BadDtype("hmoe_router x");
  if (wd < 0) return BadDtype("hmoe_router router_w");
  const int64_t T = Rows(x);
  const int D = static_cast<int>(Cols(x)), N = static_cast<int>(Cols(w));
  const int K = static_cast<int>(Cols(*top_idx));
  return Status(hmoe_router(x.untyped_data(), xd, w.untyped_data(), wd, bias.typed_data(), T, D,
                            N, K, static_cast<int>(mode), rsf, logits->typed_data(),
                            top_idx->typed_data(), gates->typed_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeRouter, RouterImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Attr<int64_t>("mode")
                                  .Attr<float>("routed_scaling_factor")
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::S32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>());

// The router and the per-token e4m3 quantisation of x in one launch (fp8
// experts on bf16 tokens): x [T, D] bf16, router_w [D, N] (f32/bf16), bias
// [N] f32 -> logits, top_idx, gates as hmoe_router, x_q [T, D] u8, x_scale
// [T] f32 as hmoe_quantize_rows_fp8.
static ffi::Error RouterQuantFp8Impl(hipStream_t stream, ffi::Buffer<ffi::BF16> x,
                                     ffi::AnyBuffer w, ffi::Buffer<ffi::F32> bias, int64_t mode,
                                     float rsf, ffi::ResultBuffer<ffi::F32> logits,
                                     ffi::ResultBuffer<ffi::S32> top_idx,
                                     ffi::ResultBuffer<ffi::F32> gates,
                                     ffi::ResultBuffer<ffi::U8> x_q,
                                     ffi::ResultBuffer<ffi::F32> x_scale) {
  const int wd = DtypeCode(w.element_type());
  if (wd < 0) return BadDtype("hmoe_router_quant_fp8 router_w");
  const int64_t T = Rows(x);
  const int D = static_cast<int>(Cols(x)), N = static_cast<int>(Cols(w));
  const int K = static_cast<int>(Cols(*top_idx));
  return Status(hmoe_router_quant_fp8(
      x.untyped_data(), HMOE_BF16, w.untyped_data(), wd, bias.typed_data(), T, D, N, K,
      static_cast<int>(mode), rsf, logits->typed_data(), top_idx->typed_data(),
      gates->typed_data(), x_q->typed_data(), x_scale->typed_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeRouterQuantFp8, RouterQuantFp8Impl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Attr<int64_t>("mode")
                                  .Attr<float>("routed_scaling_factor")
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::S32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::U8>>()
                                  .Ret<ffi::Buffer<ffi::F32>>());

// logits [T, N] f32, bias [N] f32 -> top_idx [T, K] s32, gates [T, K] f32.
static ffi::Error RouterFromLogitsImpl(hipStream_t stream, ffi::Buffer<ffi::F32> logits,
                                       ffi::Buffer<ffi::F32> bias, int64_t mode, float rsf,
                                       ffi::ResultBuffer<ffi::S32> top_idx,
                                       ffi::ResultBuffer<ffi::F32> gates) {
  return Status(hmoe_router_from_logits(
      logits.typed_data(), bias.typed_data(), Rows(logits), static_cast<int>(Cols(logits)),
      static_cast<int>(Cols(*top_idx)), static_cast<int>(mode), rsf, top_idx->typed_data(),
      gates->typed_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeRouterFromLogits, RouterFromLogitsImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Attr<int64_t>("mode")
                                  .Attr<float>("routed_scaling_factor")
                                  .Ret<ffi::Buffer<ffi::S32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>());

// ---- dispatch plan: moe.py:54-57, 80 ---------------------------------------
// top_idx [T, K] s32 -> counts [N], offsets [N+1], slot_pos [T*K],
// perm_src [rows_cap] s32, keep [T*K] u8, workspace u8.
static ffi::Error DispatchPlanImpl(hipStream_t stream, ffi::Buffer<ffi::S32> top_idx,
                                   int64_t capacity, ffi::ResultBuffer<ffi::S32> counts,
                                   ffi::ResultBuffer<ffi::S32> offsets,
                                   ffi::ResultBuffer<ffi::S32> slot_pos,
                                   ffi::ResultBuffer<ffi::S32> perm_src,
                                   ffi::ResultBuffer<ffi::U8> keep,
                                   ffi::ResultBuffer<ffi::U8> workspace) {
  return Status(hmoe_dispatch_plan(
      top_idx.typed_data(), Rows(top_idx), static_cast<int>(Cols(top_idx)),
      static_cast<int>(counts->element_count()), capacity, counts->typed_data(),
      offsets->typed_data(), slot_pos->typed_data(), perm_src->typed_data(), keep->typed_data(),
      workspace->untyped_data(), workspace->size_bytes(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeDispatchPlan, DispatchPlanImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Attr<int64_t>("capacity")
                                  .Ret<ffi::Buffer<ffi::S32>>()
                                  .Ret<ffi::Buffer<ffi::S32>>()
                                  .Ret<ffi::Buffer<ffi::S32>>()
                                  .Ret<ffi::Buffer<ffi::S32>>()
                                  .Ret<ffi::Buffer<ffi::U8>>()
                                  .Ret<ffi::Buffer<ffi::U8>>());

// ---- row permutation: moe.py:56, 198 ----------------------------------------
// x [T, D] (f32/bf16), slot_pos [T*K] s32 -> xs [rows_cap, D] (f32/bf16).
static ffi::Error PermuteRowsImpl(hipStream_t stream, ffi::AnyBuffer x,
                                  ffi::Buffer<ffi::S32> slot_pos, ffi::Result<ffi::AnyBuffer> xs) {
  const int xd = DtypeCode(x.element_type()), od = DtypeCode(xs->element_type());
  if (xd < 0 || od < 0) return BadDtype("hmoe_permute_rows");
  const int64_t T = Rows(x);
  const int K = static_cast<int>(slot_pos.element_count() / (T > 0 ? T : 1));
  return Status(hmoe_permute_rows(x.untyped_data(), xd, T, static_cast<int>(Cols(x)), K,
                                  slot_pos.typed_data(), xs->untyped_data(), od, S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoePermuteRows, PermuteRowsImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Ret<ffi::AnyBuffer>());

// x [T, D] (f32/bf16), slot_pos [T*K] -> xs_q [rows_cap, D] u8 (e4m3 codes),
// xs_scale [rows_cap] f32.
static ffi::Error PermuteRowsFp8Impl(hipStream_t stream, ffi::AnyBuffer x,
                                     ffi::Buffer<ffi::S32> slot_pos,
                                     ffi::ResultBuffer<ffi::U8> xs_q,
                                     ffi::ResultBuffer<ffi::F32> xs_scale) {
  const int xd = DtypeCode(x.element_type());
  if (xd < 0) return BadDtype("hmoe_permute_rows_fp8");
  const int64_t T = Rows(x);
  const int K = static_cast<int>(slot_pos.element_count() / (T > 0 ? T : 1));
  return Status(hmoe_permute_rows_fp8(x.untyped_data(), xd, T, static_cast<int>(Cols(x)), K,
                                      slot_pos.typed_data(), xs_q->typed_data(),
                                      xs_scale->typed_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoePermuteRowsFp8, PermuteRowsFp8Impl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Ret<ffi::Buffer<ffi::U8>>()
                                  .Ret<ffi::Buffer<ffi::F32>>());

// a [rows, cols] bf16, offsets [N+1] s32 -> q [rows, cols] u8, scale [rows] f32.
static ffi::Error QuantizeRowsFp8Impl(hipStream_t stream, ffi::Buffer<ffi::BF16> a,
                                      ffi::Buffer<ffi::S32> offsets,
                                      ffi::ResultBuffer<ffi::U8> q,
                                      ffi::ResultBuffer<ffi::F32> scale) {
  return Status(hmoe_quantize_rows_fp8(a.untyped_data(), Rows(a), static_cast<int>(Cols(a)),
                                       offsets.typed_data(),
                                       static_cast<int>(offsets.element_count() - 1),
                                       q->typed_data(), scale->typed_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeQuantizeRowsFp8, QuantizeRowsFp8Impl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Ret<ffi::Buffer<ffi::U8>>()
                                  .Ret<ffi::Buffer<ffi::F32>>());

// ---- expert weight packing: moe.py:204-206 (once per parameter update) -----
// w_gate, w_up [N, D, F] (f32/bf16) -> packed gate/up (hmoe_packed_gate_up_bytes).
static ffi::Error PackGateUpImpl(hipStream_t stream, ffi::AnyBuffer wg, ffi::AnyBuffer wu,
                                 ffi::ResultBuffer<ffi::U8> packed) {
  const int d = DtypeCode(wg.element_type());
  if (d < 0 || DtypeCode(wu.element_type()) != d) return BadDtype("hmoe_pack_gate_up");
  auto dims = wg.dimensions();
  return Status(hmoe_pack_gate_up(wg.untyped_data(), wu.untyped_data(), d,
                                  static_cast<int>(dims[0]), static_cast<int>(dims[1]),
                                  static_cast<int>(dims[2]), packed->untyped_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoePackGateUp, PackGateUpImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Ret<ffi::Buffer<ffi::U8>>());

// w_down [N, F, D] (f32/bf16) -> packed down (hmoe_packed_down_bytes).
static ffi::Error PackDownImpl(hipStream_t stream, ffi::AnyBuffer wd,
                               ffi::ResultBuffer<ffi::U8> packed) {
  const int d = DtypeCode(wd.element_type());
  if (d < 0) return BadDtype("hmoe_pack_down");
  auto dims = wd.dimensions();
  return Status(hmoe_pack_down(wd.untyped_data(), d, static_cast<int>(dims[0]),
                               static_cast<int>(dims[1]), static_cast<int>(dims[2]),
                               packed->untyped_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoePackDown, PackDownImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Ret<ffi::Buffer<ffi::U8>>());

// e4m3 packing with per-output-channel scales ([N][2F] / [N][D] f32).
static ffi::Error PackFp8GateUpImpl(hipStream_t stream, ffi::AnyBuffer wg, ffi::AnyBuffer wu,
                                    ffi::ResultBuffer<ffi::U8> packed,
                                    ffi::ResultBuffer<ffi::F32> scales) {
  const int d = DtypeCode(wg.element_type());
  if (d < 0 || DtypeCode(wu.element_type()) != d) return BadDtype("hmoe_pack_fp8_gate_up");
  auto dims = wg.dimensions();
  return Status(hmoe_pack_fp8_gate_up(wg.untyped_data(), wu.untyped_data(), d,
                                      static_cast<int>(dims[0]), static_cast<int>(dims[1]),
                                      static_cast<int>(dims[2]), packed->typed_data(),
                                      scales->typed_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoePackFp8GateUp, PackFp8GateUpImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Ret<ffi::Buffer<ffi::U8>>()
                                  .Ret<ffi::Buffer<ffi::F32>>());

static ffi::Error PackFp8DownImpl(hipStream_t stream, ffi::AnyBuffer wd,
                                  ffi::ResultBuffer<ffi::U8> packed,
                                  ffi::ResultBuffer<ffi::F32> scales) {
  const int d = DtypeCode(wd.element_type());
  if (d < 0) return BadDtype("hmoe_pack_fp8_down");
  auto dims = wd.dimensions();
  return Status(hmoe_pack_fp8_down(wd.untyped_data(), d, static_cast<int>(dims[0]),
                                   static_cast<int>(dims[1]), static_cast<int>(dims[2]),
                                   packed->typed_data(), scales->typed_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoePackFp8Down, PackFp8DownImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Ret<ffi::Buffer<ffi::U8>>()
                                  .Ret<ffi::Buffer<ffi::F32>>());

// ---- grouped expert GEMMs: moe.py:67-74 -------------------------------------
// xs [rows_cap, D] bf16, offsets [N+1], packed gate/up -> h [rows_cap, F] bf16.
static ffi::Error GroupedGateUpImpl(hipStream_t stream, ffi::Buffer<ffi::BF16> xs,
                                    ffi::Buffer<ffi::S32> offsets, ffi::Buffer<ffi::U8> w,
                                    ffi::ResultBuffer<ffi::BF16> h) {
  return Status(hmoe_grouped_gate_up(xs.untyped_data(), offsets.typed_data(),
                                     static_cast<int>(offsets.element_count() - 1), Rows(xs),
                                     static_cast<int>(Cols(xs)), static_cast<int>(Cols(*h)),
                                     w.untyped_data(), h->untyped_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedGateUp, GroupedGateUpImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Ret<ffi::Buffer<ffi::BF16>>());

// x [T, D] bf16 (rows gathered through perm_src, moe.py:56 fused), perm_src
// [rows_cap], offsets [N+1], packed gate/up -> h [rows_cap, F] bf16.
static ffi::Error GroupedGateUpGatherImpl(hipStream_t stream, ffi::Buffer<ffi::BF16> x,
                                          ffi::Buffer<ffi::S32> perm_src,
                                          ffi::Buffer<ffi::S32> offsets, ffi::Buffer<ffi::U8> w,
                                          int64_t top_k, ffi::ResultBuffer<ffi::BF16> h) {
  return Status(hmoe_grouped_gate_up_gather(
      x.untyped_data(), Rows(x), static_cast<int>(top_k), perm_src.typed_data(),
      offsets.typed_data(), static_cast<int>(offsets.element_count() - 1), Rows(*h),
      static_cast<int>(Cols(x)), static_cast<int>(Cols(*h)), w.untyped_data(), h->untyped_data(),
      S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedGateUpGather, GroupedGateUpGatherImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Attr<int64_t>("top_k")
                                  .Ret<ffi::Buffer<ffi::BF16>>());

// h [rows_cap, F] bf16, offsets, packed down -> ys [rows_cap, D] bf16.
static ffi::Error GroupedDownImpl(hipStream_t stream, ffi::Buffer<ffi::BF16> h,
                                  ffi::Buffer<ffi::S32> offsets, ffi::Buffer<ffi::U8> w,
                                  ffi::ResultBuffer<ffi::BF16> ys) {
  return Status(hmoe_grouped_down(h.untyped_data(), offsets.typed_data(),
                                  static_cast<int>(offsets.element_count() - 1), Rows(h),
                                  static_cast<int>(Cols(h)), static_cast<int>(Cols(*ys)),
                                  w.untyped_data(), ys->untyped_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedDown, GroupedDownImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Ret<ffi::Buffer<ffi::BF16>>());

// e4m3 expert GEMMs (the fp8 workload rule).
static ffi::Error GroupedGateUpFp8Impl(hipStream_t stream, ffi::Buffer<ffi::U8> xs_q,
                                       ffi::Buffer<ffi::F32> xs_scale,
                                       ffi::Buffer<ffi::S32> offsets, ffi::Buffer<ffi::U8> w,
                                       ffi::Buffer<ffi::F32> w_scales,
                                       ffi::ResultBuffer<ffi::BF16> h) {
  return Status(hmoe_grouped_gate_up_fp8(
      xs_q.typed_data(), xs_scale.typed_data(), offsets.typed_data(),
      static_cast<int>(offsets.element_count() - 1), Rows(xs_q), static_cast<int>(Cols(xs_q)),
      static_cast<int>(Cols(*h)), w.typed_data(), w_scales.typed_data(), h->untyped_data(),
      S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedGateUpFp8, GroupedGateUpFp8Impl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::BF16>>());

// Per-token codes x_q [T, D] and scales [T], perm_src, offsets, packed gate/up
// and scales -> h [rows_cap, F] bf16 (rows gathered by the GEMM's loads).
static ffi::Error GroupedGateUpFp8GatherImpl(hipStream_t stream, ffi::Buffer<ffi::U8> x_q,
                                             ffi::Buffer<ffi::F32> x_scale,
                                             ffi::Buffer<ffi::S32> perm_src,
                                             ffi::Buffer<ffi::S32> offsets, ffi::Buffer<ffi::U8> w,
                                             ffi::Buffer<ffi::F32> w_scales, int64_t top_k,
                                             ffi::ResultBuffer<ffi::BF16> h) {
  return Status(hmoe_grouped_gate_up_fp8_gather(
      x_q.typed_data(), x_scale.typed_data(), Rows(x_q), static_cast<int>(top_k),
      perm_src.typed_data(), offsets.typed_data(), static_cast<int>(offsets.element_count() - 1),
      Rows(*h), static_cast<int>(Cols(x_q)), static_cast<int>(Cols(*h)), w.typed_data(),
      w_scales.typed_data(), h->untyped_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedGateUpFp8Gather, GroupedGateUpFp8GatherImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Attr<int64_t>("top_k")
                                  .Ret<ffi::Buffer<ffi::BF16>>());

static ffi::Error GroupedDownFp8Impl(hipStream_t stream, ffi::Buffer<ffi::U8> h_q,
                                     ffi::Buffer<ffi::F32> h_scale, ffi::Buffer<ffi::S32> offsets,
                                     ffi::Buffer<ffi::U8> w, ffi::Buffer<ffi::F32> w_scales,
                                     ffi::ResultBuffer<ffi::BF16> ys) {
  return Status(hmoe_grouped_down_fp8(
      h_q.typed_data(), h_scale.typed_data(), offsets.typed_data(),
      static_cast<int>(offsets.element_count() - 1), Rows(h_q), static_cast<int>(Cols(h_q)),
      static_cast<int>(Cols(*ys)), w.typed_data(), w_scales.typed_data(), ys->untyped_data(),
      S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedDownFp8, GroupedDownFp8Impl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::BF16>>());

// Block-scaled h: the gate/up GEMMs return codes [rows, F] and biased
// exponents [rows, F / 32]; the down GEMM takes both.
static ffi::Error GroupedGateUpFp8QhImpl(hipStream_t stream, ffi::Buffer<ffi::U8> xs_q,
                                         ffi::Buffer<ffi::F32> xs_scale,
                                         ffi::Buffer<ffi::S32> offsets, ffi::Buffer<ffi::U8> w,
                                         ffi::Buffer<ffi::F32> w_scales,
                                         ffi::ResultBuffer<ffi::U8> h_q,
                                         ffi::ResultBuffer<ffi::U8> h_exp) {
  return Status(hmoe_grouped_gate_up_fp8_qh(
      xs_q.typed_data(), xs_scale.typed_data(), offsets.typed_data(),
      static_cast<int>(offsets.element_count() - 1), Rows(xs_q), static_cast<int>(Cols(xs_q)),
      static_cast<int>(Cols(*h_q)), w.typed_data(), w_scales.typed_data(), h_q->typed_data(),
      h_exp->typed_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedGateUpFp8Qh, GroupedGateUpFp8QhImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::U8>>()
                                  .Ret<ffi::Buffer<ffi::U8>>());

static ffi::Error GroupedGateUpFp8GatherQhImpl(
    hipStream_t stream, ffi::Buffer<ffi::U8> x_q, ffi::Buffer<ffi::F32> x_scale,
    ffi::Buffer<ffi::S32> perm_src, ffi::Buffer<ffi::S32> offsets, ffi::Buffer<ffi::U8> w,
    ffi::Buffer<ffi::F32> w_scales, int64_t top_k, ffi::ResultBuffer<ffi::U8> h_q,
    ffi::ResultBuffer<ffi::U8> h_exp) {
  return Status(hmoe_grouped_gate_up_fp8_gather_qh(
      x_q.typed_data(), x_scale.typed_data(), Rows(x_q), static_cast<int>(top_k),
      perm_src.typed_data(), offsets.typed_data(), static_cast<int>(offsets.element_count() - 1),
      Rows(*h_q), static_cast<int>(Cols(x_q)), static_cast<int>(Cols(*h_q)), w.typed_data(),
      w_scales.typed_data(), h_q->typed_data(), h_exp->typed_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedGateUpFp8GatherQh, GroupedGateUpFp8GatherQhImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Attr<int64_t>("top_k")
                                  .Ret<ffi::Buffer<ffi::U8>>()
                                  .Ret<ffi::Buffer<ffi::U8>>());

static ffi::Error GroupedDownFp8MxImpl(hipStream_t stream, ffi::Buffer<ffi::U8> h_q,
                                       ffi::Buffer<ffi::U8> h_exp, ffi::Buffer<ffi::S32> offsets,
                                       ffi::Buffer<ffi::U8> w, ffi::Buffer<ffi::F32> w_scales,
                                       ffi::ResultBuffer<ffi::BF16> ys) {
  return Status(hmoe_grouped_down_fp8_mx(
      h_q.typed_data(), h_exp.typed_data(), offsets.typed_data(),
      static_cast<int>(offsets.element_count() - 1), Rows(h_q), static_cast<int>(Cols(h_q)),
      static_cast<int>(Cols(*ys)), w.typed_data(), w_scales.typed_data(), ys->untyped_data(),
      S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedDownFp8Mx, GroupedDownFp8MxImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::BF16>>());

// float32 compute dtype: masters as they are.
static ffi::Error GroupedGateUpF32Impl(hipStream_t stream, ffi::Buffer<ffi::F32> xs,
                                       ffi::Buffer<ffi::S32> offsets,
                                       ffi::Buffer<ffi::F32> w_gate, ffi::Buffer<ffi::F32> w_up,
                                       ffi::ResultBuffer<ffi::F32> h) {
  return Status(hmoe_grouped_gate_up_f32(
      xs.typed_data(), offsets.typed_data(), static_cast<int>(offsets.element_count() - 1),
      Rows(xs), static_cast<int>(Cols(xs)), static_cast<int>(Cols(*h)), w_gate.typed_data(),
      w_up.typed_data(), h->typed_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedGateUpF32, GroupedGateUpF32Impl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>());

static ffi::Error GroupedDownF32Impl(hipStream_t stream, ffi::Buffer<ffi::F32> h,
                                     ffi::Buffer<ffi::S32> offsets, ffi::Buffer<ffi::F32> w_down,
                                     ffi::ResultBuffer<ffi::F32> ys) {
  return Status(hmoe_grouped_down_f32(h.typed_data(), offsets.typed_data(),
                                      static_cast<int>(offsets.element_count() - 1), Rows(h),
                                      static_cast<int>(Cols(h)), static_cast<int>(Cols(*ys)),
                                      w_down.typed_data(), ys->typed_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedDownF32, GroupedDownF32Impl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>());

// ---- combine: moe.py:80-85 (+ the shared expert's output, moe.py:249-251) ---
// ys [rows, D] (bf16/f32), slot_pos [T*K], gates [T, K] f32, residual [T, D]
// (f32/bf16; pass a zero-size buffer for none) -> out [T, D] (f32/bf16).
static ffi::Error CombineImpl(hipStream_t stream, ffi::AnyBuffer ys,
                              ffi::Buffer<ffi::S32> slot_pos, ffi::Buffer<ffi::F32> gates,
                              ffi::AnyBuffer residual, ffi::Result<ffi::AnyBuffer> out) {
  const int yd = DtypeCode(ys.element_type()), od = DtypeCode(out->element_type());
  if (yd < 0 || od < 0) return BadDtype("hmoe_combine");
  const bool has_res = residual.element_count() > 0;
  const int rd = has_res ? DtypeCode(residual.element_type()) : HMOE_F32;
  if (rd < 0) return BadDtype("hmoe_combine residual");
  return Status(hmoe_combine(ys.untyped_data(), yd, slot_pos.typed_data(), gates.typed_data(),
                             has_res ? residual.untyped_data() : nullptr, rd, Rows(gates),
                             static_cast<int>(Cols(gates)), static_cast<int>(Cols(*out)),
                             out->untyped_data(), od, S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeCombine, CombineImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Ret<ffi::AnyBuffer>());

// ---- aux outputs: moe.py:253-292 --------------------------------------------
// logits [B*S, N] f32, top_idx [B*S, K] -> losses [3] f32 (z, balance,
// entropy), expert_counts [N] f32, workspace u8 (hmoe_aux_workspace_bytes).
static ffi::Error RouterAuxImpl(hipStream_t stream, ffi::Buffer<ffi::F32> logits,
                                ffi::Buffer<ffi::S32> top_idx, int64_t batch,
                                ffi::ResultBuffer<ffi::F32> losses,
                                ffi::ResultBuffer<ffi::F32> expert_counts,
                                ffi::ResultBuffer<ffi::U8> workspace) {
  const int64_t T = Rows(logits);
  const int B = static_cast<int>(batch);
  return Status(hmoe_router_aux(logits.typed_data(), top_idx.typed_data(), B,
                                static_cast<int>(B > 0 ? T / B : 0),
                                static_cast<int>(Cols(logits)), static_cast<int>(Cols(top_idx)),
                                losses->typed_data(), expert_counts->typed_data(),
                                workspace->untyped_data(), workspace->size_bytes(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeRouterAux, RouterAuxImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Attr<int64_t>("batch")
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::U8>>());

// ---- gate/up and down in one launch: moe.py:56, 70-74 -----------------------
// x [T, D] bf16, perm_src [rows_cap], offsets [N+1], packed gate/up, packed
// down -> h [rows_cap, F] bf16, ys [rows_cap, D] bf16, workspace u8
// (hmoe_grouped_swiglu_fused_workspace_bytes).  XLA hands over a fresh
// workspace per call, so it is zero-filled on the stream first.
static ffi::Error GroupedSwigluFusedImpl(hipStream_t stream, ffi::Buffer<ffi::BF16> x,
                                         ffi::Buffer<ffi::S32> perm_src,
                                         ffi::Buffer<ffi::S32> offsets, ffi::Buffer<ffi::U8> w_gu,
                                         ffi::Buffer<ffi::U8> w_dn, int64_t top_k,
                                         ffi::ResultBuffer<ffi::BF16> h,
                                         ffi::ResultBuffer<ffi::BF16> ys,
                                         ffi::ResultBuffer<ffi::U8> workspace) {
  if (int rc = hmoe_zero_fill(workspace->untyped_data(), workspace->size_bytes() & ~size_t{3},
                              S(stream)))
    return Status(rc);
  return Status(hmoe_grouped_swiglu_fused(
      x.untyped_data(), Rows(x), static_cast<int>(top_k), perm_src.typed_data(),
      offsets.typed_data(), static_cast<int>(offsets.element_count() - 1), Rows(*h),
      static_cast<int>(Cols(x)), static_cast<int>(Cols(*h)), w_gu.untyped_data(),
      w_dn.untyped_data(), h->untyped_data(), ys->untyped_data(), workspace->untyped_data(),
      workspace->size_bytes(), 0, 0, S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedSwigluFused, GroupedSwigluFusedImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Attr<int64_t>("top_k")
                                  .Ret<ffi::Buffer<ffi::BF16>>()
                                  .Ret<ffi::Buffer<ffi::BF16>>()
                                  .Ret<ffi::Buffer<ffi::U8>>());

// =============================================================================
// Backward: the VJP that jax.value_and_grad (train.py:266) takes of
// MoE.__call__ (moe.py:170-294), bound step by step by the jax.custom_vjp in
// hanuman_amd/xla_ffi/moe_jax.py.  Routing (top-k, drops, the plan) is held
// fixed.  Gradients that the C core accumulates into an existing buffer
// (hmoe_router_aux_bwd into d_logits, hmoe_router_dx into dx) take that
// buffer as an argument aliased to their result (ffi_call's
// input_output_aliases); without the alias the handler copies it over first.
// =============================================================================

namespace {
// Makes `out` hold `in` (same size) before an accumulating kernel runs.
ffi::Error CopyIfNotAliased(hipStream_t stream, const void* in, void* out, size_t bytes) {
  if (in == out || bytes == 0) return ffi::Error::Success();
  if (hipMemcpyAsync(out, in, bytes, hipMemcpyDeviceToDevice, stream) != hipSuccess)
    return ffi::Error(ffi::ErrorCode::kInternal, "hipMemcpyAsync failed");
  return ffi::Error::Success();
}
}  // namespace

// ---- combine VJP: moe.py:80-85 ------------------------------------------------
// dy [T, D] f32, ys [rows_cap, D] bf16, slot_pos [T*K], gates [T, K] f32 ->
// d_ys [rows_cap, D] bf16, d_gates [T, K] f32, d_shared [T, D] bf16 (a
// zero-size result for no shared expert; shared_div = n_shared_experts).
static ffi::Error CombineBwdImpl(hipStream_t stream, ffi::Buffer<ffi::F32> dy,
                                 ffi::Buffer<ffi::BF16> ys, ffi::Buffer<ffi::S32> slot_pos,
                                 ffi::Buffer<ffi::F32> gates, float shared_div,
                                 ffi::ResultBuffer<ffi::BF16> d_ys,
                                 ffi::ResultBuffer<ffi::F32> d_gates,
                                 ffi::ResultBuffer<ffi::BF16> d_shared) {
  void* dsh = d_shared->element_count() > 0 ? d_shared->untyped_data() : nullptr;
  return Status(hmoe_combine_bwd(dy.typed_data(), ys.untyped_data(), slot_pos.typed_data(),
                                 gates.typed_data(), Rows(gates), static_cast<int>(Cols(gates)),
                                 static_cast<int>(Cols(dy)), d_ys->untyped_data(),
                                 d_gates->typed_data(), dsh, shared_div, S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeCombineBwd, CombineBwdImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Attr<float>("shared_div")
                                  .Ret<ffi::Buffer<ffi::BF16>>()
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::BF16>>());

// ---- expert GEMM VJPs: moe.py:70-73 ---------------------------------------------
// g and u recomputed on the gathered rows: -> gu [rows_cap, 2F] bf16.
static ffi::Error GroupedGateUpRawGatherImpl(hipStream_t stream, ffi::Buffer<ffi::BF16> x,
                                             ffi::Buffer<ffi::S32> perm_src,
                                             ffi::Buffer<ffi::S32> offsets,
                                             ffi::Buffer<ffi::U8> w, int64_t top_k,
                                             ffi::ResultBuffer<ffi::BF16> gu) {
  return Status(hmoe_grouped_gate_up_raw_gather(
      x.untyped_data(), Rows(x), static_cast<int>(top_k), perm_src.typed_data(),
      offsets.typed_data(), static_cast<int>(offsets.element_count() - 1), Rows(*gu),
      static_cast<int>(Cols(x)), static_cast<int>(Cols(*gu) / 2), w.untyped_data(),
      gu->untyped_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedGateUpRawGather, GroupedGateUpRawGatherImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Attr<int64_t>("top_k")
                                  .Ret<ffi::Buffer<ffi::BF16>>());

// The same on rows given in order (the shared expert): xs [rows, D] bf16.
static ffi::Error GroupedGateUpRawImpl(hipStream_t stream, ffi::Buffer<ffi::BF16> xs,
                                       ffi::Buffer<ffi::S32> offsets, ffi::Buffer<ffi::U8> w,
                                       ffi::ResultBuffer<ffi::BF16> gu) {
  return Status(hmoe_grouped_gate_up_raw(
      xs.untyped_data(), offsets.typed_data(), static_cast<int>(offsets.element_count() - 1),
      Rows(xs), static_cast<int>(Cols(xs)), static_cast<int>(Cols(*gu) / 2), w.untyped_data(),
      gu->untyped_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedGateUpRaw, GroupedGateUpRawImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Ret<ffi::Buffer<ffi::BF16>>());

// Recompute with the SwiGLU VJP in the epilogue: dh [rows_cap, F] bf16 ->
// dgu [rows_cap, 2F] bf16 (gathered rows of x).
static ffi::Error GroupedGateUpSwigluBwdGatherImpl(hipStream_t stream, ffi::Buffer<ffi::BF16> x,
                                                   ffi::Buffer<ffi::S32> perm_src,
                                                   ffi::Buffer<ffi::S32> offsets,
                                                   ffi::Buffer<ffi::U8> w,
                                                   ffi::Buffer<ffi::BF16> dh, int64_t top_k,
                                                   ffi::ResultBuffer<ffi::BF16> dgu) {
  return Status(hmoe_grouped_gate_up_swiglu_bwd_gather(
      x.untyped_data(), Rows(x), static_cast<int>(top_k), perm_src.typed_data(),
      offsets.typed_data(), static_cast<int>(offsets.element_count() - 1), Rows(*dgu),
      static_cast<int>(Cols(x)), static_cast<int>(Cols(dh)), w.untyped_data(), dh.untyped_data(),
      dgu->untyped_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedGateUpSwigluBwdGather, GroupedGateUpSwigluBwdGatherImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Attr<int64_t>("top_k")
                                  .Ret<ffi::Buffer<ffi::BF16>>());

// The same on rows given in order (the shared expert).
static ffi::Error GroupedGateUpSwigluBwdImpl(hipStream_t stream, ffi::Buffer<ffi::BF16> xs,
                                             ffi::Buffer<ffi::S32> offsets,
                                             ffi::Buffer<ffi::U8> w, ffi::Buffer<ffi::BF16> dh,
                                             ffi::ResultBuffer<ffi::BF16> dgu) {
  return Status(hmoe_grouped_gate_up_swiglu_bwd(
      xs.untyped_data(), offsets.typed_data(), static_cast<int>(offsets.element_count() - 1),
      Rows(xs), static_cast<int>(Cols(xs)), static_cast<int>(Cols(dh)), w.untyped_data(),
      dh.untyped_data(), dgu->untyped_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedGateUpSwigluBwd, GroupedGateUpSwigluBwdImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::U8>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Ret<ffi::Buffer<ffi::BF16>>());

// The SwiGLU VJP alone (moe.py:72): dh [rows, F], gu [rows, 2F], offsets ->
// dgu [rows, 2F] bf16.
static ffi::Error SwigluBwdImpl(hipStream_t stream, ffi::Buffer<ffi::BF16> dh,
                                ffi::Buffer<ffi::BF16> gu, ffi::Buffer<ffi::S32> offsets,
                                ffi::ResultBuffer<ffi::BF16> dgu) {
  return Status(hmoe_swiglu_bwd(dh.untyped_data(), gu.untyped_data(), offsets.typed_data(),
                                static_cast<int>(offsets.element_count() - 1), Rows(dh),
                                static_cast<int>(Cols(dh)), dgu->untyped_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeSwigluBwd, SwigluBwdImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Ret<ffi::Buffer<ffi::BF16>>());

// Backward operands, packed once per parameter update: w_down [N, F, D] ->
// [N, F, D] bf16; w_gate, w_up [N, D, F] -> [N, D, 2F] bf16.
static ffi::Error PackDownDgradImpl(hipStream_t stream, ffi::AnyBuffer wd,
                                    ffi::ResultBuffer<ffi::BF16> packed) {
  const int d = DtypeCode(wd.element_type());
  if (d < 0) return BadDtype("hmoe_pack_down_dgrad");
  auto dims = wd.dimensions();
  return Status(hmoe_pack_down_dgrad(wd.untyped_data(), d, static_cast<int>(dims[0]),
                                     static_cast<int>(dims[1]), static_cast<int>(dims[2]),
                                     packed->untyped_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoePackDownDgrad, PackDownDgradImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Ret<ffi::Buffer<ffi::BF16>>());

static ffi::Error PackGateUpDgradImpl(hipStream_t stream, ffi::AnyBuffer wg, ffi::AnyBuffer wu,
                                      ffi::ResultBuffer<ffi::BF16> packed) {
  const int d = DtypeCode(wg.element_type());
  if (d < 0 || DtypeCode(wu.element_type()) != d) return BadDtype("hmoe_pack_gate_up_dgrad");
  auto dims = wg.dimensions();
  return Status(hmoe_pack_gate_up_dgrad(wg.untyped_data(), wu.untyped_data(), d,
                                        static_cast<int>(dims[0]), static_cast<int>(dims[1]),
                                        static_cast<int>(dims[2]), packed->untyped_data(),
                                        S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoePackGateUpDgrad, PackGateUpDgradImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Ret<ffi::Buffer<ffi::BF16>>());

// dh = d_ys Wd^T: d_ys [rows_cap, D] bf16, offsets, packed [N, F, D] ->
// dh [rows_cap, F] bf16.
static ffi::Error GroupedDgradDownImpl(hipStream_t stream, ffi::Buffer<ffi::BF16> d_ys,
                                       ffi::Buffer<ffi::S32> offsets,
                                       ffi::Buffer<ffi::BF16> w_down_dgrad,
                                       ffi::ResultBuffer<ffi::BF16> dh) {
  return Status(hmoe_grouped_dgrad_down(
      d_ys.untyped_data(), offsets.typed_data(), static_cast<int>(offsets.element_count() - 1),
      Rows(d_ys), static_cast<int>(Cols(d_ys)), static_cast<int>(Cols(*dh)),
      w_down_dgrad.untyped_data(), dh->untyped_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedDgradDown, GroupedDgradDownImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Ret<ffi::Buffer<ffi::BF16>>());

// d_xs = dg Wg^T + du Wu^T: dgu [rows_cap, 2F], offsets, packed [N, D, 2F] ->
// d_xs [rows_cap, D] bf16.
static ffi::Error GroupedDgradGateUpImpl(hipStream_t stream, ffi::Buffer<ffi::BF16> dgu,
                                         ffi::Buffer<ffi::S32> offsets,
                                         ffi::Buffer<ffi::BF16> w_gu_dgrad,
                                         ffi::ResultBuffer<ffi::BF16> d_xs) {
  return Status(hmoe_grouped_dgrad_gate_up(
      dgu.untyped_data(), offsets.typed_data(), static_cast<int>(offsets.element_count() - 1),
      Rows(dgu), static_cast<int>(Cols(*d_xs)), static_cast<int>(Cols(dgu) / 2),
      w_gu_dgrad.untyped_data(), d_xs->untyped_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedDgradGateUp, GroupedDgradGateUpImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Ret<ffi::Buffer<ffi::BF16>>());

// ---- gather VJP: moe.py:56 --------------------------------------------------------
// d_xs [rows_cap, D] (f32/bf16), slot_pos [T*K], residual [T, D] (f32/bf16;
// zero-size for none) -> dx [T, D] (f32/bf16).
static ffi::Error GatherBwdImpl(hipStream_t stream, ffi::AnyBuffer d_xs,
                                ffi::Buffer<ffi::S32> slot_pos, ffi::AnyBuffer residual,
                                ffi::Result<ffi::AnyBuffer> dx) {
  const int xd = DtypeCode(d_xs.element_type()), od = DtypeCode(dx->element_type());
  if (xd < 0 || od < 0) return BadDtype("hmoe_gather_bwd");
  const bool has_res = residual.element_count() > 0;
  const int rd = has_res ? DtypeCode(residual.element_type()) : HMOE_F32;
  if (rd < 0) return BadDtype("hmoe_gather_bwd residual");
  const int64_t T = Rows(*dx);
  const int K = static_cast<int>(slot_pos.element_count() / (T > 0 ? T : 1));
  return Status(hmoe_gather_bwd(d_xs.untyped_data(), xd, slot_pos.typed_data(),
                                has_res ? residual.untyped_data() : nullptr, rd, T, K,
                                static_cast<int>(Cols(*dx)), dx->untyped_data(), od, S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGatherBwd, GatherBwdImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Ret<ffi::AnyBuffer>());

// ---- router VJPs: moe.py:175-192, 253-283 ------------------------------------------
// logits [T, N], top_idx [T, K], gates [T, K], d_gates [T, K] -> d_logits [T, N].
static ffi::Error RouterBwdImpl(hipStream_t stream, ffi::Buffer<ffi::F32> logits,
                                ffi::Buffer<ffi::S32> top_idx, ffi::Buffer<ffi::F32> gates,
                                ffi::Buffer<ffi::F32> d_gates, int64_t mode, float rsf,
                                ffi::ResultBuffer<ffi::F32> d_logits) {
  return Status(hmoe_router_bwd(logits.typed_data(), top_idx.typed_data(), gates.typed_data(),
                                d_gates.typed_data(), Rows(logits),
                                static_cast<int>(Cols(logits)), static_cast<int>(Cols(top_idx)),
                                static_cast<int>(mode), rsf, d_logits->typed_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeRouterBwd, RouterBwdImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Attr<int64_t>("mode")
                                  .Attr<float>("routed_scaling_factor")
                                  .Ret<ffi::Buffer<ffi::F32>>());

// The aux losses' VJP added into d_logits: logits [B*S, N], top_idx,
// d_losses [3] f32, d_logits_in [B*S, N] (aliased to the first result) ->
// d_logits [B*S, N], workspace u8 (hmoe_aux_bwd_workspace_bytes).
static ffi::Error RouterAuxBwdImpl(hipStream_t stream, ffi::Buffer<ffi::F32> logits,
                                   ffi::Buffer<ffi::S32> top_idx, ffi::Buffer<ffi::F32> d_losses,
                                   ffi::Buffer<ffi::F32> d_logits_in, int64_t batch,
                                   ffi::ResultBuffer<ffi::F32> d_logits,
                                   ffi::ResultBuffer<ffi::U8> workspace) {
  if (auto e = CopyIfNotAliased(stream, d_logits_in.untyped_data(), d_logits->untyped_data(),
                                d_logits->size_bytes());
      e.failure())
    return e;
  const int64_t T = Rows(logits);
  const int B = static_cast<int>(batch);
  return Status(hmoe_router_aux_bwd(logits.typed_data(), top_idx.typed_data(), B,
                                    static_cast<int>(B > 0 ? T / B : 0),
                                    static_cast<int>(Cols(logits)),
                                    static_cast<int>(Cols(top_idx)), d_losses.typed_data(),
                                    d_logits->typed_data(), 1, workspace->untyped_data(),
                                    workspace->size_bytes(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeRouterAuxBwd, RouterAuxBwdImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Attr<int64_t>("batch")
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::U8>>());

// dx += d_logits router^T: d_logits [T, N], router_w [D, N] (f32/bf16),
// dx_in [T, D] f32 (aliased to the result) -> dx [T, D] f32.
static ffi::Error RouterDxImpl(hipStream_t stream, ffi::Buffer<ffi::F32> d_logits,
                               ffi::AnyBuffer router_w, ffi::Buffer<ffi::F32> dx_in,
                               ffi::ResultBuffer<ffi::F32> dx) {
  const int wd = DtypeCode(router_w.element_type());
  if (wd < 0) return BadDtype("hmoe_router_dx router_w");
  if (auto e = CopyIfNotAliased(stream, dx_in.untyped_data(), dx->untyped_data(),
                                dx->size_bytes());
      e.failure())
    return e;
  return Status(hmoe_router_dx(d_logits.typed_data(), router_w.untyped_data(), wd,
                               Rows(d_logits), static_cast<int>(Cols(*dx)),
                               static_cast<int>(Cols(d_logits)), dx->typed_data(), 1, S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeRouterDx, RouterDxImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>());

// ---- weight gradients --------------------------------------------------------------
// dWd = h^T d_ys per segment: h [rows_cap, F], d_ys [rows_cap, D] bf16 ->
// dw_down [N, F, D] f32.
static ffi::Error GroupedWgradDownImpl(hipStream_t stream, ffi::Buffer<ffi::BF16> h,
                                       ffi::Buffer<ffi::BF16> d_ys,
                                       ffi::Buffer<ffi::S32> offsets,
                                       ffi::ResultBuffer<ffi::F32> dw_down) {
  return Status(hmoe_grouped_wgrad_down(
      h.untyped_data(), d_ys.untyped_data(), offsets.typed_data(),
      static_cast<int>(offsets.element_count() - 1), Rows(h), static_cast<int>(Cols(h)),
      static_cast<int>(Cols(d_ys)), dw_down->typed_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedWgradDown, GroupedWgradDownImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>());

// dWg | dWu = xs^T dg | du: xs [rows_cap, D], dgu [rows_cap, 2F] bf16 ->
// dw_gate, dw_up [N, D, F] f32.
static ffi::Error GroupedWgradGateUpImpl(hipStream_t stream, ffi::Buffer<ffi::BF16> xs,
                                         ffi::Buffer<ffi::BF16> dgu,
                                         ffi::Buffer<ffi::S32> offsets,
                                         ffi::ResultBuffer<ffi::F32> dw_gate,
                                         ffi::ResultBuffer<ffi::F32> dw_up) {
  return Status(hmoe_grouped_wgrad_gate_up(
      xs.untyped_data(), dgu.untyped_data(), offsets.typed_data(),
      static_cast<int>(offsets.element_count() - 1), Rows(xs), static_cast<int>(Cols(xs)),
      static_cast<int>(Cols(dgu) / 2), dw_gate->typed_data(), dw_up->typed_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedWgradGateUp, GroupedWgradGateUpImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>());

// d_router = x^T d_logits: x [T, D] (f32/bf16), d_logits [T, N] f32 ->
// d_router [D, N] f32, workspace u8 (hmoe_router_dw_workspace_bytes).
static ffi::Error RouterDwImpl(hipStream_t stream, ffi::AnyBuffer x,
                               ffi::Buffer<ffi::F32> d_logits,
                               ffi::ResultBuffer<ffi::F32> d_router,
                               ffi::ResultBuffer<ffi::U8> workspace) {
  const int xd = DtypeCode(x.element_type());
  if (xd < 0) return BadDtype("hmoe_router_dw x");
  return Status(hmoe_router_dw(x.untyped_data(), xd, d_logits.typed_data(), Rows(x),
                               static_cast<int>(Cols(x)), static_cast<int>(Cols(d_logits)),
                               d_router->typed_data(), workspace->untyped_data(),
                               workspace->size_bytes(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeRouterDw, RouterDwImpl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::U8>>());

// ---- float32 compute dtype: the same VJP on the float32 kernels -------------------
static ffi::Error CombineBwdF32Impl(hipStream_t stream, ffi::Buffer<ffi::F32> dy,
                                    ffi::Buffer<ffi::F32> ys, ffi::Buffer<ffi::S32> slot_pos,
                                    ffi::Buffer<ffi::F32> gates, float shared_div,
                                    ffi::ResultBuffer<ffi::F32> d_ys,
                                    ffi::ResultBuffer<ffi::F32> d_gates,
                                    ffi::ResultBuffer<ffi::F32> d_shared) {
  float* dsh = d_shared->element_count() > 0 ? d_shared->typed_data() : nullptr;
  return Status(hmoe_combine_bwd_f32(dy.typed_data(), ys.typed_data(), slot_pos.typed_data(),
                                     gates.typed_data(), Rows(gates),
                                     static_cast<int>(Cols(gates)), static_cast<int>(Cols(dy)),
                                     d_ys->typed_data(), d_gates->typed_data(), dsh, shared_div,
                                     S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeCombineBwdF32, CombineBwdF32Impl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Attr<float>("shared_div")
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>());

static ffi::Error GroupedDgradDownF32Impl(hipStream_t stream, ffi::Buffer<ffi::F32> d_ys,
                                          ffi::Buffer<ffi::S32> offsets,
                                          ffi::Buffer<ffi::F32> w_down,
                                          ffi::ResultBuffer<ffi::F32> dh) {
  return Status(hmoe_grouped_dgrad_down_f32(
      d_ys.typed_data(), offsets.typed_data(), static_cast<int>(offsets.element_count() - 1),
      Rows(d_ys), static_cast<int>(Cols(d_ys)), static_cast<int>(Cols(*dh)), w_down.typed_data(),
      dh->typed_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedDgradDownF32, GroupedDgradDownF32Impl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>());

static ffi::Error GroupedGateUpSwigluBwdF32Impl(hipStream_t stream, ffi::Buffer<ffi::F32> xs,
                                                ffi::Buffer<ffi::S32> offsets,
                                                ffi::Buffer<ffi::F32> w_gate,
                                                ffi::Buffer<ffi::F32> w_up,
                                                ffi::Buffer<ffi::F32> dh,
                                                ffi::ResultBuffer<ffi::F32> dgu) {
  return Status(hmoe_grouped_gate_up_swiglu_bwd_f32(
      xs.typed_data(), offsets.typed_data(), static_cast<int>(offsets.element_count() - 1),
      Rows(xs), static_cast<int>(Cols(xs)), static_cast<int>(Cols(dh)), w_gate.typed_data(),
      w_up.typed_data(), dh.typed_data(), dgu->typed_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedGateUpSwigluBwdF32, GroupedGateUpSwigluBwdF32Impl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>());

static ffi::Error GroupedDgradGateUpF32Impl(hipStream_t stream, ffi::Buffer<ffi::F32> dgu,
                                            ffi::Buffer<ffi::S32> offsets,
                                            ffi::Buffer<ffi::F32> w_gate,
                                            ffi::Buffer<ffi::F32> w_up,
                                            ffi::ResultBuffer<ffi::F32> d_xs) {
  return Status(hmoe_grouped_dgrad_gate_up_f32(
      dgu.typed_data(), offsets.typed_data(), static_cast<int>(offsets.element_count() - 1),
      Rows(dgu), static_cast<int>(Cols(*d_xs)), static_cast<int>(Cols(dgu) / 2),
      w_gate.typed_data(), w_up.typed_data(), d_xs->typed_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedDgradGateUpF32, GroupedDgradGateUpF32Impl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>());

static ffi::Error GroupedWgradGateUpF32Impl(hipStream_t stream, ffi::Buffer<ffi::F32> xs,
                                            ffi::Buffer<ffi::F32> dgu,
                                            ffi::Buffer<ffi::S32> offsets,
                                            ffi::ResultBuffer<ffi::F32> dw_gate,
                                            ffi::ResultBuffer<ffi::F32> dw_up) {
  return Status(hmoe_grouped_wgrad_gate_up_f32(
      xs.typed_data(), dgu.typed_data(), offsets.typed_data(),
      static_cast<int>(offsets.element_count() - 1), static_cast<int>(Cols(xs)),
      static_cast<int>(Cols(dgu) / 2), dw_gate->typed_data(), dw_up->typed_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedWgradGateUpF32, GroupedWgradGateUpF32Impl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>());

static ffi::Error GroupedWgradDownF32Impl(hipStream_t stream, ffi::Buffer<ffi::F32> h,
                                          ffi::Buffer<ffi::F32> d_ys,
                                          ffi::Buffer<ffi::S32> offsets,
                                          ffi::ResultBuffer<ffi::F32> dw_down) {
  return Status(hmoe_grouped_wgrad_down_f32(
      h.typed_data(), d_ys.typed_data(), offsets.typed_data(),
      static_cast<int>(offsets.element_count() - 1), static_cast<int>(Cols(h)),
      static_cast<int>(Cols(d_ys)), dw_down->typed_data(), S(stream)));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(HmoeGroupedWgradDownF32, GroupedWgradDownF32Impl,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::S32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>());
