"""MoE-layer forward benchmark on one MI355X.

Times the whole layer (router -> dispatch plan -> row permutation -> grouped
SwiGLU GEMMs -> weighted combine) on the full bf16 workload (16384 tokens,
d_model 2048, 64 experts, top-8, d_ff 1024, capacity factor 1.25), with every
input resident in HBM before the timed region.  One JSON line on stdout:

  value      tokens/s of the whole layer (1 GPU)
  roofline   the dominant kernel, the gate/up grouped GEMM with the fused SwiGLU:
             algorithmic 4*R_kept*D*F FLOP over its HIP-event time, against the
             dense bf16 (or fp8) MFMA peak; traffic = its measured HBM bytes per
             launch (profiles/hbm_traffic.json)
  grouped_gemm  gate/up + down together (6*R_kept*D*F FLOP)
  kernels    every stage's HIP-event time and roofline fraction, and its fraction of
             the ceiling measured on the box (frac_of_ceiling)
  ceilings   a 1 GiB device copy and the vendor library's dense bf16 GEMM (8192^3),
             timed in the same process after the timed steps
  cpu_baseline  the NumPy float32 restatement of the layer (oracle/) timed on
             this host's cores on up to 16384 tokens of the same workload (all of
             the headline workload)

With --backward the line is the layer backward instead (bf16 SwiGLU
workloads): data and weight gradients, timed per stage the same way, for the
cotangent of the layer output; the forward's intermediates are computed once
before the timed region.

With --train the line is one training step of the drop-in module
(hanuman_amd.moe.MoE at the workload's shape, plus its one shared expert):
forward, loss.backward() through the module's autograd node (output, z and
balance losses, as train.py:191-200), and an in-place parameter update, so
every step re-packs the expert operands as a trainer's step does.

Usage: python bench.py [--steps K] [--warmup W] [--spinup-ms MS] [--workload NAME] [--no-cpu-baseline] [--backward | --train]
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s
FP8_PEAK_TFLOPS = 5000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


FP64_PEAK_TFLOPS = 78.6       # MI355X dense fp64 MFMA
FP32_PEAK_TFLOPS = 157.3      # MI355X dense fp32 MFMA


def algorithmic(wl, kept_rows: int) -> dict:
    """Per-launch algorithmic work of each stage: (bound, amount, peak)."""
    T, D, N, K, F = wl.tokens, wl.d_model, wl.n_experts, wl.top_k, wl.d_ff
    R = T * K
    fp8 = wl.expert_dtype == "fp8"
    f32 = wl.expert_dtype == "f32"
    ex = 1 if fp8 else (4 if f32 else 2)  # dispatched activation bytes
    x_in = 4 if wl.x_dtype == "f32" else 2
    out_b = 4 if wl.out_dtype == "f32" else 2
    w_b = 2 if wl.router_w_dtype == "bf16" else 4
    mfma_peak = FP8_PEAK_TFLOPS if fp8 else (FP32_PEAK_TFLOPS if f32 else BF16_PEAK_TFLOPS)
    w = {}
    if wl.router_from_logits:
        w["router"] = ("hbm", T * N * 4 + T * K * 8, HBM_PEAK_GBS)
    else:
        # float64 matrix-core dot products (the bit-exact logit recipe)
        w["router"] = ("fp64", 2 * T * D * N, FP64_PEAK_TFLOPS)
    w["plan"] = ("hbm", 2 * R * 4 + R * 4 + R * 4 + R + N * 8, HBM_PEAK_GBS)
    # dispatch: read every token once, write the kept rows (+ scales), read the slot map
    w["permute"] = ("hbm", T * D * x_in + kept_rows * (D * ex + (4 if fp8 else 0)) + R * 4,
                    HBM_PEAK_GBS)
    # fp8 on bf16 tokens: x quantised per token (read once, codes and scales written)
    w["quant_x"] = ("hbm", T * D * x_in + T * D + T * 4, HBM_PEAK_GBS)
    # the same quantisation in the router's launch, beside its float64 MFMA
    # chains, which bound the launch: priced by the router's work
    w["router_quant_x"] = w["router"]
    if wl.expert == "swiglu":
        w["gate_up"] = ("mfma", 2 * 2 * kept_rows * D * F, mfma_peak)
        w["down"] = ("mfma", 2 * kept_rows * F * D, mfma_peak)
        # gate/up and down in one persistent launch (--fused-ffn)
        w["ffn"] = ("mfma", 6 * kept_rows * D * F, mfma_peak)
    # combine: read kept rows (bf16), write tokens, read slot map and gates
    w["combine"] = ("hbm", kept_rows * D * 2 + T * D * out_b + R * 8, HBM_PEAK_GBS)
    return w


def measured_traffic(workload: str) -> dict:
    """HBM bytes per launch by kernel name, from the counter summary committed
    in profiles/hbm_traffic.json (FETCH_SIZE/WRITE_SIZE runs calibrated against
    a 1 GiB copy); empty when the workload was not measured."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return {}
    return {k: v["total"] for k, v in data.get("workloads", {}).get(workload, {}).items()}


def measured_ceilings(dev) -> dict:
    """Ceilings measured on this GPU in this process, outside every timed
    region: a 1 GiB device-to-device copy (GB/s counting the bytes read and
    written) and the vendor library's dense bf16 GEMM at 8192^3 on random
    operands (torch.matmul, hipBLASLt).  Each runs back to back for 200 ms,
    then three batches of back-to-back calls are timed between two events;
    the median batch gives the rate."""
    import torch

    def batch_ms(fn, calls):
        t_end = time.perf_counter() + 0.2
        while time.perf_counter() < t_end:
            fn()
        torch.cuda.synchronize()
        times = []
        for _ in range(3):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(calls):
                fn()
            b.record()
            torch.cuda.synchronize()
            times.append(a.elapsed_time(b) / calls)
        return float(np.median(times))

    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    copy_ms = batch_ms(lambda: dst.copy_(src), 10)
    del src, dst
    n = 8192
    a = torch.randn(n, n, device=dev, dtype=torch.bfloat16)
    b = torch.randn(n, n, device=dev, dtype=torch.bfloat16)
    gemm_ms = batch_ms(lambda: torch.matmul(a, b), 20)
    del a, b
    torch.cuda.empty_cache()
    return {"hbm_copy_gbs": round(2 * (1 << 30) / (copy_ms / 1e3) / 1e9, 1),
            "dense_bf16_gemm_tflops": round(2 * n ** 3 / (gemm_ms / 1e3) / 1e12, 1),
            "how": "1 GiB device copy (bytes read + written), 10 back to back, and torch.matmul "
                   "bf16 8192^3 on random operands (hipBLASLt), 20 back to back; 200 ms of "
                   "spin-up each, median of 3 batches, same process, after the timed steps"}


def cpu_baseline(wl_name: str, sample_tokens: int, seed: int) -> dict:
    import oracle as O
    from hanuman_amd import workloads as W
    cores = len(os.sched_getaffinity(0))
    full = W.WORKLOADS[wl_name]
    wl = full.scaled(min(sample_tokens, full.tokens))
    inp = W.make_inputs(wl, seed=seed)
    params = {"router": inp.router, "expert_w_gate": inp.w_gate, "expert_w_up": inp.w_up,
              "expert_w_down": inp.w_down}
    kw = dict(top_k=wl.top_k, routing=wl.routing, capacity_factor=wl.capacity_factor,
              expert=wl.expert, dtype="bf16" if wl.x_dtype == "bf16" else "f32",
              precision="f32", fast_router=True,
              logits=inp.logits if wl.router_from_logits else None)
    O.moe_forward(inp.x, params, **kw)                      # warm-up
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        O.moe_forward(inp.x, params, **kw)
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    try:
        model = subprocess.run(["bash", "-c", "lscpu | grep 'Model name' | head -1"],
                               capture_output=True, text=True, timeout=10).stdout.split(":")[-1].strip()
    except Exception:  # noqa: BLE001 -- informational only
        model = "unknown"
    note = (" (float32 experts: the e4m3 expert path has no CPU-native form)"
            if wl.expert_dtype == "fp8" else "")
    return {"value": round(wl.tokens / t, 1), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": (f"{wl.tokens} tokens of the {wl_name} layer (same shape, seed {seed}), "
                       f"NumPy float32 restatement of model/moe.py with OpenBLAS{note}, median "
                       f"of 3 after 1 warm-up, {cores} threads, CPU {model}")}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--spinup-ms", type=float, default=400.0,
                    help="keep running untimed warm-up steps until this much time has passed")
    ap.add_argument("--workload", default=None)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-tokens", type=int, default=16384,
                    help="tokens of the CPU-baseline sample (capped at the workload's; the "
                         "default is the whole headline workload, ~10 s of CPU work)")
    ap.add_argument("--train", action="store_true",
                    help="time one training step of the MoE module (forward, backward, update)")
    ap.add_argument("--fused-ffn", action="store_true",
                    help="run the bf16 gate/up and down GEMMs as one persistent launch "
                         "(hmoe_grouped_swiglu_fused) instead of two")
    ap.add_argument("--backward", action="store_true",
                    help="time the data-gradient backward pass instead of the forward")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run one 1 GiB device-to-device copy before the warm-up, as the "
                         "known-size reference for HBM byte counters")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: the MoE layer holds every expert in one MI355X's HBM "
              f"and this build has no multi-GPU path (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE {world})", file=sys.stderr)
        sys.exit(2)
    cores = len(os.sched_getaffinity(0))
    os.environ.setdefault("OPENBLAS_NUM_THREADS", str(cores))

    import torch
    from hanuman_amd import workloads as W
    from hanuman_amd.layer import DeviceLayer

    name = args.workload or W.HEADLINE
    wl = W.WORKLOADS[name]
    dev = torch.device("cuda:0")
    log(f"[bench] workload {name}: T={wl.tokens} D={wl.d_model} N={wl.n_experts} "
        f"K={wl.top_k} F={wl.d_ff} CF={wl.capacity_factor}")
    inp = W.make_inputs(wl, seed=args.seed)
    layer = DeviceLayer(inp, dev, fused_ffn=args.fused_ffn)
    del inp
    torch.cuda.synchronize()

    fp8 = wl.expert_dtype == "fp8"
    if args.backward:
        bench_backward(args, name, wl, layer)
        return
    if args.train:
        del layer
        bench_train(args, name, wl)
        return
    # bf16 SwiGLU experts: the row permutation is done by the gate/up GEMM's
    # own loads (no dispatched copy of x), so there is no separate stage.
    fused = layer.fused_dispatch
    fp8_gather = layer.fp8_gather
    # fp8 on bf16 tokens: x's quantisation runs inside the router's launch
    quant_in_router = fp8_gather and layer.logits_in is None
    if fp8_gather:
        dispatch_stages = [] if quant_in_router else ["quant_x"]
    else:
        dispatch_stages = [] if fused else ["permute"]
    stages = ["router_quant_x" if quant_in_router else "router", "plan"] + dispatch_stages
    if wl.expert == "swiglu":
        stages += (["gate_up", "down"] if fp8 else
                   ["ffn"] if layer.fused_ffn else ["gate_up", "down"])
    stages += ["combine"]

    def step(ev=None):
        """One layer forward; with ``ev`` records an event after each stage."""
        import hanuman_amd.kernels as K
        marks = iter(ev) if ev is not None else None

        def mark():
            if marks is not None:
                next(marks).record()

        mark()
        logits, top_idx, gates, xq = layer.route_quant()
        mark()
        plan = K.dispatch_plan(top_idx, wl.n_experts, layer.capacity, layer.workspace)
        mark()
        if fp8 and fp8_gather:
            if xq is None:
                x_q, x_s = K.quantize_rows_fp8(layer.x)
                mark()
            else:
                x_q, x_s = xq
            h_q, h_e = K.grouped_gate_up_fp8_gather_qh(x_q, x_s, plan, layer.w_gate_up,
                                                       layer.w_gate_up_scale)
            mark()
            ys = K.grouped_down_fp8_mx(h_q, h_e, plan.offsets, layer.w_down, layer.w_down_scale)
            mark()
        elif fp8:
            xs_q, xs_s = K.permute_rows_fp8(layer.x, plan)
            mark()
            h_q, h_e = K.grouped_gate_up_fp8_qh(xs_q, xs_s, plan.offsets, layer.w_gate_up,
                                                layer.w_gate_up_scale)
            mark()
            ys = K.grouped_down_fp8_mx(h_q, h_e, plan.offsets, layer.w_down, layer.w_down_scale)
            mark()
        elif layer.fused_ffn:
            h, ys, _ = K.grouped_swiglu_fused(layer.x, plan, layer.w_gate_up, layer.w_down,
                                              layer.fused_ws)
            mark()
        elif fused:
            h = K.grouped_gate_up_gather(layer.x, plan, layer.w_gate_up)
            mark()
            ys = K.grouped_down(h, plan.offsets, layer.w_down)
            mark()
        else:
            xs = K.permute_rows(layer.x, plan, torch.float32 if layer.f32 else torch.bfloat16)
            mark()
            if wl.expert == "swiglu" and layer.f32:
                h = K.grouped_gate_up_f32(xs, plan.offsets, layer.w_gate, layer.w_up)
                mark()
                ys = K.grouped_down_f32(h, plan.offsets, layer.w_down_f32)
                mark()
            elif wl.expert == "swiglu":
                h = K.grouped_gate_up(xs, plan.offsets, layer.w_gate_up)
                mark()
                ys = K.grouped_down(h, plan.offsets, layer.w_down)
                mark()
            else:
                ys = xs
        out = K.combine(ys, plan, gates, None, layer.out_dtype)
        mark()
        return plan, out

    if args.copy_calibration:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        torch.cuda.empty_cache()

    # Warm-up: at least `warmup` steps and at least `spinup_ms` of back-to-back
    # work, because the GPU clock ramps up over tens of milliseconds of load
    # (a 20-step burst right after set-up runs ~10 % slower than steady state).
    t_warm = time.perf_counter()
    warm_steps = 0
    while warm_steps < args.warmup or (time.perf_counter() - t_warm) * 1e3 < args.spinup_ms:
        step()
        warm_steps += 1
        if warm_steps % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()

    # Timed region: exactly `steps` layer forwards back to back, as a caller
    # runs them (no events between the kernels).
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record()
    plan = None
    for s in range(args.steps):
        plan, _ = step()
    t_end.record()
    torch.cuda.synchronize()
    ms_total = t_start.elapsed_time(t_end)
    ms_per_step = ms_total / args.steps
    # Stage breakdown: the same number of steps again, outside the total, with
    # an event after every stage (each event adds a few microseconds between
    # the kernels, so the stage pass runs a little longer than the total).
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(stages) + 1)]
           for _ in range(args.steps)]
    torch.cuda.synchronize()
    for s in range(args.steps):
        step(evs[s])
    torch.cuda.synchronize()
    stage_ms = {st: float(np.mean([evs[s][j].elapsed_time(evs[s][j + 1]) for s in range(args.steps)]))
                for j, st in enumerate(stages)}
    stage_pass_ms = float(np.mean([evs[s][0].elapsed_time(evs[s][-1]) for s in range(args.steps)]))
    if layer.fused_ffn:
        import hanuman_amd.kernels as K
        # the status word holds the last launch's outcome (bit 0: a down
        # tile's bounded wait gave up and computed from an incomplete h)
        if K.fused_status(layer.fused_ws) != 0:
            raise SystemExit("bench: the fused gate/up + down launch reported a timed-out wait")
    kept = int(plan.offsets[-1].item())
    work = algorithmic(wl, kept)
    # The bf16 layer gathers its rows inside the gate/up GEMM, so the layer
    # has no separate dispatch.  The standalone dispatch kernel
    # (hmoe_permute_rows: each token row read once, written to its kept
    # slots) is timed here on the same plan, after the layer's timed region
    # and outside its total, so the line carries the dispatch HBM rate.
    dispatch_ms = None
    if fused:
        import hanuman_amd.kernels as K
        for _ in range(3):
            K.permute_rows(layer.x, plan, torch.bfloat16)
        ev_d = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        torch.cuda.synchronize()
        ev_d[0].record()
        for _ in range(args.steps):
            K.permute_rows(layer.x, plan, torch.bfloat16)
        ev_d[1].record()
        torch.cuda.synchronize()
        dispatch_ms = ev_d[0].elapsed_time(ev_d[1]) / args.steps
    ceilings = measured_ceilings(dev)
    kernels = {}
    for st in stages:
        kind, amount, peak = work[st]
        t = stage_ms[st] / 1e3
        if kind == "hbm":
            ach = amount / t / 1e9
            kernels[st] = {"ms": round(stage_ms[st], 4), "bound": "hbm", "achieved": round(ach, 1),
                           "unit": "GB/s", "peak": peak, "frac": round(ach / peak, 4), "bytes": amount,
                           "frac_of_ceiling": round(ach / ceilings["hbm_copy_gbs"], 4)}
        else:
            ach = amount / t / 1e12
            kernels[st] = {"ms": round(stage_ms[st], 4), "bound": kind, "achieved": round(ach, 1),
                           "unit": "TFLOP/s", "peak": peak, "frac": round(ach / peak, 4),
                           "flop": amount}
            if peak == BF16_PEAK_TFLOPS:
                kernels[st]["frac_of_ceiling"] = round(ach / ceilings["dense_bf16_gemm_tflops"], 4)
    if dispatch_ms is not None:
        kind, amount, peak = work["permute"]
        ach = amount / (dispatch_ms / 1e3) / 1e9
        kernels["dispatch_permute"] = {
            "ms": round(dispatch_ms, 4), "bound": "hbm", "achieved": round(ach, 1), "unit": "GB/s",
            "peak": peak, "frac": round(ach / peak, 4), "bytes": amount,
            "frac_of_ceiling": round(ach / ceilings["hbm_copy_gbs"], 4),
            "note": "hmoe_permute_rows on the step's plan, timed after the layer and outside "
                    "its total (the layer fuses the gather into the gate/up GEMM)"}
    tokens_per_s = wl.tokens / (ms_per_step / 1e3)
    traffic = measured_traffic(name)
    grouped_gemm = None
    if wl.expert == "swiglu" and layer.fused_ffn:
        # Dominant kernel: the one launch of both grouped GEMMs.
        kname = "grouped_swiglu_fused"
        flop, peak = work["ffn"][1], work["ffn"][2]
        ach = flop / (stage_ms["ffn"] / 1e3) / 1e12
        roofline = {"kernel": kname, "bound": "mfma", "achieved": round(ach, 1), "peak": peak,
                    "unit": "TFLOP/s", "frac": round(ach / peak, 4),
                    "traffic": traffic.get(kname), "flop_per_launch": flop,
                    "ms": round(stage_ms["ffn"], 4)}
        grouped_gemm = {"kernels": "gate/up + down (one launch)", "flop": flop,
                        "ms": round(stage_ms["ffn"], 4), "achieved": round(ach, 1),
                        "unit": "TFLOP/s", "frac": round(ach / peak, 4)}
    elif wl.expert == "swiglu":
        # Dominant kernel: the gate/up grouped GEMM with the fused SwiGLU
        # (register-staged bf16 kernel; direct-to-LDS kernel for e4m3).
        odd = (wl.d_model * (1 if fp8 else 2) // 128) % 2 == 1
        kname = (f"grouped_gemm_w8_fp8<true, {'true' if fp8_gather else 'false'}, true>" if fp8
                 else "grouped_gemm_f32_kernel<1, false>" if wl.expert_dtype == "f32"
                 else f"grouped_gemm_regs<true, {'true' if odd else 'false'}, "
                      f"{'true' if fused else 'false'}, false>")
        flop, peak = work["gate_up"][1], work["gate_up"][2]
        ach = flop / (stage_ms["gate_up"] / 1e3) / 1e12
        roofline = {"kernel": kname, "bound": "mfma", "achieved": round(ach, 1), "peak": peak,
                    "unit": "TFLOP/s", "frac": round(ach / peak, 4),
                    "traffic": traffic.get(kname), "flop_per_launch": flop,
                    "ms": round(stage_ms["gate_up"], 4)}
        both = work["gate_up"][1] + work["down"][1]
        t_gemm = (stage_ms["gate_up"] + stage_ms["down"]) / 1e3
        grouped_gemm = {"kernels": "gate/up + down", "flop": both, "ms": round(t_gemm * 1e3, 4),
                        "achieved": round(both / t_gemm / 1e12, 1), "unit": "TFLOP/s",
                        "frac": round(both / t_gemm / 1e12 / peak, 4)}
    else:
        # Dispatch-only workload: the dominant kernel is the combine.
        kname = "combine_kernel"
        b = work["combine"][1]
        ach = b / (stage_ms["combine"] / 1e3) / 1e9
        roofline = {"kernel": kname, "bound": "hbm", "achieved": round(ach, 1),
                    "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                    "traffic": next((v for k, v in traffic.items() if k.startswith(kname)), None),
                    "bytes_per_launch": b, "ms": round(stage_ms["combine"], 4)}
    log(f"[bench] {ms_per_step:.4f} ms/step, {tokens_per_s / 1e6:.3f} M tokens/s; stage pass "
        f"{stage_pass_ms:.4f} ms/step: " + ", ".join(f"{k} {v:.4f}" for k, v in stage_ms.items()))
    del layer
    torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu_baseline:
        log(f"[bench] cpu baseline on up to {args.cpu_sample_tokens} tokens, {cores} cores")
        cpu = cpu_baseline(name, args.cpu_sample_tokens, args.seed)
        log(f"[bench] cpu baseline {cpu['value']} tokens/s")

    line = {
        "metric": "MoE layer tokens/s (1 GPU); grouped-GEMM MFMA util %; dispatch HBM GB/s",
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_steps_run": warm_steps,
        "ms_per_step": round(ms_per_step, 5),
        "stage_pass_ms_per_step": round(stage_pass_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8-e4m3" if fp8 else ("f32" if wl.expert_dtype == "f32" else "bf16"),
        "data": "synthetic (seeded normal inputs and weights, fixed draw order)",
        "config": {"workload": name, "tokens": wl.tokens, "d_model": wl.d_model,
                   "n_experts": wl.n_experts, "top_k": wl.top_k, "d_ff": wl.d_ff,
                   "capacity_factor": wl.capacity_factor, "routing": wl.routing,
                   "kept_rows": kept, "parallelism": "single GPU, all experts resident"},
        "roofline": roofline,
        "grouped_gemm": grouped_gemm,
        "kernels": kernels,
        "dispatch_hbm_gbs": (kernels["permute"]["achieved"] if "permute" in kernels else
                             kernels["dispatch_permute"]["achieved"]
                             if "dispatch_permute" in kernels else None),
        "dispatch": ("fused into the gate/up GEMM's row loads; dispatch_hbm_gbs is the "
                     "standalone hmoe_permute_rows on the same plan, timed outside the layer "
                     "total") if fused else "hmoe_permute_rows",
        "grouped_gemm_mfma_util": grouped_gemm["frac"] if grouped_gemm else None,
        "ceilings": ceilings,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def bench_backward(args, name, wl, layer):
    """Times the layer backward (hanuman_amd.backward): data gradients, then
    the expert and router weight gradients, on `wl`."""
    import torch
    import hanuman_amd.kernels as K
    from hanuman_amd import _lib
    from hanuman_amd.backward import BackwardOperands
    from hanuman_amd import workloads as W

    if not layer.fused_dispatch:
        raise SystemExit("--backward needs a bf16 SwiGLU workload with bf16 tokens")
    inp = W.make_inputs(wl, seed=args.seed)
    dev = layer.device
    ops = BackwardOperands(torch.from_numpy(inp.w_gate).to(dev), torch.from_numpy(inp.w_up).to(dev),
                           torch.from_numpy(inp.w_down).to(dev))
    dy = torch.from_numpy(
        np.random.default_rng(args.seed + 1).standard_normal((wl.tokens, wl.d_model), dtype=np.float32)).to(dev)
    del inp
    fwd = layer.forward()
    torch.cuda.synchronize()
    plan = fwd["plan"]
    N = wl.n_experts
    # with router logits given (no router weight) the VJP ends at d_logits
    has_router = layer.router_w is not None
    stages = (["combine_bwd", "dgrad_down", "recompute_swiglu_bwd", "dgrad_gate_up",
               "gather_bwd", "router_bwd"] + (["router_dx"] if has_router else [])
              + ["permute_xs", "wgrad_gate_up", "wgrad_down"] + (["router_dw"] if has_router else []))
    dw_ws = torch.empty(max(int(_lib.lib().hmoe_router_dw_workspace_bytes(wl.tokens, wl.d_model, N)), 1),
                        dtype=torch.uint8, device=dev)

    def step(ev=None):
        marks = iter(ev) if ev is not None else None

        def mark():
            if marks is not None:
                next(marks).record()

        mark()
        d_ys, d_g, _ = K.combine_bwd(dy, fwd["ys"], plan, fwd["gates"])
        mark()
        dh = K.grouped_dgrad_down(d_ys, plan.offsets, ops.w_down_dgrad)
        mark()
        dgu = K.grouped_gate_up_swiglu_bwd_gather(layer.x, plan, layer.w_gate_up, dh)
        mark()
        d_xs = K.grouped_dgrad_gate_up(dgu, plan.offsets, ops.w_gate_up_dgrad)
        mark()
        dx = K.gather_bwd(d_xs, plan)
        mark()
        dl = K.router_bwd(fwd["logits"], fwd["top_idx"], fwd["gates"], d_g, N, layer.mode)
        mark()
        if has_router:
            K.router_dx(dl, layer.router_w, dx)
            mark()
        xs = K.permute_rows(layer.x, plan, torch.bfloat16)
        mark()
        dwg, dwu = K.grouped_wgrad_gate_up(xs, dgu, plan.offsets)
        mark()
        dwd = K.grouped_wgrad_down(fwd["h"], d_ys, plan.offsets)
        mark()
        if has_router:
            K.router_dw(layer.x, dl, dw_ws)
            mark()
        return dx, dwg, dwu, dwd

    t_warm = time.perf_counter()
    warm_steps = 0
    while warm_steps < args.warmup or (time.perf_counter() - t_warm) * 1e3 < args.spinup_ms:
        step()
        warm_steps += 1
        if warm_steps % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(stages) + 1)]
           for _ in range(args.steps)]
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()
    for s_ in range(args.steps):
        step(evs[s_])
    t1.record()
    torch.cuda.synchronize()
    ms_per_step = t0.elapsed_time(t1) / args.steps
    stage_ms = {st: float(np.mean([evs[s_][j].elapsed_time(evs[s_][j + 1])
                                   for s_ in range(args.steps)])) for j, st in enumerate(stages)}
    T, D, F, K_ = wl.tokens, wl.d_model, wl.d_ff, wl.top_k
    R = T * K_
    kept = int(plan.offsets[-1].item())
    w_b = 2 if wl.router_w_dtype == "bf16" else 4
    work = {
        "combine_bwd": ("hbm", T * D * 4 + 2 * kept * D * 2 + R * 8, HBM_PEAK_GBS),
        "dgrad_down": ("mfma", 2 * kept * D * F, BF16_PEAK_TFLOPS),
        "recompute_swiglu_bwd": ("mfma", 4 * kept * D * F, BF16_PEAK_TFLOPS),
        "dgrad_gate_up": ("mfma", 4 * kept * D * F, BF16_PEAK_TFLOPS),
        "gather_bwd": ("hbm", kept * D * 2 + T * D * 4 + R * 4, HBM_PEAK_GBS),
        "router_bwd": ("hbm", T * N * 4 * 2 + T * K_ * 12, HBM_PEAK_GBS),
        "router_dx": ("hbm", T * N * 4 + D * N * w_b + 2 * T * D * 4, HBM_PEAK_GBS),
        "permute_xs": ("hbm", T * D * 2 + kept * D * 2 + R * 4, HBM_PEAK_GBS),
        "wgrad_gate_up": ("mfma", 4 * kept * D * F, BF16_PEAK_TFLOPS),
        "wgrad_down": ("mfma", 2 * kept * D * F, BF16_PEAK_TFLOPS),
        "router_dw": ("hbm", T * D * 2 + T * N * 4 + D * N * 4, HBM_PEAK_GBS),
    }
    kernels = {}
    for st in stages:
        kind, amount, peak = work[st]
        t = stage_ms[st] / 1e3
        ach = amount / t / (1e9 if kind == "hbm" else 1e12)
        kernels[st] = {"ms": round(stage_ms[st], 4), "bound": kind, "achieved": round(ach, 1),
                       "unit": "GB/s" if kind == "hbm" else "TFLOP/s", "peak": peak,
                       "frac": round(ach / peak, 4), ("bytes" if kind == "hbm" else "flop"): amount}
    dom = "dgrad_gate_up"
    roofline = {"kernel": "grouped_gemm_regs<false, false, false, false> (dgrad gate/up)", "bound": "mfma",
                "achieved": kernels[dom]["achieved"], "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": kernels[dom]["frac"], "traffic": None, "flop_per_launch": work[dom][1],
                "ms": kernels[dom]["ms"]}
    log(f"[bench] backward {ms_per_step:.4f} ms/step, {T / ms_per_step / 1e3:.3f} M tokens/s; stages "
        + ", ".join(f"{k} {v:.4f}" for k, v in stage_ms.items()))
    line = {
        "metric": "MoE layer backward (data and weight gradients) tokens/s (1 GPU)",
        "value": round(T / (ms_per_step / 1e3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "warmup_steps_run": warm_steps,
        "ms_per_step": round(ms_per_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded normal inputs, weights and output cotangent)",
        "config": {"workload": name + " backward (data and weight gradients)", "tokens": T, "d_model": D,
                   "n_experts": N, "top_k": K_, "d_ff": F, "capacity_factor": wl.capacity_factor,
                   "kept_rows": kept, "parallelism": "single GPU, all experts resident"},
        "roofline": roofline, "kernels": kernels, "cpu_baseline": None,
        "data_gradients_ms": round(sum(stage_ms[st] for st in stages[:stages.index("permute_xs")]), 4),
        "weight_gradients_ms": round(sum(stage_ms[st] for st in stages[stages.index("permute_xs"):]), 4),
    }
    print(json.dumps(line), flush=True)


def bench_train(args, name, wl):
    """One training step of the drop-in module at `wl`'s shape."""
    import torch
    from hanuman_amd.moe import MoE

    if wl.router_from_logits or wl.expert != "swiglu" or wl.expert_dtype not in ("bf16", "f32"):
        raise SystemExit("--train needs a bf16 or float32 SwiGLU workload with a router weight")
    dt = torch.float32 if wl.expert_dtype == "f32" else torch.bfloat16
    dev = torch.device("cuda", 0)
    B = wl.batch if wl.tokens % wl.batch == 0 else 1
    S = wl.tokens // B
    m = MoE(wl.d_model, wl.d_ff, wl.n_experts, wl.top_k, 1, 0.02, 1.0, dt,
            rngs=args.seed, device=dev, routing=wl.routing, capacity_factor=wl.capacity_factor)
    params = [p.value for n, p in m.named_params().items() if n != "bias"]
    for p in params:
        p.requires_grad_(True)
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    x = torch.randn(B, S, wl.d_model, generator=gen, device=dev).to(dt)
    dy = torch.randn(B, S, wl.d_model, generator=gen, device=dev)

    def step():
        for p in params:
            p.grad = None
        out, aux = m(x)
        loss = (out * dy).sum() + 1e-3 * aux["router_z_loss"] + 1e-2 * aux["balance_loss"]
        loss.backward()
        with torch.no_grad():   # the update: every master changes, so the operands re-pack
            for p in params:
                p.add_(p.grad, alpha=-1e-9)

    t_warm = time.perf_counter()
    warm_steps = 0
    while warm_steps < args.warmup or (time.perf_counter() - t_warm) * 1e3 < args.spinup_ms:
        step()
        warm_steps += 1
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(args.steps):
        step()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    log(f"[bench] train step {ms:.4f} ms/step, {wl.tokens / ms / 1e3:.3f} M tokens/s")
    line = {
        "metric": "MoE layer training step (forward, backward, update) tokens/s (1 GPU)",
        "value": round(wl.tokens / (ms / 1e3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "warmup_steps_run": warm_steps,
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32" if dt == torch.float32 else "bf16",
        "data": "synthetic (seeded normal inputs, weights and output cotangent)",
        "config": {"workload": name + " training step (module with one shared expert)",
                   "tokens": wl.tokens, "d_model": wl.d_model, "n_experts": wl.n_experts,
                   "top_k": wl.top_k, "d_ff": wl.d_ff, "capacity_factor": wl.capacity_factor,
                   "n_shared_experts": 1, "parallelism": "single GPU, all experts resident"},
        "roofline": None, "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
