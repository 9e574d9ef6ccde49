"""Throughput of the MI355X MoE FFN layer on its headline workload.

Workload: one Qwen3-30B-A3B-shaped MoE layer (hidden 2048, 128 experts of SwiGLU
2048->768->2048, top-8 softmax with renormalisation), Q8_0 experts, at decode
batch 64 with i.i.d. U(0,1) router logits (the router GEMV is not part of this
workload).  A step is one layer forward over the batch (route, dispatch, fused
dequant + gate/up, fused dequant + down, combine) with the inputs already
resident in HBM, its kernels launched directly on the library's stream (the
time with one HIP graph per call is reported beside it).  Steps rotate over
`--copies` device copies of the layer so the 256 MB Infinity Cache cannot serve
the weights between steps.

Prints ONE JSON line (rank 0, N=1) with the throughput, the roofline of the
dominant kernel (the fused dequant + gate/up GEMV: its mean launch time over
back-to-back launches, HIP events on the library's stream), and the CPU
restatement of the reference path timed on the host cores on a bounded sample of
the same batch.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, TFLOP/s
METRIC = "MoE-layer tok/s + % HBM roofline (decode), % MFMA peak (prefill), 30B-A3B shape"


def log(msg: str):
    print(msg, file=sys.stderr, flush=True)


def gateup_bytes(spec, touched: int, T: int) -> float:
    """Algorithmic HBM bytes of one fused dequant + gate/up launch (no K split at
    this size): the touched experts' gate and up weights once, the f16 activations
    once, the f16 SwiGLU output of every (token, slot) once."""
    from anedvd_amd import workloads as W
    w = touched * spec.inter * spec.hidden * (W.bytes_per_weight(spec.gate_type) + W.bytes_per_weight(spec.up_type))
    return w + T * spec.hidden * 2 + T * spec.k * spec.inter * 2


def read_traffic(name: str):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3
    --pmc summary (FETCH_SIZE + WRITE_SIZE, calibrated on a copy kernel)."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def cpu_baseline(spec, L, h, logits, budget_s: float):
    """The oracle's streaming forward (Engine.forward's per-token decode path:
    route, dequantise each selected expert, SwiGLU GEMVs) on 1 core, over as
    many tokens of the batch as fit in about `budget_s` seconds."""
    from oracle import oracle as O
    ol = O.OracleLayer(spec, L)
    t0 = time.perf_counter()
    ref1 = ol.forward(h[:1], logits[:1], streaming=True)
    per_tok = time.perf_counter() - t0
    n = int(max(1, min(h.shape[0], budget_s / max(per_tok, 1e-6))))
    t0 = time.perf_counter()
    ref = ol.forward(h[:n], logits[:n], streaming=True)
    dt = time.perf_counter() - t0
    return {"value": round(n / dt, 3), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"oracle/moe_oracle.c streaming decode (per token: route, dequantise 8 Q8_0 experts to f32, "
                      f"SwiGLU GEMVs), first {n} tokens of the batch, {dt:.1f} s, gcc -O2, 1 thread"}, ref, n


CONFIGS = {
    # name: (spec attribute, tokens, routing, device copies rotated, layers timed as a stack)
    "qwen3-q4km-512": ("QWEN3_30B_A3B_Q4_K_M", 512, "zipf", 2, 1),
    "mixtral-q4_0-2048": ("MIXTRAL_8X7B_Q4_0", 2048, "normal", 3, 1),
    "mixtral-q4_0-1": ("MIXTRAL_8X7B_Q4_0", 1, "normal", 3, 1),
    "deepseek-v2-lite-32-x26": ("DEEPSEEK_V2_LITE_Q8_0", 32, "uniform", 26, 26),
    "deepseek-v2-lite-1024-x26": ("DEEPSEEK_V2_LITE_Q8_0", 1024, "uniform", 26, 26),
}
_LAYERS = {}  # spec name -> resident layer copies, shared by the configs of one spec


def resident_layers(ctx, spec, copies: int) -> list:
    """`copies` device copies of one synthetic layer of `spec` (seed 0): each copy
    is a distinct HBM allocation, so rotating through them defeats the Infinity
    Cache as a stack of distinct layers would."""
    from anedvd_amd import moe, synth
    have = _LAYERS.setdefault(spec.name, [])
    if len(have) < copies:
        L = synth.make_layer(spec, seed=0)
        while len(have) < copies:
            have.append(moe.MoeLayer(ctx, spec, L))
    return have[:copies]


def free_layers():
    for ls in _LAYERS.values():
        for l in ls:
            l.free()
    _LAYERS.clear()


def run_config(name: str, ctx, warmup: int, steps: int) -> dict:
    """One workload beside the headline: a layer call (route + dispatch + expert
    products + shared expert + combine, router logits given), rotated over device
    copies of the layer.  For a stack, call j runs layer j mod n of n distinct
    resident layers and the stack time is n times the mean call.  Reports tokens/s,
    the layer's algorithmic HBM bytes/s and useful MFMA-path FLOP/s against the peaks."""
    from anedvd_amd import moe, synth
    from anedvd_amd import workloads as W
    attr, T, routing, copies, stack = CONFIGS[name]
    spec = getattr(W, attr)
    t0 = time.perf_counter()
    layers = resident_layers(ctx, spec, copies)
    h = synth.activations(spec, T, seed=1)
    if routing == "zipf":
        lg = synth.zipf_logits(spec, T, seed=1)
    elif routing == "uniform":
        lg = synth.uniform_logits(spec, T, seed=1)
    else:
        lg = synth.activations(spec, T, seed=2)[:, :spec.n_experts]
    lg = np.ascontiguousarray(lg, dtype=np.float32)
    _, st = layers[0].forward(h, lg, stats=True)
    d_h, d_lg = ctx.to_device(h), ctx.to_device(lg)
    d_out = ctx.alloc(T * spec.hidden * 4)
    steps = max(steps, 2 * copies) // copies * copies
    warmup = max(warmup, copies)
    ms, _ = moe.time_forward(layers, d_h, T, d_lg, d_out, warmup, steps)
    _, stages = moe.time_forward(layers, d_h, T, d_lg, d_out, 1, steps, stages=True)
    _, solo = moe.time_forward(layers, d_h, T, d_lg, d_out, 1, steps, solo=True)
    for p in (d_h, d_lg, d_out):
        ctx.free(p)
    t = ms / 1e3 / steps
    flops = spec.call_flops(T, with_router=False)
    lbytes = spec.call_bytes(st["touched_experts"], T, with_router=False)
    r = {"name": name, "workload": spec.name, "tokens": T, "routing": routing, "layer_copies_rotated": copies,
         "touched_experts": st["touched_experts"], "max_group": st["max_group"],
         "path": "grouped GEMM" if st["path"] else "decode GEMV",
         "ms_per_call": round(ms / steps, 4), "tokens_per_s": round(T / t, 1),
         "TFLOPs": round(flops / t / 1e12, 2), "mfma_frac": round(flops / t / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
         "layer_GBps": round(lbytes / t / 1e9, 1), "hbm_frac": round(lbytes / t / 1e9 / HBM_PEAK_GBS, 4),
         "stage_ms": dict(zip(["route_dispatch", "gate_up", "down", "shared", "combine", "total"],
                              [round(x, 4) for x in stages])),
         "solo_launch_ms": {"gate_up": round(solo[1], 4), "down": round(solo[2], 4)}}
    gu_flops = 2 * 2 * T * spec.k * spec.hidden * spec.inter  # the routed gate and up products
    r["gate_up_mfma_frac"] = round(gu_flops / (solo[1] / 1e3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)
    if stack > 1:
        r["stack_layers"] = stack
        r["stack_ms"] = round(ms / steps * stack, 4)
        r["stack_tokens_per_s"] = round(T / (t * stack), 1)
    log(f"[bench] {name}: {r['ms_per_call'] * 1e3:.1f} us/call ({r['path']}), {r['tokens_per_s']:.0f} tok/s, "
        f"{r['TFLOPs']} TFLOP/s ({100 * r['mfma_frac']:.1f}% of fp16 MFMA peak), {r['layer_GBps']} GB/s "
        f"({100 * r['hbm_frac']:.1f}% of HBM), touched {r['touched_experts']}, max group {r['max_group']}"
        + (f", {stack}-layer stack {r['stack_ms']:.3f} ms" if stack > 1 else "")
        + f", event stages {r['stage_ms']}, solo launches {r['solo_launch_ms']} "
        f"(setup {time.perf_counter() - t0:.1f} s)")
    return r


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--copies", type=int, default=8, help="device copies of the layer rotated per step")
    ap.add_argument("--sweep", default="1,8,32", help="extra decode batches reported beside the headline ('' = none)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU-baseline budget (0 = skip)")
    ap.add_argument("--configs", default=",".join(CONFIGS),
                    help="further workloads reported beside the headline ('' = none): " + ", ".join(CONFIGS))
    ap.add_argument("--configs-only", action="store_true", help="run only the --configs workloads (profiling)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="first run 3 device-to-device copies of MIB MiB (a plain copy kernel of known size, "
                         "for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build runs the MoE layer on one GPU; multi-GPU (expert-parallel) runs "
                                   "are not part of it", "n_gpus": args.gpus}))
        sys.exit(2)

    from anedvd_amd import moe, synth
    from anedvd_amd import workloads as W

    if args.calibrate_copy:
        import torch
        src = torch.ones(args.calibrate_copy << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] calibration: 3 device copies of {args.calibrate_copy} MiB")
        del src, dst

    if args.configs_only:
        ctx = moe.MoeContext(0)
        out = [run_config(name, ctx, args.warmup, args.steps) for name in args.configs.split(",") if name.strip()]
        print(json.dumps({"configs": out}), flush=True)
        free_layers()
        ctx.close()
        return

    spec = W.QWEN3_30B_A3B_Q8_0
    B = args.batch
    t0 = time.perf_counter()
    L = synth.make_layer(spec, seed=0)
    log(f"[bench] synthetic layer {spec.name}: {sum(v.nbytes for v in L.values()) / 1e6:.1f} MB in "
        f"{time.perf_counter() - t0:.1f} s")
    ctx = moe.MoeContext(0)
    layers = [moe.MoeLayer(ctx, spec, L) for _ in range(args.copies)]
    log(f"[bench] {len(layers)} resident copies, {layers[0].device_bytes() / 1e6:.1f} MB each")

    def run(T: int, steps: int, warmup: int):
        h = synth.activations(spec, T, seed=0)
        lg = synth.uniform_logits(spec, T, seed=0)
        out_host, st = layers[0].forward(h, lg, stats=True)
        d_h, d_lg = ctx.to_device(h), ctx.to_device(lg)
        d_out = ctx.alloc(T * spec.hidden * 4)
        ms, _ = moe.time_forward(layers, d_h, T, d_lg, d_out, warmup, steps)
        ms_graph, _ = moe.time_forward(layers, d_h, T, d_lg, d_out, warmup, steps, graph=True)
        _, stages = moe.time_forward(layers, d_h, T, d_lg, d_out, 2, steps, stages=True)
        _, solo = moe.time_forward(layers, d_h, T, d_lg, d_out, 2, steps, solo=True)
        for p in (d_h, d_lg, d_out):
            ctx.free(p)
        touched = st["touched_experts"]
        layer_s = ms / 1e3 / steps
        lbytes = spec.call_bytes(touched, T, with_router=False)
        r = {"batch": T, "touched_experts": touched, "ms_per_step": ms / steps, "graph_ms_per_step": ms_graph / steps,
             "tokens_per_s": T / layer_s, "layer_GBps": lbytes / layer_s / 1e9,
             "layer_hbm_frac": lbytes / layer_s / 1e9 / HBM_PEAK_GBS,
             "stage_ms": dict(zip(["route_dispatch", "gate_up", "down", "shared", "combine", "total"],
                                  [round(x, 5) for x in stages])),
             "solo_launch_ms": {"gate_up": round(solo[1], 5), "down": round(solo[2], 5)}}
        log(f"[bench] B={T}: {ms / steps * 1e3:.1f} us/step ({ms_graph / steps * 1e3:.1f} as graphs), "
            f"{r['tokens_per_s']:.0f} tok/s, "
            f"{r['layer_GBps']:.0f} GB/s ({100 * r['layer_hbm_frac']:.1f}% of HBM), touched {touched}, "
            f"event stages {r['stage_ms']}, solo launches {r['solo_launch_ms']}")
        return r, h, lg, out_host

    sweep = []
    for T in [int(s) for s in args.sweep.split(",") if s.strip()]:
        sweep.append(run(T, max(10, args.steps // 2), args.warmup)[0])

    head, h, lg, out_gpu = run(B, args.steps, args.warmup)
    ms_step = head["ms_per_step"]
    gu_ms = head["solo_launch_ms"]["gate_up"]
    gu_bytes = gateup_bytes(spec, head["touched_experts"], B)
    achieved = gu_bytes / (gu_ms / 1e3) / 1e9
    roofline = {"bound": "hbm", "kernel": "k_mm_gateup<MQ8_0> (fused Q8_0 dequant + gate/up + SwiGLU on MFMA)",
                "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": read_traffic("pmc_k_mm_gateup_q8_0_decode_b64.md"),
                "bytes_per_launch": gu_bytes, "avg_launch_ms": gu_ms}

    configs = []
    for name in [x for x in args.configs.split(",") if x.strip()]:
        configs.append(run_config(name, ctx, args.warmup, max(10, args.steps // 4)))
    free_layers()

    cpu = None
    parity = None
    if args.cpu_seconds > 0:
        cpu, ref, n = cpu_baseline(spec, L, h, lg, args.cpu_seconds)
        parity = {"tokens_checked": n, "rel_l2": moe.rel_l2(out_gpu[:n], ref),
                  "max_abs": float(np.abs(out_gpu[:n].astype(np.float64) - ref).max())}
        log(f"[bench] cpu baseline {cpu['value']} tok/s; GPU vs oracle on {n} tokens: rel-L2 {parity['rel_l2']:.2e}")

    line = {
        "metric": METRIC, "value": round(head["tokens_per_s"], 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic (seeded Q8_0 experts, N(0,1) activations, U(0,1) router logits)",
        "config": {"workload": "qwen3-30b-a3b moe layer, q8_0 experts, decode batch %d" % B, "hidden": spec.hidden,
                   "experts": spec.n_experts, "inter": spec.inter, "top_k": spec.k, "batch": B,
                   "weights": "q8_0", "layer_copies_rotated": args.copies,
                   "arithmetic": "f16 dot products of exact dequantised weights, f32 accumulation"},
        "graph_ms_per_step": round(head["graph_ms_per_step"], 5),
        "layer_GBps": round(head["layer_GBps"], 1), "layer_hbm_frac": round(head["layer_hbm_frac"], 4),
        "touched_experts": head["touched_experts"], "stage_ms": head["stage_ms"],
        "solo_launch_ms": head["solo_launch_ms"],
        "roofline": roofline, "cpu_baseline": cpu, "parity_vs_oracle": parity,
        "sweep": [{k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()} for r in sweep],
        "configs": configs,
    }
    print(json.dumps(line), flush=True)
    for l in layers:
        l.free()
    ctx.close()


if __name__ == "__main__":
    main()
