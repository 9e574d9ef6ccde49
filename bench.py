"""Throughput of the MI355X MoE FFN layer on its headline workload, with every
benchmarked workload beside it.

Headline: one Qwen3-30B-A3B-shaped MoE layer (hidden 2048, 128 experts of SwiGLU
2048->768->2048, top-8 softmax with renormalisation), Q8_0 experts, at decode
batch 64 with i.i.d. U(0,1) router logits (the router GEMV is timed on its own).
A step is one layer forward over the batch (route, dispatch, fused dequant +
gate/up, fused dequant + down, combine) with the inputs already resident in HBM,
its kernels launched directly on the library's stream (the time with one HIP
graph per call is reported beside it).  Steps rotate over `--copies` device
copies of the layer so the 256 MB Infinity Cache cannot serve the weights.

Beside it (`configs`): the Qwen3 Q4_K_M 512-token prefill with Zipf routing,
Mixtral-8x7B Q4_0 at 1 and 2048 tokens, and the DeepSeek-V2-Lite 26-layer stack
(26 distinct layers chained x += proj, at decode batch 32 and a 1024-token
prefill); the Mixtral and DeepSeek calls run their layer's router GEMV on their
own input inside the timed call.  Every workload's output is checked against the oracle on sampled
tokens of the same run (a stack layer by layer), and the oracle (the CPU
restatement of the reference path, AVX2 build) is timed on one pinned host core in
two modes: streaming (the engine's expert reads, per token or per 128-token
prefill chunk) and resident f32 experts.

Prints ONE JSON line (rank 0, N=1).
"""
from __future__ import annotations

import argparse
import contextlib
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, TFLOP/s
METRIC = "MoE-layer tok/s + % HBM roofline (decode), % MFMA peak (prefill), 30B-A3B shape"
CPU_RUNS = 5                   # the CPU baseline reports the median of this many runs
CPU_RUNS_LONG = 3              # ... or of this many when one run takes longer than CPU_LONG_S
CPU_LONG_S = 3.0


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


# ------------------------------------------------------------------ CPU baseline

def host_cpu() -> dict:
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count(), "cores_allowed": len(os.sched_getaffinity(0))}


@contextlib.contextmanager
def pinned_core():
    """Pins the calling thread to one core (the last one it may use) while timing."""
    old = os.sched_getaffinity(0)
    core = max(old)
    os.sched_setaffinity(0, {core})
    try:
        yield core
    finally:
        os.sched_setaffinity(0, old)


def cpu_median(fn) -> tuple:
    t0 = time.perf_counter()
    fn()  # warm-up
    runs = CPU_RUNS_LONG if time.perf_counter() - t0 > CPU_LONG_S else CPU_RUNS
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts), ts


def cpu_baseline(spec, L, h, lg, mode_a: tuple, n_b: int) -> dict:
    """The oracle timed on one pinned core, median of CPU_RUNS runs after a warm-up
    (CPU_RUNS_LONG when the warm-up run takes more than CPU_LONG_S).
    Mode A is the engine's streaming path: ("stream", n) runs the per-token decode
    loop (engine.zig:705-779: route, read each selected expert's three projections
    from the GGUF bytes to f32, moeExpertAccumF32) over n tokens; ("chunk", n) runs
    the batched prefill (engine.zig:1158-1268: each routed expert read once for the
    chunk, then every token it serves) on one n-token chunk.  Mode B holds the
    experts the sample touches as resident f32 (dequantised before timing) and runs
    the decode loop over n_b tokens: the expert products alone."""
    from oracle import oracle as O
    ol = O.OracleLayer(spec, L)
    kind, n_a = mode_a
    ha, la = h[:n_a], (None if lg is None else lg[:n_a])
    hb, lb = h[:n_b], (None if lg is None else lg[:n_b])
    _, _, ia = ol.route(ha, n_a, la)
    _, _, ib = ol.route(hb, n_b, lb)
    touched_a = len(np.unique(ia))
    exp_b = spec.expert_bytes()
    out = {}
    with pinned_core() as core:
        ta, tsa = cpu_median(lambda: ol.forward(ha, la, streaming=(kind == "stream"), fast=True))
        R = ol.resident(np.unique(ib), fast=True)
        tb, tsb = cpu_median(lambda: R.forward(hb, lb))
        R.free()
    # bytes the CPU path reads: streaming, every (token, slot) reads its expert; a
    # prefill chunk reads each touched expert once; resident, f32 weights per slot
    bytes_a = (n_a * spec.k if kind == "stream" else touched_a) * exp_b + n_a * spec.shared_bytes()
    bytes_b = n_b * spec.k * 3 * spec.inter * spec.hidden * 4
    out["mode_a"] = {"tokens_per_s": round(n_a / ta, 3), "GBps": round(bytes_a / ta / 1e9, 3),
                     "median_s": round(ta, 4), "runs": len(tsa),
                     "sample": (f"per-token streaming decode of {n_a} tokens" if kind == "stream" else
                                f"batched prefill of one {n_a}-token chunk ({touched_a} experts read once)")}
    out["mode_b"] = {"tokens_per_s": round(n_b / tb, 3), "GBps": round(bytes_b / tb / 1e9, 3),
                     "median_s": round(tb, 4), "runs": len(tsb),
                     "sample": f"decode loop over {n_b} tokens on resident f32 experts ({len(np.unique(ib))} held)"}
    out.update({"cores": 1, "core": core, "kind": "port",
                "build": "oracle/moe_oracle.c, gcc -O3 -mavx2 -mno-fma -ffp-contract=off (8-lane loops vectorised, "
                         "results bit-identical to the portable build)"})
    return out


# ------------------------------------------------------------------ workloads

CONFIGS = {
    # spec: workloads attribute; T tokens; routing: the logits given to the call (zipf,
    # uniform) or "router": none, the layer routes each call from its own input with
    # its router GEMV inside the timed call (main.zig:493, engine.zig:715, 1178);
    # copies of the layer rotated (stack: distinct chained layers); parity: tokens
    # sampled against the oracle; cpu_a: mode A of the CPU baseline (prefill: one
    # 128-token chunk, the engine's prefill chunk, engine.zig:45); cpu_b: tokens of mode B
    "qwen3-q4km-512": dict(spec="QWEN3_30B_A3B_Q4_K_M", T=512, routing="zipf", copies=2, parity=32,
                           cpu_a=("chunk", 128), cpu_b=32),
    "mixtral-q4_0-2048": dict(spec="MIXTRAL_8X7B_Q4_0", T=2048, routing="router", copies=3, parity=16,
                              cpu_a=("chunk", 128), cpu_b=4),
    "mixtral-q4_0-1": dict(spec="MIXTRAL_8X7B_Q4_0", T=1, routing="router", copies=8, parity=1,
                           cpu_a=("stream", 1), cpu_b=1),
    "deepseek-v2-lite-32-x26": dict(spec="DEEPSEEK_V2_LITE_Q8_0", T=32, routing="router", stack=26, parity=6,
                                    cpu_a=("stream", 8), cpu_b=16),
    "deepseek-v2-lite-1024-x26": dict(spec="DEEPSEEK_V2_LITE_Q8_0", T=1024, routing="router", stack=26, parity=6,
                                      cpu_a=("chunk", 128), cpu_b=16),
}
_LAYERS = {}  # (spec name, kind) -> resident layers and their host arrays


def logits_for(spec, routing: str, T: int, seed: int):
    """The router logits a call is given, or None: the layer's own router GEMV."""
    from anedvd_amd import synth
    if routing == "router":
        return None
    if routing == "zipf":
        lg = synth.zipf_logits(spec, T, seed=seed)
    elif routing == "uniform":
        lg = synth.uniform_logits(spec, T, seed=seed)
    else:
        lg = synth.activations(spec, T, seed=seed + 1)[:, :spec.n_experts]
    return np.ascontiguousarray(lg, dtype=np.float32)


def resident_copies(ctx, spec, copies: int):
    """`copies` device copies of one synthetic layer of `spec` (seed 0): distinct
    HBM allocations, so rotating through them defeats the Infinity Cache."""
    from anedvd_amd import moe, synth
    key = (spec.name, "copies")
    if key not in _LAYERS:
        _LAYERS[key] = (synth.make_layer(spec, seed=0), [])
    L, have = _LAYERS[key]
    while len(have) < copies:
        have.append(moe.MoeLayer(ctx, spec, L))
    return L, have[:copies]


def resident_stack(ctx, spec, n: int):
    """n distinct layers of `spec` (layer seeds 0..n-1), resident."""
    from anedvd_amd import moe, synth
    key = (spec.name, "stack")
    if key not in _LAYERS:
        t0 = time.perf_counter()
        Ls, layers = [], []
        for i in range(n):
            Ls.append(synth.make_layer(spec, seed=0, layer=i))
            layers.append(moe.MoeLayer(ctx, spec, Ls[-1]))
        _LAYERS[key] = (Ls, layers)
        log(f"[bench] {n} distinct {spec.name} layers generated and resident in {time.perf_counter() - t0:.1f} s")
    return _LAYERS[key]


def free_layers():
    for _, ls in _LAYERS.values():
        for l in ls:
            l.free()
    _LAYERS.clear()


def parity_of(got: np.ndarray, want: np.ndarray, n: int) -> dict:
    """rel-L2 and max-abs error of `got` against the oracle's `want`, with the
    reference's largest magnitude beside max-abs (its scale)."""
    from anedvd_amd import moe
    return {"tokens_checked": n, "rel_l2": moe.rel_l2(got, want),
            "max_abs": float(np.abs(got.astype(np.float64) - want).max()),
            "ref_max_abs": float(np.abs(want).max())}


def sample_rows(T: int, n: int) -> np.ndarray:
    return np.unique(np.linspace(0, T - 1, n).round().astype(np.int64)) if n < T else np.arange(T)


def run_config(name: str, ctx, warmup: int, steps: int, with_parity: bool) -> dict:
    """One workload beside the headline: a layer call (route + dispatch + expert
    products + shared expert + combine; the router GEMV too where the workload does
    not give logits), rotated over device copies of the layer, or a chained stack of
    distinct layers each routing its own input.  Reports tokens/s,
    the algorithmic HBM bytes/s and useful MFMA-path FLOP/s against the peaks, and
    the oracle's agreement on sampled tokens of the same inputs."""
    from anedvd_amd import moe, synth
    from anedvd_amd import workloads as W
    from oracle import oracle as O
    c = CONFIGS[name]
    spec, T, stack = getattr(W, c["spec"]), c["T"], c.get("stack", 0)
    t0 = time.perf_counter()
    h = synth.activations(spec, T, seed=1)
    rows = sample_rows(T, c["parity"])
    r = {"name": name, "workload": spec.name, "tokens": T, "routing": c["routing"]}
    if stack:
        Ls, layers = resident_stack(ctx, spec, stack)
        lgl = [logits_for(spec, c["routing"], T, seed=1 + i) for i in range(stack)]
        routed = lgl[0] is None
        _, st = layers[0].forward(h, lgl[0], stats=True)
        d_h, d_out = ctx.to_device(h), ctx.alloc(T * spec.hidden * 4)
        d_lg = None if routed else ctx.to_device(np.stack(lgl))
        passes = max(2, steps // stack)
        ms, _ = moe.time_forward(layers, d_h, T, d_lg, d_out, stack, stack * passes, chain=True)
        _, stages = moe.time_forward(layers, d_h, T, d_lg, d_out, 0, stack, stages=True, chain=True)
        got = ctx.from_device(d_out, (T, spec.hidden), np.float32)  # one whole pass from d_h
        for p in (d_h, d_lg, d_out):
            if p:
                ctx.free(p)
        n_calls = stack * passes
        if with_parity:
            # Layer by layer on the GPU (host calls over all T tokens: the kernels of the
            # timed call), each layer checked against the oracle on the GPU's own input
            # rows.  A layer that routes its own x picks its experts from that x, so both
            # sides see the same x and the router's bit-exact logits: the check is one
            # layer's arithmetic.  (A chained oracle would drift to another expert choice
            # wherever two logits tie within the stack's accumulated rounding.)
            x, worst = h.copy(), None
            for i in range(stack):
                proj = layers[i].forward(x, lgl[i])
                want = O.OracleLayer(spec, Ls[i]).forward(x[rows], None if routed else lgl[i][rows], fast=True)
                p_i = parity_of(proj[rows], want, len(rows))
                if worst is None or p_i["rel_l2"] > worst["rel_l2"]:
                    worst = dict(p_i, layer=i)
                x = x + proj
            r["parity"] = dict(worst, check="each layer on the GPU's own input rows; the worst layer",
                               chained_vs_layer_by_layer_max_abs=float(np.abs(got[rows] - x[rows]).max()))
        r.update({"stack_layers": stack, "layers": f"{stack} distinct layers, chained x += proj",
                  "stack_ms": round(ms / passes, 4), "stack_tokens_per_s": round(T / (ms / passes / 1e3), 1)})
        L = Ls[0]
        lg = lgl[0]
        solo = None
    else:
        L, layers = resident_copies(ctx, spec, c["copies"])
        lg = logits_for(spec, c["routing"], T, seed=1)
        routed = lg is None
        out_host, st = layers[0].forward(h, lg, stats=True)
        d_h, d_out = ctx.to_device(h), ctx.alloc(T * spec.hidden * 4)
        d_lg = None if routed else ctx.to_device(lg)
        n_calls = max(steps, 2 * c["copies"]) // c["copies"] * c["copies"]
        ms, _ = moe.time_forward(layers, d_h, T, d_lg, d_out, max(warmup, c["copies"]), n_calls)
        _, stages = moe.time_forward(layers, d_h, T, d_lg, d_out, 1, n_calls, stages=True)
        _, solo = moe.time_forward(layers, d_h, T, d_lg, d_out, 1, n_calls, solo=True)
        for p in (d_h, d_lg, d_out):
            if p:
                ctx.free(p)
        if with_parity:
            want = O.OracleLayer(spec, L).forward(h[rows], None if routed else lg[rows], fast=True)
            r["parity"] = parity_of(out_host[rows], want, len(rows))
        r["layer_copies_rotated"] = c["copies"]
    r["router_in_call"] = routed
    t = ms / 1e3 / n_calls  # one layer call
    flops = spec.call_flops(T, with_router=routed)
    lbytes = spec.call_bytes(st["touched_experts"], T, with_router=routed)
    r.update({"touched_experts": st["touched_experts"], "max_group": st["max_group"],
              "path": "grouped GEMM" if st["path"] else "decode MFMA kernels",
              "ms_per_call": round(ms / n_calls, 4), "tokens_per_s": round(T / t, 1),
              "TFLOPs": round(flops / t / 1e12, 2), "mfma_frac": round(flops / t / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
              "layer_GBps": round(lbytes / t / 1e9, 1), "hbm_frac": round(lbytes / t / 1e9 / HBM_PEAK_GBS, 4),
              "stage_ms": dict(zip(["route_dispatch", "gate_up", "down", "shared", "combine", "total"],
                                   [round(x, 4) for x in stages]))})
    if solo is not None:
        r["solo_launch_ms"] = {"gate_up": round(solo[1], 4), "down": round(solo[2], 4)}
        gu_flops = 2 * 2 * T * spec.k * spec.hidden * spec.inter  # the routed gate and up products
        r["gate_up_mfma_frac"] = round(gu_flops / (solo[1] / 1e3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)
    r["_cpu"] = (spec, L, h, lg, c["cpu_a"], c["cpu_b"])
    log(f"[bench] {name}: {r['ms_per_call'] * 1e3:.1f} us/call ({r['path']}), {r['tokens_per_s']:.0f} tok/s, "
        f"{r['TFLOPs']} TFLOP/s ({100 * r['mfma_frac']:.1f}% of fp16 MFMA peak), {r['layer_GBps']} GB/s "
        f"({100 * r['hbm_frac']:.1f}% of HBM), touched {r['touched_experts']}, max group {r['max_group']}"
        + (f", {stack}-layer stack {r['stack_ms']:.3f} ms" if stack else "")
        + (f", parity rel-L2 {r['parity']['rel_l2']:.2e}, max-abs {r['parity']['max_abs']:.3g} of |ref| "
           f"{r['parity']['ref_max_abs']:.3g} on {r['parity']['tokens_checked']} tokens" if "parity" in r else "")
        + (", router GEMV in the call" if routed else ", logits given")
        + f", event stages {r['stage_ms']} (setup {time.perf_counter() - t0:.1f} s)")
    return r


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--copies", type=int, default=8, help="device copies of the layer rotated per step")
    ap.add_argument("--sweep", default="1,8,32", help="extra decode batches reported beside the headline ('' = none)")
    ap.add_argument("--cpu", type=int, default=1, help="time the CPU baseline (0 = skip)")
    ap.add_argument("--parity", type=int, default=1, help="check every workload against the oracle (0 = skip)")
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

    names = [x for x in args.configs.split(",") if x.strip()]
    if args.configs_only:
        ctx = moe.MoeContext(0)
        out = [run_config(name, ctx, args.warmup, args.steps, bool(args.parity)) for name in names]
        for r in out:
            r.pop("_cpu")
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
        rb = spec.n_experts * spec.hidden * 2 + T * spec.hidden * 4 + T * spec.n_experts * 4
        r = {"batch": T, "touched_experts": touched, "ms_per_step": ms / steps, "graph_ms_per_step": ms_graph / steps,
             "tokens_per_s": T / layer_s, "layer_GBps": lbytes / layer_s / 1e9,
             "layer_hbm_frac": lbytes / layer_s / 1e9 / HBM_PEAK_GBS,
             "stage_ms": dict(zip(["route_dispatch", "gate_up", "down", "shared", "combine", "total"],
                                  [round(x, 5) for x in stages])),
             "solo_launch_ms": {"gate_up": round(solo[1], 5), "down": round(solo[2], 5)},
             "router_gemv": {"us": round(solo[0] * 1e3, 3), "bytes": rb,
                             "GBps": round(rb / (solo[0] / 1e3) / 1e9, 1)}}
        log(f"[bench] B={T}: {ms / steps * 1e3:.1f} us/step ({ms_graph / steps * 1e3:.1f} as graphs), "
            f"{r['tokens_per_s']:.0f} tok/s, "
            f"{r['layer_GBps']:.0f} GB/s ({100 * r['layer_hbm_frac']:.1f}% of HBM), touched {touched}, "
            f"event stages {r['stage_ms']}, solo launches {r['solo_launch_ms']}, router GEMV {r['router_gemv']}")
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
                "traffic": read_traffic("pmc_k_mm_q8_0_decode_b1_b8_b32_b64.md"),
                "bytes_per_launch": gu_bytes, "avg_launch_ms": gu_ms}
    for l in layers:
        l.free()

    configs = [run_config(name, ctx, args.warmup, max(10, args.steps // 4), bool(args.parity)) for name in names]
    free_layers()

    parity = None
    if args.parity:
        from oracle import oracle as O
        rows = sample_rows(B, 16)
        want = O.OracleLayer(spec, L).forward(h[rows], lg[rows], fast=True)
        parity = parity_of(out_gpu[rows], want, len(rows))
        log(f"[bench] headline vs oracle on {len(rows)} tokens: rel-L2 {parity['rel_l2']:.2e}, "
            f"max-abs {parity['max_abs']:.2e} of |ref| {parity['ref_max_abs']:.3g}")

    cpu = None
    if args.cpu:
        hw = host_cpu()
        base = cpu_baseline(spec, L, h, lg, ("stream", 16), 32)
        a = base["mode_a"]
        cpu = {"value": a["tokens_per_s"], "unit": "tokens/s", "cores": 1, "kind": "port",
               "sample": f"oracle streaming decode (per token: route, read the 8 selected Q8_0 experts to f32, "
                         f"SwiGLU GEMVs) over the first 16 tokens of the batch, median of {CPU_RUNS} runs on one "
                         f"pinned core of {hw['cpu_model']} ({hw['nproc']} logical CPUs)",
               "GBps": a["GBps"], "mode_b": base["mode_b"], "build": base["build"], **hw}
        log(f"[bench] cpu baseline: streaming {a['tokens_per_s']} tok/s ({a['GBps']} GB/s), resident f32 "
            f"{base['mode_b']['tokens_per_s']} tok/s on {hw['cpu_model']}")
        for r in configs:
            r["cpu_baseline"] = cpu_baseline(*r["_cpu"])
            log(f"[bench] cpu baseline {r['name']}: mode A {r['cpu_baseline']['mode_a']['tokens_per_s']} tok/s, "
                f"mode B {r['cpu_baseline']['mode_b']['tokens_per_s']} tok/s")
    for r in configs:
        r.pop("_cpu")

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
        "solo_launch_ms": head["solo_launch_ms"], "router_gemv": head["router_gemv"],
        "roofline": roofline, "cpu_baseline": cpu, "parity_vs_oracle": parity,
        "sweep": [{k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()} for r in sweep],
        "configs": configs,
    }
    print(json.dumps(line), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
