"""GPU parity at the benchmarked workloads' real shapes, and the invariants the
reference's engine tests pin (engine.zig:1885-2032).

Each token's output depends only on its own row of h (and logits), so a call's
sampled tokens are checked against the oracle run on just those rows: the GPU
call runs at full size, the oracle at a size it finishes in seconds.
Tolerance: rel-L2 <= 2e-3 against the oracle's f32 composition, max-abs printed.
"""
import dataclasses

import numpy as np
import pytest

from anedvd_amd import moe, synth
from anedvd_amd import workloads as W
from oracle import oracle as O

pytestmark = pytest.mark.gpu

REL_L2_TOL = 2e-3


@pytest.fixture(scope="module")
def ctx():
    c = moe.MoeContext(0)
    yield c
    c.close()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def sample_rows(T: int, n: int, seed: int = 0) -> np.ndarray:
    """n distinct token rows of a T-token call, always including the first and last."""
    if n >= T:
        return np.arange(T)
    rng = np.random.default_rng(seed)
    idx = rng.choice(np.arange(1, T - 1), n - 2, replace=False)
    return np.sort(np.concatenate([[0, T - 1], idx]))


def check_sampled(spec, L, h, lg, got, n_sample, what):
    rows = sample_rows(h.shape[0], n_sample)
    want = O.OracleLayer(spec, L).forward(h[rows], None if lg is None else lg[rows])
    err = moe.rel_l2(got[rows], want)
    mabs = float(np.abs(got[rows].astype(np.float64) - want).max())
    print(f"\n{what}: {len(rows)} of {h.shape[0]} tokens, rel-L2 {err:.3e} max-abs {mabs:.3e} "
          f"(|ref|max {np.abs(want).max():.3e})")
    assert err <= REL_L2_TOL
    return err


# ------------------------------------------------------- the benchmarked shapes

@pytest.fixture(scope="module")
def mixtral(ctx):
    spec = W.MIXTRAL_8X7B_Q4_0
    L = synth.make_layer(spec, seed=0)
    layer = moe.MoeLayer(ctx, spec, L)
    yield spec, L, layer
    layer.free()


def test_mixtral_full_width_one_token(mixtral):
    """Mixtral-8x7B at its real width (hidden 4096, experts 4096->14336->4096, Q4_0),
    one token (the GEMV regime), against the whole oracle."""
    spec, L, layer = mixtral
    for seed in (1, 2):
        h = synth.activations(spec, 1, seed=seed)
        got, st = layer.forward(h, stats=True)
        assert st["path"] == 0
        want = O.OracleLayer(spec, L).forward(h)
        err = moe.rel_l2(got, want)
        print(f"\nmixtral T=1 seed {seed}: rel-L2 {err:.3e} max-abs {np.abs(got - want).max():.3e}")
        assert err <= REL_L2_TOL


def test_mixtral_full_width_2048_tokens(mixtral):
    """Mixtral at 2048 tokens (the grouped GEMM on MFMA, groups of ~512 tokens)
    with the benchmark's logits, 16 sampled tokens against the oracle."""
    spec, L, layer = mixtral
    h = synth.activations(spec, 2048, seed=1)
    lg = np.ascontiguousarray(synth.activations(spec, 2048, seed=2)[:, :spec.n_experts])
    got, st = layer.forward(h, lg, stats=True)
    assert st["path"] == 1 and st["max_group"] > 300
    check_sampled(spec, L, h, lg, got, 16, "mixtral T=2048")


def test_qwen3_q4_k_m_512_token_prefill_zipf(ctx):
    """The Q4_K_M layer (gate/up Q4_K, down Q6_K) at its benchmarked 512-token
    prefill with Zipf-skewed routing: 64 sampled tokens against the oracle."""
    spec = W.QWEN3_30B_A3B_Q4_K_M
    L = synth.make_layer(spec, seed=0)
    layer = moe.MoeLayer(ctx, spec, L)
    h = synth.activations(spec, 512, seed=1)
    lg = synth.zipf_logits(spec, 512, seed=1)
    got, st = layer.forward(h, lg, stats=True)
    assert st["path"] == 1 and st["max_group"] > 150
    check_sampled(spec, L, h, lg, got, 64, "qwen3 q4_k_m T=512 zipf")
    layer.free()


@pytest.mark.parametrize("T,n_sample", [(32, 32), (1024, 48)])
def test_deepseek_v2_lite_with_merged_shared_expert(ctx, T, n_sample):
    """DeepSeek-V2-Lite layer (64 experts of 1408, top-6 without renormalisation,
    shared SwiGLU of width 2816 cut into two merged expert-width pieces) at the
    benchmarked decode batch and 1024-token prefill."""
    spec = W.DEEPSEEK_V2_LITE_Q8_0
    L = synth.make_layer(spec, seed=0)
    layer = moe.MoeLayer(ctx, spec, L)
    h = synth.activations(spec, T, seed=1)
    lg = synth.uniform_logits(spec, T, seed=1)
    got, st = layer.forward(h, lg, stats=True)
    assert st["path"] == (1 if T == 1024 else 0)
    check_sampled(spec, L, h, lg, got, n_sample, f"deepseek T={T}")
    layer.free()


@pytest.mark.parametrize("T", [20, 300])
def test_chained_stack_matches_layer_by_layer(ctx, T):
    """The timed stack (ANEDVD_TIME_CHAIN: layer j takes the previous layer's x and
    writes x + its block output, x += proj as main.zig:519 adds it) equals running
    the distinct layers one after another from the host and adding the residual,
    bit for bit; and a second pass from the same input gives the same result."""
    spec = dataclasses.replace(W.DEEPSEEK_V2_LITE_Q8_0, name="stack", hidden=512, inter=512, n_experts=8, k=2,
                               shared_inter=1024, shared_gated=True)
    n = 3
    Ls = [synth.make_layer(spec, seed=0, layer=i) for i in range(n)]
    layers = [moe.MoeLayer(ctx, spec, L) for L in Ls]
    h = synth.activations(spec, T, seed=2)
    lgs = np.stack([synth.uniform_logits(spec, T, seed=10 + i) for i in range(n)])
    x = h.copy()
    for i in range(n):
        x = x + layers[i].forward(x, lgs[i])
    d_h, d_lg, d_out = ctx.to_device(h), ctx.to_device(lgs), ctx.alloc(T * spec.hidden * 4)
    for passes in (1, 2):
        moe.time_forward(layers, d_h, T, d_lg, d_out, 0, n * passes, chain=True)
        got = ctx.from_device(d_out, (T, spec.hidden), np.float32)
        assert np.array_equal(bits(got), bits(x)), passes
    for p in (d_h, d_lg, d_out):
        ctx.free(p)
    for layer in layers:
        layer.free()


# ------------------------------------------------------------------ invariants

INVARIANT_SPECS = [
    dataclasses.replace(W.QWEN3_30B_A3B_Q4_K_M, name="q8_0-merged-shared", hidden=1024, inter=1024, n_experts=16,
                        k=4, gate_type=W.Q8_0, up_type=W.Q8_0, down_type=W.Q8_0, shared_inter=1024,
                        shared_type=W.Q8_0, shared_gated=True, scale_sigma=0.02),
    dataclasses.replace(W.QWEN3_30B_A3B_Q4_K_M, name="q4_k_m-separate-shared", hidden=1024, inter=1024, n_experts=16,
                        k=4, shared_inter=1024, shared_type=W.Q8_0, shared_gated=True),
]


@pytest.mark.parametrize("spec", INVARIANT_SPECS, ids=lambda s: s.name)
def test_prefill_agrees_with_per_token_decode(ctx, spec):
    """engine.zig:1885-2032: the batched prefill and per-token decode of the same
    tokens agree.  600 tokens in one call take the grouped GEMM; the same tokens
    in 16-token calls take the decode kernels and, every 8th token alone, the
    one-token path.  Routing is identical bit for bit; every token is within the
    tolerance of the batched result, and both are checked against the oracle."""
    L = synth.make_layer(spec, seed=21)
    layer = moe.MoeLayer(ctx, spec, L)
    T = 600
    h = synth.activations(spec, T, seed=21)
    whole, st = layer.forward(h, stats=True)
    assert st["path"] >= 1
    _, p_all, i_all = layer.route(h)
    pieces = []
    for t0 in range(0, T, 16):
        y, s16 = layer.forward(h[t0:t0 + 16], stats=True)
        assert s16["path"] == 0
        pieces.append(y)
        _, p16, i16 = layer.route(h[t0:t0 + 16])
        assert np.array_equal(i16, i_all[t0:t0 + 16]) and np.array_equal(bits(p16), bits(p_all[t0:t0 + 16]))
    dec = np.concatenate(pieces)
    for t in range(0, T, 8):
        one = layer.forward(h[t:t + 1])
        assert moe.rel_l2(one[0], dec[t]) <= REL_L2_TOL, t
    per_token = [moe.rel_l2(dec[t], whole[t]) for t in range(T)]
    print(f"\n{spec.name}: per-token rel-L2 prefill vs decode: max {max(per_token):.3e}")
    assert max(per_token) <= REL_L2_TOL
    check_sampled(spec, L, h, None, whole, 40, f"{spec.name} prefill")
    check_sampled(spec, L, h, None, dec, 40, f"{spec.name} decode")
    layer.free()


def test_chunked_prefill_equals_whole_call(ctx):
    """Engine.prefill runs a prompt in chunks of Options.chunk = 128 tokens
    (engine.zig:45, 1158-1268): four 128-token calls agree with one 512-token call
    token by token (Qwen3 Q4_K_M layer, Zipf routing)."""
    spec = W.QWEN3_30B_A3B_Q4_K_M
    L = synth.make_layer(spec, seed=4)
    layer = moe.MoeLayer(ctx, spec, L)
    h = synth.activations(spec, 512, seed=4)
    lg = synth.zipf_logits(spec, 512, seed=4)
    whole = layer.forward(h, lg)
    chunks = np.concatenate([layer.forward(h[c:c + 128], lg[c:c + 128]) for c in range(0, 512, 128)])
    per_token = np.array([moe.rel_l2(chunks[t], whole[t]) for t in range(512)])
    print(f"\nchunked vs whole 512-token prefill: per-token rel-L2 max {per_token.max():.3e}")
    assert per_token.max() <= REL_L2_TOL
    layer.free()


# ------------------------------------------------------------------ gelu

@pytest.mark.parametrize("shape,T", [("decode", 16), ("grouped", 600)])
def test_forward_gelu(ctx, shape, T):
    """use_gelu (cpu.zig:434-437; Gemma, load_gguf.zig:158): geluTanh(gate) * up in
    the decode kernels and the grouped GEMM, with a gated shared expert, against
    the oracle; and not the SiLU result."""
    spec = dataclasses.replace(W.TINY_Q8_0, name="gelu", hidden=512, inter=2048 if shape == "grouped" else 512,
                               n_experts=4 if shape == "grouped" else 8, k=2, use_gelu=True, shared_inter=512,
                               shared_gated=True)
    L = synth.make_layer(spec, seed=17)
    h = synth.activations(spec, T, seed=17)
    layer = moe.MoeLayer(ctx, spec, L)
    got, st = layer.forward(h, stats=True)
    assert st["path"] == (1 if shape == "grouped" else 0)
    want = O.OracleLayer(spec, L).forward(h)
    err = moe.rel_l2(got, want)
    print(f"\ngelu {shape} T={T}: rel-L2 {err:.3e} max-abs {np.abs(got - want).max():.3e}")
    assert err <= REL_L2_TOL
    silu = O.OracleLayer(dataclasses.replace(spec, use_gelu=False), L).forward(h)
    assert moe.rel_l2(got, silu) > 10 * REL_L2_TOL
    layer.free()


def test_layer_from_gemma_gguf_runs_gelu(ctx):
    """A gemma-architecture GGUF loads with use_gelu set (load_gguf.zig:145-158)."""
    spec = dataclasses.replace(W.TINY_Q8_0, name="gemma-moe", hidden=512, inter=512, n_experts=8, k=2,
                               norm_topk_prob=False, use_gelu=True)
    img, Ls = synth.moe_gguf(spec, 1, seed=5, arch="gemma2")
    layer = moe.MoeLayer.from_gguf(ctx, img, 0)
    assert layer.spec.use_gelu
    h = synth.activations(spec, 8, seed=5)
    err = moe.rel_l2(layer.forward(h), O.OracleLayer(spec, Ls[0]).forward(h))
    assert err <= REL_L2_TOL
    layer.free()


def test_layer_from_gguf_with_transposed_shared_expert(ctx):
    """Shared-expert tensors stored {out, in} as F16 load through loadLinear's
    transposition (load_gguf.zig:374-384): the layer holds them as f16 [out][in]
    and matches the oracle, which holds the shared expert as the same f16 values."""
    spec = dataclasses.replace(W.DEEPSEEK_V2_LITE_Q8_0, name="gguf-shared-transposed", hidden=512, inter=512,
                               n_experts=8, k=2, shared_inter=1024, shared_gated=True)
    img, Ls = synth.moe_gguf(spec, 1, seed=6, shared_transposed=True)
    layer = moe.MoeLayer.from_gguf(ctx, img, 0, norm_topk_prob=spec.norm_topk_prob)
    assert layer.spec.shared_type == W.F16
    for T in (3, 300):
        h = synth.activations(spec, T, seed=6)
        err = moe.rel_l2(layer.forward(h), O.OracleLayer(spec, Ls[0]).forward(h))
        assert err <= REL_L2_TOL, T
    layer.free()


# ------------------------------------------------------- op-level mirrors

@pytest.mark.parametrize("types", [(W.Q8_0, W.Q8_0, W.Q8_0), (W.Q4_K, W.Q4_K, W.Q6_K), (W.Q4_0, W.Q4_0, W.Q4_0),
                                   (W.Q5_K, W.Q5_K, W.Q2_K), (W.F16, W.F16, W.F16)])
def test_load_expert_f16_bit_exact(ctx, types):
    """readExpertF16 (gguf.zig:499-531) of the resident layer equals the oracle's
    chunked dequantise-then-round, bit for bit, for all three projections."""
    spec = dataclasses.replace(W.TINY_Q8_0, hidden=512, inter=768, n_experts=4, gate_type=types[0],
                               up_type=types[1], down_type=types[2], scale_sigma=0.5)
    L = synth.make_layer(spec, seed=7)
    layer = moe.MoeLayer(ctx, spec, L)
    n = spec.inter * spec.hidden
    for which, (nm, t) in enumerate((("gate", types[0]), ("up", types[1]), ("down", types[2]))):
        for e in (0, 3):
            rc, want = O.read_expert_f16(t, L[nm], e, spec.n_experts, n)
            assert rc == O.OK
            assert np.array_equal(layer.load_expert_f16(which, e).view(np.uint16), want), (nm, e)
    with pytest.raises(moe.MoeError) as ei:
        layer.load_expert_f16(0, spec.n_experts)
    assert ei.value.name == "TensorDataOutOfRange"
    layer.free()


@pytest.mark.parametrize("gelu", [False, True])
def test_expert_accum_on_weight_slices(ctx, gelu):
    """cpu.moeExpertAccumF32 and cpu.moeExpertAccum on caller weight slices (the
    op-level drop-ins): against the oracle, and a second call accumulates."""
    spec = W.TINY_Q8_0
    L = synth.make_layer(spec, seed=2)
    H, I = spec.hidden, spec.inter
    h = synth.activations(spec, 1, seed=2)[0]
    g, u, d = (O.read_expert_f32(W.Q8_0, L[nm], 5, 8, I * H)[1] for nm in ("gate", "up", "down"))
    want = O.moe_expert_accum_f32(np.zeros(H, np.float32), h, g, u, d, I, H, 0.75, gelu)
    got = ctx.moe_expert_accum_f32(np.zeros(H, np.float32), h, g, u, d, I, H, 0.75, gelu)
    assert moe.rel_l2(got, want) <= 1e-5
    ctx.moe_expert_accum_f32(got, h, g, u, d, I, H, 1.5, gelu)
    assert moe.rel_l2(got, 3 * want) <= 1e-5
    g16, u16, d16 = (a.astype(np.float16) for a in (g, u, d))
    want16 = O.moe_expert_accum_f16(np.zeros(H, np.float32), h, g16, u16, d16, I, H, 0.75, gelu)
    got16 = ctx.moe_expert_accum_f16(np.zeros(H, np.float32), h, g16, u16, d16, I, H, 0.75, gelu)
    assert moe.rel_l2(got16, want16) <= 1e-5


# ------------------------------------------------------- limits and fallbacks

@pytest.mark.parametrize("E,k,Is", [(256, 8, 256), (64, 30, 1024)])
def test_shared_expert_that_cannot_merge_runs_separately(ctx, E, k, Is):
    """A shared expert of the routed type and a multiple of their width is merged
    as extra experts and slots only while E + pieces <= 256 and k + pieces <= 32
    (the route and dispatch limits); past either it keeps its own matrices and the
    forward still runs, decode and grouped."""
    spec = dataclasses.replace(W.TINY_Q8_0, name="no-merge", hidden=256, inter=256, n_experts=E, k=k,
                               shared_inter=Is, shared_type=W.Q8_0, shared_gated=True)
    L = synth.make_layer(spec, seed=9)
    layer = moe.MoeLayer(ctx, spec, L)
    for T in (4, 300):
        h = synth.activations(spec, T, seed=9)
        got = layer.forward(h)
        err = moe.rel_l2(got, O.OracleLayer(spec, L).forward(h))
        print(f"\nE={E} k={k} Is={Is} T={T}: rel-L2 {err:.3e}")
        assert err <= REL_L2_TOL
    layer.free()


def test_call_above_the_token_limit_is_rejected(ctx):
    """A call whose activations would pass the kernels' 32-bit offsets is refused
    with InvalidArgument before any launch (and one at the limit's edge is not)."""
    spec = dataclasses.replace(W.TINY_Q8_0, hidden=512, inter=512, n_experts=8, k=2)
    layer = moe.MoeLayer(ctx, spec, synth.make_layer(spec, seed=1))
    lim = layer.max_tokens()
    assert lim == min(((1 << 31) - 1) // (2 * 512), ((1 << 31) - 1) // (2 * 512) // 2 - 64, 1 << 20)
    d_h = ctx.alloc(4)  # never read: the call is refused first
    with pytest.raises(moe.MoeError) as ei:
        layer.forward_device(d_h, lim + 1, None, d_h)
    assert ei.value.name == "InvalidArgument"
    ctx.free(d_h)
    layer.free()


@pytest.mark.parametrize("T", [1, 64, 300])
def test_forward_f16_activations(ctx, T):
    """fp16 activations (the Mixtral-8x7B workload's input option): the f16 entry
    widens each value exactly, so it computes the f32 entry's bits on the widened
    rows, at decode (1, 64 tokens) and grouped-GEMM (300 tokens) sizes; and the
    oracle agrees on the widened rows."""
    spec = dataclasses.replace(W.MIXTRAL_8X7B_Q4_0, name="f16-activations", inter=2048)
    L = synth.make_layer(spec, seed=41)
    h16 = (synth.activations(spec, T, seed=41) * 0.75).astype(np.float16)
    h32 = h16.astype(np.float32)
    layer = moe.MoeLayer(ctx, spec, L)
    n = T * spec.hidden
    d16, d32, o16, o32 = ctx.to_device(h16.view(np.uint16)), ctx.to_device(h32), ctx.alloc(n * 4), ctx.alloc(n * 4)
    layer.forward_device_f16(d16, T, None, o16)
    layer.forward_device(d32, T, None, o32)
    got = ctx.from_device(o16, (T, spec.hidden), np.float32)
    ref = ctx.from_device(o32, (T, spec.hidden), np.float32)
    for p in (d16, d32, o16, o32):
        ctx.free(p)
    layer.free()
    assert np.array_equal(bits(got), bits(ref))
    rows = sample_rows(T, min(T, 16), seed=41)
    want = O.OracleLayer(spec, L).forward(h32[rows], fast=True)
    err = moe.rel_l2(got[rows], want)
    print(f"\nf16 activations T={T}: rel-L2 {err:.3e} on {len(rows)} tokens")
    assert err <= REL_L2_TOL
