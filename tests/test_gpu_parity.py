"""GPU parity: every entry point of the C ABI against the CPU oracle.

Bit-exact: dequantised values (reference fixtures and resident experts), router
logits, routing indices and probabilities, dispatch permutations.
Tolerance: MoE layer outputs within rel-L2 <= 2e-3 of the oracle's f32
composition (the bar the path is specified to), max-abs error printed.
"""
import dataclasses
import os

import numpy as np
import pytest

from anedvd_amd import moe, synth
from anedvd_amd import workloads as W
from oracle import oracle as O

pytestmark = pytest.mark.gpu

REL_L2_TOL = 2e-3
FIXTURES = ["f32", "f16", "bf16", "q4_0", "q4_1", "q5_0", "q5_1", "q8_0", "q8_1", "q2_k", "q3_k",
            "q4_k", "q5_k", "q6_k", "q8_k"]
TYPE = {n: t for t, n in W.TYPE_NAMES.items()}


@pytest.fixture(scope="module")
def ctx():
    c = moe.MoeContext(0)
    yield c
    c.close()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ------------------------------------------------------------------ dequant

@pytest.mark.parametrize("name", FIXTURES)
def test_dequant_fixtures_bit_exact(ctx, golden_dir, name):
    src = open(os.path.join(golden_dir, "dequant", name + ".bin"), "rb").read()
    want = np.frombuffer(open(os.path.join(golden_dir, "dequant", name + ".f32"), "rb").read(), dtype=np.uint32)
    got = ctx.dequantize(TYPE[name], src)
    assert np.array_equal(bits(got), want)


def test_dequant_range_errors_and_chunks(ctx, golden_dir):
    src = open(os.path.join(golden_dir, "dequant", "q6_k.bin"), "rb").read()
    want = np.frombuffer(open(os.path.join(golden_dir, "dequant", "q6_k.f32"), "rb").read(), dtype=np.uint32)
    got = np.concatenate([ctx.dequantize_range(W.Q6_K, src, off, 256) for off in (0, 256)])
    assert np.array_equal(bits(got), want)
    for args, err in [((W.Q6_K, src, 64, 256), "InvalidTensorShape"), ((W.Q6_K, src[:300], 0, 512), "TruncatedFile"),
                      ((99, src, 0, 256), "UnsupportedType")]:
        with pytest.raises(moe.MoeError) as ei:
            ctx.dequantize_range(*args)
        assert ei.value.name == err


@pytest.mark.parametrize("t", [W.Q8_0, W.Q8_1, W.Q4_0, W.Q4_1, W.Q5_0, W.Q5_1, W.Q2_K, W.Q3_K, W.Q4_K, W.Q5_K,
                               W.Q6_K])
def test_dequant_random_blocks_bit_exact(ctx, t):
    src = synth.quant_matrix(t, 5, 9, 256 * 64, 0.3)
    assert np.array_equal(bits(ctx.dequantize(t, src)), bits(O.dequantize(t, src)))


@pytest.mark.parametrize("types", [(W.Q8_0, W.Q8_0, W.Q8_0), (W.Q4_K, W.Q4_K, W.Q6_K), (W.Q4_0, W.Q4_0, W.Q4_0),
                                   (W.Q5_K, W.Q5_K, W.Q6_K), (W.Q5_K, W.Q5_K, W.Q5_K), (W.Q4_1, W.Q4_1, W.Q8_1),
                                   (W.Q5_0, W.Q5_0, W.Q5_1), (W.Q2_K, W.Q2_K, W.Q3_K), (W.Q3_K, W.Q3_K, W.Q2_K),
                                   (W.F16, W.F16, W.F16)])
def test_resident_experts_bit_exact(ctx, types):
    """The tile repack keeps every dequantised weight: readExpertF32 of the
    resident layer equals the oracle's on the GGUF payload, all three projections."""
    spec = dataclasses.replace(W.TINY_Q8_0, hidden=512, inter=768, n_experts=4, gate_type=types[0], up_type=types[1],
                               down_type=types[2])
    L = synth.make_layer(spec, seed=3)
    layer = moe.MoeLayer(ctx, spec, L)
    n = spec.inter * spec.hidden
    for which, (nm, t) in enumerate((("gate", types[0]), ("up", types[1]), ("down", types[2]))):
        for e in (0, 3):
            rc, want = O.read_expert_f32(t, L[nm], e, spec.n_experts, n)
            assert rc == O.OK
            assert np.array_equal(bits(layer.load_expert_f32(which, e)), bits(want)), (nm, e)
    layer.free()


# ------------------------------------------------------------------ routing

@pytest.mark.parametrize("out_dim,in_dim,n", [(128, 2048, 1), (128, 2048, 64), (8, 512, 16), (64, 2048, 3),
                                              (7, 300, 5), (8, 4096, 2), (64, 2048, 1024), (128, 2048, 512),
                                              (100, 1003, 700), (8, 4096, 300), (70, 5, 3), (64, 2048, 1025),
                                              (100, 1003, 5), (8, 64, 70000), (256, 1024, 300)])
def test_matmul_f16_bit_exact(ctx, out_dim, in_dim, n):
    """The router GEMV (cpu.matmulF16's chains) at the shapes of both launch forms:
    a token and an expert per lane, and two of each (>= 64 experts and >= 65536
    token-expert pairs: (64, 2048, 1024), (128, 2048, 512), and (100, 1003, 700) with
    a partial second expert half and a partial last 8-j block plus a scalar tail; an
    odd token count, whose last workgroup has one token), a hidden size below one
    block (70, 5, 3), more token blocks than a grid's y dimension takes (8, 64,
    70000: tokens run on x), and four 64-expert groups at two experts per lane (256,
    1024, 300)."""
    w = (synth.normal(1, out_dim, out_dim * in_dim) * 0.02).astype(np.float16).reshape(out_dim, in_dim)
    x = synth.normal(2, in_dim, n * in_dim).astype(np.float32).reshape(n, in_dim)
    got = ctx.matmul_f16(w, x)
    want = np.stack([O.matmul_f16(w, x[i]) for i in range(n)])
    assert np.array_equal(bits(got), bits(want))


def test_moe_route_reference_kat(ctx):
    vals = np.array([1.0, -2.0, -3.0, 5.0, -4.0, 0.5, -5.0, 3.0], dtype=np.float32)
    p, idx = ctx.moe_route(vals, 4, False)
    assert list(idx) == [3, 7, 0, 5]
    op, _ = O.moe_route(vals, 4, False)
    assert np.array_equal(bits(p), bits(op))
    p, idx = ctx.moe_route(vals, 4, True)
    assert abs(float(p.sum()) - 1.0) <= 1e-6
    _, idx = ctx.moe_route(np.full(4, 2.0, np.float32), 4, False)
    assert list(idx) == [0, 1, 2, 3]


@pytest.mark.parametrize("E,k,norm,T", [(8, 2, True, 64), (128, 8, True, 512), (64, 6, False, 256),
                                        (60, 4, False, 100), (256, 8, True, 64), (128, 1, False, 64),
                                        (128, 8, False, 16), (128, 8, True, 17), (64, 6, False, 48),
                                        (16, 4, True, 33), (100, 24, True, 40)])
def test_moe_route_bit_exact(ctx, E, k, norm, T):
    """Up to 16 tokens route in the layer's small-call kernel (routing and dispatch
    in one launch), beyond that in the route launch: both against cpu.moeRoute bit
    for bit."""
    lg = (synth.normal(7, E, T * E) * 2.0).astype(np.float32).reshape(T, E)
    lg[::3] = np.round(lg[::3] * 4) / 4   # coarse logits: many exact ties
    lg[1::7] = synth.uniform(8, E, lg[1::7].size).astype(np.float32).reshape(-1, E)
    p, idx = ctx.moe_route(lg, k, norm)
    for t in range(T):
        op, oi = O.moe_route(lg[t], k, norm)
        assert np.array_equal(idx[t], oi), t
        assert np.array_equal(bits(p[t]), bits(op)), t


@pytest.mark.parametrize("reps", [1, 4])
@pytest.mark.parametrize("E", [60, 128, 256])
def test_moe_route_special_values(ctx, E, reps):
    """NaN, +-inf, underflowing exps and all-tied rows route as cpu.moeRoute does
    (cpu.zig:1244-1288: @max skips NaN, NaN probabilities are never chosen, an
    empty slot gets (0, expert 0))."""
    base = np.linspace(-3.0, 3.0, E).astype(np.float32)
    rows = [base.copy()]
    r = base.copy(); r[5] = np.nan; r[E - 3] = np.nan; rows.append(r)
    r = np.full(E, -np.inf, np.float32); r[3] = 1.0; rows.append(r)      # one finite logit
    rows.append(np.full(E, np.nan, np.float32))                           # every logit NaN
    rows.append(np.full(E, -np.inf, np.float32))                          # every logit -inf
    r = np.zeros(E, np.float32); r[9] = np.inf; rows.append(r)            # +inf: the sum is NaN
    r = np.zeros(E, np.float32); r[::2] = -200.0; rows.append(r)          # half the exps underflow
    rows.append(np.zeros(E, np.float32))                                  # all tied
    r = base.copy(); r[-1] = 7.0; r[0] = 7.0; rows.append(r)              # tie between first and last
    lg = np.concatenate([np.stack(rows)] * reps)  # 9 or 36 tokens: the small-call kernel or the route launch
    rows = rows * reps
    for k, norm in [(8, True), (8, False), (1, False), (32, True)]:
        p, idx = ctx.moe_route(lg, k, norm)
        for t in range(len(rows)):
            op, oi = O.moe_route(lg[t], k, norm)
            assert np.array_equal(idx[t], oi), (t, k, norm)
            assert np.array_equal(bits(p[t]), bits(op)), (t, k, norm)


@pytest.mark.parametrize("T,E,k", [(1, 8, 2), (16, 8, 2), (64, 128, 8), (128, 128, 8), (96, 256, 8), (128, 256, 8),
                                   (512, 128, 8), (2048, 8, 2), (1024, 64, 6), (1000, 256, 16), (4096, 128, 8)])
def test_dispatch_bit_exact(ctx, T, E, k):
    """Stable counting sort, against the oracle, on every path: up to 1024 entries
    one workgroup ranks them, with the one-pass bitmap while E rows of ceil(P/32)
    words fit in LDS (64x8 and 128x8 of 128) and by per-wavefront segments beyond
    (96x8 and 128x8 of 256: a 128-token prefill chunk of a 256-expert model); larger
    calls go to k_dispatch_multi, one workgroup per 1024-entry block (512x8 of 128,
    2048x2 of 8, 1024x6 of 64, 1000x16 of 256, 4096x8 of 128)."""
    lg = synth.normal(11, T, T * E).astype(np.float32).reshape(T, E)
    idx = np.stack([O.moe_route(lg[t], k, True)[1] for t in range(T)])
    got = ctx.dispatch(idx, T, k, E)
    want = O.dispatch(idx, T, k, E)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)


@pytest.mark.parametrize("T,k,E", [(1, 2, 8), (512, 8, 128), (4096, 8, 128)])
def test_dispatch_rejects_bad_expert_ids(ctx, T, k, E):
    idx = (np.arange(T * k, dtype=np.uint32) % E).reshape(T, k)
    idx[T // 2, k - 1] = E + 1
    with pytest.raises(moe.MoeError):
        ctx.dispatch(idx, T, k, E)


def test_forward_256_experts_segment_dispatch(ctx):
    """A whole forward call whose dispatch ranks by segments (256 experts, top-8,
    a 128-token chunk: 1024 entries, 256 rows of 32 bitmap words do not fit in LDS),
    against the oracle."""
    spec = dataclasses.replace(W.QWEN3_30B_A3B_Q8_0, name="e256-top8", hidden=256, inter=256, n_experts=256)
    L = synth.make_layer(spec, seed=17)
    h = synth.activations(spec, 128, seed=17)
    layer = moe.MoeLayer(ctx, spec, L)
    got = layer.forward(h)
    layer.free()
    want = O.OracleLayer(spec, L).forward(h, fast=True)
    err = moe.rel_l2(got, want)
    print(f"\n256 experts, 128 tokens: rel-L2 {err:.3e}, max-abs {np.abs(got - want).max():.3e}")
    assert err <= REL_L2_TOL


@pytest.mark.parametrize("spec,T", [(W.TINY_Q8_0, 16), (W.QWEN3_30B_A3B_Q8_0, 64)])
def test_layer_route_bit_exact(ctx, spec, T):
    L = synth.make_layer(spec, seed=0)
    h = synth.activations(spec, T, seed=0)
    layer = moe.MoeLayer(ctx, spec, L)
    logits, probs, idx = layer.route(h)
    ol, op, oi = O.OracleLayer(spec, L).route(h, T)
    assert np.array_equal(bits(logits), bits(ol))
    assert np.array_equal(idx, oi)
    assert np.array_equal(bits(probs), bits(op))
    layer.free()


# ------------------------------------------------------------------ experts

def test_expert_accum_matches_oracle(ctx):
    spec = W.TINY_Q8_0
    L = synth.make_layer(spec, seed=2)
    layer = moe.MoeLayer(ctx, spec, L)
    h = synth.activations(spec, 1, seed=2)[0]
    n = spec.inter * spec.hidden
    g = O.read_expert_f32(W.Q8_0, L["gate"], 5, 8, n)[1]
    u = O.read_expert_f32(W.Q8_0, L["up"], 5, 8, n)[1]
    d = O.read_expert_f32(W.Q8_0, L["down"], 5, 8, n)[1]
    want = O.moe_expert_accum_f32(np.zeros(spec.hidden, np.float32), h, g, u, d, spec.inter, spec.hidden, 0.75)
    got = layer.expert_accum(np.zeros(spec.hidden, np.float32), 5, h, 0.75)
    assert moe.rel_l2(got, want) <= REL_L2_TOL
    # a second call accumulates (cpu.zig:1384-1387)
    layer.expert_accum(got, 5, h, 1.5)
    assert moe.rel_l2(got, 3 * want) <= REL_L2_TOL
    layer.free()


def _forward_case(ctx, spec, T, seed=0, logits=None, layer_arrays=None):
    L = layer_arrays if layer_arrays is not None else synth.make_layer(spec, seed=seed)
    h = synth.activations(spec, T, seed=seed)
    layer = moe.MoeLayer(ctx, spec, L)
    got, st = layer.forward(h, logits, stats=True)
    want = O.OracleLayer(spec, L).forward(h, logits)
    err = moe.rel_l2(got, want)
    mabs = float(np.abs(got.astype(np.float64) - want).max())
    print(f"\n{spec.name} T={T}: rel-L2 {err:.3e} max-abs {mabs:.3e} (|ref|max {np.abs(want).max():.3e}) "
          f"touched {st['touched_experts']}")
    layer.free()
    return got, want, err, st


@pytest.mark.parametrize("T", [1, 16])
def test_forward_tiny_q8_0(ctx, T):
    _, _, err, _ = _forward_case(ctx, W.TINY_Q8_0, T)
    assert err <= REL_L2_TOL


@pytest.mark.parametrize("T", [1, 8, 32, 64])
def test_forward_qwen3_30b_a3b_q8_0(ctx, T):
    spec = W.QWEN3_30B_A3B_Q8_0
    got, want, err, st = _forward_case(ctx, spec, T)
    assert err <= REL_L2_TOL
    _, oi = O.OracleLayer(spec, synth.make_layer(spec, 0)).route(synth.activations(spec, T, 0), T)[1:]
    assert st["touched_experts"] == len(np.unique(oi))


@pytest.mark.parametrize("T", [2, 8])
def test_forward_k_split_finished_in_down_crowded(ctx, T):
    """Decode batches whose gate/up splits K and whose down kernel finishes the
    partials in its prologue, with every token routed to the same eight experts:
    chunks of T tokens, the most (token, step) pieces that prologue takes."""
    spec = W.QWEN3_30B_A3B_Q8_0
    rng = np.random.default_rng(43)
    lg = rng.uniform(-6.0, -5.0, size=(T, spec.n_experts)).astype(np.float32)
    lg[:, 17:25] = rng.uniform(1.0, 2.0, size=(T, 8)).astype(np.float32)
    _, _, err, st = _forward_case(ctx, spec, T, seed=43, logits=lg)
    assert err <= REL_L2_TOL
    assert st["touched_experts"] == 8 and st["max_group"] == T


@pytest.mark.parametrize("T", [1, 64])
def test_forward_qwen3_uniform_logits(ctx, T):
    """The decode workload routes i.i.d. U(0,1) logits instead of the router GEMV."""
    spec = W.QWEN3_30B_A3B_Q8_0
    lg = synth.uniform_logits(spec, T, seed=4)
    _, _, err, _ = _forward_case(ctx, spec, T, seed=4, logits=lg)
    assert err <= REL_L2_TOL


def test_forward_shared_expert_deepseek_shape(ctx):
    spec = W.DEEPSEEK_V2_LITE_Q8_0
    _, _, err, _ = _forward_case(ctx, spec, 32)
    assert err <= REL_L2_TOL


def test_forward_shared_expert_separate_grouped(ctx):
    """A shared expert of another type than the routed experts keeps matrices of
    its own and runs on the second stream: here (width 4096, 512 tokens) on the
    grouped GEMM while the small routed experts take the decode kernels."""
    spec = dataclasses.replace(W.DEEPSEEK_V2_LITE_Q8_0, name="shared-separate", hidden=512, inter=512, n_experts=8,
                               k=2, shared_inter=4096, shared_type=W.Q4_0, shared_gated=True)
    _, _, err, st = _forward_case(ctx, spec, 512, seed=12)
    assert err <= REL_L2_TOL
    assert st["path"] == 0


@pytest.mark.parametrize("T", [1, 600])
def test_forward_shared_expert_merged(ctx, T):
    """A shared expert of the routed type and twice their width is cut into two
    expert-width pieces that every token takes as extra slots; at 600 tokens the
    routed experts and the pieces share the grouped GEMM launches."""
    spec = dataclasses.replace(W.DEEPSEEK_V2_LITE_Q8_0, name="shared-merged", hidden=512, inter=1024, n_experts=8,
                               k=2, shared_inter=2048, shared_gated=True)
    _, _, err, st = _forward_case(ctx, spec, T, seed=13)
    assert err <= REL_L2_TOL
    assert (st["path"] >= 1) == (T == 600)
    assert st["touched_experts"] <= spec.n_experts


def test_forward_gated_shared_expert(ctx):
    spec = dataclasses.replace(W.TINY_Q8_0, shared_inter=1024, shared_gated=True)
    _, _, err, _ = _forward_case(ctx, spec, 16, seed=6)
    assert err <= REL_L2_TOL


def test_forward_is_deterministic_and_order_equivariant(ctx):
    """Size-independent properties at the full decode shape: two calls are bit
    identical, and permuting the tokens permutes the outputs bit for bit (the
    per-token combine is a fixed-order gather, not atomics)."""
    spec = W.QWEN3_30B_A3B_Q8_0
    L = synth.make_layer(spec, seed=1)
    h = synth.activations(spec, 64, seed=1)
    layer = moe.MoeLayer(ctx, spec, L)
    a = layer.forward(h)
    b = layer.forward(h)
    assert np.array_equal(bits(a), bits(b))
    perm = np.random.default_rng(0).permutation(64)
    c = layer.forward(h[perm])
    assert np.array_equal(bits(c), bits(a[perm]))
    layer.free()


def test_forward_zero_input_gives_zero(ctx):
    spec = W.TINY_Q8_0
    layer = moe.MoeLayer(ctx, spec, synth.make_layer(spec, seed=0))
    out = layer.forward(np.zeros((3, spec.hidden), np.float32))
    assert np.all(out == 0)
    layer.free()


# --------------------------------------------------- other block formats

FORMATS = [(W.Q4_0, W.Q4_0, W.Q4_0), (W.Q4_K, W.Q4_K, W.Q6_K), (W.Q8_0, W.Q8_0, W.Q6_K), (W.Q4_K, W.Q4_K, W.Q4_K),
           (W.Q6_K, W.Q6_K, W.Q8_0), (W.Q5_K, W.Q5_K, W.Q6_K), (W.Q8_0, W.Q8_0, W.Q5_K), (W.Q4_1, W.Q4_1, W.Q5_1),
           (W.Q5_0, W.Q5_0, W.Q8_1), (W.Q2_K, W.Q2_K, W.Q3_K), (W.Q3_K, W.Q3_K, W.Q4_K), (W.F16, W.F16, W.F16),
           (W.F16, W.F16, W.Q8_0)]


@pytest.mark.parametrize("types", FORMATS, ids=lambda t: "/".join(W.TYPE_NAMES[x] for x in t))
@pytest.mark.parametrize("T", [1, 5, 64, 160])
def test_forward_block_formats(ctx, types, T):
    """Fused dequant + SwiGLU for every supported GGUF block format, at group sizes
    from 1 token (K split over workgroups) through several 16-token chunks per
    expert (T=64) to the grouped GEMM's 64-token chunks with partial last chunks
    (T=160: 640 entries over 16 experts)."""
    spec = dataclasses.replace(W.QWEN3_30B_A3B_Q4_K_M, name="formats", hidden=1024, inter=512, n_experts=16, k=4,
                               gate_type=types[0], up_type=types[1], down_type=types[2], scale_sigma=0.01)
    _, _, err, _ = _forward_case(ctx, spec, T, seed=T)
    assert err <= REL_L2_TOL


@pytest.mark.parametrize("types", FORMATS, ids=lambda t: "/".join(W.TYPE_NAMES[x] for x in t))
def test_forward_grouped_large_groups(ctx, types):
    """Groups of ~300 tokens (600 tokens, top-2 of 4 experts) take the grouped GEMM:
    several 64-token chunks per expert and a partial last one (expert width 2048, so
    the grouped grid has the 256 workgroups the planner asks for)."""
    spec = dataclasses.replace(W.QWEN3_30B_A3B_Q4_K_M, name="formats", hidden=512, inter=2048, n_experts=4, k=2,
                               gate_type=types[0], up_type=types[1], down_type=types[2], scale_sigma=0.01)
    _, _, err, st = _forward_case(ctx, spec, 600, seed=11)
    assert err <= REL_L2_TOL
    assert st["path"] == 1


@pytest.mark.parametrize("types", FORMATS, ids=lambda t: "/".join(W.TYPE_NAMES[x] for x in t))
def test_forward_grouped_partial_chunks(ctx, types):
    """The grouped GEMM with 1, 2 and 3 live 16-token tiles per 64-token chunk (one
    loop instantiation per count): 300 tokens, top-4 of 32 experts, groups of
    ~37 tokens (expert width 2048 for the grid size), every block format."""
    spec = dataclasses.replace(W.QWEN3_30B_A3B_Q4_K_M, name="partial", hidden=256, inter=2048, n_experts=32, k=4,
                               gate_type=types[0], up_type=types[1], down_type=types[2], scale_sigma=0.01)
    _, _, err, st = _forward_case(ctx, spec, 300, seed=17)
    assert err <= REL_L2_TOL
    assert st["path"] == 1


def _logits_for_groups(sizes, seed):
    """Router logits under which expert e receives exactly sizes[e] of the tokens
    (top-2, sum(sizes) even): the expert slots sorted by expert and slot i paired
    with slot i + T, which names a different expert while no group exceeds T."""
    slots = np.repeat(np.arange(len(sizes)), sizes)
    T = len(slots) // 2
    assert len(slots) == 2 * T and max(sizes) <= T
    rng = np.random.default_rng(seed)
    lg = rng.uniform(-1.0, 0.0, size=(T, len(sizes))).astype(np.float32)
    perm = rng.permutation(T)  # the tokens in no particular order
    lg[perm, slots[:T]] = 3.0 + rng.uniform(0.0, 0.5, T).astype(np.float32)
    lg[perm, slots[T:]] = 2.0 + rng.uniform(0.0, 0.5, T).astype(np.float32)
    return lg


@pytest.mark.parametrize("types", FORMATS, ids=lambda t: "/".join(W.TYPE_NAMES[x] for x in t))
def test_forward_grouped_every_live_tile_count(ctx, types):
    """Groups of 128 + r tokens, r giving a last chunk with 1 to 8 live 16-token
    tiles: the 128-token workgroups of the types that have them (Q8_0, Q4_0, F16,
    the 32-element formats; every count 1..8; Q8_0's down product keeps 64-token
    ones) and the 64-token workgroups of the others (counts 1..4, whole and empty
    halves of 128-token chunks)."""
    sizes = [128 + r for r in (5, 20, 40, 60, 70, 90, 100, 121)]
    lg = _logits_for_groups(sizes, seed=23)
    spec = dataclasses.replace(W.MIXTRAL_8X7B_Q4_0, name="live-tiles", hidden=256, inter=4096,
                               gate_type=types[0], up_type=types[1], down_type=types[2], scale_sigma=0.01)
    _, _, err, st = _forward_case(ctx, spec, lg.shape[0], seed=23, logits=lg)
    assert err <= REL_L2_TOL
    assert st["path"] == 1 and st["max_group"] == max(sizes)
    wide_gu = types[0] in (W.Q8_0, W.Q8_1, W.F16, W.Q4_0, W.Q4_1, W.Q5_0, W.Q5_1)
    wide_dn = types[2] in (W.F16, W.Q4_0, W.Q4_1, W.Q5_0, W.Q5_1)
    assert st["chunk"] == (128 if wide_gu or wide_dn else 64)  # gate/up and down pick their widths apart


@pytest.mark.parametrize("types", [(W.Q4_0, W.Q4_0, W.Q4_0), (W.Q4_K, W.Q4_K, W.Q6_K), (W.Q8_0, W.Q8_0, W.Q5_K)],
                         ids=lambda t: "/".join(W.TYPE_NAMES[x] for x in t))
def test_forward_grouped_split_k_down(ctx, types):
    """A down K of 128 steps (expert width 8192) over a grid of a few workgroups:
    the grouped down kernel splits K in two (two planes the combine adds), in
    128- and 64-token workgroups."""
    sizes = [70, 90, 100, 130, 40, 60, 80, 110]
    lg = _logits_for_groups(sizes, seed=29)
    spec = dataclasses.replace(W.MIXTRAL_8X7B_Q4_0, name="split-k", hidden=256, inter=8192,
                               gate_type=types[0], up_type=types[1], down_type=types[2], scale_sigma=0.01)
    L = synth.make_layer(spec, seed=29)
    h = synth.activations(spec, lg.shape[0], seed=29)
    layer = moe.MoeLayer(ctx, spec, L)
    got, st = layer.forward(h, lg, stats=True)
    layer.free()
    want = O.OracleLayer(spec, L).forward(h, lg, fast=True)
    err = moe.rel_l2(got, want)
    print(f"\nsplit-k {types}: rel-L2 {err:.3e}, chunk {st['chunk']}, down_ks {st['down_ks']}")
    assert err <= REL_L2_TOL
    assert st["path"] == 1 and st["down_ks"] == 2


@pytest.mark.parametrize("k", [1, 3])
def test_forward_large_call_combine_partial_pass(ctx, k):
    """The large-call combine loads 2, 4 or 8 slots per pass: top-1 and top-3 leave
    part of a pass empty (300 tokens x 1024 columns, one thread per column group)."""
    spec = dataclasses.replace(W.QWEN3_30B_A3B_Q8_0, name=f"combine-k{k}", hidden=1024, inter=512, n_experts=16, k=k)
    _, _, err, st = _forward_case(ctx, spec, 300, seed=53)
    assert err <= REL_L2_TOL


@pytest.mark.parametrize("sizes", [[400] * 8, [1600, 320, 320, 320, 320, 160, 80, 80]], ids=["whole", "one-too-big"])
def test_forward_grouped_xcd_ranges(ctx, sizes):
    """Large groups over few experts (the contiguous workgroup order): the dispatch
    cuts the work list into 8 XCD ranges of whole experts where each fits (eight
    groups of 4 chunks), and into even ranges when one group has more chunks than
    a range holds (13 chunks against 5)."""
    lg = _logits_for_groups(sizes, seed=47)
    spec = dataclasses.replace(W.MIXTRAL_8X7B_Q4_0, name="xcd-ranges", hidden=256, inter=4096, scale_sigma=0.01)
    L = synth.make_layer(spec, seed=47)
    h = synth.activations(spec, lg.shape[0], seed=47)
    layer = moe.MoeLayer(ctx, spec, L)
    got, st = layer.forward(h, lg, stats=True)
    layer.free()
    want = O.OracleLayer(spec, L).forward(h, lg, fast=True)
    err = moe.rel_l2(got, want)
    print(f"\nxcd ranges {sizes[:2]}: rel-L2 {err:.3e}, chunk {st['chunk']}")
    assert err <= REL_L2_TOL
    assert st["path"] == 1 and st["chunk"] == 128 and st["max_group"] == max(sizes)


# Sixteen groups averaging 42.5 tokens (the grouped GEMM), six of them of 1 to 16
# tokens (the grouped launches' small-group workgroups).
SMALL_SIZES = [1, 3, 8, 16, 17, 30, 64, 65, 90, 120, 130, 10, 5, 50, 40, 31]
SMALL_SHARED = [dataclasses.replace(W.DEEPSEEK_V2_LITE_Q8_0, name="small-shared-merged", hidden=256, inter=4096,
                                    n_experts=16, k=2, shared_inter=4096, shared_gated=True),
                dataclasses.replace(W.DEEPSEEK_V2_LITE_Q8_0, name="small-shared-separate", hidden=256, inter=4096,
                                    n_experts=16, k=2, shared_inter=2048, shared_type=W.Q4_0, shared_gated=True)]


@pytest.mark.parametrize("types", FORMATS, ids=lambda t: "/".join(W.TYPE_NAMES[x] for x in t))
def test_forward_grouped_small_groups(ctx, types):
    """A skewed call on the grouped GEMM: the groups of at most 16 tokens go to the
    dispatch's second work list and run in the same launches on one 16-token tile
    each (activations read straight from memory), the rest on the staged grouped
    GEMM, every format."""
    lg = _logits_for_groups(SMALL_SIZES, seed=31)
    spec = dataclasses.replace(W.MIXTRAL_8X7B_Q4_0, name="small-groups", hidden=256, inter=4096, n_experts=16,
                               gate_type=types[0], up_type=types[1], down_type=types[2], scale_sigma=0.01)
    L = synth.make_layer(spec, seed=31)
    h = synth.activations(spec, lg.shape[0], seed=31)
    layer = moe.MoeLayer(ctx, spec, L)
    got, st = layer.forward(h, lg, stats=True)
    layer.free()
    want = O.OracleLayer(spec, L).forward(h, lg, fast=True)
    err = moe.rel_l2(got, want)
    print(f"\nsmall groups {types}: rel-L2 {err:.3e}, small groups {st['small_groups']}")
    assert err <= REL_L2_TOL
    assert st["path"] == 1 and st["max_group"] == max(SMALL_SIZES)
    assert st["small_groups"] == sum(1 for n in SMALL_SIZES if n <= 16)


ROUTER_IN_ROUTING = [
    (dataclasses.replace(W.MIXTRAL_8X7B_Q4_0, name="mixtral-router", inter=256), (1, 2, 16)),
    (dataclasses.replace(W.DEEPSEEK_V2_LITE_Q8_0, name="deepseek-router", inter=256, shared_inter=512), (1, 2)),
    (dataclasses.replace(W.QWEN3_30B_A3B_Q8_0, name="qwen3-router", inter=256), (1,)),
    (W.TINY_Q8_0, (1, 5, 16)),
]


@pytest.mark.parametrize("spec,Ts", ROUTER_IN_ROUTING, ids=lambda v: v.name if hasattr(v, "name") else str(v))
def test_router_in_the_routing_launch_is_bit_exact(ctx, spec, Ts):
    """A call of a few tokens without logits forms the router logits inside the
    routing launch (a chain per thread, T E 8 <= 1024) instead of the router
    GEMV launch: its output must equal, bit for bit, the same call given the
    oracle's logits (cpu.matmulF16's order, which the router GEMV matches bit for
    bit), so every logit bit is the same.  Shapes of Mixtral (H 4096, 8 experts),
    DeepSeek-V2-Lite (64 experts and merged shared pieces), Qwen3 (128 experts at
    one token) and the tiny layer (H 512: the largest T)."""
    L = synth.make_layer(spec, seed=61)
    layer = moe.MoeLayer(ctx, spec, L)
    ol = O.OracleLayer(spec, L)
    for T in Ts:
        h = synth.activations(spec, T, seed=61 + T)
        lg = ol.route(h, T)[0]
        fused = layer.forward(h)
        given = layer.forward(h, lg)
        assert np.array_equal(bits(fused), bits(given)), T
        err = moe.rel_l2(fused, ol.forward(h, lg, fast=True))
        assert err <= REL_L2_TOL, (T, err)
    layer.free()


def test_route_counts_match_the_routing(ctx):
    """Engine.route_counts through the drop-in (engine.zig:726-731, 1190-1195): after
    a forward call the layer's per-expert choices of that call are added to the
    caller's counts, k per token, and the call's tokens to route_tokens.  Checked
    against the oracle's routing (the router GEMV of the call, bit-exact), over two
    calls (host and device entry points) that accumulate, on a layer with merged
    shared pieces (not counted), and refused for a layer whose call was not the last."""
    spec = W.TINY_Q8_0
    L = synth.make_layer(spec, seed=5)
    layer = moe.MoeLayer(ctx, spec, L)
    h = synth.activations(spec, 16, seed=5)
    _, _, oidx = O.OracleLayer(spec, L).route(h, 16)
    want = np.bincount(oidx.ravel(), minlength=spec.n_experts).astype(np.uint32)
    layer.forward(h)
    counts, n = layer.route_counts()
    assert np.array_equal(counts, want) and n == 16
    d_h, d_out = ctx.to_device(h), ctx.alloc(16 * spec.hidden * 4)
    layer.forward_device(d_h, 16, None, d_out)
    counts, n = layer.route_counts(counts)
    assert np.array_equal(counts, 2 * want) and n == 16
    for p in (d_h, d_out):
        ctx.free(p)
    spec2 = SMALL_SHARED[0]  # the shared expert merged as pieces after the routed experts
    lg = _logits_for_groups(SMALL_SIZES, seed=41)
    L2 = synth.make_layer(spec2, seed=41)
    other = moe.MoeLayer(ctx, spec2, L2)
    other.forward(synth.activations(spec2, lg.shape[0], seed=41), lg)
    c2, n2 = other.route_counts()
    assert np.array_equal(c2, np.array(SMALL_SIZES, dtype=np.uint32)) and n2 == lg.shape[0]
    before = counts.copy()
    with pytest.raises(moe.MoeError) as ei:
        layer.route_counts(counts)  # the last call on the context was the other layer's
    assert ei.value.name == "InvalidArgument" and np.array_equal(counts, before)
    other.free()
    layer.free()


@pytest.mark.parametrize("spec", SMALL_SHARED, ids=lambda s: s.name)
def test_forward_small_groups_with_shared_expert(ctx, spec):
    """Small groups beside a shared expert merged as pieces (large groups of their
    own) and beside a separate one (on the second stream, one join); the
    stage-timed call (one stream) and the HIP-graph replay compute the same bits
    as the direct call."""
    lg = _logits_for_groups(SMALL_SIZES, seed=37)
    T = lg.shape[0]
    L = synth.make_layer(spec, seed=37)
    h = synth.activations(spec, T, seed=37)
    layer = moe.MoeLayer(ctx, spec, L)
    got, st = layer.forward(h, lg, stats=True)
    want = O.OracleLayer(spec, L).forward(h, lg, fast=True)
    err = moe.rel_l2(got, want)
    print(f"\n{spec.name}: rel-L2 {err:.3e}, small groups {st['small_groups']}")
    assert err <= REL_L2_TOL
    assert st["path"] == 1 and st["small_groups"] == sum(1 for n in SMALL_SIZES if n <= 16)
    d_h, d_lg, d_out = ctx.to_device(h), ctx.to_device(lg), ctx.alloc(T * spec.hidden * 4)
    for kw in (dict(stages=True), dict(graph=True), dict()):
        moe.time_forward([layer], d_h, T, d_lg, d_out, 0, 2, **kw)
        again = ctx.from_device(d_out, (T, spec.hidden), np.float32)
        assert np.array_equal(bits(again), bits(got)), kw
    for p in (d_h, d_lg, d_out):
        ctx.free(p)
    layer.free()


@pytest.mark.parametrize("T", [1, 16, 160])
def test_forward_mixtral_shape_q4_0(ctx, T):
    """Mixtral-8x7B proportions (hidden 4096, top-2 of 8) with the expert width cut to
    2048 so the oracle stays fast."""
    spec = dataclasses.replace(W.MIXTRAL_8X7B_Q4_0, inter=2048)
    _, _, err, _ = _forward_case(ctx, spec, T, seed=2)
    assert err <= REL_L2_TOL


def test_forward_qwen3_q4_k_m_prefill_zipf(ctx):
    """A 300-token prefill of the Q4_K_M layer with Zipf-skewed routing (skewed
    groups up to ~200 tokens); more than 256 tokens also takes the unfused
    route/dispatch path.  (300 rather than 512 tokens keeps the oracle to seconds.)"""
    spec = W.QWEN3_30B_A3B_Q4_K_M
    lg = synth.zipf_logits(spec, 300, seed=0)
    got, want, err, st = _forward_case(ctx, spec, 300, seed=0, logits=lg)
    assert err <= REL_L2_TOL
    assert st["max_group"] > 60


def test_forward_many_passes_tiny(ctx):
    """Groups of ~16 tokens per expert: two passes of 8 tokens over the weights."""
    _, _, err, _ = _forward_case(ctx, W.TINY_Q8_0, 64, seed=9)
    assert err <= REL_L2_TOL


def test_forward_repeat_calls_keep_counters_clean(ctx):
    """The K-split completion counters are left at zero: many B=1 calls in a row (the
    path that splits K) stay identical to the first."""
    spec = W.QWEN3_30B_A3B_Q8_0
    L = synth.make_layer(spec, seed=5)
    layer = moe.MoeLayer(ctx, spec, L)
    h = synth.activations(spec, 1, seed=5)
    first = layer.forward(h)
    for _ in range(20):
        assert np.array_equal(bits(layer.forward(h)), bits(first))
    layer.free()


GRAPH_SPECS = [W.QWEN3_30B_A3B_Q8_0,
               dataclasses.replace(W.DEEPSEEK_V2_LITE_Q8_0, name="shared-gated", hidden=512, inter=512, n_experts=8,
                                   k=2, shared_inter=1024, shared_gated=True)]


@pytest.mark.parametrize("spec", GRAPH_SPECS, ids=lambda s: s.name.split()[0])
def test_graph_replay_matches_direct_forward(ctx, spec):
    """The timed loop's HIP-graph replay computes what the directly launched
    forward computes, replay after replay, with direct launches in between (with a
    shared expert, the graph holds the fork to the second stream and the join)."""
    L = synth.make_layer(spec, seed=8)
    layer = moe.MoeLayer(ctx, spec, L)
    for T in (1, 64):
        h = synth.activations(spec, T, seed=8)
        lg = synth.uniform_logits(spec, T, seed=8)
        want = layer.forward(h, lg)
        d_h, d_lg, d_out = ctx.to_device(h), ctx.to_device(lg), ctx.alloc(T * spec.hidden * 4)
        for _ in range(3):
            moe.time_forward([layer], d_h, T, d_lg, d_out, 0, 2, graph=True)
            got = ctx.from_device(d_out, (T, spec.hidden), np.float32)
            assert np.array_equal(bits(got), bits(want))
            assert np.array_equal(bits(layer.forward(h, lg)), bits(want))
        for p in (d_h, d_lg, d_out):
            ctx.free(p)
    layer.free()


# ------------------------------------------------------------------ GGUF loading

GGUF_SPECS = [
    dataclasses.replace(W.TINY_Q8_0, name="gguf-q8_0", hidden=512, inter=512, n_experts=8, k=2),
    dataclasses.replace(W.QWEN3_30B_A3B_Q4_K_M, name="gguf-q4_k-q6_k", hidden=512, inter=512, n_experts=8, k=2),
    dataclasses.replace(W.DEEPSEEK_V2_LITE_Q8_0, name="gguf-shared-merged", hidden=512, inter=512, n_experts=8, k=2,
                        shared_inter=1024, shared_gated=True),
    dataclasses.replace(W.DEEPSEEK_V2_LITE_Q8_0, name="gguf-shared-separate", hidden=512, inter=512, n_experts=8,
                        k=2, shared_inter=1024, shared_type=W.Q4_0, shared_gated=True),
]


@pytest.mark.parametrize("spec", GGUF_SPECS, ids=lambda s: s.name)
@pytest.mark.parametrize("router", ["f32", "f16-transposed"])
def test_layer_from_gguf_matches_layer_from_arrays(ctx, spec, router):
    """loadMoeLayerStreaming (load_gguf.zig:767-826) through the C++ GGUF loader:
    block 1 of a two-block file computes bit for bit what the same arrays handed
    to layer_create compute, and matches the oracle."""
    rt, tr = (W.F32, False) if router == "f32" else (W.F16, True)
    img, Ls = synth.moe_gguf(spec, 2, seed=3, router_type=rt, router_transposed=tr)
    a = moe.MoeLayer.from_gguf(ctx, img, 1, norm_topk_prob=spec.norm_topk_prob)
    b = moe.MoeLayer(ctx, spec, Ls[1])
    assert (a.spec.hidden, a.spec.inter, a.spec.n_experts, a.spec.k) == (spec.hidden, spec.inter, spec.n_experts,
                                                                         spec.k)
    for T in (1, 24):
        h = synth.activations(spec, T, seed=3)
        ya, sa = a.forward(h, stats=True)
        yb, sb = b.forward(h, stats=True)
        assert np.array_equal(bits(ya), bits(yb))
        assert sa == sb
        want = O.OracleLayer(spec, Ls[1]).forward(h)
        assert moe.rel_l2(ya, want) <= REL_L2_TOL
    a.free()
    b.free()


def test_layer_from_gguf_rejects_truncated_data(ctx):
    spec = GGUF_SPECS[0]
    img, _ = synth.moe_gguf(spec, 1, seed=3)
    with pytest.raises(moe.MoeError) as e:
        moe.MoeLayer.from_gguf(ctx, img[:-100], 0)
    assert e.value.name == "TensorDataOutOfRange"
