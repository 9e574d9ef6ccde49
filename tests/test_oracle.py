"""Pins the CPU oracle before anything is compared against it.

Golden vectors and known answers come from the reference's own tests
(gguf.zig:1424-1570, gguf.zig:1648-1715, gguf.zig:1771-1792, cpu.zig:1290-1400);
the rest are brute force and closed forms, chosen so that a dropped term, a
wrong sign or index, or a transposed operand fails one of them.
"""
import os
import struct

import numpy as np
import pytest

from anedvd_amd import synth
from anedvd_amd import workloads as W
from anedvd_amd.gguf import Gguf
from oracle import oracle as O

FIXTURE_TYPES = {"f32": W.F32, "f16": W.F16, "bf16": W.BF16, "q4_0": W.Q4_0, "q4_1": W.Q4_1,
                 "q5_0": W.Q5_0, "q5_1": W.Q5_1, "q8_0": W.Q8_0, "q8_1": W.Q8_1, "q2_k": W.Q2_K,
                 "q3_k": W.Q3_K, "q4_k": W.Q4_K, "q5_k": W.Q5_K, "q6_k": W.Q6_K, "q8_k": W.Q8_K}

SHA256 = {  # published digests of the four hot-path fixtures
    "q8_0.bin": "16f7e2116b9e4d2a6c1d0fd71aa5c679031faf72fc084dc043ca369219c84653",
    "q8_0.f32": "f1330301cfbb20eb66bb83b43e69c0a173f566bd73b56f95ffc3bd88ea361f7b",
    "q4_0.bin": "27e6f80d97d44b4a27bae89f6dd38f66579e7def3e9265559823bffd06f90030",
    "q4_0.f32": "fed5dae21d05a22e30673c75f369678591202dc5479685c22aab3164fa380d6d",
    "q4_k.bin": "387afa5b897a3dc97d06c3864cfa11b383e4f6b1eede0e848df50b9e233f4ea7",
    "q4_k.f32": "81c2125b48b20718716c4186df48cc5343e9c5bdca8d7790ebe584e40807aab9",
    "q6_k.bin": "f933da4144febb7f11bf0611e38ae4363d5f6d61d9626bb723fc953c990cc3d5",
    "q6_k.f32": "0dd0a2303609bf0a7eb815558054ce75240d16e61365820681ab5ffac8f1ec02",
}


def fixture(golden_dir, name):
    with open(os.path.join(golden_dir, "dequant", name), "rb") as f:
        return f.read()


def test_fixture_digests(golden_dir):
    import hashlib
    for name, digest in SHA256.items():
        assert hashlib.sha256(fixture(golden_dir, name)).hexdigest() == digest, name


@pytest.mark.parametrize("name", sorted(FIXTURE_TYPES))
def test_dequant_bit_exact_against_reference_fixtures(golden_dir, name):
    """gguf.zig:1528-1570: every type equals the ggml fixture bit for bit."""
    t = FIXTURE_TYPES[name]
    src = fixture(golden_dir, name + ".bin")
    want = np.frombuffer(fixture(golden_dir, name + ".f32"), dtype=np.uint32)
    got = O.dequantize(t, src).view(np.uint32)
    assert got.shape == want.shape
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{name}: first differing element {bad[:5]}"


def test_dequant_hand_blocks():
    """gguf.zig:1424-1488: hand-computed legacy blocks."""
    z = lambda n: bytes(n)
    _, o = O.dequantize_range(W.Q4_0, bytes([0x00, 0x38, 0x21]) + z(15), 0, 32)
    assert (o[0], o[16], o[1], o[17], o[31]) == (-3.5, -3.0, -4.0, -4.0, -4.0)
    _, o = O.dequantize_range(W.Q4_1, bytes([0x00, 0x38, 0x00, 0x34, 0x21]) + z(15), 0, 32)
    assert (o[0], o[16], o[1]) == (0.75, 1.25, 0.25)
    _, o = O.dequantize_range(W.Q5_0, bytes([0x00, 0x34, 0x01, 0x00, 0x01, 0x00, 0x21]) + z(15), 0, 32)
    assert (o[0], o[16], o[1], o[17]) == (0.25, 0.5, -4.0, -4.0)
    _, o = O.dequantize_range(W.Q5_1, bytes([0x00, 0x38, 0x00, 0x3C, 0x01, 0x00, 0x01, 0x00, 0x21]) + z(15), 0, 32)
    assert (o[0], o[16], o[1]) == (9.5, 10.0, 1.0)
    _, o = O.dequantize_range(W.Q8_0, bytes([0x00, 0x34, 0x80, 0x7F, 0xFF]) + z(29), 0, 32)
    assert (o[0], o[1], o[2], o[3]) == (-32.0, 31.75, -0.25, 0.0)
    _, o = O.dequantize_range(W.Q8_1, bytes([0x00, 0x34, 0x00, 0x00, 0x80, 0x7F, 0xFF]) + z(29), 0, 32)
    assert (o[0], o[1], o[2]) == (-32.0, 31.75, -0.25)
    _, o = O.dequantize_range(W.F16, bytes([0x00, 0x3C, 0x00, 0xC0, 0x00, 0x38]), 0, 3)
    assert list(o) == [1.0, -2.0, 0.5]
    _, o = O.dequantize_range(W.BF16, bytes([0x80, 0x3F, 0x00, 0xC0, 0x00, 0x80]), 0, 3)
    assert list(o) == [1.0, -2.0, 0.0] and np.signbit(o[2])


def test_dequant_hand_q4_k_block():
    """gguf.zig:1490-1526."""
    blk = bytearray(144)
    blk[0:4] = bytes([0x00, 0x3C, 0x00, 0x38])
    blk[4:8] = bytes([2, 3, 4, 5])
    blk[8] = 1
    blk[12:16] = bytes([6, 7, 8, 9])
    blk[16] = 0x21
    blk[16 + 32] = 0x0F
    _, o = O.dequantize_range(W.Q4_K, bytes(blk), 0, 256)
    assert (o[0], o[1], o[31], o[32], o[33], o[64], o[96], o[128], o[255]) == (1.5, -0.5, -0.5, 6.0, 0.0, 60.0, 0.0, 0.0, 0.0)


def test_dequant_errors_and_chunking(golden_dir):
    """dequantizeRange checks (gguf.zig:694-728) and chunked Q6_K (gguf.zig:1771-1792)."""
    src = fixture(golden_dir, "q6_k.bin")
    want = np.frombuffer(fixture(golden_dir, "q6_k.f32"), dtype=np.uint32)
    got = np.concatenate([O.dequantize_range(W.Q6_K, src, off, 256)[1] for off in range(0, 512, 256)])
    assert np.array_equal(got.view(np.uint32), want)
    assert O.dequantize_range(W.Q6_K, src, 64, 256)[0] == O.ERR_SHAPE
    assert O.dequantize_range(W.Q6_K, src, 0, 100)[0] == O.ERR_SHAPE
    assert O.dequantize_range(W.Q6_K, src[:300], 0, 512)[0] == O.ERR_TRUNCATED
    assert O.dequantize_range(W.Q6_K, src, 512, 256)[0] == O.ERR_TRUNCATED
    assert O.dequantize_range(99, src, 0, 256)[0] == O.ERR_UNSUPPORTED
    assert O.dequantize_range(W.Q6_K, src, 0, 0)[0] == O.OK


def test_tiny_v3_gguf_values(golden_dir):
    """gguf.zig:1648-1715: values of the reference's hand-written GGUF fixture."""
    g = Gguf.load(os.path.join(golden_dir, "gguf", "tiny_v3.gguf"))
    assert g.version == 3 and len(g.order) == 4 and g.arch() == "llama"
    assert g.kv["fixture.u64"] == 1234567890123 and g.kv["fixture.u32_array"] == [1, 2, 3]
    t = g.tensor("w.f32")
    assert list(O.dequantize(t.ttype, g.tensor_bytes(t))) == [1.5, -2.0, 3.25, 0.5]
    t = g.tensor("w.f16")
    assert t.dims == (2, 3) and list(O.dequantize(t.ttype, g.tensor_bytes(t))) == [1.0, 2.5, -0.75, 4.0, -1.5, 0.25]
    q4 = O.dequantize(W.Q4_0, g.tensor_bytes(g.tensor("w.q4_0")))
    assert (q4[0], q4[16], q4[31]) == (-3.5, -3.0, -4.0)
    q8 = O.dequantize(W.Q8_0, g.tensor_bytes(g.tensor("w.q8_0")))
    assert (q8[0], q8[1], q8[31]) == (-32.0, -31.75, -24.25)


@pytest.mark.parametrize("t", [W.Q8_0, W.Q4_0, W.Q4_K, W.Q6_K])
def test_dequant_closed_form_exactness(t):
    """Every block product is exact in f32 (Q4_K rounds once, at the subtraction):
    y/d must be an integer for Q8_0/Q4_0, y/(d*sc) for Q6_K."""
    n = 4096 if t in (W.Q8_0, W.Q4_0) else 4096
    src = synth.quant_matrix(t, 7, 3, n, 0.5)
    y = O.dequantize(t, src).astype(np.float64)
    epb, bpb = W.BLOCK[t]
    blocks = src.reshape(-1, bpb)
    if t == W.Q8_0:
        d = blocks[:, 0:2].copy().view(np.float16).astype(np.float64)
        q = y.reshape(-1, 32) / d
        assert np.array_equal(q, blocks[:, 2:].view(np.int8).astype(np.float64))
    elif t == W.Q4_0:
        d = blocks[:, 0:2].copy().view(np.float16).astype(np.float64)
        q = y.reshape(-1, 32) / d
        assert np.all(q == np.round(q)) and q.min() >= -8 and q.max() <= 7
    elif t == W.Q6_K:
        d = blocks[:, 208:210].copy().view(np.float16).astype(np.float64)
        sc = blocks[:, 192:208].view(np.int8).astype(np.float64)  # 16 scales of 16 elements
        yy = y.reshape(-1, 2, 4, 2, 16)  # half, quarter (32 rows apart), is, l
        s = sc.reshape(-1, 2, 4, 2)  # [blk][half][quarter][is]: sc[is + 2*quarter]
        den = d[:, :, None, None, None] * s[..., None]
        ok = np.broadcast_to(den != 0, yy.shape)
        q = yy[ok] / np.broadcast_to(den, yy.shape)[ok]
        assert np.all(yy[~ok] == 0)
        assert np.all(q == np.round(q)) and q.min() >= -32 and q.max() <= 31
    else:  # Q4_K: (y + m1) / d1 is an integer nibble
        assert np.all(np.isfinite(y))


def test_matmul_f16_lane_order_known_answer():
    """cpu.matmulF16 sums in 8 strided lanes, then the lanes in order: with
    x = [2^24, 1 x7, -2^24, 1 x7] lane 0 cancels exactly and lanes 1..7 each hold 2,
    so the answer is 14; a sequential sum would lose the ones next to 2^24."""
    x = np.array([2.0 ** 24] + [1.0] * 7 + [-(2.0 ** 24)] + [1.0] * 7, dtype=np.float32)
    w = np.ones((1, 16), dtype=np.float16)
    assert O.matmul_f16(w, x)[0] == 14.0
    assert O.matmul_f16(w, x, scalar=True)[0] != 14.0


def test_matmul_against_f64():
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((37, 300)) * 0.1).astype(np.float16)
    x = rng.standard_normal(300).astype(np.float32)
    ref = w.astype(np.float64) @ x.astype(np.float64)
    bound = np.abs(w.astype(np.float64)) @ np.abs(x.astype(np.float64))
    for got in (O.matmul_f16(w, x), O.matmul_f16(w, x, scalar=True), O.matmul_f32(w.astype(np.float32), x)):
        assert np.all(np.abs(got - ref) <= 1e-6 * bound + 1e-30)


def test_moe_route_reference_kat():
    """cpu.zig:1290-1336."""
    vals = np.array([1.0, -2.0, -3.0, 5.0, -4.0, 0.5, -5.0, 3.0], dtype=np.float32)
    e = np.exp(vals.astype(np.float64) - 5.0)
    expect_p = e[[3, 7, 0, 5]] / e.sum()
    p, idx = O.moe_route(vals, 4, False)
    assert list(idx) == [3, 7, 0, 5]
    assert np.all(np.abs(p - expect_p) <= 1e-6)
    p, idx = O.moe_route(vals, 4, True)
    assert abs(float(p.sum()) - 1.0) <= 1e-6
    p, idx = O.moe_route(vals, 1, False)
    assert idx[0] == 3
    p, idx = O.moe_route(np.full(4, 2.0, np.float32), 4, False)
    assert sorted(idx) == [0, 1, 2, 3] and list(idx) == [0, 1, 2, 3]


def _route_brute_force(lg, k, norm):
    """Rank by (p desc, index asc) with p = f32(expf(v - max)) * f32(1/sum): a
    full sort, not the reference's k-pass scan."""
    lg = lg.astype(np.float32)
    mx = np.float32(lg.max())
    ex = np.array([O.expf(float(np.float32(v - mx))) for v in lg], dtype=np.float32)
    s = np.float32(0)
    for v in ex:
        s = np.float32(s + v)
    inv = np.float32(1) / s
    p = (ex * inv).astype(np.float32)
    order = sorted(range(len(lg)), key=lambda e: (-p[e], e))[:k]
    probs = p[order]
    if norm:
        t = np.float32(0)
        for v in probs:
            t = np.float32(t + v)
        probs = (probs / t).astype(np.float32)
    return probs, np.array(order, dtype=np.uint32)


@pytest.mark.parametrize("E,k,norm", [(8, 2, True), (128, 8, True), (64, 6, False), (60, 4, False)])
def test_moe_route_brute_force(E, k, norm):
    for t in range(20):
        lg = (synth.normal(3, t, E) * (0.3 if t % 2 else 3.0)).astype(np.float32)
        if t % 5 == 0:  # force ties: quantise logits coarsely
            lg = (np.round(lg * 2) / 2).astype(np.float32)
        p, idx = O.moe_route(lg, k, norm)
        bp, bidx = _route_brute_force(lg, k, norm)
        assert np.array_equal(idx, bidx)
        assert np.array_equal(p.view(np.uint32), bp.view(np.uint32))


def _lcg_weights(n, seed):
    out = np.empty(n, dtype=np.float16)
    for i in range(n):
        seed = (seed * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float16(np.float32(np.float32(seed >> 8) / np.float32(8388608.0) - np.float32(1.0)))
    return out, seed


def test_moe_expert_accum_reference_kat():
    """cpu.zig:1338-1388: H=4, I=3, LCG seed 99 weights; a second call with weight 2 gives 3x."""
    H, I = 4, 3
    h = np.array([0.5, -0.25, 1.0, 0.0], dtype=np.float32)
    gate, s = _lcg_weights(I * H, 99)
    up, s = _lcg_weights(I * H, s)
    down, s = _lcg_weights(H * I, s)
    g = gate.astype(np.float64).reshape(I, H) @ h
    u = up.astype(np.float64).reshape(I, H) @ h
    act = g / (1 + np.exp(-g)) * u
    want = down.astype(np.float64).reshape(H, I) @ act
    out = np.zeros(H, dtype=np.float32)
    O.moe_expert_accum_f16(out, h, gate, up, down, I, H, 1.0)
    assert np.all(np.abs(out - want) <= 1e-5)
    O.moe_expert_accum_f16(out, h, gate, up, down, I, H, 2.0)
    assert np.all(np.abs(out - 3 * want) <= 1e-5)
    out32 = np.zeros(H, dtype=np.float32)
    O.moe_expert_accum_f32(out32, h, gate.astype(np.float32), up.astype(np.float32), down.astype(np.float32), I, H, 1.0)
    assert np.array_equal(out32, O.moe_expert_accum_f16(np.zeros(H, np.float32), h, gate, up, down, I, H, 1.0))


def test_expert_accum_and_mlp_against_f64():
    rng = np.random.default_rng(5)
    H, I = 96, 40
    h = rng.standard_normal(H).astype(np.float32)
    gate, up, down = [(rng.standard_normal(s) * 0.2).astype(np.float16) for s in ((I, H), (I, H), (H, I))]
    g = gate.astype(np.float64) @ h
    u = up.astype(np.float64) @ h
    ref = down.astype(np.float64) @ (g / (1 + np.exp(-g)) * u)
    out = O.moe_expert_accum_f32(np.zeros(H, np.float32), h, gate.astype(np.float32), up.astype(np.float32),
                                 down.astype(np.float32), I, H, 0.75)
    assert np.abs(out - 0.75 * ref).max() <= 1e-5 * np.abs(ref).max()
    mlp = O.mlp_forward(h, gate, up, down, I, H)
    assert np.abs(mlp - ref).max() <= 1e-5 * np.abs(ref).max()


def test_sigmoid_reference_kat():
    """cpu.zig:1390-1400."""
    assert abs(O.sigmoid(0.0) - 0.5) <= 1e-6
    assert O.sigmoid(100.0) > 0.999 and O.sigmoid(-100.0) < 0.001
    assert O.sigmoid(1000.0) == 1.0
    assert 0.0 <= O.sigmoid(-1000.0) < 1e-30


def test_gelu_tanh_reference_kat():
    """cpu.zig:1434-1449: the six reference values within 1e-6, and gelu is not SiLU
    at -3 (they differ by more than 0.13)."""
    for x, want in ((0.0, 0.0), (1.0, 0.84119199), (-1.0, -0.15880796), (3.0, 2.99636241), (-3.0, -0.00363739),
                    (0.5, 0.34571400)):
        assert abs(O.gelu_tanh(x) - want) <= 1e-6, x
    assert abs(O.gelu_tanh(-3.0) - (-3.0 / (1.0 + np.exp(3.0)))) > 0.13


def test_gelu_tanh_closed_forms():
    """What the formula 0.5 x (1 + tanh(c (x + 0.044715 x^3))) fixes: gelu(0) = 0;
    tanh saturates, so gelu(x) = x exactly for large x and -0 for very negative x;
    tanh is odd, so gelu(x) - gelu(-x) = x; and the f64 formula within 1e-6 over a
    sweep (a wrong constant, sign or factor fails one of them)."""
    assert O.gelu_tanh(0.0) == 0.0
    for x in (10.0, 20.0, 1e3):
        assert O.gelu_tanh(x) == x
    for x in (-10.0, -20.0, -1e3):
        assert O.gelu_tanh(x) == 0.0
    xs = np.linspace(-8.0, 8.0, 4001).astype(np.float32)
    got = np.array([O.gelu_tanh(float(x)) for x in xs], dtype=np.float64)
    x64 = xs.astype(np.float64)
    want = 0.5 * x64 * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x64 + 0.044715 * x64 ** 3)))
    assert np.abs(got - want).max() <= 1e-6 * np.maximum(1.0, np.abs(want)).max()
    odd = np.array([O.gelu_tanh(float(x)) - O.gelu_tanh(float(-x)) for x in xs[::40]])
    assert np.abs(odd - xs[::40]).max() <= 2e-6 * np.abs(xs).max()


def test_layer_forward_gelu_against_f64():
    """use_gelu runs geluTanh(gate) * up in every expert (cpu.zig:434-437) and in the
    shared expert (cpu.zig:1207): the layer against an f64 composition."""
    import dataclasses
    spec = dataclasses.replace(W.TINY_Q8_0, use_gelu=True)
    L = synth.make_layer(spec, seed=3)
    h = synth.activations(spec, 6, seed=3)
    got = O.OracleLayer(spec, L).forward(h)
    ref = _layer_f64(spec, L, h, gelu=True)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-6
    silu = O.OracleLayer(dataclasses.replace(spec, use_gelu=False), L).forward(h)
    assert np.linalg.norm(silu - ref) / np.linalg.norm(ref) > 1e-2


@pytest.mark.parametrize("T,E,k", [(1, 8, 2), (16, 8, 2), (64, 128, 8), (37, 64, 6)])
def test_dispatch_is_stable_sort_by_expert(T, E, k):
    rng = np.random.default_rng(T * 100 + E)
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.uint32)
    offsets, rows, slots = O.dispatch(idx, T, k, E)
    flat = idx.reshape(-1)
    order = np.argsort(flat, kind="stable")  # (expert, token, slot) order
    assert np.array_equal(rows, (order // k).astype(np.int32))
    assert np.array_equal(slots, (order % k).astype(np.int32))
    assert np.array_equal(offsets, np.searchsorted(flat[order], np.arange(E + 1)).astype(np.int32))


def test_read_expert_slices_whole_tensor():
    """Expert e of a stacked tensor is bytes [e*per, (e+1)*per) and dequantises to rows
    e*out .. (e+1)*out-1 of the whole tensor (gguf.zig:474-552)."""
    E, per = 4, 256 * 3
    for t in (W.Q8_0, W.Q4_0, W.Q4_K, W.Q6_K):
        payload = synth.quant_matrix(t, 11, 1, E * per, 0.1)
        whole = O.dequantize(t, payload)
        for e in range(E):
            rc, got = O.read_expert_f32(t, payload, e, E, per)
            assert rc == O.OK and np.array_equal(got.view(np.uint32), whole[e * per:(e + 1) * per].view(np.uint32))
        assert O.read_expert_f32(t, payload, E, E, per)[0] == O.ERR_RANGE
        assert O.read_expert_f32(t, payload, 0, E, per + W.BLOCK[t][0])[0] == O.ERR_DIMENSION


def test_f32_to_f16_round_to_nearest_even():
    """f32ToF16Slice (gguf.zig:682-692) against numpy's IEEE conversion, bit for
    bit: every finite f16 value, the midpoint between each pair of neighbours (the
    ties: even wins), values just off the midpoints, the subnormal range, the
    overflow edge (65504 stays, 65520 becomes inf) and random f32 bit patterns."""
    allh = np.arange(0x10000, dtype=np.uint32).astype(np.uint16).view(np.float16)
    fin = allh[np.isfinite(allh)].astype(np.float32)
    pos = np.unique(np.abs(fin))
    mid = ((pos[:-1].astype(np.float64) + pos[1:]) / 2).astype(np.float32)  # exact in f32
    near = np.concatenate([np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(0))])
    rng = np.random.default_rng(0)
    rnd = rng.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    rnd = rnd[np.isfinite(rnd)]
    edge = np.array([65504.0, 65519.99, 65520.0, 1e9, -1e9, 2.0 ** -25, 2.0 ** -24, 3 * 2.0 ** -26, 2.0 ** -26,
                     1e-30, -0.0, 0.0, np.inf, -np.inf], dtype=np.float32)
    for x in (fin, mid, -mid, near, rnd, edge):
        with np.errstate(over="ignore"):
            want = x.astype(np.float16).view(np.uint16)
        assert np.array_equal(O.f32_to_f16(x), want)
    nan = O.f32_to_f16(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7C00) == 0x7C00 and (nan & 0x3FF) != 0


def test_read_expert_f16_is_dequant_then_round():
    """readExpertF16 (gguf.zig:499-531) in 2048-element chunks equals the whole
    expert dequantised and rounded, with readExpertF32's checks."""
    E, per = 3, 256 * 24
    for t in (W.Q8_0, W.Q4_0, W.Q4_K, W.Q6_K, W.Q5_K):
        payload = synth.quant_matrix(t, 13, 2, E * per, 0.3)
        for e in range(E):
            rc, f32 = O.read_expert_f32(t, payload, e, E, per)
            rc16, f16 = O.read_expert_f16(t, payload, e, E, per)
            assert rc == rc16 == O.OK
            assert np.array_equal(f16, f32.astype(np.float16).view(np.uint16))
        assert O.read_expert_f16(t, payload, E, E, per)[0] == O.ERR_RANGE
        assert O.read_expert_f16(t, payload, 0, E, per + W.BLOCK[t][0])[0] == O.ERR_DIMENSION


def _layer_f64(spec, L, h, logits=None, gelu=False):
    """f64 composition of the block (main.zig:488-520) from the oracle's routing."""
    ol = O.OracleLayer(spec, L)
    _, probs, idx = ol.route(h, h.shape[0], logits)
    H, I, E = spec.hidden, spec.inter, spec.n_experts
    out = np.zeros((h.shape[0], H))
    cache = {}
    for t in range(h.shape[0]):
        for s in range(spec.k):
            e = int(idx[t, s])
            if e not in cache:
                cache[e] = [O.read_expert_f32(tt, L[nm], e, E, I * H)[1].astype(np.float64)
                            for nm, tt in (("gate", spec.gate_type), ("up", spec.up_type), ("down", spec.down_type))]
            g_w, u_w, d_w = cache[e]
            x = h[t].astype(np.float64)
            g = g_w.reshape(I, H) @ x
            u = u_w.reshape(I, H) @ x
            if gelu:
                act = 0.5 * g * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (g + 0.044715 * g ** 3)))
            else:
                act = g / (1 + np.exp(-g))
            out[t] += probs[t, s] * (d_w.reshape(H, I) @ (act * u))
    return out


def test_layer_forward_streaming_equals_expert_major_and_f64():
    spec = W.TINY_Q8_0
    L = synth.make_layer(spec, seed=0)
    h = synth.activations(spec, 16, seed=0)
    ol = O.OracleLayer(spec, L)
    a = ol.forward(h)
    b = ol.forward(h, streaming=True)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    ref = _layer_f64(spec, L, h)
    assert np.linalg.norm(a - ref) / np.linalg.norm(ref) < 1e-6


def test_fast_build_and_resident_mode_are_bit_identical():
    """The CPU baseline's builds and modes compute the same bits: the AVX2 build of
    the oracle (vectorised 8-lane loops, no FMA, no reassociation) equals the
    portable build, and the resident-f32 decode loop equals the streaming one."""
    import dataclasses
    spec = dataclasses.replace(W.DEEPSEEK_V2_LITE_Q8_0, hidden=512, inter=512, n_experts=16, k=4,
                               shared_inter=1024, shared_gated=True)
    L = synth.make_layer(spec, seed=4)
    h = synth.activations(spec, 12, seed=4)
    ol = O.OracleLayer(spec, L)
    ref = ol.forward(h, streaming=True)
    for fast in (False, True):
        assert np.array_equal(ol.forward(h, streaming=True, fast=fast).view(np.uint32), ref.view(np.uint32))
        assert np.array_equal(ol.forward(h, fast=fast).view(np.uint32), ref.view(np.uint32))
        R = ol.resident(range(spec.n_experts), fast=fast)
        assert np.array_equal(R.forward(h).view(np.uint32), ref.view(np.uint32))
        R.free()
    _, _, idx = ol.route(h, 12)
    R = ol.resident([int(idx[0, 0])])
    with pytest.raises(RuntimeError):  # a token routed to an expert that is not held
        R.forward(h)
    R.free()


def test_layer_forward_shared_expert_gate():
    """With shared_gate_lin = 0 the shared expert joins at half weight
    (engine.zig:2100-2105); with no gate it joins at weight 1.0 (engine.zig:687-691)."""
    import dataclasses
    spec = dataclasses.replace(W.TINY_Q8_0, shared_inter=256, shared_gated=True)
    L = synth.make_layer(spec, seed=1)
    h = synth.activations(spec, 3, seed=1)
    routed = O.OracleLayer(dataclasses.replace(spec, shared_inter=0), L).forward(h)
    sh = np.stack([O.mlp_forward(h[t], O.dequantize(W.Q8_0, L["shared_gate"]).astype(np.float16).reshape(256, 512),
                                 O.dequantize(W.Q8_0, L["shared_up"]).astype(np.float16).reshape(256, 512),
                                 O.dequantize(W.Q8_0, L["shared_down"]).astype(np.float16).reshape(512, 256), 256, 512)
                   for t in range(3)])
    L0 = dict(L, shared_gate_lin=np.zeros(512, np.float16))
    half = O.OracleLayer(spec, L0).forward(h)
    assert np.allclose(half, routed + 0.5 * sh, rtol=1e-6, atol=1e-6)
    ungated = O.OracleLayer(dataclasses.replace(spec, shared_gated=False), {k: v for k, v in L.items() if k != "shared_gate_lin"}).forward(h)
    assert np.allclose(ungated, routed + sh, rtol=1e-6, atol=1e-6)
