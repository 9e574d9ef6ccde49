"""Seeded synthetic MoE layers and activations, reproducible on any host.

Every random value is a pure function of (seed, stream, index): a SplitMix64
finaliser over a counter, so the same bytes come out whether a whole tensor or
one expert of it is generated, and on whichever host generates it.

Quantised tensors are written in GGUF byte layout (the block structs of
gguf.zig:763-1059), stacked `[E][rows][cols]` with the expert axis slowest, as
`blk.N.ffn_*_exps.weight` is stored (gguf.zig:474-488).
"""
from __future__ import annotations

import numpy as np

from . import workloads as W

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)
_GOLD = np.uint64(0x9E3779B97F4A7C15)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def _key(seed: int, stream: int) -> np.uint64:
    with np.errstate(over="ignore"):
        s = np.array([(seed * 0x100000001B3 + stream * 0xC2B2AE3D27D4EB4F) & 0xFFFFFFFFFFFFFFFF], dtype=np.uint64)
        return _mix(s + _GOLD)[0]


def u64(seed: int, stream: int, n: int, offset: int = 0) -> np.ndarray:
    """n uniform 64-bit words of stream `stream`, starting at counter `offset`."""
    i = np.arange(offset, offset + n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix(i * _GOLD + _key(seed, stream))


def uniform(seed: int, stream: int, n: int, offset: int = 0) -> np.ndarray:
    """Doubles in [0, 1)."""
    return (u64(seed, stream, n, offset) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normal(seed: int, stream: int, n: int, offset: int = 0) -> np.ndarray:
    """Standard normals (Box-Muller on two counters per value), float64."""
    w = u64(seed, stream, 2 * n, 2 * offset)
    u1 = ((w[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
    u2 = (w[1::2] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def rand_bytes(seed: int, stream: int, n: int, offset: int = 0) -> np.ndarray:
    """n uniform bytes (8 per counter)."""
    c0, c1 = offset // 8, (offset + n + 7) // 8
    b = u64(seed, stream, c1 - c0, c0).view(np.uint8)
    s = offset - c0 * 8
    return b[s:s + n].copy()


def _f16_abs_normal(seed, stream, n, sigma, offset=0, div=1.0):
    return (np.abs(normal(seed, stream, n, offset)) * sigma / div).astype(np.float16)


# ----------------------------------------------------------------- quant blocks

def q8_0(seed: int, stream: int, n_blocks: int, sigma: float = 0.02, offset: int = 0) -> np.ndarray:
    """Q8_0 blocks: d = f16(|N(0,sigma)|/127), qs uniform int8 in [-127, 127]."""
    blk = np.empty((n_blocks, 34), dtype=np.uint8)
    blk[:, 0:2] = _f16_abs_normal(seed, stream, n_blocks, sigma, offset, 127.0).view(np.uint8).reshape(n_blocks, 2)
    # 16-bit draws reduced mod 255 -> [-127, 127]
    w = u64(seed, stream + 1, n_blocks * 8, offset * 8).view(np.uint16).astype(np.int32)
    q = (w % 255 - 127).astype(np.int8)
    blk[:, 2:] = q.view(np.uint8).reshape(n_blocks, 32)
    return blk


def q4_0(seed: int, stream: int, n_blocks: int, sigma: float = 0.01, offset: int = 0) -> np.ndarray:
    """Q4_0 blocks: d = f16(|N(0,sigma)|), random nibbles."""
    blk = np.empty((n_blocks, 18), dtype=np.uint8)
    blk[:, 0:2] = _f16_abs_normal(seed, stream, n_blocks, sigma, offset).view(np.uint8).reshape(n_blocks, 2)
    blk[:, 2:] = rand_bytes(seed, stream + 1, n_blocks * 16, offset * 16).reshape(n_blocks, 16)
    return blk


def q8_1(seed: int, stream: int, n_blocks: int, sigma: float = 0.02, offset: int = 0) -> np.ndarray:
    """Q8_1 blocks: d = f16(|N(0,sigma)|/127), s = f16(d * sum(qs)), qs uniform int8 in [-127, 127]."""
    b0 = q8_0(seed, stream, n_blocks, sigma, offset)
    blk = np.empty((n_blocks, 36), dtype=np.uint8)
    blk[:, 0:2] = b0[:, 0:2]
    qs = b0[:, 2:].view(np.int8).astype(np.float32)
    d = b0[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    blk[:, 2:4] = (d * qs.sum(axis=1)).astype(np.float16).view(np.uint8).reshape(n_blocks, 2)
    blk[:, 4:] = b0[:, 2:]
    return blk


def q4_1(seed: int, stream: int, n_blocks: int, sigma: float = 0.01, offset: int = 0) -> np.ndarray:
    """Q4_1 blocks: d = f16(|N(0,sigma)|), m = f16(N(0,sigma) * 8), random nibbles."""
    blk = np.empty((n_blocks, 20), dtype=np.uint8)
    blk[:, 0:2] = _f16_abs_normal(seed, stream, n_blocks, sigma, offset).view(np.uint8).reshape(n_blocks, 2)
    m = (normal(seed, stream + 1, n_blocks, offset) * sigma * 8).astype(np.float16)
    blk[:, 2:4] = m.view(np.uint8).reshape(n_blocks, 2)
    blk[:, 4:] = rand_bytes(seed, stream + 2, n_blocks * 16, offset * 16).reshape(n_blocks, 16)
    return blk


def q5_0(seed: int, stream: int, n_blocks: int, sigma: float = 0.01, offset: int = 0) -> np.ndarray:
    """Q5_0 blocks: d = f16(|N(0,sigma)|), random qh and nibbles."""
    blk = np.empty((n_blocks, 22), dtype=np.uint8)
    blk[:, 0:2] = _f16_abs_normal(seed, stream, n_blocks, sigma, offset).view(np.uint8).reshape(n_blocks, 2)
    blk[:, 2:] = rand_bytes(seed, stream + 2, n_blocks * 20, offset * 20).reshape(n_blocks, 20)
    return blk


def q5_1(seed: int, stream: int, n_blocks: int, sigma: float = 0.01, offset: int = 0) -> np.ndarray:
    """Q5_1 blocks: d = f16(|N(0,sigma)|), m = f16(N(0,sigma) * 16), random qh and nibbles."""
    blk = np.empty((n_blocks, 24), dtype=np.uint8)
    blk[:, 0:2] = _f16_abs_normal(seed, stream, n_blocks, sigma, offset).view(np.uint8).reshape(n_blocks, 2)
    m = (normal(seed, stream + 1, n_blocks, offset) * sigma * 16).astype(np.float16)
    blk[:, 2:4] = m.view(np.uint8).reshape(n_blocks, 2)
    blk[:, 4:] = rand_bytes(seed, stream + 2, n_blocks * 20, offset * 20).reshape(n_blocks, 20)
    return blk


def q4_k(seed: int, stream: int, n_blocks: int, sigma: float = 0.01, offset: int = 0) -> np.ndarray:
    """Q4_K super-blocks: d, dmin = f16(|N(0,sigma)|); random 12-byte packed 6-bit
    scales/mins; random 4-bit quants."""
    blk = np.empty((n_blocks, 144), dtype=np.uint8)
    blk[:, 0:2] = _f16_abs_normal(seed, stream, n_blocks, sigma, offset).view(np.uint8).reshape(n_blocks, 2)
    blk[:, 2:4] = _f16_abs_normal(seed, stream + 1, n_blocks, sigma, offset).view(np.uint8).reshape(n_blocks, 2)
    blk[:, 4:] = rand_bytes(seed, stream + 2, n_blocks * 140, offset * 140).reshape(n_blocks, 140)
    return blk


def q6_k(seed: int, stream: int, n_blocks: int, sigma: float = 0.01, offset: int = 0) -> np.ndarray:
    """Q6_K super-blocks: random ql/qh, random int8 sub-block scales, d = f16(|N(0,sigma)|)."""
    blk = np.empty((n_blocks, 210), dtype=np.uint8)
    blk[:, 0:208] = rand_bytes(seed, stream + 1, n_blocks * 208, offset * 208).reshape(n_blocks, 208)
    blk[:, 208:210] = _f16_abs_normal(seed, stream, n_blocks, sigma, offset).view(np.uint8).reshape(n_blocks, 2)
    return blk


def q5_k(seed: int, stream: int, n_blocks: int, sigma: float = 0.01, offset: int = 0) -> np.ndarray:
    """Q5_K super-blocks: d, dmin = f16(|N(0,sigma)|); random 12-byte packed 6-bit
    scales/mins, random high bits qh[32] and 4-bit quants qs[128]."""
    blk = np.empty((n_blocks, 176), dtype=np.uint8)
    blk[:, 0:2] = _f16_abs_normal(seed, stream, n_blocks, sigma, offset).view(np.uint8).reshape(n_blocks, 2)
    blk[:, 2:4] = _f16_abs_normal(seed, stream + 1, n_blocks, sigma, offset).view(np.uint8).reshape(n_blocks, 2)
    blk[:, 4:] = rand_bytes(seed, stream + 2, n_blocks * 172, offset * 172).reshape(n_blocks, 172)
    return blk


def q2_k(seed: int, stream: int, n_blocks: int, sigma: float = 0.01, offset: int = 0) -> np.ndarray:
    """Q2_K super-blocks: random scale|min bytes[16] and 2-bit quants qs[64];
    d, dmin = f16(|N(0,sigma)|/8)."""
    blk = np.empty((n_blocks, 84), dtype=np.uint8)
    blk[:, 0:80] = rand_bytes(seed, stream + 2, n_blocks * 80, offset * 80).reshape(n_blocks, 80)
    blk[:, 80:82] = _f16_abs_normal(seed, stream, n_blocks, sigma, offset, 8.0).view(np.uint8).reshape(n_blocks, 2)
    blk[:, 82:84] = _f16_abs_normal(seed, stream + 1, n_blocks, sigma, offset, 8.0).view(np.uint8).reshape(n_blocks, 2)
    return blk


def q3_k(seed: int, stream: int, n_blocks: int, sigma: float = 0.01, offset: int = 0) -> np.ndarray:
    """Q3_K super-blocks: random hmask[32], 2-bit quants qs[64] and 12 bytes of packed
    6-bit scales; d = f16(|N(0,sigma)|/16)."""
    blk = np.empty((n_blocks, 110), dtype=np.uint8)
    blk[:, 0:108] = rand_bytes(seed, stream + 1, n_blocks * 108, offset * 108).reshape(n_blocks, 108)
    blk[:, 108:110] = _f16_abs_normal(seed, stream, n_blocks, sigma, offset, 16.0).view(np.uint8).reshape(n_blocks, 2)
    return blk


def f16(seed: int, stream: int, n_blocks: int, sigma: float = 0.02, offset: int = 0) -> np.ndarray:
    """F16 weights (blocks of one value): N(0, sigma) rounded to f16."""
    v = (normal(seed, stream, n_blocks, offset) * sigma).astype(np.float16)
    return v.view(np.uint8).reshape(n_blocks, 2)


_GEN = {W.F16: f16, W.Q8_0: q8_0, W.Q8_1: q8_1, W.Q4_0: q4_0, W.Q4_1: q4_1, W.Q5_0: q5_0, W.Q5_1: q5_1, W.Q2_K: q2_k,
        W.Q3_K: q3_k, W.Q4_K: q4_k, W.Q5_K: q5_k, W.Q6_K: q6_k}


_CHUNK_BLOCKS = 1 << 20


def _workers() -> int:
    import os
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def quant_matrix(t: int, seed: int, stream: int, n_elems: int, sigma: float, elem_offset: int = 0) -> np.ndarray:
    """GGUF blocks of type t for elements [elem_offset, elem_offset + n_elems) of a
    stream.  Every block is a pure function of its index, so large tensors are
    generated in chunks on a thread pool (numpy's element-wise work runs outside
    the GIL) with the same bytes as one call."""
    epb, bpb = W.BLOCK[t]
    assert n_elems % epb == 0 and elem_offset % epb == 0
    nb, b0 = n_elems // epb, elem_offset // epb
    if nb <= _CHUNK_BLOCKS:
        return _GEN[t](seed, stream, nb, sigma, b0).reshape(-1)
    from concurrent.futures import ThreadPoolExecutor
    out = np.empty(nb * bpb, dtype=np.uint8)

    def part(c0):
        n = min(_CHUNK_BLOCKS, nb - c0)
        out[c0 * bpb:(c0 + n) * bpb] = _GEN[t](seed, stream, n, sigma, b0 + c0).reshape(-1)

    with ThreadPoolExecutor(_workers()) as ex:
        list(ex.map(part, range(0, nb, _CHUNK_BLOCKS)))
    return out


# ------------------------------------------------------------------- layers

_STREAM = {"gate": 100, "up": 200, "down": 300, "router": 400, "sh_gate": 500, "sh_up": 600,
           "sh_down": 700, "sh_gate_lin": 800, "x": 900, "logits": 1000}


def layer_seed(seed: int, layer: int) -> int:
    return seed * 1000003 + layer


def expert_tensor(spec: W.LayerSpec, which: str, seed: int, experts: range | None = None) -> np.ndarray:
    """GGUF payload bytes of a stacked expert tensor, or of a contiguous range of
    its experts (the bytes are identical to slicing the whole payload)."""
    t = {"gate": spec.gate_type, "up": spec.up_type, "down": spec.down_type}[which]
    per = spec.inter * spec.hidden
    experts = experts if experts is not None else range(spec.n_experts)
    sigma = spec.scale_sigma
    return quant_matrix(t, seed, _STREAM[which], per * len(experts), sigma, per * experts.start)


def router_f16(spec: W.LayerSpec, seed: int) -> np.ndarray:
    """fp32 N(0, router_sigma) router, rounded to f16 as the loader does (loadLinear -> readF16)."""
    r = (normal(seed, _STREAM["router"], spec.n_experts * spec.hidden) * spec.router_sigma).astype(np.float32)
    return r.astype(np.float16).reshape(spec.n_experts, spec.hidden)


def make_layer(spec: W.LayerSpec, seed: int = 0, layer: int = 0) -> dict:
    s = layer_seed(seed, layer)
    L = {
        "gate": expert_tensor(spec, "gate", s),
        "up": expert_tensor(spec, "up", s),
        "down": expert_tensor(spec, "down", s),
        "router": router_f16(spec, s),
    }
    if spec.shared_inter:
        n = spec.shared_inter * spec.hidden
        L["shared_gate"] = quant_matrix(spec.shared_type, s, _STREAM["sh_gate"], n, spec.scale_sigma)
        L["shared_up"] = quant_matrix(spec.shared_type, s, _STREAM["sh_up"], n, spec.scale_sigma)
        L["shared_down"] = quant_matrix(spec.shared_type, s, _STREAM["sh_down"], n, spec.scale_sigma)
        if spec.shared_gated:
            L["shared_gate_lin"] = (normal(s, _STREAM["sh_gate_lin"], spec.hidden) * 0.02).astype(np.float32).astype(np.float16)
    return L


def activations(spec: W.LayerSpec, n_tokens: int, seed: int = 0) -> np.ndarray:
    """fp32 N(0,1) activations [T][H]; RMS-normalised with unit weight and eps 1e-5
    (cpu.rmsnorm, cpu.zig:11-18) when the workload asks for it."""
    x = normal(seed, _STREAM["x"], n_tokens * spec.hidden).astype(np.float32).reshape(n_tokens, spec.hidden)
    if spec.rms_normalise_input:
        ms = (x.astype(np.float64) ** 2).mean(axis=1, keepdims=True)
        x = (x / np.sqrt(ms + 1e-5)).astype(np.float32)
    return x


def uniform_logits(spec: W.LayerSpec, n_tokens: int, seed: int = 0) -> np.ndarray:
    """Router logits ~ U(0,1) i.i.d. (the decode workload's routing)."""
    return uniform(seed, _STREAM["logits"], n_tokens * spec.n_experts).astype(np.float32).reshape(n_tokens, spec.n_experts)


# Zipf-skewed prefill routing: logits = N(0,1) + alpha * log(p_e), p_e proportional to
# rank^-1.1 over a seeded permutation of the experts.  alpha = 0.44 puts the busiest
# expert at ~300 of 512 tokens with top-8 of 128 (299 for seed 0, 286 for seed 1;
# tests/test_workloads.py keeps it in range).
ZIPF_S = 1.1
ZIPF_ALPHA = 0.44


def zipf_logits(spec: W.LayerSpec, n_tokens: int, seed: int = 0, alpha: float = ZIPF_ALPHA) -> np.ndarray:
    E = spec.n_experts
    perm = np.argsort(u64(seed, _STREAM["logits"] + 1, E))
    rank = np.empty(E, dtype=np.float64)
    rank[perm] = np.arange(1, E + 1)
    p = rank ** -ZIPF_S
    p /= p.sum()
    bias = alpha * np.log(p)
    z = normal(seed, _STREAM["logits"] + 2, n_tokens * E).reshape(n_tokens, E)
    return (z + bias[None, :]).astype(np.float32)


def dequantize_host(t: int, payload: np.ndarray) -> np.ndarray:
    """f32 values of F16, Q8_0 or Q4_0 blocks (gguf.zig:763-776, 827-840: every
    product d * q is exact in f32), for writing test files."""
    b = np.ascontiguousarray(payload, dtype=np.uint8)
    if t == W.F16:
        return b.view(np.float16).astype(np.float32)
    if t == W.Q8_0:
        blk = b.reshape(-1, 34)
        d = blk[:, :2].copy().view(np.float16).astype(np.float32)
        return (d * blk[:, 2:].view(np.int8).astype(np.float32)).reshape(-1)
    if t == W.Q4_0:
        blk = b.reshape(-1, 18)
        d = blk[:, :2].copy().view(np.float16).astype(np.float32)
        qs = blk[:, 2:]
        q = np.concatenate([(qs & 15).astype(np.int32) - 8, (qs >> 4).astype(np.int32) - 8], axis=1)
        return (d * q.astype(np.float32)).reshape(-1)
    raise ValueError(f"dequantize_host: type {t} not handled")


def moe_gguf(spec: W.LayerSpec, n_layers: int, seed: int = 0, arch: str = "qwen3moe", router_type: int = W.F32,
             router_transposed: bool = False, extra_metadata: dict | None = None, drop: tuple = (),
             shared_transposed: bool = False) -> tuple:
    """A GGUF image of `n_layers` MoE blocks of `spec` in llama.cpp's tensor naming
    (the names load_gguf.zig:767-826 reads): blk.N.ffn_gate_inp.weight {H, E}
    (`router_type` F32 or F16; {E, H} when `router_transposed`),
    blk.N.ffn_{gate,up}_exps.weight {H, I, E}, blk.N.ffn_down_exps.weight {I, H, E},
    and the shared expert's blk.N.ffn_{gate,up}_shexp {H, Is}, ffn_down_shexp {Is, H}
    and ffn_gate_inp_shexp {H} (F32).  With `shared_transposed` the shared expert's
    three tensors are F16 stored the other way round ({Is, H}, {H, Is}: the
    dequantised values rounded to f16 and transposed), which loadLinear also takes.
    Block N holds make_layer(spec, seed, N).  `drop` lists metadata keys or tensor
    names left out.  Returns (image bytes, [per-layer arrays])."""
    from . import gguf as G
    H, I, E, Is = spec.hidden, spec.inter, spec.n_experts, spec.shared_inter
    meta = {"general.architecture": arch, "general.alignment": 32, f"{arch}.block_count": n_layers,
            f"{arch}.embedding_length": H, f"{arch}.feed_forward_length": 4 * H, f"{arch}.expert_count": E,
            f"{arch}.expert_used_count": spec.k, f"{arch}.expert_feed_forward_length": I}
    if Is:
        meta[f"{arch}.expert_shared_feed_forward_length"] = Is
    meta.update(extra_metadata or {})
    meta = {k: v for k, v in meta.items() if k not in drop}
    tensors, layers = [], []
    for n in range(n_layers):
        L = make_layer(spec, seed=seed, layer=n)
        layers.append(L)
        r = L["router"].astype(np.float32)
        if router_transposed:
            r, rdims = np.ascontiguousarray(r.T), (E, H)
        else:
            rdims = (H, E)
        rb = (r.astype(np.float16) if router_type == W.F16 else r).tobytes()
        tensors += [(f"blk.{n}.ffn_gate_inp.weight", rdims, router_type, rb),
                    (f"blk.{n}.ffn_gate_exps.weight", (H, I, E), spec.gate_type, L["gate"].tobytes()),
                    (f"blk.{n}.ffn_up_exps.weight", (H, I, E), spec.up_type, L["up"].tobytes()),
                    (f"blk.{n}.ffn_down_exps.weight", (I, H, E), spec.down_type, L["down"].tobytes())]
        if Is:
            lin = L.get("shared_gate_lin")
            lin = np.zeros(H, np.float32) if lin is None else lin.astype(np.float32)
            if shared_transposed:
                def tr(nm, rows, cols):  # [rows][cols] values -> f16 stored [cols][rows], dims {rows, cols}
                    v = dequantize_host(spec.shared_type, L[nm]).reshape(rows, cols)
                    return np.ascontiguousarray(v.astype(np.float16).T).tobytes()
                tensors += [(f"blk.{n}.ffn_gate_shexp.weight", (Is, H), W.F16, tr("shared_gate", Is, H)),
                            (f"blk.{n}.ffn_up_shexp.weight", (Is, H), W.F16, tr("shared_up", Is, H)),
                            (f"blk.{n}.ffn_down_shexp.weight", (H, Is), W.F16, tr("shared_down", H, Is))]
            else:
                tensors += [(f"blk.{n}.ffn_gate_shexp.weight", (H, Is), spec.shared_type, L["shared_gate"].tobytes()),
                            (f"blk.{n}.ffn_up_shexp.weight", (H, Is), spec.shared_type, L["shared_up"].tobytes()),
                            (f"blk.{n}.ffn_down_shexp.weight", (Is, H), spec.shared_type,
                             L["shared_down"].tobytes())]
            tensors += [(f"blk.{n}.ffn_gate_inp_shexp.weight", (H,), W.F32, lin.tobytes())]
    tensors = [t for t in tensors if t[0] not in drop]
    return G.write(meta, tensors), layers
