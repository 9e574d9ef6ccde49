"""ctypes wrapper of the CPU oracle (oracle/moe_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's CPU-baseline leg, never by the product package.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_moe.so")

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_sz = C.c_size_t

OK, ERR_UNSUPPORTED, ERR_SHAPE, ERR_TRUNCATED, ERR_DIMENSION, ERR_RANGE = 0, -1, -2, -3, -4, -5


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


AVX2_PATH = os.path.join(HERE, "liboracle_moe_avx2.so")
_lib = None
_lib_fast = None


def has_avx2() -> bool:
    try:
        return any(line.startswith("flags") and " avx2" in line for line in open("/proc/cpuinfo"))
    except OSError:
        return False


def lib_fast():
    """The AVX2 build of the same source (bit-identical results), for timing the
    CPU baseline; the portable build where the host lacks AVX2."""
    global _lib_fast
    if _lib_fast is None:
        _lib_fast = _load(AVX2_PATH) if has_avx2() and os.path.exists(AVX2_PATH) else lib()
    return _lib_fast


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = _load(LIB_PATH)
    return _lib


def _load(path):
    if True:
        L = C.CDLL(path)
        L.or_block_elems.restype = _sz
        L.or_block_elems.argtypes = [C.c_int]
        L.or_block_bytes.restype = _sz
        L.or_block_bytes.argtypes = [C.c_int]
        L.or_f16_to_f32.restype = C.c_float
        L.or_f16_to_f32.argtypes = [C.c_uint16]
        L.or_dequantize_range.restype = C.c_int
        L.or_dequantize_range.argtypes = [C.c_int, C.c_void_p, _sz, C.c_uint64, _f32p, _sz]
        L.or_read_expert_f32.restype = C.c_int
        L.or_read_expert_f32.argtypes = [C.c_int, C.c_void_p, _sz, C.c_uint32, C.c_uint32, _f32p, _sz]
        L.or_read_expert_f16.restype = C.c_int
        L.or_read_expert_f16.argtypes = [C.c_int, C.c_void_p, _sz, C.c_uint32, C.c_uint32, _u16p, _sz]
        L.or_f32_to_f16_slice.restype = None
        L.or_f32_to_f16_slice.argtypes = [_f32p, _u16p, _sz]
        for name in ("or_matmul_f16", "or_matmul_f16_scalar"):
            getattr(L, name).restype = None
            getattr(L, name).argtypes = [_f32p, _u16p, _f32p, _sz, _sz]
        L.or_matmul_f32.restype = None
        L.or_matmul_f32.argtypes = [_f32p, _f32p, _f32p, _sz, _sz]
        L.or_moe_route.restype = None
        L.or_moe_route.argtypes = [_f32p, _sz, _sz, C.c_int, _f32p, _u32p]
        L.or_moe_expert_accum_f32.restype = None
        L.or_moe_expert_accum_f32.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _sz, _sz, C.c_float, C.c_int]
        L.or_moe_expert_accum_f16.restype = None
        L.or_moe_expert_accum_f16.argtypes = [_f32p, _f32p, _f32p, _f32p, _u16p, _u16p, _u16p, _sz, _sz, C.c_float, C.c_int]
        L.or_mlp_forward.restype = None
        L.or_mlp_forward.argtypes = [_f32p, _f32p, _f32p, _u16p, _u16p, _u16p, _sz, _sz, C.c_int]
        L.or_sigmoid.restype = C.c_float
        L.or_sigmoid.argtypes = [C.c_float]
        L.or_gelu_tanh.restype = C.c_float
        L.or_gelu_tanh.argtypes = [C.c_float]
        L.or_expf.restype = C.c_float
        L.or_expf.argtypes = [C.c_float]
        L.or_dispatch.restype = None
        L.or_dispatch.argtypes = [_u32p, _sz, _sz, _sz, _i32p, _i32p, _i32p]
        L.or_layer_route.restype = None
        L.or_layer_route.argtypes = [C.c_void_p, C.c_void_p, _sz, C.c_void_p, C.c_void_p, _f32p, _u32p]
        L.or_layer_forward.restype = C.c_int
        L.or_layer_forward.argtypes = [C.c_void_p, _f32p, _sz, C.c_void_p, _f32p]
        L.or_layer_forward_streaming.restype = C.c_int
        L.or_layer_forward_streaming.argtypes = [C.c_void_p, _f32p, _sz, C.c_void_p, _f32p]
        L.or_resident_create.restype = C.c_void_p
        L.or_resident_create.argtypes = [C.c_void_p, _u8p]
        L.or_resident_free.restype = None
        L.or_resident_free.argtypes = [C.c_void_p]
        L.or_layer_forward_resident.restype = C.c_int
        L.or_layer_forward_resident.argtypes = [C.c_void_p, _f32p, _sz, C.c_void_p, _f32p]
    return L


def _bytes_arg(src):
    a = np.ascontiguousarray(np.frombuffer(src, dtype=np.uint8) if isinstance(src, (bytes, bytearray)) else src).view(np.uint8)
    return a, a.ctypes.data_as(C.c_void_p), a.nbytes


# ------------------------------------------------------------------ ops

def dequantize_range(t: int, src, elem_offset: int, n: int):
    """gguf.dequantizeRange: returns (status, f32 array)."""
    a, p, nb = _bytes_arg(src)
    out = np.zeros(n, dtype=np.float32)
    rc = lib().or_dequantize_range(t, p, nb, elem_offset, out, n)
    return rc, out


def dequantize(t: int, src) -> np.ndarray:
    a, _, nb = _bytes_arg(src)
    epb, bpb = lib().or_block_elems(t), lib().or_block_bytes(t)
    rc, out = dequantize_range(t, a, 0, nb // bpb * epb)
    if rc != OK:
        raise ValueError(f"dequantize failed: {rc}")
    return out


def read_expert_f32(t: int, payload, expert: int, n_experts: int, per_expert: int):
    a, p, nb = _bytes_arg(payload)
    out = np.zeros(per_expert, dtype=np.float32)
    rc = lib().or_read_expert_f32(t, p, nb, expert, n_experts, out, per_expert)
    return rc, out


def read_expert_f16(t: int, payload, expert: int, n_experts: int, per_expert: int):
    """Gguf.readExpertF16: returns (status, f16 bits as uint16)."""
    a, p, nb = _bytes_arg(payload)
    out = np.zeros(per_expert, dtype=np.uint16)
    rc = lib().or_read_expert_f16(t, p, nb, expert, n_experts, out, per_expert)
    return rc, out


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    """f32ToF16Slice: f16 bits (uint16) of each value, round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.zeros(x.size, dtype=np.uint16)
    lib().or_f32_to_f16_slice(x, out, x.size)
    return out


def matmul_f16(w_f16: np.ndarray, x: np.ndarray, scalar: bool = False) -> np.ndarray:
    w = np.ascontiguousarray(w_f16, dtype=np.float16).view(np.uint16)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out_dim, in_dim = w.shape
    out = np.zeros(out_dim, dtype=np.float32)
    (lib().or_matmul_f16_scalar if scalar else lib().or_matmul_f16)(out, w, x, out_dim, in_dim)
    return out


def matmul_f32(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.zeros(w.shape[0], dtype=np.float32)
    lib().or_matmul_f32(out, w, np.ascontiguousarray(x, dtype=np.float32), w.shape[0], w.shape[1])
    return out


def moe_route(logits: np.ndarray, k: int, norm_topk_prob: bool):
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    probs = np.zeros(k, dtype=np.float32)
    idx = np.zeros(k, dtype=np.uint32)
    lib().or_moe_route(lg, lg.size, k, int(norm_topk_prob), probs, idx)
    return probs, idx


def moe_expert_accum_f32(out, h, gate, up, down, inter, hidden, weight, use_gelu=False):
    hs = np.zeros(inter, dtype=np.float32)
    sc = np.zeros(inter, dtype=np.float32)
    lib().or_moe_expert_accum_f32(out, hs, sc, np.ascontiguousarray(h, np.float32), np.ascontiguousarray(gate, np.float32),
                                  np.ascontiguousarray(up, np.float32), np.ascontiguousarray(down, np.float32),
                                  inter, hidden, weight, int(use_gelu))
    return out


def moe_expert_accum_f16(out, h, gate, up, down, inter, hidden, weight, use_gelu=False):
    hs = np.zeros(inter, dtype=np.float32)
    sc = np.zeros(inter, dtype=np.float32)
    f = lambda a: np.ascontiguousarray(a, dtype=np.float16).view(np.uint16)
    lib().or_moe_expert_accum_f16(out, hs, sc, np.ascontiguousarray(h, np.float32), f(gate), f(up), f(down),
                                  inter, hidden, weight, int(use_gelu))
    return out


def mlp_forward(h, gate, up, down, inter, hidden, use_gelu=False):
    out = np.zeros(hidden, dtype=np.float32)
    gs = np.zeros(inter, dtype=np.float32)
    f = lambda a: np.ascontiguousarray(a, dtype=np.float16).view(np.uint16)
    lib().or_mlp_forward(out, gs, np.ascontiguousarray(h, np.float32), f(gate), f(up), f(down), inter, hidden, int(use_gelu))
    return out


def sigmoid(x: float) -> float:
    return lib().or_sigmoid(x)


def gelu_tanh(x: float) -> float:
    return lib().or_gelu_tanh(x)


def expf(x: float) -> float:
    return lib().or_expf(x)


def dispatch(idx: np.ndarray, n_tokens: int, k: int, n_experts: int):
    idx = np.ascontiguousarray(idx, dtype=np.uint32).reshape(-1)
    offsets = np.zeros(n_experts + 1, dtype=np.int32)
    rows = np.zeros(n_tokens * k, dtype=np.int32)
    slots = np.zeros(n_tokens * k, dtype=np.int32)
    lib().or_dispatch(idx, n_tokens, k, n_experts, offsets, rows, slots)
    return offsets, rows, slots


# ------------------------------------------------------------------ layers

class _OrLayer(C.Structure):
    _fields_ = [
        ("hidden", C.c_uint32), ("inter", C.c_uint32), ("n_experts", C.c_uint32), ("k", C.c_uint32),
        ("norm_topk_prob", C.c_int32), ("use_gelu", C.c_int32),
        ("gate_type", C.c_int32), ("up_type", C.c_int32), ("down_type", C.c_int32),
        ("gate", C.c_void_p), ("up", C.c_void_p), ("down", C.c_void_p),
        ("gate_len", C.c_size_t), ("up_len", C.c_size_t), ("down_len", C.c_size_t),
        ("router", C.c_void_p),
        ("shared_inter", C.c_uint32),
        ("shared_gate", C.c_void_p), ("shared_up", C.c_void_p), ("shared_down", C.c_void_p),
        ("shared_gate_lin", C.c_void_p),
    ]


class OracleLayer:
    """One MoE layer held by the oracle.  `arrays` is the dict from synth.make_layer."""

    def __init__(self, spec, arrays: dict):
        self.spec = spec
        self._keep = []
        keep = lambda a: (self._keep.append(a), a.ctypes.data_as(C.c_void_p))[1]
        s = _OrLayer()
        s.hidden, s.inter, s.n_experts, s.k = spec.hidden, spec.inter, spec.n_experts, spec.k
        s.norm_topk_prob, s.use_gelu = int(spec.norm_topk_prob), int(spec.use_gelu)
        s.gate_type, s.up_type, s.down_type = spec.gate_type, spec.up_type, spec.down_type
        for nm in ("gate", "up", "down"):
            a = np.ascontiguousarray(arrays[nm], dtype=np.uint8)
            setattr(s, nm, keep(a))
            setattr(s, nm + "_len", a.nbytes)
        s.router = keep(np.ascontiguousarray(arrays["router"], dtype=np.float16).view(np.uint16))
        s.shared_inter = spec.shared_inter
        if spec.shared_inter:
            # The reference holds the shared expert as f16 (loadLinear -> readF16):
            # dequantise to f32, then round to nearest f16.
            for nm in ("gate", "up", "down"):
                f = dequantize(spec.shared_type, arrays["shared_" + nm]).astype(np.float16)
                setattr(s, "shared_" + nm, keep(np.ascontiguousarray(f).view(np.uint16)))
            if "shared_gate_lin" in arrays:
                s.shared_gate_lin = keep(np.ascontiguousarray(arrays["shared_gate_lin"], dtype=np.float16).view(np.uint16))
        self.s = s
        self.ptr = C.cast(C.pointer(s), C.c_void_p)

    def route(self, h: np.ndarray | None, n_tokens: int, logits_in: np.ndarray | None = None):
        E, k = self.spec.n_experts, self.spec.k
        hp = None if h is None else np.ascontiguousarray(h, np.float32)
        lp = None if logits_in is None else np.ascontiguousarray(logits_in, np.float32)
        logits = np.zeros((n_tokens, E), dtype=np.float32)
        probs = np.zeros((n_tokens, k), dtype=np.float32)
        idx = np.zeros((n_tokens, k), dtype=np.uint32)
        lib().or_layer_route(self.ptr, None if hp is None else hp.ctypes.data_as(C.c_void_p), n_tokens,
                             None if lp is None else lp.ctypes.data_as(C.c_void_p),
                             logits.ctypes.data_as(C.c_void_p), probs.reshape(-1), idx.reshape(-1))
        return logits, probs, idx

    def forward(self, h: np.ndarray, logits_in: np.ndarray | None = None, streaming: bool = False,
                fast: bool = False) -> np.ndarray:
        """The block for T tokens.  streaming: the engine's per-token decode loop
        (expert reads per token and slot); else experts dequantised once per call
        (the engine's batched prefill, engine.zig:1204-1264).  fast: the AVX2 build."""
        h = np.ascontiguousarray(h, np.float32)
        T = h.shape[0]
        lp = None if logits_in is None else np.ascontiguousarray(logits_in, np.float32)
        out = np.zeros((T, self.spec.hidden), dtype=np.float32)
        L = lib_fast() if fast else lib()
        fn = L.or_layer_forward_streaming if streaming else L.or_layer_forward
        rc = fn(self.ptr, h.reshape(-1), T, None if lp is None else lp.ctypes.data_as(C.c_void_p), out.reshape(-1))
        if rc != OK:
            raise RuntimeError(f"oracle layer forward failed: {rc}")
        return out

    def resident(self, need, fast: bool = False) -> "Resident":
        """Mode B: experts with need[e] dequantised to f32 once and held."""
        return Resident(self, need, fast)


class Resident:
    """Resident f32 experts of an OracleLayer (or_resident_create)."""

    def __init__(self, layer: OracleLayer, need, fast: bool):
        self.layer = layer
        self.L = lib_fast() if fast else lib()
        mask = np.zeros(layer.spec.n_experts, np.uint8)
        mask[np.asarray(need, dtype=np.int64)] = 1
        self.h = self.L.or_resident_create(layer.ptr, mask)
        if not self.h:
            raise RuntimeError("or_resident_create failed")

    def forward(self, h: np.ndarray, logits_in: np.ndarray | None = None) -> np.ndarray:
        h = np.ascontiguousarray(h, np.float32)
        T = h.shape[0]
        lp = None if logits_in is None else np.ascontiguousarray(logits_in, np.float32)
        out = np.zeros((T, self.layer.spec.hidden), dtype=np.float32)
        rc = self.L.or_layer_forward_resident(self.h, h.reshape(-1), T,
                                              None if lp is None else lp.ctypes.data_as(C.c_void_p), out.reshape(-1))
        if rc != OK:
            raise RuntimeError(f"oracle resident forward failed: {rc}")
        return out

    def free(self):
        if self.h:
            self.L.or_resident_free(self.h)
            self.h = None

    def __del__(self):
        self.free()
