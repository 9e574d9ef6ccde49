"""Host-side mirror of ANEDVD's MoE call surface over the gfx950 C ABI
(include/anedvd_moe.h).

Function names and argument meaning follow src/cpu.zig and src/gguf.zig:
`dequantize_range` (gguf.zig:694), `matmul_f16` (cpu.zig:461), `moe_route`
(cpu.zig:1236), `dispatch` (engine.zig:1204-1216), `MoeLayer.load_expert_f32`
(model.zig:519), `MoeLayer.expert_accum` (cpu.zig:416), `MoeLayer.forward`
(main.zig:488-520).  Errors raise `MoeError` carrying the reference's error name.

This module only loads the HIP library; there is no CPU fallback.  If the
library is missing or no gfx950 device is present, every entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os
import weakref

import numpy as np

from . import workloads as W

HERE = os.path.dirname(os.path.abspath(__file__))
# ANEDVD_MOE_LIB selects another build of the library (e.g. one compiled with
# different tuning options); the default is the in-tree build.
LIB_PATH = os.environ.get("ANEDVD_MOE_LIB") or os.path.join(HERE, "libanedvd_moe_hip.so")

STATUS = {0: "OK", -1: "UnsupportedType", -2: "InvalidTensorShape", -3: "TruncatedFile",
          -4: "DimensionMismatch", -5: "TensorDataOutOfRange", -6: "InvalidArgument", -7: "HipError",
          -8: "NoDevice", -9: "NotGgufFile", -10: "UnsupportedVersion", -11: "InvalidMetadata",
          -12: "MissingTensor"}


class MoeError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status
        self.name = STATUS.get(status, str(status))


class LayerDesc(C.Structure):
    _fields_ = [
        ("hidden", C.c_uint32), ("inter", C.c_uint32), ("n_experts", C.c_uint32), ("k", C.c_uint32),
        ("norm_topk_prob", C.c_int32), ("use_gelu", C.c_int32),
        ("gate_type", C.c_int32), ("up_type", C.c_int32), ("down_type", C.c_int32),
        ("gate", C.c_void_p), ("gate_bytes", C.c_size_t),
        ("up", C.c_void_p), ("up_bytes", C.c_size_t),
        ("down", C.c_void_p), ("down_bytes", C.c_size_t),
        ("router", C.c_void_p),
        ("shared_inter", C.c_uint32), ("shared_type", C.c_int32),
        ("shared_gate", C.c_void_p), ("shared_gate_bytes", C.c_size_t),
        ("shared_up", C.c_void_p), ("shared_up_bytes", C.c_size_t),
        ("shared_down", C.c_void_p), ("shared_down_bytes", C.c_size_t),
        ("shared_gate_lin", C.c_void_p),
    ]


class GgufMoeCfg(C.Structure):
    _fields_ = [
        ("arch", C.c_char * 64), ("version", C.c_uint32), ("n_tensors", C.c_uint64), ("data_offset", C.c_uint64),
        ("hidden", C.c_uint32), ("n_layers", C.c_uint32), ("n_experts", C.c_uint32), ("k", C.c_uint32),
        ("inter", C.c_uint32), ("shared_inter", C.c_uint32),
        ("gate_type", C.c_int32), ("up_type", C.c_int32), ("down_type", C.c_int32), ("router_type", C.c_int32),
        ("shared_type", C.c_int32), ("has_shared_gate_lin", C.c_int32), ("use_gelu", C.c_int32),
        ("shared_as_f16", C.c_int32),
    ]


class GgufMoeOpts(C.Structure):
    _fields_ = [("norm_topk_prob", C.c_int32), ("use_gelu", C.c_int32)]


class Stats(C.Structure):
    _fields_ = [("n_tokens", C.c_uint32), ("touched_experts", C.c_uint32), ("weight_bytes", C.c_uint64),
                ("max_group", C.c_uint32), ("path", C.c_uint32), ("chunk", C.c_uint32),
                ("down_ks", C.c_uint32), ("small_groups", C.c_uint32)]


# every symbol include/anedvd_moe.h declares, with its ctypes signature
_vp, _sz, _i, _f = C.c_void_p, C.c_size_t, C.c_int, C.c_float
SIGNATURES = {
    "anedvd_moe_last_error": (C.c_char_p, []),
    "anedvd_moe_abi_version": (_i, []),
    "anedvd_moe_open": (_i, [_i, C.POINTER(_vp)]),
    "anedvd_moe_close": (None, [_vp]),
    "anedvd_moe_layer_create": (_i, [_vp, C.POINTER(LayerDesc), C.POINTER(_vp)]),
    "anedvd_moe_layer_free": (None, [_vp]),
    "anedvd_moe_layer_device_bytes": (C.c_uint64, [_vp]),
    "anedvd_dequantize_range": (_i, [_vp, _i, _vp, _sz, C.c_uint64, _vp, _sz]),
    "anedvd_moe_layer_max_tokens": (_sz, [_vp]),
    "anedvd_moe_load_expert_f32": (_i, [_vp, _i, C.c_uint32, _vp, _sz]),
    "anedvd_moe_load_expert_f16": (_i, [_vp, _i, C.c_uint32, _vp, _sz]),
    "anedvd_moe_expert_accum_f32": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _f, _i]),
    "anedvd_moe_expert_accum_f16": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _f, _i]),
    "anedvd_matmul_f16": (_i, [_vp, _vp, _vp, _vp, _sz, _sz, _sz]),
    "anedvd_moe_route": (_i, [_vp, _vp, _sz, _sz, _sz, _i, _vp, _vp]),
    "anedvd_moe_dispatch": (_i, [_vp, _vp, _sz, _sz, _sz, _vp, _vp, _vp]),
    "anedvd_moe_expert_accum": (_i, [_vp, C.c_uint32, _vp, _f, _vp]),
    "anedvd_moe_layer_route": (_i, [_vp, _vp, _sz, _vp, _vp, _vp]),
    "anedvd_moe_layer_forward": (_i, [_vp, _vp, _sz, _vp, _vp, C.POINTER(Stats)]),
    "anedvd_moe_layer_route_counts": (_i, [_vp, _vp, _vp]),
    "anedvd_moe_layer_forward_device": (_i, [_vp, _vp, _sz, _vp, _vp]),
    "anedvd_moe_layer_forward_device_noalloc": (_i, [_vp, _vp, _sz, _vp, _vp]),
    "anedvd_moe_layer_forward_device_f16": (_i, [_vp, _vp, _sz, _vp, _vp]),
    "anedvd_moe_device_alloc": (_i, [_vp, _sz, C.POINTER(_vp)]),
    "anedvd_moe_device_free": (_i, [_vp, _vp]),
    "anedvd_moe_memcpy_h2d": (_i, [_vp, _vp, _vp, _sz]),
    "anedvd_moe_memcpy_d2h": (_i, [_vp, _vp, _vp, _sz]),
    "anedvd_moe_synchronize": (_i, [_vp]),
    "anedvd_moe_time_forward": (_i, [C.POINTER(_vp), _sz, _vp, _sz, _vp, _vp, _i, _i, _i, C.POINTER(_f),
                                     C.POINTER(_f)]),
    "anedvd_gguf_moe_info": (_i, [_vp, _sz, C.c_uint32, C.POINTER(GgufMoeCfg)]),
    "anedvd_moe_layer_create_gguf": (_i, [_vp, _vp, _sz, C.c_uint32, C.POINTER(GgufMoeOpts), C.POINTER(_vp)]),
}

_lib = None


def lib():
    """The loaded HIP library.  Raises if it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MoeError(-8, f"{LIB_PATH} is not built; run __graft_entry__.build() (make -C anedvd_amd/csrc)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _check(rc: int):
    if rc != 0:
        raise MoeError(rc, lib().anedvd_moe_last_error().decode())


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


class MoeContext:
    """One device and its stream (anedvd_moe_open)."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        _check(lib().anedvd_moe_open(device, C.byref(h)))
        self.h = h
        self._layers = weakref.WeakSet()  # freed before the context closes

    def close(self):
        if self.h:
            for layer in list(self._layers):
                layer.free()
            lib().anedvd_moe_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- op-level mirrors

    def dequantize_range(self, t: int, src, elem_offset: int, n: int) -> np.ndarray:
        a = np.frombuffer(bytes(src), dtype=np.uint8) if not isinstance(src, np.ndarray) else _c(src, np.uint8)
        out = np.zeros(n, dtype=np.float32)
        _check(lib().anedvd_dequantize_range(self.h, t, _p(a) if a.size else None, a.nbytes, elem_offset, _p(out), n))
        return out

    def dequantize(self, t: int, src) -> np.ndarray:
        a = np.frombuffer(bytes(src), dtype=np.uint8) if not isinstance(src, np.ndarray) else _c(src, np.uint8)
        epb, bpb = W.BLOCK[t]
        return self.dequantize_range(t, a, 0, a.nbytes // bpb * epb)

    def matmul_f16(self, w_f16: np.ndarray, x: np.ndarray) -> np.ndarray:
        """cpu.matmulF16 over a batch: x [n_vec][in] (or [in]) -> [n_vec][out]."""
        w = _c(w_f16, np.float16)
        x = _c(x, np.float32)
        xv = x.reshape(-1, w.shape[1])
        out = np.zeros((xv.shape[0], w.shape[0]), dtype=np.float32)
        _check(lib().anedvd_matmul_f16(self.h, _p(out), _p(w), _p(xv), w.shape[0], w.shape[1], xv.shape[0]))
        return out.reshape(x.shape[:-1] + (w.shape[0],))

    def moe_route(self, logits: np.ndarray, k: int, norm_topk_prob: bool):
        lg = _c(logits, np.float32)
        lg2 = lg.reshape(-1, lg.shape[-1])
        T, E = lg2.shape
        probs = np.zeros((T, k), dtype=np.float32)
        idx = np.zeros((T, k), dtype=np.uint32)
        _check(lib().anedvd_moe_route(self.h, _p(lg2), T, E, k, int(norm_topk_prob), _p(probs), _p(idx)))
        if lg.ndim == 1:
            return probs[0], idx[0]
        return probs, idx

    def moe_expert_accum_f32(self, out: np.ndarray, h: np.ndarray, gate: np.ndarray, up: np.ndarray,
                             down: np.ndarray, inter: int, hidden: int, weight: float,
                             use_gelu: bool = False) -> np.ndarray:
        """cpu.moeExpertAccumF32 (cpu.zig:416-452): out[hidden] += weight * expert(h),
        f32 weight slices gate/up [inter][hidden], down [hidden][inter]."""
        assert out.dtype == np.float32 and out.flags.c_contiguous and out.size == hidden
        g, u, d = (_c(a, np.float32) for a in (gate, up, down))
        assert g.size == u.size == d.size == inter * hidden
        hh = _c(h, np.float32)
        _check(lib().anedvd_moe_expert_accum_f32(self.h, _p(out), _p(hh), _p(g), _p(u), _p(d), inter, hidden,
                                                 weight, int(use_gelu)))
        return out

    def moe_expert_accum_f16(self, out: np.ndarray, h: np.ndarray, gate: np.ndarray, up: np.ndarray,
                             down: np.ndarray, inter: int, hidden: int, weight: float,
                             use_gelu: bool = False) -> np.ndarray:
        """cpu.moeExpertAccum (cpu.zig:1141-1185): the same with f16 weight slices."""
        assert out.dtype == np.float32 and out.flags.c_contiguous and out.size == hidden
        g, u, d = (_c(a, np.float16) for a in (gate, up, down))
        assert g.size == u.size == d.size == inter * hidden
        hh = _c(h, np.float32)
        _check(lib().anedvd_moe_expert_accum_f16(self.h, _p(out), _p(hh), _p(g), _p(u), _p(d), inter, hidden,
                                                 weight, int(use_gelu)))
        return out

    def dispatch(self, idx: np.ndarray, n_tokens: int, k: int, n_experts: int):
        i = _c(idx, np.uint32).reshape(-1)
        offsets = np.zeros(n_experts + 1, dtype=np.int32)
        rows = np.zeros(n_tokens * k, dtype=np.int32)
        slots = np.zeros(n_tokens * k, dtype=np.int32)
        _check(lib().anedvd_moe_dispatch(self.h, _p(i), n_tokens, k, n_experts, _p(offsets), _p(rows), _p(slots)))
        return offsets, rows, slots

    # ---- device memory

    def alloc(self, nbytes: int) -> int:
        p = C.c_void_p()
        _check(lib().anedvd_moe_device_alloc(self.h, nbytes, C.byref(p)))
        return p.value

    def free(self, ptr: int):
        _check(lib().anedvd_moe_device_free(self.h, ptr))

    def to_device(self, a: np.ndarray) -> int:
        a = np.ascontiguousarray(a)
        p = self.alloc(max(a.nbytes, 4))
        _check(lib().anedvd_moe_memcpy_h2d(self.h, p, _p(a), a.nbytes))
        return p

    def from_device(self, ptr: int, shape, dtype) -> np.ndarray:
        out = np.zeros(shape, dtype=dtype)
        _check(lib().anedvd_moe_memcpy_d2h(self.h, _p(out), ptr, out.nbytes))
        return out

    def synchronize(self):
        _check(lib().anedvd_moe_synchronize(self.h))


def _gguf_image(src):
    """A GGUF image as a contiguous uint8 array: a path is memory-mapped, bytes are
    viewed in place."""
    if isinstance(src, (str, os.PathLike)):
        return np.memmap(src, dtype=np.uint8, mode="r")
    return np.frombuffer(src, dtype=np.uint8)


def gguf_moe_config(src, layer: int = 0) -> dict:
    """The MoE configuration of a GGUF file (load_gguf.zig:109-128, 251-289) and the
    tensor types of block `layer`, as anedvd_gguf_moe_info derives them (host only)."""
    img = _gguf_image(src)
    cfg = GgufMoeCfg()
    _check(lib().anedvd_gguf_moe_info(_p(img), img.nbytes, layer, C.byref(cfg)))
    out = {name: getattr(cfg, name) for name, _ in GgufMoeCfg._fields_}
    out["arch"] = cfg.arch.decode()
    return out


class MoeLayer:
    """One resident MoE layer (anedvd_moe_layer_create).  `arrays` is the dict of
    GGUF payloads from synth.make_layer (or a GGUF loader)."""

    def __init__(self, ctx: MoeContext, spec: W.LayerSpec, arrays: dict):
        self.ctx, self.spec = ctx, spec
        keep = []

        def ptr(a, dt):
            a = _c(a, dt)
            keep.append(a)
            return _p(a), a.nbytes

        d = LayerDesc()
        d.hidden, d.inter, d.n_experts, d.k = spec.hidden, spec.inter, spec.n_experts, spec.k
        d.norm_topk_prob, d.use_gelu = int(spec.norm_topk_prob), int(spec.use_gelu)
        d.gate_type, d.up_type, d.down_type = spec.gate_type, spec.up_type, spec.down_type
        d.gate, d.gate_bytes = ptr(arrays["gate"], np.uint8)
        d.up, d.up_bytes = ptr(arrays["up"], np.uint8)
        d.down, d.down_bytes = ptr(arrays["down"], np.uint8)
        d.router = ptr(np.asarray(arrays["router"], dtype=np.float16).view(np.uint16), np.uint16)[0]
        if spec.shared_inter:
            d.shared_inter, d.shared_type = spec.shared_inter, spec.shared_type
            d.shared_gate, d.shared_gate_bytes = ptr(arrays["shared_gate"], np.uint8)
            d.shared_up, d.shared_up_bytes = ptr(arrays["shared_up"], np.uint8)
            d.shared_down, d.shared_down_bytes = ptr(arrays["shared_down"], np.uint8)
            if "shared_gate_lin" in arrays:
                d.shared_gate_lin = ptr(np.asarray(arrays["shared_gate_lin"], dtype=np.float16).view(np.uint16), np.uint16)[0]
        h = C.c_void_p()
        _check(lib().anedvd_moe_layer_create(ctx.h, C.byref(d), C.byref(h)))
        self.h = h
        ctx._layers.add(self)

    @classmethod
    def from_gguf(cls, ctx: MoeContext, src, layer: int, norm_topk_prob: bool | None = None,
                  use_gelu: bool | None = None) -> "MoeLayer":
        """Block `layer` of a GGUF file (path, or the image's bytes) loaded the way
        loadMoeLayerStreaming does (load_gguf.zig:767-826); None keeps the
        reference GGUF loader's value of an option (norm_topk_prob false; use_gelu
        true for the gemma architectures, load_gguf.zig:145-158)."""
        c = gguf_moe_config(src, layer)
        img = _gguf_image(src)
        opts = GgufMoeOpts(-1 if norm_topk_prob is None else int(norm_topk_prob),
                           -1 if use_gelu is None else int(use_gelu))
        h = C.c_void_p()
        _check(lib().anedvd_moe_layer_create_gguf(ctx.h, _p(img), img.nbytes, layer, C.byref(opts), C.byref(h)))
        self = cls.__new__(cls)
        self.ctx = ctx
        self.spec = W.LayerSpec(f"{c['arch']} blk.{layer}", c["hidden"], c["inter"], c["n_experts"], c["k"],
                                bool(norm_topk_prob), c["gate_type"], c["up_type"], c["down_type"],
                                shared_inter=c["shared_inter"],
                                shared_type=(W.F16 if c["shared_as_f16"] else c["shared_type"])
                                if c["shared_type"] >= 0 else W.Q8_0,
                                shared_gated=bool(c["has_shared_gate_lin"]),
                                use_gelu=bool(c["use_gelu"] if use_gelu is None else use_gelu))
        self.h = h
        ctx._layers.add(self)
        return self

    def free(self):
        if self.h:
            if self.ctx.h:
                lib().anedvd_moe_layer_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def device_bytes(self) -> int:
        return lib().anedvd_moe_layer_device_bytes(self.h)

    def load_expert_f32(self, which: int, expert: int) -> np.ndarray:
        s = self.spec
        n = s.inter * s.hidden
        out = np.zeros(n, dtype=np.float32)
        _check(lib().anedvd_moe_load_expert_f32(self.h, which, expert, _p(out), n))
        return out

    def load_expert_f16(self, which: int, expert: int) -> np.ndarray:
        """readExpertF16 / loadExpert (gguf.zig:499-531): f16 values as np.float16."""
        s = self.spec
        n = s.inter * s.hidden
        out = np.zeros(n, dtype=np.uint16)
        _check(lib().anedvd_moe_load_expert_f16(self.h, which, expert, _p(out), n))
        return out.view(np.float16)

    def max_tokens(self) -> int:
        return int(lib().anedvd_moe_layer_max_tokens(self.h))

    def expert_accum(self, out: np.ndarray, expert: int, h: np.ndarray, weight: float) -> np.ndarray:
        assert out.dtype == np.float32 and out.flags.c_contiguous
        hh = _c(h, np.float32)
        _check(lib().anedvd_moe_expert_accum(self.h, expert, _p(hh), weight, _p(out)))
        return out

    def route(self, h: np.ndarray):
        hh = _c(h, np.float32)
        T = hh.shape[0]
        s = self.spec
        logits = np.zeros((T, s.n_experts), dtype=np.float32)
        probs = np.zeros((T, s.k), dtype=np.float32)
        idx = np.zeros((T, s.k), dtype=np.uint32)
        _check(lib().anedvd_moe_layer_route(self.h, _p(hh), T, _p(logits), _p(probs), _p(idx)))
        return logits, probs, idx

    def forward(self, h: np.ndarray, logits: np.ndarray | None = None, stats: bool = False):
        hh = _c(h, np.float32)
        T = hh.shape[0]
        out = np.zeros((T, self.spec.hidden), dtype=np.float32)
        lp = None
        if logits is not None:
            lg = _c(logits, np.float32)
            lp = _p(lg)
        st = Stats()
        _check(lib().anedvd_moe_layer_forward(self.h, _p(hh), T, lp, _p(out), C.byref(st)))
        if stats:
            return out, {"touched_experts": st.touched_experts, "weight_bytes": st.weight_bytes,
                         "max_group": st.max_group, "path": st.path, "chunk": st.chunk,
                         "down_ks": st.down_ks, "small_groups": st.small_groups}
        return out

    def forward_device(self, d_h: int, n_tokens: int, d_logits: int | None, d_out: int):
        _check(lib().anedvd_moe_layer_forward_device(self.h, d_h, n_tokens, d_logits, d_out))

    def route_counts(self, counts: np.ndarray | None = None) -> tuple:
        """Engine.route_counts for this layer (engine.zig:726-731, 1190-1195): adds
        the last forward call's per-expert choices into `counts` (uint32 [E], a
        new zero array if None) and returns (counts, tokens of that call)."""
        if counts is None:
            counts = np.zeros(self.spec.n_experts, dtype=np.uint32)
        if counts.dtype != np.uint32 or counts.shape != (self.spec.n_experts,) or not counts.flags.c_contiguous:
            raise ValueError("counts must be a contiguous uint32 array of n_experts entries")
        n = C.c_uint32(0)
        _check(lib().anedvd_moe_layer_route_counts(self.h, _p(counts), C.byref(n)))
        return counts, n.value

    def forward_device_f16(self, d_h16: int, n_tokens: int, d_logits: int | None, d_out: int):
        """forward_device with [T][H] f16 activations (bits), widened exactly on the device."""
        _check(lib().anedvd_moe_layer_forward_device_f16(self.h, d_h16, n_tokens, d_logits, d_out))

    def forward_device_noalloc(self, d_h: int, n_tokens: int, d_logits: int | None, d_out: int):
        """forward_device on the library's static per-GPU scratch: no allocation."""
        _check(lib().anedvd_moe_layer_forward_device_noalloc(self.h, d_h, n_tokens, d_logits, d_out))


TIME_GRAPH = 1
TIME_EXPERT_SOLO = 2


TIME_CHAIN = 4


def time_forward(layers: list, d_h: int, n_tokens: int, d_logits: int | None, d_out: int,
                 warmup: int, iters: int, stages: bool = False, graph: bool = False, solo: bool = False,
                 chain: bool = False):
    """Runs the timed loop inside the library (HIP events on the context's stream),
    replaying per-layer HIP graphs when `graph`.  Returns (total_ms, per-stage mean
    ms or None); with `solo` the gate/up and down entries are single-launch means
    from back-to-back launches of that stage alone, and entry 0 the router GEMV's.
    With `chain` the layers are a stack (x += proj from one layer to the next,
    d_logits [n_layers][T][E])."""
    arr = (C.c_void_p * len(layers))(*[l.h.value for l in layers])
    ms = C.c_float()
    km = (C.c_float * 6)()
    flags = (TIME_GRAPH if graph else 0) | (TIME_EXPERT_SOLO if solo else 0) | (TIME_CHAIN if chain else 0)
    _check(lib().anedvd_moe_time_forward(arr, len(layers), d_h, n_tokens, d_logits, d_out, warmup, iters,
                                         flags, C.byref(ms), km if (stages or solo) else None))
    return ms.value, (list(km) if (stages or solo) else None)


def rel_l2(got: np.ndarray, ref: np.ndarray) -> float:
    ref64 = ref.astype(np.float64)
    return float(np.linalg.norm(got.astype(np.float64) - ref64) / max(np.linalg.norm(ref64), 1e-300))
