"""The C++ GGUF loader's host side (anedvd_gguf_moe_info; no GPU): the container
rules of Gguf.parse (gguf.zig:587-657) and the MoE configuration rules of
load_gguf.zig:109-128 and 251-289, on synthetic MoE files written by
anedvd_amd.gguf.write and on the reference's own fixture tests/golden/gguf/tiny_v3.gguf
(gguf.zig:1648-1715)."""
import ctypes as C
import dataclasses
import os
import struct

import numpy as np
import pytest

from anedvd_amd import gguf as G
from anedvd_amd import moe, synth
from anedvd_amd import workloads as W

TINY = dataclasses.replace(W.TINY_Q8_0, hidden=256, inter=256, n_experts=4, k=2)
SHARED = dataclasses.replace(TINY, shared_inter=512, shared_gated=True)


def raw_info(img: bytes, layer: int = 0):
    cfg = moe.GgufMoeCfg()
    buf = C.create_string_buffer(img, len(img))
    rc = moe.lib().anedvd_gguf_moe_info(C.cast(buf, C.c_void_p), len(img), layer, C.byref(cfg))
    return rc, cfg


def status_of(img: bytes, layer: int = 0) -> str:
    return moe.STATUS[raw_info(img, layer)[0]]


def test_config_of_a_synthetic_qwen3moe_file():
    img, _ = synth.moe_gguf(TINY, 3)
    c = moe.gguf_moe_config(img, 2)
    assert c["arch"] == "qwen3moe" and c["version"] == 3 and c["n_layers"] == 3
    assert (c["hidden"], c["inter"], c["n_experts"], c["k"], c["shared_inter"]) == (256, 256, 4, 2, 0)
    assert (c["gate_type"], c["up_type"], c["down_type"], c["router_type"]) == (W.Q8_0, W.Q8_0, W.Q8_0, W.F32)
    assert c["shared_type"] == -1 and c["has_shared_gate_lin"] == 0
    g = G.Gguf.from_bytes(img)  # the Python reader agrees on the container
    assert c["data_offset"] == g.data_offset and c["n_tensors"] == len(g.order)


def test_shared_expert_config():
    img, _ = synth.moe_gguf(SHARED, 1)
    c = moe.gguf_moe_config(img)
    assert c["shared_inter"] == 512 and c["shared_type"] == W.Q8_0 and c["has_shared_gate_lin"] == 1


def test_shared_width_comes_from_the_tensor_without_metadata():
    """load_gguf.zig:279-286: no expert_shared_feed_forward_length -> dims[1] of
    blk.0.ffn_gate_shexp.weight (not dims[0], the hidden size)."""
    img, _ = synth.moe_gguf(SHARED, 1, drop=("qwen3moe.expert_shared_feed_forward_length",))
    assert moe.gguf_moe_config(img)["shared_inter"] == 512


def test_no_shared_expert_without_metadata_or_tensor():
    img, _ = synth.moe_gguf(TINY, 1, drop=("qwen3moe.expert_shared_feed_forward_length",))
    assert moe.gguf_moe_config(img)["shared_inter"] == 0


def test_expert_used_count_defaults_to_two():
    """load_gguf.zig:255-259: experts declared, no expert_used_count -> 2."""
    spec = dataclasses.replace(TINY, k=3)
    img, _ = synth.moe_gguf(spec, 1, drop=("qwen3moe.expert_used_count",))
    assert moe.gguf_moe_config(img)["k"] == 2


def test_tensor_expert_count_wins_over_metadata():
    """load_gguf.zig:268-273: expert_count disagrees with ffn_gate_exps -> the tensor."""
    img, _ = synth.moe_gguf(TINY, 1, extra_metadata={"qwen3moe.expert_count": 7})
    assert moe.gguf_moe_config(img)["n_experts"] == 4


def test_expert_width_from_the_tensor_not_the_metadata():
    """load_gguf.zig:262-275: the tensor shapes are authoritative."""
    img, _ = synth.moe_gguf(TINY, 1, extra_metadata={"qwen3moe.expert_feed_forward_length": 999})
    assert moe.gguf_moe_config(img)["inter"] == 256


def test_metadata_value_types_and_typed_counts():
    """asU32 (gguf.zig:197-211) takes any integer type that fits, and bool."""
    img, _ = synth.moe_gguf(TINY, 1, extra_metadata={"qwen3moe.expert_used_count": (G.U64, 2),
                                                     "qwen3moe.block_count": (G.I32, 1)})
    c = moe.gguf_moe_config(img)
    assert c["k"] == 2 and c["n_layers"] == 1


def test_the_reference_fixture_parses_and_is_not_moe():
    """tiny_v3.gguf carries every metadata value type; the container parses (same
    version, tensor count and data offset as the Python reader) and the file is
    refused for lack of llama.embedding_length, as load_gguf.zig:109-112 refuses it."""
    path = os.path.join(os.path.dirname(__file__), "golden", "gguf", "tiny_v3.gguf")
    img = open(path, "rb").read()
    rc, cfg = raw_info(img)
    g = G.Gguf.load(path)
    assert moe.STATUS[rc] == "MissingTensor"
    assert cfg.version == 3 and cfg.n_tensors == len(g.order) and cfg.data_offset == g.data_offset
    with pytest.raises(moe.MoeError):
        moe.gguf_moe_config(img)


def test_container_errors():
    img, _ = synth.moe_gguf(TINY, 1)
    assert status_of(b"XXXX" + img[4:]) == "NotGgufFile"
    assert status_of(img[:4] + struct.pack("<I", 1) + img[8:]) == "UnsupportedVersion"
    assert status_of(img[:4] + struct.pack("<I", 4) + img[8:]) == "UnsupportedVersion"
    for cut in (3, 10, 40, 200):
        assert status_of(img[:cut]) == "TruncatedFile", cut
    # 6 bytes after the counts cannot hold 9 entries: the count check comes first
    assert status_of(img[:30]) == "InvalidMetadata"  # TooManyMetadataEntries
    assert status_of(b"") == "TruncatedFile"
    huge = img[:8] + struct.pack("<Q", 1 << 40) + img[16:]
    assert status_of(huge) == "InvalidMetadata"  # TooManyTensors


def test_bad_alignment_is_invalid_metadata():
    img, _ = synth.moe_gguf(TINY, 1, extra_metadata={"general.alignment": 3})
    assert status_of(img) == "InvalidMetadata"


def test_missing_pieces():
    img, _ = synth.moe_gguf(TINY, 2, drop=("blk.1.ffn_up_exps.weight",))
    assert status_of(img, 0) == "OK" and status_of(img, 1) == "MissingTensor"
    img, _ = synth.moe_gguf(TINY, 1, drop=("qwen3moe.embedding_length",))
    assert status_of(img) == "MissingTensor"
    img, _ = synth.moe_gguf(TINY, 1, drop=("qwen3moe.expert_count",))
    assert status_of(img) == "InvalidMetadata"
    img, _ = synth.moe_gguf(SHARED, 1, drop=("blk.0.ffn_gate_inp_shexp.weight",))
    assert status_of(img) == "MissingTensor"
    img, _ = synth.moe_gguf(TINY, 2)
    assert status_of(img, 2) == "InvalidArgument"  # past block_count


def test_wrong_shapes_are_dimension_mismatch():
    spec = dataclasses.replace(TINY, inter=512)
    img, _ = synth.moe_gguf(spec, 1)
    g = G.Gguf.from_bytes(img)
    meta = dict(g.kv)
    tensors = [(t.name, t.dims, t.ttype, bytes(g.tensor_bytes(t))) for t in g.order]
    # down stored as {H, I, E} instead of {I, H, E}: same bytes, axes swapped
    bad = [(n, (256, 512, 4) if n.endswith("ffn_down_exps.weight") else d, tt, b) for n, d, tt, b in tensors]
    assert status_of(G.write(meta, bad)) == "DimensionMismatch"
    # a router with 3 rows for 4 experts
    router = lambda n: n.endswith("ffn_gate_inp.weight")  # noqa: E731
    bad = [(n, (256, 3) if router(n) else d, tt, b[:256 * 3 * 4] if router(n) else b) for n, d, tt, b in tensors]
    assert status_of(G.write(meta, bad)) == "DimensionMismatch"


def test_router_in_either_orientation_passes_the_shape_check():
    img, _ = synth.moe_gguf(TINY, 1, router_transposed=True, router_type=W.F16)
    c = moe.gguf_moe_config(img)
    assert c["router_type"] == W.F16


def test_gemma_architecture_sets_use_gelu():
    """load_gguf.zig:145-158: every gemma* architecture runs geluTanh(gate) * up;
    the others keep SiLU (load_gguf.zig:1093, 1132)."""
    for arch, want in (("gemma2", 1), ("gemma3", 1), ("qwen3moe", 0), ("mixtral", 0), ("deepseek2", 0)):
        img, _ = synth.moe_gguf(TINY, 1, arch=arch)
        assert moe.gguf_moe_config(img)["use_gelu"] == want, arch


def test_shared_expert_as_stored_keeps_its_payloads():
    img, _ = synth.moe_gguf(SHARED, 1)
    c = moe.gguf_moe_config(img)
    assert c["shared_type"] == W.Q8_0 and c["shared_as_f16"] == 0


def test_transposed_shared_expert_is_read_as_f16():
    """loadLinear (load_gguf.zig:374-384) takes a shared-expert tensor stored
    {out, in} too and transposes it; the loader then holds the shared expert as
    f16 [out][in], as the reference does."""
    img, _ = synth.moe_gguf(SHARED, 1, shared_transposed=True)
    c = moe.gguf_moe_config(img)
    assert c["shared_inter"] == 512 and c["shared_type"] == W.F16 and c["shared_as_f16"] == 1


def test_shared_expert_of_mixed_types_is_read_as_f16():
    img, _ = synth.moe_gguf(SHARED, 1)
    g = G.Gguf.from_bytes(img)
    tensors = []
    for t in g.order:
        b = bytes(g.tensor_bytes(t))
        if t.name.endswith("ffn_up_shexp.weight"):  # up as F16 of the same values
            tensors.append((t.name, t.dims, W.F16, synth.dequantize_host(W.Q8_0, np.frombuffer(b, np.uint8))
                            .astype(np.float16).tobytes()))
        else:
            tensors.append((t.name, t.dims, t.ttype, b))
    c = moe.gguf_moe_config(G.write(dict(g.kv), tensors))
    assert c["shared_as_f16"] == 1


def test_shared_expert_of_wrong_size_is_dimension_mismatch():
    img, _ = synth.moe_gguf(SHARED, 1)
    g = G.Gguf.from_bytes(img)
    tensors = [(t.name, (256, 256) if t.name.endswith("ffn_gate_shexp.weight") else t.dims, t.ttype,
                bytes(g.tensor_bytes(t))[:256 * 256 // 32 * 34] if t.name.endswith("ffn_gate_shexp.weight")
                else bytes(g.tensor_bytes(t))) for t in g.order]
    assert status_of(G.write(dict(g.kv), tensors)) == "DimensionMismatch"
