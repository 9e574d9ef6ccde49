"""The no-allocation forward (anedvd_moe_layer_forward_device_noalloc) computes
what anedvd_moe_layer_forward_device computes, bit for bit, through the C ABI:
two calls in a row on each layer, the second smaller than the first (the static
scratch keeps the first call's contents), on the decode kernels, the grouped
GEMM (with Zipf routing also its groups of a few tokens, run in the grouped
launches) and a separately run shared expert (the context's second stream); and a
call whose scratch exceeds the array is refused; the no-allocation call also runs
first on a fresh context, before its workspace ever grows."""
import dataclasses
import re

import numpy as np
import pytest

from anedvd_amd import moe, synth
from anedvd_amd import workloads as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = moe.MoeContext(0)
    yield c
    c.close()


def run(ctx, layer, spec, T, seed, noalloc, routing="uniform"):
    h = synth.activations(spec, T, seed=seed)
    lg = (synth.zipf_logits if routing == "zipf" else synth.uniform_logits)(spec, T, seed=seed)
    d_h, d_lg, d_out = ctx.to_device(h), ctx.to_device(lg), ctx.alloc(T * spec.hidden * 4)
    (layer.forward_device_noalloc if noalloc else layer.forward_device)(d_h, T, d_lg, d_out)
    out = ctx.from_device(d_out, (T, spec.hidden), np.float32)
    for p in (d_h, d_lg, d_out):
        ctx.free(p)
    return out


SPECS = [
    (W.QWEN3_30B_A3B_Q8_0, (64, 8), "uniform"),
    (W.QWEN3_30B_A3B_Q4_K_M, (512, 64), "uniform"),
    (W.QWEN3_30B_A3B_Q4_K_M, (512, 300), "zipf"),
    (dataclasses.replace(W.DEEPSEEK_V2_LITE_Q8_0, name="separate-shared", hidden=512, inter=512, n_experts=8, k=2,
                         shared_inter=1024, shared_type=W.Q4_0, shared_gated=True), (300, 16), "uniform"),
]


@pytest.mark.parametrize("spec,sizes,routing", SPECS,
                         ids=lambda x: x.name.split()[0] if hasattr(x, "name") else str(x))
def test_noalloc_forward_matches_forward_device(ctx, spec, sizes, routing):
    layer = moe.MoeLayer(ctx, spec, synth.make_layer(spec, seed=3))
    if routing == "zipf":  # the case exists: skewed routing leaves groups of at most 16 tokens
        h = synth.activations(spec, sizes[0], seed=30)
        _, st = layer.forward(h, synth.zipf_logits(spec, sizes[0], seed=30), stats=True)
        assert st["path"] == 1 and st["small_groups"] > 0, st
    for i, T in enumerate(sizes):
        want = run(ctx, layer, spec, T, 30 + i, noalloc=False, routing=routing)
        got = run(ctx, layer, spec, T, 30 + i, noalloc=True, routing=routing)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (spec.name, T, routing)
    layer.free()


def test_noalloc_first_on_a_fresh_context():
    """The no-allocation call made first on a context whose workspace was never grown
    (a call that fell back to the context's workspace would find none), then the
    allocating call on the same inputs: the same bits."""
    spec = W.QWEN3_30B_A3B_Q8_0
    c = moe.MoeContext(0)
    layer = moe.MoeLayer(c, spec, synth.make_layer(spec, seed=4))
    T = 32
    h = synth.activations(spec, T, seed=4)
    d_h, d_out = c.to_device(h), c.alloc(T * spec.hidden * 4)
    layer.forward_device_noalloc(d_h, T, None, d_out)  # router GEMV in the call as well
    got = c.from_device(d_out, (T, spec.hidden), np.float32)
    layer.forward_device(d_h, T, None, d_out)
    want = c.from_device(d_out, (T, spec.hidden), np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for p in (d_h, d_out):
        c.free(p)
    layer.free()
    c.close()


def test_noalloc_refuses_calls_beyond_its_scratch(ctx):
    spec = W.QWEN3_30B_A3B_Q8_0
    layer = moe.MoeLayer(ctx, spec, synth.make_layer(spec, seed=3))
    T = 4096
    d_h = ctx.alloc(T * spec.hidden * 4)
    with pytest.raises(moe.MoeError) as ei:
        layer.forward_device_noalloc(d_h, T, None, d_h)
    assert ei.value.name == "InvalidArgument"
    most = int(re.search(r"at most (\d+) tokens", str(ei.value)).group(1))
    print(f"\nno-allocation forward: at most {most} tokens per call at the Qwen3-30B-A3B shape")
    assert 64 <= most < T
    ctx.free(d_h)
    layer.free()
