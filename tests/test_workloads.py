"""The synthetic workloads have the shapes and statistics the benchmark configs name."""
import numpy as np
import pytest

from anedvd_amd import synth
from anedvd_amd import workloads as W


@pytest.mark.parametrize("seed", [0, 1])
def test_zipf_prefill_groups_reach_about_300_tokens(seed):
    """Q4_K_M prefill: 512 tokens, top-8 of 128 experts, Zipf(1.1) router bias; the
    busiest expert gets ~300 tokens and the group sizes spread from a few upward."""
    spec = W.QWEN3_30B_A3B_Q4_K_M
    lg = synth.zipf_logits(spec, 512, seed=seed)
    top = np.argsort(-lg, axis=1, kind="stable")[:, :spec.k]
    counts = np.bincount(top.ravel(), minlength=spec.n_experts)
    assert counts.sum() == 512 * spec.k
    assert 250 <= counts.max() <= 350
    assert counts.min() <= 10


def test_shapes_match_the_configs():
    q = W.QWEN3_30B_A3B_Q8_0
    assert (q.hidden, q.inter, q.n_experts, q.k, q.norm_topk_prob) == (2048, 768, 128, 8, True)
    m = W.MIXTRAL_8X7B_Q4_0
    assert (m.hidden, m.inter, m.n_experts, m.k) == (4096, 14336, 8, 2)
    d = W.DEEPSEEK_V2_LITE_Q8_0
    assert (d.hidden, d.inter, d.n_experts, d.k, d.shared_inter, d.norm_topk_prob) == (2048, 1408, 64, 6, 2816, False)
    t = W.TINY_Q8_0
    assert (t.hidden, t.inter, t.n_experts, t.k) == (512, 1024, 8, 2)
