"""MoE layer shapes and synthetic-data recipes for the workloads this library is
measured and checked on.

Each `LayerSpec` is one MoE FFN layer in the storage contract of ANEDVD's
`MoeWeights` (model.zig:414-470): router `[E][H]` f16, gate/up `[E][I][H]`,
down `[E][H][I]`, expert axis slowest, blocks along the input dimension
(gguf.zig:474-488), optional shared expert and shared-expert gate.
"""
from __future__ import annotations

from dataclasses import dataclass, field

# ggml type ids (gguf.zig:30-46)
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1 = 0, 1, 2, 3, 6, 7, 8, 9
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K, BF16 = 10, 11, 12, 13, 14, 15, 30

TYPE_NAMES = {F32: "f32", F16: "f16", Q4_0: "q4_0", Q4_1: "q4_1", Q5_0: "q5_0", Q5_1: "q5_1",
              Q8_0: "q8_0", Q8_1: "q8_1", Q2_K: "q2_k", Q3_K: "q3_k", Q4_K: "q4_k",
              Q5_K: "q5_k", Q6_K: "q6_k", Q8_K: "q8_k", BF16: "bf16"}

# GgmlType.blockElems / blockBytes (gguf.zig:49-77)
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22),
         Q5_1: (32, 24), Q8_0: (32, 34), Q8_1: (32, 36), Q2_K: (256, 84), Q3_K: (256, 110),
         Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), Q8_K: (256, 292)}


def bytes_per_weight(t: int) -> float:
    e, b = BLOCK[t]
    return b / e


@dataclass(frozen=True)
class LayerSpec:
    name: str
    hidden: int
    inter: int
    n_experts: int
    k: int
    norm_topk_prob: bool
    gate_type: int
    up_type: int
    down_type: int
    # scale of the |N(0, sigma)| block scales (Q8_0 divides it by 127)
    scale_sigma: float = 0.02
    router_sigma: float = 0.02
    shared_inter: int = 0
    shared_type: int = Q8_0
    shared_gated: bool = False
    rms_normalise_input: bool = False
    use_gelu: bool = False  # geluTanh(gate) * up (cpu.zig:78-81, 434-437) instead of SiLU
    layers: int = 1
    tokens: tuple = field(default_factory=tuple)

    def expert_bytes(self) -> float:
        H, I = self.hidden, self.inter
        return (I * H * (bytes_per_weight(self.gate_type) + bytes_per_weight(self.up_type))
                + H * I * bytes_per_weight(self.down_type))

    def shared_bytes(self) -> float:
        if not self.shared_inter:
            return 0.0
        return 3 * self.hidden * self.shared_inter * bytes_per_weight(self.shared_type)

    def call_bytes(self, touched: int, n_tokens: int, with_router: bool = True) -> float:
        """Algorithmic HBM bytes of one layer call: every touched expert's weights
        once, the router, the shared expert, activations in and out."""
        b = touched * self.expert_bytes() + self.shared_bytes() + n_tokens * self.hidden * 4 * 2
        if with_router:
            b += self.n_experts * self.hidden * 2
        return b

    def call_flops(self, n_tokens: int, with_router: bool = True) -> float:
        f = n_tokens * self.k * 6 * self.hidden * self.inter + 6 * n_tokens * self.hidden * self.shared_inter
        if with_router:
            f += 2 * n_tokens * self.n_experts * self.hidden
        return f


# Tiny random-init layer used for parity: H=512, 8 experts of 512->1024->512, top-2, renorm.
TINY_Q8_0 = LayerSpec("tiny-moe h512 e8 i1024 top2 q8_0", 512, 1024, 8, 2, True, Q8_0, Q8_0, Q8_0,
                      rms_normalise_input=True, tokens=(1, 16))

# Qwen3-30B-A3B-shaped layer: H=2048, 128 experts of 2048->768->2048, top-8, renorm, Q8_0.
QWEN3_30B_A3B_Q8_0 = LayerSpec("qwen3-30b-a3b moe layer h2048 e128 i768 top8 q8_0", 2048, 768, 128, 8, True,
                               Q8_0, Q8_0, Q8_0, layers=48, tokens=(1, 8, 32, 64))

# Same shape in Q4_K_M layout (gate/up Q4_K, down Q6_K), 512-token prefill, Zipf-skewed routing.
QWEN3_30B_A3B_Q4_K_M = LayerSpec("qwen3-30b-a3b moe layer h2048 e128 i768 top8 q4_k/q6_k", 2048, 768, 128, 8, True,
                                 Q4_K, Q4_K, Q6_K, scale_sigma=0.01, layers=48, tokens=(512,))

# Mixtral-8x7B-shaped layer: H=4096, 8 experts of 4096->14336->4096, top-2, Q4_0.
MIXTRAL_8X7B_Q4_0 = LayerSpec("mixtral-8x7b moe layer h4096 e8 i14336 top2 q4_0", 4096, 14336, 8, 2, True,
                              Q4_0, Q4_0, Q4_0, scale_sigma=0.01, layers=32, tokens=(1, 2048))

# DeepSeek-V2-Lite-shaped layer: H=2048, 64 experts of 2048->1408->2048, top-6 without renorm,
# plus two ungated shared experts of the same shape (= one shared SwiGLU of width 2816).
DEEPSEEK_V2_LITE_Q8_0 = LayerSpec("deepseek-v2-lite moe layer h2048 e64 i1408 top6 + shared 2816 q8_0", 2048, 1408,
                                  64, 6, False, Q8_0, Q8_0, Q8_0, shared_inter=2816, shared_type=Q8_0,
                                  layers=26, tokens=(32, 1024))

ALL = [TINY_Q8_0, QWEN3_30B_A3B_Q8_0, QWEN3_30B_A3B_Q4_K_M, MIXTRAL_8X7B_Q4_0, DEEPSEEK_V2_LITE_Q8_0]
