"""Seeded synthetic inputs for the BASELINE configurations.

Tensors are drawn on the CPU from ``torch.Generator`` so that the oracle (CPU)
and the HIP kernels (copied to the GPU) see identical values.
"""
from __future__ import annotations

import math

import torch

BF16 = torch.bfloat16


def gen(seed: int) -> torch.Generator:
    return torch.Generator(device="cpu").manual_seed(seed)


def randn(shape, g, scale: float = 1.0, dtype=BF16) -> torch.Tensor:
    x = torch.randn(*shape, generator=g)
    if scale != 1.0:
        x = x * scale
    return x.to(dtype)


def full_attention_weights(g: torch.Generator, std: float = 0.02) -> dict:
    """Config 1 weights of one gated GQA layer, N(0, 0.02) bf16."""
    return {
        "q_proj": randn((8192, 2048), g, std),
        "k_proj": randn((512, 2048), g, std),
        "v_proj": randn((512, 2048), g, std),
        "o_proj": randn((2048, 4096), g, std),
        "q_norm": randn((256,), g, std),
        "k_norm": randn((256,), g, std),
    }


def linear_attention_weights(g: torch.Generator, std: float = 0.02,
                             a_max: float = 16.0) -> dict:
    """One Gated-DeltaNet layer.  A ~ U(0, a_max), A_log = log A (the
    Qwen3-Next initialisation); conv taps N(0, 0.5) so the conv output keeps a
    useful scale."""
    a = torch.rand(32, generator=g) * a_max
    return {
        "in_proj_qkv": randn((8192, 2048), g, std),
        "in_proj_z": randn((4096, 2048), g, std),
        "in_proj_a": randn((32, 2048), g, std),
        "in_proj_b": randn((32, 2048), g, std),
        "conv1d": randn((8192, 4), g, 0.5),
        "A_log": torch.log(a.clamp_min(1e-4)).float(),
        "dt_bias": torch.zeros(32),
        "norm": randn((128,), g, std),
        "out_proj": randn((2048, 4096), g, std),
    }


def gdn_core_inputs(t: int, g: torch.Generator, a_max: float = 16.0, qk_heads: int = 16):
    """Config 4 delta-rule inputs: q, k [T, qk_heads, 128], v [T, 32, 128]
    bf16 N(0,1); beta = sigmoid(N(0,1)); g = -softplus(N(0,1)) * A with
    A ~ U(0, a_max) per head (fp32)."""
    q = randn((t, qk_heads, 128), g)
    k = randn((t, qk_heads, 128), g)
    v = randn((t, 32, 128), g)
    beta = torch.sigmoid(torch.randn(t, 32, generator=g))
    a = torch.rand(32, generator=g) * a_max
    gg = -torch.nn.functional.softplus(torch.randn(t, 32, generator=g)) * a
    return q, k, v, gg.float(), beta.float()


def causal_pairs(q_tokens: int, kv_tokens: int) -> int:
    """Unmasked (q, k) pairs of a bottom-right causal mask, diagonal included."""
    off = kv_tokens - q_tokens
    return q_tokens * off + q_tokens * (q_tokens + 1) // 2


def rope_inv_freq_reference() -> list[float]:
    return [1.0 / math.pow(1.0e7, 2.0 * i / 64.0) for i in range(32)]


def moe_weights(g: torch.Generator, n_experts: int = 256, std: float = 0.02,
                router_std: float = 0.05) -> dict:
    """One MoE block (Qwen3.6-35B-A3B geometry: hidden 2048, expert and
    shared intermediate 512, top-8), N(0, std) bf16; the post-attention norm
    weight is N(0, 0.1) (it enters as w + 1)."""
    return {
        "post_attention_layernorm": randn((2048,), g, 0.1),
        "router": randn((n_experts, 2048), g, router_std),
        "expert_gate_up": randn((n_experts, 1024, 2048), g, std),
        "expert_down": randn((n_experts, 2048, 512), g, std),
        "shared_gate": randn((1, 2048), g, std),
        "shared_gate_proj": randn((512, 2048), g, std),
        "shared_up_proj": randn((512, 2048), g, std),
        "shared_down_proj": randn((2048, 512), g, std),
    }
