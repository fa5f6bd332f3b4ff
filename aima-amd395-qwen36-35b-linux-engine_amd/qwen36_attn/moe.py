"""Host-side mirror of the MoE block that follows attention in every layer
(four_layer_mini_engine.py:8479-8650: residual add, post-attention RMSNorm,
router top-8 :7775-7789, routed experts :7791-7803, shared expert
:8240-8300), with the one-token decode in ``libqwen36_attn.so``
(``qwen36_moe_decode``, three launches).

``weights``: post_attention_layernorm [2048], router [E, 2048],
expert_gate_up [E, 1024, 2048] (gate rows then up rows), expert_down
[E, 2048, 512], shared_gate [1, 2048], shared_gate_proj [512, 2048],
shared_up_proj [512, 2048], shared_down_proj [2048, 512]; all bf16."""
from __future__ import annotations

import torch

from . import _lib
from ._tensors import ptr, require, scratch, stream_handle

HIDDEN, INTER, TOP_K = 2048, 512, 8
WS_IDS, WS_RW, WS_LOGITS = 8192, 8224, 17472   # byte offsets in the workspace


class MoEBlock:
    def __init__(self, weights: dict) -> None:
        self.w = weights
        self.n_experts = weights["router"].shape[0]
        if not (TOP_K <= self.n_experts <= 256):
            raise ValueError("8 <= num_experts <= 256")
        for name in ("expert_gate_up", "expert_down", "shared_down_proj",
                     "post_attention_layernorm"):
            require(weights[name], name, torch.bfloat16)
        # fused decode input rows: router | shared_gate | shared gate_proj | shared up_proj
        self.w_in = torch.cat([weights["router"], weights["shared_gate"],
                               weights["shared_gate_proj"], weights["shared_up_proj"]],
                              dim=0).contiguous()

    def decode(self, inp: torch.Tensor, attn_out: torch.Tensor,
               out: torch.Tensor | None = None, debug: bool = False):
        """One token: returns after + MoE(rmsnorm(after)) [1, 2048] bf16 with
        after = inp + attn_out.  ``debug`` also returns (expert ids [8],
        routing weights [8] fp32, router logits [E] bf16) read back from the
        workspace."""
        for name, x in (("inp", inp), ("attn_out", attn_out)):
            require(x, name, torch.bfloat16)
            if x.numel() != HIDDEN:
                raise ValueError(f"{name} must hold 2048 values")
        dev = inp.device
        if out is None:
            out = torch.empty(1, HIDDEN, dtype=torch.bfloat16, device=dev)
        lib = _lib.load(("qwen36_moe_decode",))
        nb = lib.qwen36_moe_decode_workspace_bytes()
        ws = scratch("moe_decode", nb, dev)
        w = self.w
        _lib.call("qwen36_moe_decode", ptr(inp), ptr(attn_out), ptr(w["post_attention_layernorm"]),
                  ptr(self.w_in), ptr(w["expert_gate_up"]), ptr(w["expert_down"]),
                  ptr(w["shared_down_proj"]), self.n_experts, ptr(out), ptr(ws), ws.numel(),
                  stream_handle(dev))
        if not debug:
            return out
        ids = ws[WS_IDS:WS_IDS + 4 * TOP_K].view(torch.int32).clone()
        rw = ws[WS_RW:WS_RW + 4 * TOP_K].view(torch.float32).clone()
        logits = ws[WS_LOGITS:WS_LOGITS + 2 * self.n_experts].view(torch.bfloat16).clone()
        return out, ids, rw, logits

    def prefill(self, inp: torch.Tensor, attn_out: torch.Tensor,
                out: torch.Tensor | None = None, debug: bool = False):
        """T tokens (``qwen36_moe_prefill``): returns after + MoE(rmsnorm(after))
        [T, 2048] bf16 with after = inp + attn_out.  ``debug`` also returns
        (expert ids [T, 8] int32, routing weights [T, 8] fp32, router logits
        [T, E] bf16, shared-gate logits [T] bf16) read back from the
        workspace."""
        for name, x in (("inp", inp), ("attn_out", attn_out)):
            require(x, name, torch.bfloat16)
            if x.dim() != 2 or x.shape[1] != HIDDEN:
                raise ValueError(f"{name} must be [T, 2048]")
        t = inp.shape[0]
        if attn_out.shape[0] != t or t == 0:
            raise ValueError("inp and attn_out must hold the same T >= 1 rows")
        dev = inp.device
        if out is None:
            out = torch.empty(t, HIDDEN, dtype=torch.bfloat16, device=dev)
        lib = _lib.load(("qwen36_moe_prefill", "qwen36_moe_prefill_workspace_bytes"))
        nb = lib.qwen36_moe_prefill_workspace_bytes(t, self.n_experts)
        if nb == 0:
            raise ValueError("unsupported token count or expert count")
        ws = scratch("moe_prefill", nb, dev)
        w = self.w
        _lib.call("qwen36_moe_prefill", ptr(inp), ptr(attn_out), ptr(w["post_attention_layernorm"]),
                  ptr(self.w_in), ptr(w["expert_gate_up"]), ptr(w["expert_down"]),
                  ptr(w["shared_down_proj"]), self.n_experts, t, ptr(out), ptr(ws), ws.numel(),
                  stream_handle(dev))
        if not debug:
            return out

        def region(offset, nbytes):
            return ws[offset:offset + nbytes], (offset + nbytes + 255) // 256 * 256

        ld = (self.n_experts + 8) & ~7
        ids, o = region(0, 4 * TOP_K * t)
        rw, o = region(o, 4 * TOP_K * t)
        logits, _ = region(o, 2 * ld * t)
        ids = ids.view(torch.int32).view(t, TOP_K).clone()
        rw = rw.view(torch.float32).view(t, TOP_K).clone()
        logits = logits.view(torch.bfloat16).view(t, ld)
        return out, ids, rw, logits[:, :self.n_experts].clone(), logits[:, self.n_experts].clone()
