"""Write the small golden fixtures in this directory from the oracle.

    python tests/golden/make_fixtures.py

The reference's own tests hold no fixtures for this path, and its Python
implementation lives in closures that need the full checkpoint, so these
vectors come from the oracle restatement (itself pinned by
tests/test_oracle.py).  They freeze the oracle's outputs on tiny seeded inputs
so that GPU tests and later oracle edits are checked against fixed data.
Format: safetensors (no code executes on load).
"""
import os
import sys

import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "aima-amd395-qwen36-35b-linux-engine_amd"))

from oracle import attention_oracle as O  # noqa: E402
from qwen36_attn import synthetic as syn  # noqa: E402

OUT = os.path.join(HERE, "fixtures.safetensors")


def build() -> dict:
    f = {}
    g = syn.gen(2024)
    # prefill: 5 new tokens over a 4-token prefix (bottom-right mask)
    q = syn.randn((5, 16, 256), g)
    k = syn.randn((9, 2, 256), g)
    v = syn.randn((9, 2, 256), g)
    f.update({"prefill.q": q, "prefill.k": k, "prefill.v": v,
              "prefill.out_f32": O.prefill_attention(q, k, v, 4, out_dtype=torch.float32),
              "prefill.out_bf16": O.prefill_attention(q, k, v, 4)})
    # decode over 33 cached rows
    qd = syn.randn((1, 16, 256), g)
    kc = syn.randn((33, 2, 256), g)
    vc = syn.randn((33, 2, 256), g)
    f.update({"decode.q": qd, "decode.k": kc, "decode.v": vc,
              "decode.out_bf16": O.decode_attention_grouped_bf16(qd, kc, vc, 33)})
    # head norm + rope at positions 7..9
    qg = syn.randn((3, 8192), g)
    kr = syn.randn((3, 512), g)
    qw = syn.randn((256,), g, 0.5)
    kw = syn.randn((256,), g, 0.5)
    cos, sin = O.rope_cos_sin(7, 3)
    qh, _ = O.split_q_gate(qg)
    f.update({"norm_rope.q_gate": qg, "norm_rope.k": kr, "norm_rope.q_w": qw, "norm_rope.k_w": kw,
              "norm_rope.q_out": O.apply_rope(O.head_rmsnorm(qh, qw), cos, sin),
              "norm_rope.k_out": O.apply_rope(O.head_rmsnorm(kr.view(3, 2, 256), kw), cos, sin)})
    # conv1d with a carried state
    x = syn.randn((6, 8192), g)
    w = syn.randn((8192, 4), g, 0.5)
    st = syn.randn((8192, 3), g)
    co, cs = O.causal_conv1d(x, st, w)
    f.update({"conv.x": x, "conv.w": w, "conv.state": st, "conv.out": co, "conv.new_state": cs})
    # delta rule: 20 tokens, zero state; states kept for v-heads 0 and 31
    qq, kk, vv, gg, beta = syn.gdn_core_inputs(20, g, a_max=1.0)
    R = O.repeat_kv_heads
    args = (R(qq).unsqueeze(0), R(kk).unsqueeze(0), vv.unsqueeze(0), gg.unsqueeze(0),
            beta.unsqueeze(0), torch.zeros(1, 32, 128, 128))
    co_, cs_ = O.chunk_gated_delta_rule(*args)
    ro_, rs_ = O.recurrent_gated_delta_rule(*args)
    f.update({"gdn.q": qq, "gdn.k": kk, "gdn.v": vv, "gdn.g": gg, "gdn.beta": beta,
              "gdn.chunk_out": co_[0], "gdn.chunk_state_h0_h31": cs_[0, [0, 31]].contiguous(),
              "gdn.recurrent_out": ro_[0],
              "gdn.recurrent_state_h0_h31": rs_[0, [0, 31]].contiguous()})
    return {k_: v_.contiguous() for k_, v_ in f.items()}


if __name__ == "__main__":
    save_file(build(), OUT)
    print(OUT, os.path.getsize(OUT))
