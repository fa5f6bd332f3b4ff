#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path (one GPU).

Headline (BASELINE.json metric "decode attn us/tok + HBM GB/s @128K ctx;
prefill attn TFLOP/s @8K tokens"):
  * one *step* = one decode token through the 10 gated GQA full-attention
    layers at KV length 131072 (config 5), each layer with its own resident
    bf16 KV cache (10 distinct caches, 2.7 GB, so the 256 MB Infinity Cache
    cannot serve the stream); the step includes the new-row KV write.
  * ``value`` = microseconds per token for that step (lower is better).
Also reported (``extra``): decode at 32768 (config 2) and 262143, prefill FMHA
TFLOP/s for 8192 causal tokens and for 8192 new tokens over a 4096-token
prefix (config 3), Gated-DeltaNet recurrent step and chunked prefill.

Inputs are synthetic bf16 N(0,1), seeded, already resident in HBM when the
timed region starts.  The CPU baseline is the oracle restatement timed on a
bounded sample on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "aima-amd395-qwen36-35b-linux-engine_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
DECODE_BYTES_PER_TOKEN = 2048          # K + V bytes per cached token per layer
PREFILL_FLOP_PER_PAIR = 16384          # 4 * Hq * D
N_FULL_LAYERS = 10


def _parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-graph", action="store_true", help="time eager launches")
    p.add_argument("--only", choices=["decode", "prefill", "prefill_8k", "prefill_c3", "gdn", "moe",
                                      "moe_1k", "moe_decode", "gemm", "copy", "launch"], default=None,
                   help="run one leg only (for counter collection); prints no JSON line")
    return p.parse_args()


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_gqa_128k_traffic.md")


def measured_traffic():
    """HBM bytes per decode launch at S=131072, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (line 'traffic_bytes_per_launch: N')."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def _cpu_info():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return model


class Timer:
    """HIP-event timing on the stream the kernels are launched on."""

    def __init__(self, torch):
        self.torch = torch

    def time(self, fn, iters, warmup=2, warm_seconds=0.2):
        """Mean ms per call over `iters` calls, after `warmup` calls and at
        least `warm_seconds` of back-to-back calls: an idle MI355X runs at a
        low clock for the first few milliseconds of work, which would
        otherwise be charged to the timed region."""
        torch = self.torch
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        t_end = time.perf_counter() + warm_seconds
        while time.perf_counter() < t_end:
            for _ in range(4):
                fn()
            torch.cuda.synchronize()
        s = torch.cuda.current_stream()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(iters):
            fn()
        e1.record(s)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / iters  # ms


def make_graph(torch, fn):
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm allocations outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def decode_setup(torch, fa, dev, cache_end, layers, seed):
    gen = torch.Generator(device="cpu").manual_seed(seed)
    caches = []
    for _ in range(layers):
        k = torch.empty(cache_end, 2, 256, dtype=torch.bfloat16, device=dev)
        v = torch.empty_like(k)
        # fill on device in slices from a seeded CPU stream (keeps host RAM low)
        step = 16384
        for s0 in range(0, cache_end, step):
            n = min(step, cache_end - s0)
            k[s0:s0 + n].copy_(torch.randn(n, 2, 256, generator=gen).to(torch.bfloat16))
            v[s0:s0 + n].copy_(torch.randn(n, 2, 256, generator=gen).to(torch.bfloat16))
        caches.append((k, v))
    q = [torch.randn(16, 256, generator=gen).to(torch.bfloat16).to(dev) for _ in range(layers)]
    kn = [torch.randn(2, 256, generator=gen).to(torch.bfloat16).to(dev) for _ in range(layers)]
    vn = [torch.randn(2, 256, generator=gen).to(torch.bfloat16).to(dev) for _ in range(layers)]
    outs = [torch.empty(1, 4096, dtype=torch.bfloat16, device=dev) for _ in range(layers)]
    # per-layer workspaces so a captured graph holds fixed pointers
    ws = []
    lib = fa._lib.load()
    for _ in range(layers):
        nb = lib.qwen36_decode_gqa_workspace_bytes(cache_end, 0)
        ws.append(torch.zeros(nb, dtype=torch.uint8, device=dev))

    def step():
        for i in range(layers):
            k, v = caches[i]
            fa._lib.call("qwen36_decode_gqa", q[i].data_ptr(), kn[i].data_ptr(), vn[i].data_ptr(),
                         k.data_ptr(), v.data_ptr(), cache_end - 1, cache_end, cache_end,
                         None, 0, outs[i].data_ptr(), ws[i].data_ptr(), ws[i].numel(), 0,
                         torch.cuda.current_stream().cuda_stream)
    return step, caches


def bench_decode(torch, fa, dev, cache_end, layers, iters, warmup, use_graph, seed=0):
    step, caches = decode_setup(torch, fa, dev, cache_end, layers, seed)
    t = Timer(torch)
    run = step
    if use_graph:
        g = make_graph(torch, step)
        run = g.replay
    ms = t.time(run, iters, warmup)
    us_tok = ms * 1000.0
    nbytes = DECODE_BYTES_PER_TOKEN * cache_end * layers
    del caches
    return {"cache_end": cache_end, "layers": layers, "us_per_token": us_tok,
            "hbm_gbs": nbytes / (us_tok * 1e-6) / 1e9,
            "frac_hbm": nbytes / (us_tok * 1e-6) / 1e9 / HBM_PEAK_GBS}


def bench_decode_layer_step(torch, fa, dev, cache_end, layers, iters, warmup, use_graph,
                            fused=True, seed=5):
    """The full-attention part of a decode token between the projections and
    o_proj, through ``layers`` layers at KV length ``cache_end``: head norm +
    RoPE of q and the new k, the KV-row write, split-K attention and the
    output gate -- fused into the decode launches (``fused``) or as the
    separate head-norm/RoPE launch followed by the decode core."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    cap = cache_end
    layer_t = []
    for _ in range(layers):
        k = torch.empty(cap, 2, 256, dtype=torch.bfloat16, device=dev)
        v = torch.empty_like(k)
        step = 16384
        for s0 in range(0, cap, step):
            n = min(step, cap - s0)
            k[s0:s0 + n].copy_(torch.randn(n, 2, 256, generator=gen).to(torch.bfloat16))
            v[s0:s0 + n].copy_(torch.randn(n, 2, 256, generator=gen).to(torch.bfloat16))
        layer_t.append(dict(
            k=k, v=v, q_gate=torch.randn(1, 8192, generator=gen).to(torch.bfloat16).to(dev),
            kr=torch.randn(1, 512, generator=gen).to(torch.bfloat16).to(dev),
            vr=torch.randn(1, 512, generator=gen).to(torch.bfloat16).to(dev),
            qn=(torch.randn(256, generator=gen) * 0.1).to(torch.bfloat16).to(dev),
            kn=(torch.randn(256, generator=gen) * 0.1).to(torch.bfloat16).to(dev),
            out=torch.empty(1, 4096, dtype=torch.bfloat16, device=dev),
            q=torch.empty(1, 16, 256, dtype=torch.bfloat16, device=dev)))
    pos = cache_end - 1

    def step():
        for d in layer_t:
            if fused:
                fa.decode_step(d["q_gate"], d["kr"], d["vr"], d["qn"], d["kn"], d["k"], d["v"],
                               pos, cache_end, out=d["out"])
            else:
                fa.head_norm_rope_kv_write(d["q_gate"], d["kr"], d["vr"], d["qn"], d["kn"],
                                           d["k"], d["v"], pos, q_out=d["q"])
                fa.decode_gqa(d["q"], d["k"], d["v"], pos, cache_end,
                              gate=d["q_gate"].view(16, 512)[:, 256:], out=d["out"])
    run = make_graph(torch, step).replay if use_graph else step
    ms = Timer(torch).time(run, iters, warmup)
    us = ms * 1000.0
    nbytes = DECODE_BYTES_PER_TOKEN * cache_end * layers
    del layer_t
    return {"cache_end": cache_end, "layers": layers, "launches_per_layer": 2 if fused else 3,
            "us_per_token": us, "hbm_gbs": nbytes / (us * 1e-6) / 1e9,
            "frac_hbm": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}


def bench_prefix_cache(torch, dev, tokens, iters, warmup):
    """Exact-prefix cache at model scale: the state of 10 full-attention
    layers (K and V caches, capacity = ``tokens``) and 30 Gated-DeltaNet
    layers (conv + recurrent state) captured for a ``tokens``-token prompt and
    restored, each as one batched copy launch.  Bandwidth counts read + write
    of the copied bytes."""
    import ctypes
    from qwen36_attn import _lib
    lib = _lib.load(("qwen36_prefix_cache_create",))
    pool = lib.qwen36_prefix_cache_create(tokens, 4096, 1)
    bufs = []
    for _ in range(N_FULL_LAYERS):
        for _kv in range(2):
            t = torch.empty(tokens, 2, 256, dtype=torch.bfloat16, device=dev)
            bufs.append(t)
            _lib.call("qwen36_prefix_cache_add_slice", pool, t.data_ptr(), t.numel() * 2, 1024)
    for _ in range(GDN_LAYERS):
        c = torch.empty(8192, 3, dtype=torch.bfloat16, device=dev)
        s_ = torch.empty(32, 128, 128, dtype=torch.float32, device=dev)
        bufs += [c, s_]
        _lib.call("qwen36_prefix_cache_add_slice", pool, c.data_ptr(), c.numel() * 2, 0)
        _lib.call("qwen36_prefix_cache_add_slice", pool, s_.data_ptr(), s_.numel() * 4, 0)
    _lib.call("qwen36_prefix_cache_finalize", pool, None)
    hidden = torch.empty(2048, dtype=torch.bfloat16, device=dev)
    toks = (ctypes.c_uint * tokens)(*range(tokens))
    st = torch.cuda.current_stream().cuda_stream
    nbytes = ctypes.c_ulonglong(0)

    def capture():
        _lib.call("qwen36_prefix_cache_capture", pool, toks, tokens, hidden.data_ptr(), st,
                  None, ctypes.byref(nbytes))

    def restore():
        _lib.call("qwen36_prefix_cache_restore", pool, 0, st, None)
    t_cap = Timer(torch).time(capture, iters, warmup)
    t_res = Timer(torch).time(restore, iters, warmup)
    moved = nbytes.value
    lib.qwen36_prefix_cache_destroy(pool)
    del bufs
    res = {"tokens": tokens, "bytes": moved, "capture_us": t_cap * 1e3, "restore_us": t_res * 1e3,
           "restore_gbs_rw": 2 * moved / (t_res * 1e-3) / 1e9}
    res["frac_hbm"] = res["restore_gbs_rw"] / HBM_PEAK_GBS
    return res


def bench_decode_projections(torch, dev, iters, warmup, use_graph, native=True, seed=6):
    """One decode token's projection GEMVs through the 40-layer stack: 10
    full-attention layers (fused q|gate,k,v [9216,2048] + o_proj [2048,4096])
    and 30 Gated-DeltaNet layers (fused qkv|z|b|a [12352,2048] + out_proj
    [2048,4096]), distinct weights per layer (2.57 GB), with the HIP GEMV
    (``native``) or torch.matmul."""
    from qwen36_attn.projections import gemv
    gen = torch.Generator(device="cpu").manual_seed(seed)
    shapes = [(9216, 2048), (2048, 4096)] * N_FULL_LAYERS + [(12352, 2048), (2048, 4096)] * GDN_LAYERS
    ws = []
    for n, k in shapes:
        w = torch.empty(n, k, dtype=torch.bfloat16, device=dev)
        w.copy_((torch.randn(n, k, generator=gen) * 0.02).to(torch.bfloat16))
        ws.append(w)
    xs = {k: torch.randn(1, k, generator=gen).to(torch.bfloat16).to(dev) for k in (2048, 4096)}
    outs = [torch.empty(1, n, dtype=torch.bfloat16, device=dev) for n, _ in shapes]

    def step():
        for w, o in zip(ws, outs):
            x = xs[w.shape[1]]
            if native:
                gemv(w, x, out=o)
            else:
                torch.matmul(x, w.t(), out=o)
    run = make_graph(torch, step).replay if use_graph else step
    ms = Timer(torch).time(run, iters, warmup)
    us = ms * 1000.0
    nbytes = sum(n * k * 2 for n, k in shapes)
    del ws
    return {"gemvs": len(shapes), "weight_bytes": nbytes, "us_per_token": us,
            "hbm_gbs": nbytes / (us * 1e-6) / 1e9, "frac_hbm": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}


PREFILL_PROJ_SHAPES = [(9216, 2048), (2048, 4096), (12352, 2048), (2048, 4096)]


def bench_prefill_projections(torch, dev, t, iters, warmup, native=True, seed=13,
                              backend="auto"):
    """The prefill projections of one full-attention layer (fused q|gate,k,v
    [9216, 2048] and o_proj [2048, 4096]) and one Gated-DeltaNet layer
    (fused qkv|z|b|a [12352, 2048] and out_proj [2048, 4096]) for a prompt
    of t tokens: the library's ``linear`` (``native``; ``backend`` "auto" =
    its hipBLASLt entry point, "native" = its MFMA kernel) or torch.matmul."""
    from qwen36_attn.prefill_gemm import linear
    gen = torch.Generator(device=dev).manual_seed(seed)
    ws = [(torch.randn(n, k, generator=gen, device=dev) * 0.02).to(torch.bfloat16)
          for n, k in PREFILL_PROJ_SHAPES]
    xs = {k: (torch.randn(t, k, generator=gen, device=dev) * 0.5).to(torch.bfloat16)
          for k in (2048, 4096)}
    outs = [torch.empty(t, n, dtype=torch.bfloat16, device=dev) for n, _ in PREFILL_PROJ_SHAPES]

    def step():
        for w, o in zip(ws, outs):
            x = xs[w.shape[1]]
            if native:
                linear(x, w, out=o, backend=backend)
            else:
                torch.matmul(x, w.t(), out=o)
    ms = Timer(torch).time(step, iters, warmup)
    flop = sum(2 * t * n * k for n, k in PREFILL_PROJ_SHAPES)
    del ws, xs, outs
    return {"tokens": t, "gemms": len(PREFILL_PROJ_SHAPES), "ms": ms,
            "tflops": flop / (ms * 1e-3) / 1e12,
            "frac_bf16_mfma": flop / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS}


def bench_moe_decode(torch, dev, layers, iters, warmup, use_graph, seed=7):
    """One decode token through the MoE blocks of ``layers`` layers (256
    experts, top-8, intermediate 512, shared expert), distinct weights per
    layer (1.5 GB each, generated on the device).  Bytes per layer-token =
    router + shared input rows (1281 x 4 KiB) + 8 experts x 6 MiB + shared
    down (2 MiB)."""
    from qwen36_attn.moe import MoEBlock
    gen = torch.Generator(device=dev).manual_seed(seed)

    def rnd(shape, std):
        return (torch.randn(*shape, generator=gen, device=dev) * std).to(torch.bfloat16)
    blocks = []
    for _ in range(layers):
        w = {"post_attention_layernorm": rnd((2048,), 0.1), "router": rnd((256, 2048), 0.05),
             "expert_gate_up": rnd((256, 1024, 2048), 0.02), "expert_down": rnd((256, 2048, 512), 0.02),
             "shared_gate": rnd((1, 2048), 0.02), "shared_gate_proj": rnd((512, 2048), 0.02),
             "shared_up_proj": rnd((512, 2048), 0.02), "shared_down_proj": rnd((2048, 512), 0.02)}
        blocks.append(MoEBlock(w))
    xs = [rnd((1, 2048), 0.5) for _ in range(layers)]
    at = [rnd((1, 2048), 0.5) for _ in range(layers)]
    outs = [torch.empty(1, 2048, dtype=torch.bfloat16, device=dev) for _ in range(layers)]

    def step():
        for b, x, a, o in zip(blocks, xs, at, outs):
            b.decode(x, a, out=o)
    run = make_graph(torch, step).replay if use_graph else step
    ms = Timer(torch).time(run, iters, warmup)
    us = ms * 1000.0
    per_layer = (256 + 1 + 1024) * 2048 * 2 + 8 * (1024 * 2048 + 2048 * 512) * 2 + 2048 * 512 * 2
    nbytes = per_layer * layers
    del blocks
    torch.cuda.empty_cache()
    return {"layers": layers, "bytes_per_token": nbytes, "us_per_token": us,
            "hbm_gbs": nbytes / (us * 1e-6) / 1e9, "frac_hbm": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}


def moe_prefill_flops(tokens, n_experts=256):
    """Algorithmic FLOP of one MoE block over `tokens` tokens: router +
    shared-gate GEMM (E + 1 rows) and, for 8 routed rows plus the shared
    expert per token, gate/up (2 x 2048 x 1024) and down (2 x 512 x 2048)."""
    return tokens * (2 * 2048 * (n_experts + 1) + 9 * (2 * 2048 * 1024 + 2 * 512 * 2048))


def bench_moe_prefill(torch, dev, tokens, iters, warmup, native=True, seed=11):
    """One MoE block over `tokens` prefill tokens (256 experts, top-8).  The
    torch leg runs the same routed rows as a loop of per-expert hipBLASLt
    GEMMs (torch.matmul) after the native kernel's routing, which it does not
    time."""
    from qwen36_attn.moe import MoEBlock
    import torch.nn.functional as F
    gen = torch.Generator(device=dev).manual_seed(seed)

    def rnd(shape, std):
        return (torch.randn(*shape, generator=gen, device=dev) * std).to(torch.bfloat16)
    w = {"post_attention_layernorm": rnd((2048,), 0.1), "router": rnd((256, 2048), 0.05),
         "expert_gate_up": rnd((256, 1024, 2048), 0.02), "expert_down": rnd((256, 2048, 512), 0.02),
         "shared_gate": rnd((1, 2048), 0.02), "shared_gate_proj": rnd((512, 2048), 0.02),
         "shared_up_proj": rnd((512, 2048), 0.02), "shared_down_proj": rnd((2048, 512), 0.02)}
    block = MoEBlock(w)
    x = rnd((tokens, 2048), 0.5)
    a = rnd((tokens, 2048), 0.5)
    out = torch.empty(tokens, 2048, dtype=torch.bfloat16, device=dev)
    if native:
        fn = lambda: block.prefill(x, a, out=out)  # noqa: E731
    else:
        _, ids, rw, _, _ = block.prefill(x, a, debug=True)
        flat = ids.view(-1).long()
        groups = [(e, (flat == e).nonzero().squeeze(1)) for e in range(256)]
        groups = [(e, r) for e, r in groups if r.numel()]
        rwb = rw.view(-1, 1).to(torch.bfloat16)
        y = torch.empty(tokens * 8, 2048, dtype=torch.bfloat16, device=dev)

        def fn():
            after = x + a
            h2 = (after.float() * torch.rsqrt(after.float().pow(2).mean(-1, keepdim=True) + 1e-6)
                  * (w["post_attention_layernorm"].float() + 1)).to(torch.bfloat16)
            h2 @ block.w_in[:257].t()
            for e, rows in groups:
                gu = h2[rows // 8] @ w["expert_gate_up"][e].t()
                act = (F.silu(gu[:, :512].float()) * gu[:, 512:].float()).to(torch.bfloat16)
                y[rows] = act @ w["expert_down"][e].t()
            moe = (y * rwb).view(tokens, 8, 2048).sum(1)
            su = h2 @ block.w_in[257:].t()
            sact = (F.silu(su[:, :512].float()) * su[:, 512:].float()).to(torch.bfloat16)
            out.copy_(after + (moe + sact @ w["shared_down_proj"].t()))
    ms = Timer(torch).time(fn, iters, warmup)
    flops = moe_prefill_flops(tokens)
    wbytes = 256 * (1024 * 2048 + 2048 * 512) * 2
    del block, w
    torch.cuda.empty_cache()
    return {"tokens": tokens, "ms": ms, "tflops": flops / (ms * 1e-3) / 1e12,
            "frac_mfma": flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
            "expert_weight_bytes": wbytes}


def causal_pairs(t, s):
    off = s - t
    return t * off + t * (t + 1) // 2


def bench_prefill(torch, fa, dev, t, s, iters, warmup, seed=1):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(t, 16, 256, generator=gen).to(torch.bfloat16).to(dev)
    k = torch.randn(s, 2, 256, generator=gen).to(torch.bfloat16).to(dev)
    v = torch.randn(s, 2, 256, generator=gen).to(torch.bfloat16).to(dev)
    out = torch.empty(t, 4096, dtype=torch.float32, device=dev)
    ms = Timer(torch).time(lambda: fa.fmha_prefill(q, k, v, out=out), iters, warmup)
    flop = PREFILL_FLOP_PER_PAIR * causal_pairs(t, s)
    tf = flop / (ms * 1e-3) / 1e12
    return {"q_tokens": t, "kv_tokens": s, "ms": ms, "tflops": tf,
            "frac_bf16_mfma": tf / BF16_PEAK_TFLOPS}


def bench_prefill_gated(torch, fa, dev, t, s, iters, warmup, seed=1):
    """The prefill attention with the layer's sigmoid output gate: the gate
    applied in the FMHA launches (bf16 rows out) against the two-launch
    form (fp32 FMHA rows, then the gate kernel) -- the reference's provider
    FMHA + full_attention_gate_kernel pair."""
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(t, 16, 256, generator=gen).to(torch.bfloat16).to(dev)
    k = torch.randn(s, 2, 256, generator=gen).to(torch.bfloat16).to(dev)
    v = torch.randn(s, 2, 256, generator=gen).to(torch.bfloat16).to(dev)
    fused_rows = torch.randn(t, 9216, generator=gen).to(torch.bfloat16).to(dev)
    q_gate = fused_rows[:, :8192]
    out = torch.empty(t, 4096, dtype=torch.bfloat16, device=dev)
    a32 = torch.empty(t, 4096, dtype=torch.float32, device=dev)
    tm = Timer(torch)
    fused = tm.time(lambda: fa.fmha_prefill_gated(q, k, v, q_gate, out=out), iters, warmup)
    two = tm.time(lambda: fa.output_gate(fa.fmha_prefill(q, k, v, out=a32), q_gate, out=out),
                  iters, warmup)
    flop = PREFILL_FLOP_PER_PAIR * causal_pairs(t, s)
    return {"q_tokens": t, "kv_tokens": s, "fused_ms": fused, "fmha_then_gate_ms": two,
            "fused_frac_bf16_mfma": flop / (fused * 1e-3) / 1e12 / BF16_PEAK_TFLOPS}


GDN_STATE_BYTES = 2 * 32 * 128 * 128 * 4     # fp32 state read + write per layer step
GDN_LAYERS = 30


def bench_gdn_recurrent(torch, dev, layers, iters, warmup, use_graph, seed=2):
    """Config 5 GDN part: one recurrent decode step through 30 layers, each
    with its own fp32 state (state updated in place)."""
    from qwen36_attn import _lib
    from qwen36_attn import synthetic as syn
    g = syn.gen(seed)
    q, k, v, gg, beta = [x.to(dev) for x in syn.gdn_core_inputs(layers, g, a_max=16.0)]
    states = [torch.randn(32, 128, 128, generator=g).to(dev) for _ in range(layers)]
    outs = [torch.empty(1, 32, 128, dtype=torch.bfloat16, device=dev) for _ in range(layers)]

    def step():
        st = torch.cuda.current_stream().cuda_stream
        for i in range(layers):
            _lib.call("qwen36_gdn_recurrent", q[i].data_ptr(), k[i].data_ptr(), v[i].data_ptr(),
                      16, 2048, 4096, gg[i].data_ptr(), beta[i].data_ptr(), states[i].data_ptr(),
                      states[i].data_ptr(), outs[i].data_ptr(), 1, st)
    run = make_graph(torch, step).replay if use_graph else step
    ms = Timer(torch).time(run, iters, warmup)
    us = ms * 1000.0
    nbytes = GDN_STATE_BYTES * layers
    return {"layers": layers, "us_per_token": us, "hbm_gbs": nbytes / (us * 1e-6) / 1e9,
            "frac_hbm": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}


def bench_gdn_fused_gating_update(torch, dev, layers, iters, warmup, use_graph, seed=5):
    """vLLM-orientation decode update (gating fused, [Hv, dv, dk] state,
    qwen36_gdn_fused_gating_update) for one token through 30 layers with their
    own states updated in place -- the same state traffic as
    bench_gdn_recurrent, in the orientation the reference's decode keeps."""
    from qwen36_attn import _lib
    from qwen36_attn import synthetic as syn
    g = syn.gen(seed)
    mixed = [syn.randn((1, 8192), g).to(dev) for _ in range(layers)]
    ab = [syn.randn((1, 64), g).to(dev) for _ in range(layers)]
    a_log = torch.log(torch.rand(32, generator=g) * 16 + 1e-4).float().to(dev)
    dtb = torch.randn(32, generator=g).float().to(dev)
    states = [(torch.randn(32, 128, 128, generator=g) * 0.2).to(dev) for _ in range(layers)]
    outs = [torch.empty(1, 32, 128, dtype=torch.bfloat16, device=dev) for _ in range(layers)]

    def step():
        st = torch.cuda.current_stream().cuda_stream
        for i in range(layers):
            base = mixed[i].data_ptr()
            _lib.call("qwen36_gdn_fused_gating_update", a_log.data_ptr(), ab[i].data_ptr(),
                      ab[i].data_ptr() + 64, 64, dtb.data_ptr(), base, base + 4096, 16, 8192,
                      base + 8192, 8192, states[i].data_ptr(), states[i].data_ptr(),
                      outs[i].data_ptr(), 1, 128 ** -0.5, 1, st)
    run = make_graph(torch, step).replay if use_graph else step
    ms = Timer(torch).time(run, iters, warmup)
    us = ms * 1000.0
    nbytes = GDN_STATE_BYTES * layers
    return {"layers": layers, "us_per_token": us, "hbm_gbs": nbytes / (us * 1e-6) / 1e9,
            "frac_hbm": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}


def bench_gdn_decode_step(torch, dev, layers, iters, warmup, use_graph, fused=True, seed=4):
    """Everything between a GDN layer's input projections and out_proj for
    one decode token (conv, gating, l2norm, recurrent delta rule, gated
    RMSNorm), through 30 layers with their own states: one fused launch per
    layer (``fused``) or the four-launch sequence conv / gating / recurrent /
    gated norm."""
    from qwen36_attn import gated_deltanet as G
    from qwen36_attn import synthetic as syn
    g = syn.gen(seed)
    L = []
    for _ in range(layers):
        L.append(dict(
            mixed=syn.randn((1, 8192), g).to(dev), conv_w=syn.randn((8192, 4), g, 0.5).to(dev),
            conv_a=syn.randn((8192, 3), g).to(dev), conv_b=syn.randn((8192, 3), g).to(dev),
            a=syn.randn((1, 32), g).to(dev), b=syn.randn((1, 32), g).to(dev),
            a_log=torch.log(torch.rand(32, generator=g) * 16 + 1e-4).float().to(dev),
            dt_bias=torch.randn(32, generator=g).float().to(dev), z=syn.randn((1, 4096), g).to(dev),
            norm=syn.randn((128,), g, 0.5).to(dev),
            ssm=(torch.randn(32, 128, 128, generator=g) * 0.2).to(dev),
            out=torch.empty(1, 4096, dtype=torch.bfloat16, device=dev)))

    def step():
        for d in L:
            if fused:
                G.gdn_decode_step(d["mixed"], d["conv_a"], d["conv_b"], d["conv_w"], d["a"], d["b"],
                                  d["a_log"], d["dt_bias"], d["z"], d["norm"], d["ssm"],
                                  out=d["out"])
            else:
                conv_out, _ = G.causal_conv1d(d["mixed"], d["conv_a"], d["conv_w"],
                                              new_state=d["conv_b"])
                q = conv_out[:, :2048].view(1, 16, 128)
                k = conv_out[:, 2048:4096].view(1, 16, 128)
                v = conv_out[:, 4096:].view(1, 32, 128)
                gg, beta = G.gating(d["a"], d["b"], d["a_log"], d["dt_bias"])
                core, _ = G.recurrent_gated_delta_rule(q, k, v, gg, beta, d["ssm"],
                                                       final_state=d["ssm"])
                d["out"] = G.gated_rmsnorm(core, d["z"], d["norm"])
    run = make_graph(torch, step).replay if use_graph else step
    ms = Timer(torch).time(run, iters, warmup)
    us = ms * 1000.0
    nbytes = GDN_STATE_BYTES * layers
    return {"layers": layers, "launches_per_layer": 1 if fused else 4, "us_per_token": us,
            "hbm_gbs": nbytes / (us * 1e-6) / 1e9,
            "frac_hbm": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}


def bench_config1_layers(torch, dev, t, iters, warmup, seed=12):
    """Config 1: one gated full-attention layer and one Gated-DeltaNet layer
    (random weights of the model's shapes) prefilling T tokens from an empty
    cache / zero state -- every launch from this library: the prefill GEMMs
    over the fused projection rows, norms/RoPE/KV write, FMHA, the GDN conv,
    gating, chunked rule and gated norm -- and one decode step of each after
    the prompt (fused projection GEMVs, fused step kernels).  Times are per
    layer call."""
    from qwen36_attn import synthetic as syn
    from qwen36_attn.full_attention import FullAttentionLayer
    from qwen36_attn.gated_deltanet import LinearAttentionLayer
    g = syn.gen(seed)
    wf = {k: v.to(dev) for k, v in syn.full_attention_weights(g).items()}
    wl = {k: v.to(dev) for k, v in syn.linear_attention_weights(g, a_max=1.0).items()}
    fl = FullAttentionLayer(wf, t + 64, dev)
    ll = LinearAttentionLayer(wl, dev)
    x = syn.randn((t, 2048), g, 0.5).to(dev)
    x1 = syn.randn((1, 2048), g, 0.5).to(dev)
    tm = Timer(torch)
    res = {"tokens": t}
    res["full_attention_prefill_us"] = tm.time(lambda: fl.forward(x, 0, "prefill"), iters, warmup) * 1000
    res["linear_attention_prefill_us"] = tm.time(lambda: ll.forward(x, "prefill"), iters, warmup) * 1000
    fl.forward(x, 0, "prefill")
    res["full_attention_decode_us"] = tm.time(lambda: fl.forward(x1, t, "decode"), iters, warmup) * 1000
    res["linear_attention_decode_us"] = tm.time(lambda: ll.forward(x1, "decode"), iters, warmup) * 1000
    del fl, ll, wf, wl
    torch.cuda.empty_cache()
    return res


def _config1_sequence(layer_fn, x, steps):
    """Config 1's sequence: a causal prefill of the prompt, then ``steps``
    decode steps, each feeding the layer's own last output row back as the
    next input (a single layer has no greedy token to embed)."""
    out = layer_fn(x, 0, "prefill")
    t = x.shape[0]
    for i in range(steps):
        out = layer_fn(out[-1:].contiguous(), t + i, "decode")
    return out


def bench_config1_sequence(torch, dev, t=1024, steps=16, iters=10, warmup=2, seed=21):
    """Config 1 exactly as BASELINE defines it, on the GPU: one gated
    full-attention layer (random N(0, 0.02) weights, x ~ N(0,1)*0.5), a
    1,024-token causal prefill then 16 decode steps appending to the KV
    cache; wall time of the whole sequence (eager launches)."""
    from qwen36_attn import synthetic as syn
    from qwen36_attn.full_attention import FullAttentionLayer
    g = syn.gen(seed)
    wf = {k: v.to(dev) for k, v in syn.full_attention_weights(g).items()}
    fl = FullAttentionLayer(wf, t + steps + 64, dev)
    x = syn.randn((t, 2048), g, 0.5).to(dev)
    tm = Timer(torch)
    ms = tm.time(lambda: _config1_sequence(fl.forward, x, steps), iters, warmup)
    del fl, wf
    torch.cuda.empty_cache()
    return {"tokens": t, "decode_steps": steps, "ms": ms}


def cpu_config1_baseline(torch, t=1024, steps=16, seed=21):
    """Config 1 on this host's cores, the reference's CPU plumbing path: the
    oracle's gated full-attention layer (torch CPU, bf16 weights and
    activations as fle:6546-6653) over the same sequence as
    bench_config1_sequence; median of at least 3 whole sequences."""
    from oracle import attention_oracle as O
    from qwen36_attn import synthetic as syn
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    g = syn.gen(seed)
    w = syn.full_attention_weights(g)
    x = syn.randn((t, 2048), g, 0.5)
    k_cache = torch.zeros(t + steps, 2, 256, dtype=torch.bfloat16)
    v_cache = torch.zeros_like(k_cache)
    fn = lambda inp, pos, mode: O.full_attention(inp, w, k_cache, v_cache, pos, mode)
    med, n = _median_time(lambda: _config1_sequence(fn, x, steps), min_runs=3, budget_s=20.0)
    return {"value": med * 1e3, "unit": "ms", "cores": threads, "kind": "port",
            "sample": f"median of {n} whole config-1 sequences ({t}-token prefill + {steps} "
                      f"decode steps, one layer) through the oracle (torch CPU, {_cpu_info()})"}


def cpu_decode_32k_baseline(torch, cache_end=32768):
    """Config 2 on this host's cores: the oracle's grouped bf16 decode of one
    layer at S = 32768, median of at least 3; and x10 for the model's 10
    full-attention layers."""
    from oracle import attention_oracle as O
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(8)
    k = torch.randn(cache_end, 2, 256, generator=gen).to(torch.bfloat16)
    v = torch.randn(cache_end, 2, 256, generator=gen).to(torch.bfloat16)
    q = torch.randn(1, 16, 256, generator=gen).to(torch.bfloat16)
    med, n = _median_time(lambda: O.decode_attention_grouped_bf16(q, k, v, cache_end),
                          min_runs=5, budget_s=5.0, max_runs=50)
    return {"us_per_layer": med * 1e6, "us_10layers": med * 1e6 * N_FULL_LAYERS,
            "cores": threads, "kind": "port",
            "sample": f"median of {n} single-layer grouped-bf16 decodes at S={cache_end} "
                      f"(oracle, torch CPU, {_cpu_info()})"}


def bench_gdn_prefill(torch, dev, t, iters, warmup, seed=3):
    """Config 4: chunked delta-rule prefill of T tokens from zero state."""
    from qwen36_attn import gated_deltanet as G
    from qwen36_attn import synthetic as syn
    g = syn.gen(seed)
    q, k, v, gg, beta = [x.to(dev) for x in syn.gdn_core_inputs(t, g, a_max=16.0)]
    fs = torch.empty(32, 128, 128, dtype=torch.float32, device=dev)
    ms = Timer(torch).time(lambda: G.chunk_gated_delta_rule(q, k, v, gg, beta, None, final_state=fs),
                           iters, warmup)
    flop, nbytes = gdn_prefill_work(t)
    # Two rooflines (the pass is neither purely MFMA- nor HBM-bound): the
    # algorithmic FLOP against the bf16 dense MFMA peak, and the essential
    # bytes (q, k, v, o, g, beta, state) against HBM.  The kernels issue
    # about 3x the algorithmic products (fp32-accurate bf16 hi/lo splits),
    # which neither fraction credits.
    return {"tokens": t, "ms": ms, "tflops": flop / (ms * 1e-3) / 1e12,
            "frac_bf16_mfma": flop / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
            "hbm_gbs_algorithmic": nbytes / (ms * 1e-3) / 1e9,
            "frac_hbm": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}


def gdn_prefill_work(t, c=64):
    """Algorithmic FLOP and essential HBM bytes of a chunked delta-rule
    prefill of t tokens (32 v-heads, dk = dv = 128): per (chunk, v-head)
    6 x 2C^2 d + 4 x 2C d^2 + C^3 / 3; bytes = q, k (16 heads) and v, o (32
    heads) in bf16, g and beta in fp32, the fp32 state written once."""
    flop_per_unit = 6 * 2 * c * c * 128 + 4 * 2 * c * 128 * 128 + c ** 3 // 3
    flop = flop_per_unit * ((t + c - 1) // c) * 32
    nbytes = 2 * t * 16 * 128 * 2 + t * 32 * 128 * 2 * 2 + t * 32 * 4 * 2 + 32 * 128 * 128 * 4
    return flop, nbytes


def cpu_baseline(torch, cache_end):
    """Oracle grouped bf16 decode on this host's cores: a bounded sample of
    whole layers at the headline cache length, scaled to the 10-layer step."""
    from oracle import attention_oracle as O
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(7)
    k = torch.randn(cache_end, 2, 256, generator=gen).to(torch.bfloat16)
    v = torch.randn(cache_end, 2, 256, generator=gen).to(torch.bfloat16)
    q = torch.randn(1, 16, 256, generator=gen).to(torch.bfloat16)
    O.decode_attention_grouped_bf16(q, k, v, cache_end)  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < 10.0 and len(times) < 50):
        t0 = time.perf_counter()
        O.decode_attention_grouped_bf16(q, k, v, cache_end)
        times.append(time.perf_counter() - t0)
    times.sort()
    per_layer_s = times[len(times) // 2]
    return {"value": per_layer_s * N_FULL_LAYERS * 1e6, "unit": "us/token",
            "cores": threads, "kind": "port",
            "sample": f"median of {len(times)} single-layer grouped-bf16 decodes at "
                      f"S={cache_end} (oracle, torch CPU, {_cpu_info()}), x{N_FULL_LAYERS} layers"}


def _median_time(fn, min_runs=3, budget_s=8.0, max_runs=20):
    fn()  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < min_runs or (time.perf_counter() - t_start < budget_s and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_prefill_baseline(torch, rows=8192):
    """Config 3 on this host's cores: the oracle's SDPA (fp32 evaluation of
    the bf16 inputs, as the FMHA provider returns fp32) for the last ``rows``
    query rows of the 8192-token block over the 12288-row cache (the whole
    block by default; fewer rows are the ones with the most keys, scaled to
    the whole block by unmasked (q, k) pairs)."""
    from oracle import attention_oracle as O
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(17)
    t_full, s_full = 8192, 12288
    q = torch.randn(rows, 16, 256, generator=gen).to(torch.bfloat16)
    k = torch.randn(s_full, 2, 256, generator=gen).to(torch.bfloat16)
    v = torch.randn(s_full, 2, 256, generator=gen).to(torch.bfloat16)
    med, n = _median_time(lambda: O.prefill_attention(q, k, v, s_full - rows, out_dtype=torch.float32))
    scale = causal_pairs(t_full, s_full) / causal_pairs(rows, s_full)
    ms = med * scale * 1e3
    flop = PREFILL_FLOP_PER_PAIR * causal_pairs(t_full, s_full)
    what = (f"the whole block ({t_full} query rows x {s_full} keys)" if rows == t_full else
            f"the last {rows} query rows x {s_full} keys, scaled x{scale:.1f} by unmasked pairs to "
            f"8192 rows over a 4096-token prefix")
    return {"value": ms, "unit": "ms", "tflops": flop / (ms * 1e-3) / 1e12, "cores": threads,
            "kind": "port",
            "sample": f"median of {n} oracle SDPA runs (torch CPU fp32, {_cpu_info()}) over {what}"}


def cpu_gdn_baseline(torch, chunk_tokens=8192, steps=64):
    """Config 4 on this host's cores: the oracle's chunked delta rule
    (fp32, chunk 64, 32 v-heads) over ``chunk_tokens`` tokens (the whole
    8192 by default; fewer are scaled linearly -- the chunk loop is
    sequential and every chunk costs the same), plus ``steps`` recurrent
    steps (config 4's 64 by default), reported per step."""
    from oracle import attention_oracle as O
    from qwen36_attn import synthetic as syn
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    g = syn.gen(19)
    q, k, v, gg, beta = syn.gdn_core_inputs(chunk_tokens + steps, g, a_max=16.0)
    R = O.repeat_kv_heads
    qr, kr = R(q).unsqueeze(0), R(k).unsqueeze(0)
    vv, gb, bb = v.unsqueeze(0), gg.unsqueeze(0), beta.unsqueeze(0)
    s0 = torch.zeros(1, 32, 128, 128)
    c = chunk_tokens
    med_c, n_c = _median_time(lambda: O.chunk_gated_delta_rule(
        qr[:, :c], kr[:, :c], vv[:, :c], gb[:, :c], bb[:, :c], s0))
    med_r, n_r = _median_time(lambda: O.recurrent_gated_delta_rule(
        qr[:, c:], kr[:, c:], vv[:, c:], gb[:, c:], bb[:, c:], s0))
    prefill_ms = med_c * (8192 / c) * 1e3
    decode_us = med_r / steps * 1e6
    flop, _ = gdn_prefill_work(8192)
    return {"prefill_8k_ms": prefill_ms, "prefill_tflops": flop / (prefill_ms * 1e-3) / 1e12,
            "recurrent_us_per_step": decode_us, "cores": threads, "kind": "port",
            "sample": f"median of {n_c} oracle chunked-rule runs over {c} tokens"
                      + (f" scaled x{8192 // c} to 8192" if c != 8192 else "")
                      + f", median of {n_r} runs of {steps} recurrent steps (torch CPU fp32, "
                      f"{_cpu_info()})"}


def bench_launch_cost(torch, dev, launches=30, iters=50, warmup=5):
    """The fixed cost of one kernel node in a HIP graph: ``launches``
    back-to-back launches of a one-element kernel (torch's fill, and this
    library's output gate over one row), replayed as one graph; reported
    per launch.  Every per-layer latency in a decode step pays this once
    per kernel."""
    from qwen36_attn import _lib
    x = torch.zeros(1, device=dev)
    attn = torch.zeros(1, 4096, dtype=torch.bfloat16, device=dev)
    qg = torch.zeros(1, 8192, dtype=torch.bfloat16, device=dev)
    out = torch.empty(1, 4096, dtype=torch.bfloat16, device=dev)

    def fills():
        for _ in range(launches):
            x.zero_()

    def gates():
        st = torch.cuda.current_stream().cuda_stream
        for _ in range(launches):
            _lib.call("qwen36_output_gate", attn.data_ptr(), 0, qg.data_ptr(), 8192,
                      out.data_ptr(), 1, st)
    tm = Timer(torch)
    res = {"launches": launches}
    for name, fn in (("torch_fill", fills), ("output_gate_1row", gates)):
        res[name + "_us_per_launch"] = tm.time(make_graph(torch, fn).replay, iters, warmup) * 1e3 / launches
    return res


def run_only(torch, fa, dev, args):
    """Single legs for counter runs (rocprofv3 --pmc): the decode headline
    (10 layers x S=131072, eager launches), the prefill configs, the GDN legs,
    or a 256 MiB device copy used to calibrate FETCH_SIZE/WRITE_SIZE."""
    if args.only == "decode":
        r = bench_decode(torch, fa, dev, 131072, N_FULL_LAYERS, args.steps, args.warmup, False)
    elif args.only == "prefill":
        r = [bench_prefill(torch, fa, dev, 8192, 8192, args.steps, args.warmup),
             bench_prefill(torch, fa, dev, 8192, 12288, args.steps, args.warmup),
             bench_prefill(torch, fa, dev, 1024, 1024, args.steps, args.warmup),
             bench_prefill(torch, fa, dev, 1024, 5120, args.steps, args.warmup),
             bench_prefill_gated(torch, fa, dev, 8192, 8192, args.steps, args.warmup),
             bench_prefill_gated(torch, fa, dev, 1024, 1024, args.steps, args.warmup)]
    elif args.only == "prefill_8k":
        r = bench_prefill(torch, fa, dev, 8192, 8192, args.steps, args.warmup)
    elif args.only == "prefill_c3":
        r = bench_prefill(torch, fa, dev, 8192, 12288, args.steps, args.warmup)
    elif args.only == "gemm":
        r = bench_prefill_projections(torch, dev, 8192, args.steps, args.warmup)
    elif args.only == "gdn":
        r = [bench_gdn_recurrent(torch, dev, GDN_LAYERS, args.steps, args.warmup, False),
             bench_gdn_fused_gating_update(torch, dev, GDN_LAYERS, args.steps, args.warmup, False),
             bench_gdn_decode_step(torch, dev, GDN_LAYERS, args.steps, args.warmup, False),
             bench_gdn_prefill(torch, dev, 8192, args.steps, args.warmup)]
    elif args.only == "launch":
        r = bench_launch_cost(torch, dev)
    elif args.only == "moe":
        r = [bench_moe_prefill(torch, dev, 8192, args.steps, args.warmup)]
    elif args.only == "moe_1k":
        r = [bench_moe_prefill(torch, dev, 1024, args.steps, args.warmup)]
    elif args.only == "moe_decode":
        r = [bench_moe_decode(torch, dev, 40, args.steps, args.warmup, False)]
    else:
        x = torch.empty(64 * 1024 * 1024, dtype=torch.float32, device=dev)
        x.fill_(1.0)
        y = torch.empty_like(x)
        for _ in range(args.steps):
            y.copy_(x)
        torch.cuda.synchronize()
        r = {"copy_bytes_read": x.numel() * 4, "copy_bytes_written": y.numel() * 4}
    print(r, file=sys.stderr)


def main():
    args = _parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(every box has one MI355X); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    from qwen36_attn import full_attention as fa
    fa._lib.load()
    dev = torch.device("cuda:0")
    use_graph = not args.no_graph
    if args.only is not None:
        run_only(torch, fa, dev, args)
        return

    head = bench_decode(torch, fa, dev, 131072, N_FULL_LAYERS, args.steps, args.warmup, use_graph)
    extra = {
        "decode_128k": head,
        "decode_32k_1layer": bench_decode(torch, fa, dev, 32768, 1, 50, 5, use_graph),
        "decode_32k_10layers": bench_decode(torch, fa, dev, 32768, N_FULL_LAYERS, 20, 3, use_graph),
        "decode_262143": bench_decode(torch, fa, dev, 262143, N_FULL_LAYERS, 10, 2, use_graph),
        "decode_layer_step_128k_fused": bench_decode_layer_step(torch, fa, dev, 131072, N_FULL_LAYERS,
                                                               20, 3, use_graph),
        "decode_layer_step_128k_unfused": bench_decode_layer_step(torch, fa, dev, 131072,
                                                                 N_FULL_LAYERS, 20, 3, use_graph,
                                                                 fused=False),
        "prefill_8k_causal": bench_prefill(torch, fa, dev, 8192, 8192, 10, 2),
        "prefill_8k_over_4k_prefix": bench_prefill(torch, fa, dev, 8192, 12288, 10, 2),
        "prefill_8k_gated": bench_prefill_gated(torch, fa, dev, 8192, 8192, 10, 2),
        "prefill_1k_gated": bench_prefill_gated(torch, fa, dev, 1024, 1024, 20, 3),
        "graph_launch_cost": bench_launch_cost(torch, dev),
        "gdn_recurrent_30layers": bench_gdn_recurrent(torch, dev, GDN_LAYERS, 50, 5, use_graph),
        "gdn_fused_gating_update_30layers": bench_gdn_fused_gating_update(torch, dev, GDN_LAYERS,
                                                                          50, 5, use_graph),
        "prefix_cache_32k": bench_prefix_cache(torch, dev, 32768, 20, 3),
        "decode_projections_40layers": bench_decode_projections(torch, dev, 20, 3, use_graph),
        "moe_decode_40layers": bench_moe_decode(torch, dev, 40, 20, 3, use_graph),
        "decode_projections_40layers_torch": bench_decode_projections(torch, dev, 20, 3, use_graph,
                                                                      native=False),
        "gdn_decode_step_30layers": bench_gdn_decode_step(torch, dev, GDN_LAYERS, 50, 5, use_graph),
        "gdn_decode_unfused_30layers": bench_gdn_decode_step(torch, dev, GDN_LAYERS, 50, 5,
                                                             use_graph, fused=False),
        "gdn_chunk_prefill_8k": bench_gdn_prefill(torch, dev, 8192, 10, 2),
        "config1_layers_1k": bench_config1_layers(torch, dev, 1024, 20, 3),
        "prefill_layers_8k": bench_config1_layers(torch, dev, 8192, 10, 2),
        "config1_sequence": bench_config1_sequence(torch, dev),
        "prefill_projections_1k": bench_prefill_projections(torch, dev, 1024, 20, 3),
        "prefill_projections_1k_torch": bench_prefill_projections(torch, dev, 1024, 20, 3,
                                                                  native=False),
        "prefill_projections_8k": bench_prefill_projections(torch, dev, 8192, 10, 2),
        "prefill_projections_8k_torch": bench_prefill_projections(torch, dev, 8192, 10, 2,
                                                                  native=False),
        "prefill_projections_8k_mfma_kernel": bench_prefill_projections(torch, dev, 8192, 10, 2,
                                                                        backend="native"),
        "prefill_projections_1k_mfma_kernel": bench_prefill_projections(torch, dev, 1024, 20, 3,
                                                                        backend="native"),
        "moe_prefill_8k": bench_moe_prefill(torch, dev, 8192, 10, 2),
        "moe_prefill_1k": bench_moe_prefill(torch, dev, 1024, 20, 3),
        "moe_prefill_8k_torch_expert_loop": bench_moe_prefill(torch, dev, 8192, 3, 1, native=False),
    }
    extra["attention_us_per_token_128k"] = (head["us_per_token"]
                                            + extra["gdn_recurrent_30layers"]["us_per_token"])
    torch.cuda.empty_cache()
    # Roofline of the dominant kernel (split-K decode), per layer launch.
    per_layer_us = head["us_per_token"] / N_FULL_LAYERS
    alg_bytes = DECODE_BYTES_PER_TOKEN * 131072
    achieved = alg_bytes / (per_layer_us * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": achieved / HBM_PEAK_GBS, "traffic": measured_traffic(),
                "kernel": "qwen36_decode_gqa (write_kv_row + decode_gqa_split + decode_gqa_combine)",
                "algorithmic_bytes_per_launch": alg_bytes}
    cpu = None if args.no_cpu else cpu_baseline(torch, 131072)
    if not args.no_cpu:
        extra["cpu_prefill_config3"] = cpu_prefill_baseline(torch)
        extra["cpu_gdn_config4"] = cpu_gdn_baseline(torch)
        extra["cpu_config1"] = cpu_config1_baseline(torch)
        extra["cpu_decode_config2"] = cpu_decode_32k_baseline(torch)
    line = {
        "metric": "decode attn us/tok + HBM GB/s @128K ctx; prefill attn TFLOP/s @8K tokens",
        "value": head["us_per_token"], "unit": "us/token", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": head["us_per_token"] / 1000.0,
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 q/K/V, resident in HBM)",
        "config": {"workload": "config5: 10 gated-GQA decode layers, 16q/2kv heads, D=256, "
                               "KV length 131072, distinct caches", "graph": use_graph},
        "roofline": roofline, "cpu_baseline": cpu, "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
