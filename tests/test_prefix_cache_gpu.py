"""Exact-prefix cache (qwen36_prefix_cache_*, the reference's
NativeExactPrefixCache + entry pool, native_resident_engine.hip.cpp:121-296,
:553-560, :706-719, :826-836, :1197-1214) over a stack of one Gated-DeltaNet
and one gated full-attention layer."""
import pytest
import torch

from qwen36_attn import synthetic as syn

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _stack(gpu, capacity, seed=0):
    from qwen36_attn.full_attention import FullAttentionLayer
    from qwen36_attn.gated_deltanet import LinearAttentionLayer
    g = syn.gen(seed)
    wl = {k: v.to(gpu) for k, v in syn.linear_attention_weights(g, a_max=1.0).items()}
    wf = {k: v.to(gpu) for k, v in syn.full_attention_weights(g).items()}
    return [LinearAttentionLayer(wl, gpu), FullAttentionLayer(wf, capacity, gpu)]


def _run(layers, x, pos, mode):
    h = x
    for layer in layers:
        h = layer.forward(h, mode) if not hasattr(layer, "k_cache") else layer.forward(h, pos, mode)
    return h


def test_capture_restore_replays_decode_bit_exact(gpu):
    from qwen36_attn.prefix_cache import ExactPrefixCachePool
    cap, t = 1024, 300
    layers = _stack(gpu, cap)
    pool = ExactPrefixCachePool(cap, layers)
    assert pool.entries == 4
    g = syn.gen(1)
    prompt = syn.randn((t, 2048), g, 0.5).to(gpu)
    steps = [syn.randn((1, 2048), g, 0.5).to(gpu) for _ in range(3)]
    tokens = list(range(1000, 1000 + t))
    print("prefix cache: prefill + capture", flush=True)
    h = _run(layers, prompt, 0, "prefill")
    idx, nbytes = pool.capture(tokens, h[-1])
    assert nbytes == 2 * t * 1024 + 8192 * 3 * 2 + 32 * 128 * 128 * 4 + 4096
    first = [_run(layers, s, t + i, "decode").clone() for i, s in enumerate(steps)]
    states = [layers[0].ssm_state.clone(), layers[1].k_cache[:t + 3].clone()]
    matched, index = pool.lookup(tokens + [7, 8])
    assert (matched, index) == (t, idx)
    pool.restore(index)
    again = [_run(layers, s, t + i, "decode") for i, s in enumerate(steps)]
    torch.cuda.synchronize()
    for a, b in zip(first, again):
        assert torch.equal(a, b)
    assert torch.equal(layers[0].ssm_state, states[0])
    assert torch.equal(layers[1].k_cache[:t + 3], states[1])
    term = torch.empty(2048, dtype=torch.bfloat16, device=gpu)
    pool.terminal_hidden(idx, term)
    torch.cuda.synchronize()
    assert torch.equal(term, h[-1])
    pool.close()


def test_prefix_hit_then_suffix_prefill_matches_full_prefill(gpu):
    """Restore a 256-token prefix, prefill only the 100-token suffix: the
    suffix rows equal those of one prefill over all 356 tokens (GDN state
    carried across a chunk boundary; bottom-right causal FMHA)."""
    from qwen36_attn.prefix_cache import ExactPrefixCachePool
    cap, t1, t2 = 512, 256, 100
    g = syn.gen(3)
    x = syn.randn((t1 + t2, 2048), g, 0.5).to(gpu)
    tokens = list(range(t1 + t2))
    full_layers = _stack(gpu, cap, seed=9)
    ref = _run(full_layers, x, 0, "prefill")
    layers = _stack(gpu, cap, seed=9)
    pool = ExactPrefixCachePool(cap, layers, entries=2)
    print("prefix cache: prefix + suffix", flush=True)
    h = _run(layers, x[:t1], 0, "prefill")
    pool.capture(tokens[:t1], h[-1])
    _run(layers, syn.randn((40, 2048), g, 0.5).to(gpu), 0, "prefill")   # clobber the live state
    matched, index = pool.lookup(tokens)
    assert matched == t1
    pool.restore(index)
    got = _run(layers, x[t1:], t1, "prefill")
    torch.cuda.synchronize()
    assert (got.float() - ref[t1:].float()).abs().max().item() <= TOL
    pool.close()


def test_lookup_longest_prefix_and_lru_capture_slot(gpu):
    from qwen36_attn.prefix_cache import ExactPrefixCachePool
    cap = 256
    layers = _stack(gpu, cap, seed=4)
    pool = ExactPrefixCachePool(cap, layers, entries=2)
    hid = torch.zeros(2048, dtype=torch.bfloat16, device=gpu)
    p1, p2, p3, p4 = ([i] * n for i, n in ((1, 10), (2, 20), (3, 30), (4, 40)))
    print("prefix cache: lru", flush=True)
    assert pool.lookup(p1) == (0, pool.entries)                  # empty pool: miss
    assert pool.capture(p1, hid)[0] == 0                         # first empty entry
    assert pool.capture(p2, hid)[0] == 1
    assert pool.lookup(p1 + [5]) == (10, 0)                      # prefix extension
    assert pool.lookup(p2[:15]) == (0, pool.entries)             # shorter than stored
    assert pool.lookup(p2) == (20, 1)                            # exact
    assert pool.capture(p3, hid)[0] == 0                         # evicts the LRU (p1)
    assert pool.lookup(p1) == (0, pool.entries)
    pool.restore(1)                                              # p2 becomes most recent
    assert pool.capture(p4, hid)[0] == 0                         # evicts p3, not p2
    assert pool.lookup(p2 + p4) == (20, 1)
    torch.cuda.synchronize()
    from qwen36_attn._lib import KernelError
    with pytest.raises(KernelError):
        pool.restore(5)
    pool.close()


def test_finalize_failure_leaves_pool_unfinalized_and_frees(gpu):
    """An entry snapshot that cannot be allocated (a 1 TiB fixed slice) makes
    finalize return the allocation error; whatever it had allocated (the
    device slice table, earlier snapshots) is freed and the pool stays
    unfinalized (capture / restore refuse it), so nothing leaks."""
    import ctypes
    from qwen36_attn import _lib
    lib = _lib.load()
    buf = torch.zeros(4096, dtype=torch.uint8, device=gpu)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info(gpu)
    pool = lib.qwen36_prefix_cache_create(1024, 4096, 2)
    assert pool
    assert lib.qwen36_prefix_cache_add_slice(pool, buf.data_ptr(), 1 << 40, 0) == 0
    nbytes = ctypes.c_ulonglong(0)
    assert lib.qwen36_prefix_cache_finalize(pool, ctypes.byref(nbytes)) != 0
    free1, _ = torch.cuda.mem_get_info(gpu)
    assert abs(free1 - free0) < (64 << 20)
    toks = (ctypes.c_uint * 4)(1, 2, 3, 4)
    idx = ctypes.c_uint(0)
    assert lib.qwen36_prefix_cache_capture(pool, toks, 4, buf.data_ptr(), None, ctypes.byref(idx),
                                           None) != 0
    assert lib.qwen36_prefix_cache_restore(pool, 0, None, None) != 0
    assert lib.qwen36_prefix_cache_destroy(pool) == 0
