"""qwen36_decode_gqa_noalloc (library-owned split scratch, no allocation)
against qwen36_decode_gqa (caller workspace) through the C ABI: two calls in
a row, the second on a smaller cache, bit-identical outputs and cache rows;
split counts past the scratch are rejected."""
import ctypes

import pytest
import torch

from qwen36_attn import synthetic as syn

pytestmark = pytest.mark.gpu


def _call_both(lib, gpu, s, cap, pos, split_tokens, seed, with_gate):
    g = syn.gen(seed)
    q = syn.randn((16, 256), g).to(gpu)
    kc = syn.randn((cap, 2, 256), g).to(gpu)
    vc = syn.randn((cap, 2, 256), g).to(gpu)
    kn = syn.randn((2, 256), g).to(gpu)
    vn = syn.randn((2, 256), g).to(gpu)
    gate = syn.randn((16, 512), g).to(gpu) if with_gate else None
    gp = gate[:, 256:].data_ptr() if with_gate else None
    gs = 512 if with_gate else 0
    stream = torch.cuda.current_stream(gpu).cuda_stream
    kc2, vc2 = kc.clone(), vc.clone()
    out_ref = torch.empty(1, 4096, dtype=torch.bfloat16, device=gpu)
    out_na = torch.full((1, 4096), 7.0, dtype=torch.bfloat16, device=gpu)
    nb = lib.qwen36_decode_gqa_workspace_bytes(s, split_tokens)
    ws = torch.empty(nb, dtype=torch.uint8, device=gpu)
    rc = lib.qwen36_decode_gqa(q.data_ptr(), kn.data_ptr(), vn.data_ptr(), kc.data_ptr(),
                               vc.data_ptr(), pos, s, cap, gp, gs, out_ref.data_ptr(),
                               ws.data_ptr(), nb, split_tokens, stream)
    assert rc == 0
    rc = lib.qwen36_decode_gqa_noalloc(q.data_ptr(), kn.data_ptr(), vn.data_ptr(), kc2.data_ptr(),
                                       vc2.data_ptr(), pos, s, cap, gp, gs, out_na.data_ptr(),
                                       split_tokens, stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(out_na, out_ref)
    assert torch.equal(kc2, kc) and torch.equal(vc2, vc)


def test_noalloc_decode_matches_workspace_decode(gpu):
    from qwen36_attn import _lib
    lib = _lib.load(("qwen36_decode_gqa_noalloc",))
    print("noalloc decode: S=131072 then S=3000", flush=True)
    _call_both(lib, gpu, 131072, 131072, 131071, 0, 71, True)
    _call_both(lib, gpu, 3000, 4096, 2999, 0, 72, False)
    # the most splits a call can ask for (256) fits; more are rejected
    print("noalloc decode: 256 splits, then 257 rejected", flush=True)
    _call_both(lib, gpu, 256 * 128, 256 * 128, 5000, 128, 73, True)
    z = torch.zeros(1, dtype=torch.bfloat16, device=gpu).data_ptr()
    assert lib.qwen36_decode_gqa_noalloc(z, None, None, z, z, 0, 257 * 128, 257 * 128, None, 0,
                                         z, 128, None) == 1
