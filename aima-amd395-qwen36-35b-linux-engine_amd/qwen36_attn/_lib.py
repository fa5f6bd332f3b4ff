"""ctypes binding of the C-ABI library ``libqwen36_attn.so``.

The library is the product: every op in this package calls into it.  There is
no CPU fallback -- if the library is missing or a symbol is absent, loading
fails loudly.
"""
from __future__ import annotations

import ctypes
import os

from .build import LIB_PATH

_vp = ctypes.c_void_p
_u32 = ctypes.c_uint
_i32 = ctypes.c_int
_sz = ctypes.c_size_t
_f32 = ctypes.c_float
_u64 = ctypes.c_ulonglong
_pu32 = ctypes.POINTER(ctypes.c_uint)
_pu64 = ctypes.POINTER(ctypes.c_ulonglong)

# name -> (restype, argtypes).  Mirrors include/qwen36_attn.h.
SIGNATURES: dict[str, tuple] = {
    # FMHA provider ABI (drop-in for qrt_ck_fmha_*)
    "qrt_ck_fmha_prepare": (_i32, [_u32]),
    "qrt_ck_fmha_bf16_launch": (_i32, [_vp, _vp, _vp, _vp, _u32, _vp]),
    "qrt_ck_fmha_bf16_launch_ex": (_i32, [_vp, _vp, _vp, _vp, _u32, _u32, _vp]),
    "qrt_ck_fmha_release": (_i32, []),
    "qwen36_fmha_prefill_workspace_bytes": (_sz, [_u32, _u32]),
    "qwen36_fmha_prefill": (_i32, [_vp, _vp, _vp, _vp, _u32, _u32, _vp, _sz, _vp]),
    "qwen36_fmha_prefill_gated": (_i32, [_vp, _vp, _vp, _vp, _u32, _vp, _u32, _u32, _vp, _sz, _vp]),
    "qrt_ck_fmha_q8192_prepare": (_i32, []),
    "qrt_ck_fmha_q8192_bf16_launch": (_i32, [_vp, _vp, _vp, _vp, _vp]),
    "qrt_ck_fmha_q8192_f32_launch": (_i32, [_vp, _vp, _vp]),
    "qrt_ck_fmha_q8192_release": (_i32, []),
    # decode
    "qwen36_decode_gqa_workspace_bytes": (_sz, [_u32, _u32]),
    "qwen36_decode_gqa": (_i32, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32,
                                 _vp, _u32, _vp, _vp, _sz, _u32, _vp]),
    "qwen36_decode_gqa_noalloc": (_i32, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32,
                                         _vp, _u32, _vp, _u32, _vp]),
    "qwen36_decode_step": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32,
                                  _vp, _vp, _sz, _u32, _vp]),
    # pointwise (full attention)
    "qwen36_rotary_table": (_i32, [_vp, _vp, _u32, _u32, _vp]),
    "qwen36_head_norm_rope": (_i32, [_vp, _u32, _vp, _u32, _vp, _u32, _vp, _vp,
                                     _u32, _u32, _vp, _vp, _vp, _vp]),
    "qwen36_output_gate": (_i32, [_vp, _i32, _vp, _u32, _vp, _u32, _vp]),
    # Gated DeltaNet
    "qwen36_gdn_conv1d": (_i32, [_vp, _u32, _vp, _vp, _vp, _vp, _u32, _vp]),
    "qwen36_gdn_gating": (_i32, [_vp, _vp, _u32, _vp, _vp, _vp, _vp, _u32, _u32, _vp]),
    "qwen36_gdn_recurrent": (_i32, [_vp, _vp, _vp, _u32, _u32, _u32, _vp, _vp,
                                    _vp, _vp, _vp, _u32, _vp]),
    "qwen36_gdn_chunk_prefill_workspace_bytes": (_sz, [_u32]),
    "qwen36_gdn_chunk_prefill": (_i32, [_vp, _vp, _vp, _u32, _u32, _u32, _vp, _vp,
                                        _vp, _vp, _vp, _u32, _vp, _sz, _vp]),
    "qwen36_gdn_chunk_prefill_ex": (_i32, [_vp, _vp, _vp, _u32, _u32, _u32, _vp, _vp,
                                           _vp, _vp, _vp, _u32, _u32, _vp, _sz, _vp]),
    "qwen36_gdn_fused_gating_update": (_i32, [_vp, _vp, _vp, _u32, _vp, _vp, _vp, _u32, _u32,
                                              _vp, _u32, _vp, _vp, _vp, _u32, _f32, _u32, _vp]),
    "qwen36_gdn_fused_gating_update_varlen": (_i32, [_vp, _vp, _vp, _u32, _vp, _vp, _vp, _u32,
                                                     _u32, _vp, _u32, _vp, _vp, _vp, _u32, _vp,
                                                     _vp, _u32, _u32, _f32, _u32, _vp]),
    "qwen36_gdn_gated_norm": (_i32, [_vp, _vp, _u32, _vp, _vp, _u32, _vp]),
    # prefill projections
    "qwen36_prefill_gemm_lt_workspace_bytes": (_sz, []),
    "qwen36_prefill_gemm_bf16_lt": (_i32, [_vp, _u32, _vp, _vp, _u32, _u32, _u32, _u32, _vp, _sz,
                                           _vp]),
    "qwen36_prefill_gemm_bf16": (_i32, [_vp, _u32, _vp, _vp, _u32, _u32, _u32, _u32, _vp]),
    "qwen36_prefill_gemm_workspace_bytes": (_sz, [_u32, _u32, _u32]),
    "qwen36_prefill_gemm_bf16_ws": (_i32, [_vp, _u32, _vp, _vp, _u32, _u32, _u32, _u32, _vp, _sz,
                                           _vp]),
    # decode projections
    "qwen36_gemv_bf16": (_i32, [_vp, _u32, _u32, _vp, _vp, _vp]),
    # MoE block
    "qwen36_moe_decode_workspace_bytes": (_sz, []),
    "qwen36_moe_decode": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _vp, _vp, _sz, _vp]),
    "qwen36_moe_prefill_workspace_bytes": (_sz, [_u32, _u32]),
    "qwen36_moe_prefill": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _vp, _vp, _sz,
                                  _vp]),
    # exact-prefix cache
    "qwen36_prefix_cache_create": (_vp, [_u32, _u64, _u32]),
    "qwen36_prefix_cache_entries": (_u32, [_vp]),
    "qwen36_prefix_cache_add_slice": (_i32, [_vp, _vp, _u64, _u64]),
    "qwen36_prefix_cache_finalize": (_i32, [_vp, _pu64]),
    "qwen36_prefix_cache_lookup": (_i32, [_vp, _pu32, _u32, _pu32, _pu32]),
    "qwen36_prefix_cache_restore": (_i32, [_vp, _u32, _vp, _pu64]),
    "qwen36_prefix_cache_capture": (_i32, [_vp, _pu32, _u32, _vp, _vp, _pu32, _pu64]),
    "qwen36_prefix_cache_copy_terminal": (_i32, [_vp, _u32, _vp, _vp]),
    "qwen36_prefix_cache_destroy": (_i32, [_vp]),
    "qwen36_gdn_decode_step": (_i32, [_vp, _u32, _vp, _vp, _vp, _vp, _vp, _u32, _vp,
                                      _vp, _vp, _u32, _vp, _vp, _vp, _vp, _u32, _vp]),
}

_LIB = None


class KernelError(RuntimeError):
    """A C-ABI entry point returned a non-zero hipError_t."""


def library_path() -> str:
    return os.environ.get("QWEN36_ATTN_LIB", LIB_PATH)


def load(required: tuple[str, ...] | None = None) -> ctypes.CDLL:
    """Load the library once; raise if it (or a required symbol) is missing."""
    global _LIB
    if _LIB is None:
        path = library_path()
        if not os.path.isfile(path):
            raise RuntimeError(
                f"qwen36_attn HIP library not built: {path} is missing "
                "(run __graft_entry__.build() or python -m qwen36_attn.build)")
        lib = ctypes.CDLL(path, mode=ctypes.RTLD_LOCAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
        _LIB = lib
    for name in required or ():
        if getattr(_LIB, name, None) is None:
            raise RuntimeError(f"{library_path()} does not export {name}")
    return _LIB


def call(name: str, *args) -> int:
    fn = getattr(load((name,)), name)
    status = fn(*args)
    if status != 0:
        raise KernelError(f"{name} failed: hip_status={status}")
    return status
