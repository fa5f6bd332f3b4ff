"""Exact-prefix cache mirror of the reference's ``NativeExactPrefixCache``
and the resident engine's entry pool
(native/src/native_resident_engine.hip.cpp:121-296 cache, :553-560 pool size,
:706-719 lookup, :826-836 restore, :1197-1214 capture slot).

The pool, its bookkeeping and the batched device copies live in
``libqwen36_attn.so`` (``qwen36_prefix_cache_*``); this class binds them and
registers the state buffers of a stack of attention layers:
  * a full-attention layer's K and V caches are per-token slices (a capture
    stores only the prompt's rows: 1 KiB per token each);
  * a Gated-DeltaNet layer's conv state [8192,3] bf16 and recurrent state
    [32,128,128] fp32 are fixed slices (stored whole).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._tensors import stream_handle
from .full_attention import FullAttentionLayer, HKV, HEAD_DIM
from .gated_deltanet import LinearAttentionLayer

KV_BYTES_PER_TOKEN = HKV * HEAD_DIM * 2        # one cache row of K (or V), bf16
HIDDEN_BYTES = 2048 * 2                         # terminal hidden row, bf16


def default_entries(capacity: int) -> int:
    """The reference's pool size (native_resident_engine.hip.cpp:553-556)."""
    return 4 if capacity <= 32768 else (2 if capacity <= 131072 else 1)


class ExactPrefixCachePool:
    """Pool of exact-prefix snapshots over the layers' live state buffers.

    ``lookup(tokens)`` returns (matched_tokens, index) for the entry with the
    longest stored prefix of ``tokens`` (index == entries on a miss);
    ``restore(index)`` copies that entry back into the live buffers;
    ``capture(tokens, terminal_hidden)`` stores the current state for the
    prompt ``tokens`` in the first empty entry, else the least recently used.
    Copies are asynchronous on the current stream."""

    def __init__(self, capacity: int, layers, entries: int = 0,
                 terminal_bytes: int = HIDDEN_BYTES) -> None:
        lib = _lib.load(("qwen36_prefix_cache_create",))
        self._lib = lib
        self.capacity = capacity
        self.terminal_bytes = terminal_bytes
        self._pool = lib.qwen36_prefix_cache_create(capacity, terminal_bytes, entries)
        if not self._pool:
            raise ValueError("native exact-prefix context is unsupported")
        self.entries = lib.qwen36_prefix_cache_entries(self._pool)
        self.layers = list(layers)
        for layer in self.layers:
            if isinstance(layer, FullAttentionLayer):
                if layer.capacity != capacity:
                    raise ValueError("layer KV capacity differs from the cache capacity")
                for t in (layer.k_cache, layer.v_cache):
                    self._add(t, KV_BYTES_PER_TOKEN)
            elif isinstance(layer, LinearAttentionLayer):
                layer.normalize_state()
                self._add(layer.conv_state, 0)
                self._add(layer.ssm_state, 0)
            else:
                raise TypeError(f"unsupported layer type {type(layer).__name__}")
        total = ctypes.c_ulonglong(0)
        _lib.call("qwen36_prefix_cache_finalize", self._pool, ctypes.byref(total))
        self.device_bytes = total.value

    def _add(self, t: torch.Tensor, bytes_per_token: int) -> None:
        if not t.is_contiguous():
            raise ValueError("prefix-cache slices must be contiguous")
        nbytes = t.numel() * t.element_size()
        _lib.call("qwen36_prefix_cache_add_slice", self._pool, t.data_ptr(), nbytes,
                  bytes_per_token)

    @staticmethod
    def _tokens(tokens) -> tuple[ctypes.Array, int]:
        vals = [int(x) for x in tokens]
        return (ctypes.c_uint * max(len(vals), 1))(*vals), len(vals)

    def lookup(self, tokens) -> tuple[int, int]:
        arr, n = self._tokens(tokens)
        matched, index = ctypes.c_uint(0), ctypes.c_uint(0)
        _lib.call("qwen36_prefix_cache_lookup", self._pool, arr, n, ctypes.byref(matched),
                  ctypes.byref(index))
        return matched.value, index.value

    def _normalize(self) -> None:
        for layer in self.layers:
            if isinstance(layer, LinearAttentionLayer):
                layer.normalize_state()

    def restore(self, index: int) -> int:
        """Copy entry ``index`` into the live buffers; returns the bytes copied."""
        self._normalize()
        nbytes = ctypes.c_ulonglong(0)
        dev = torch.device("cuda", torch.cuda.current_device())
        _lib.call("qwen36_prefix_cache_restore", self._pool, index, stream_handle(dev),
                  ctypes.byref(nbytes))
        return nbytes.value

    def capture(self, tokens, terminal_hidden: torch.Tensor) -> tuple[int, int]:
        """Store the live state for prompt ``tokens`` with its terminal hidden
        row; returns (entry index, bytes copied)."""
        if terminal_hidden.numel() * terminal_hidden.element_size() != self.terminal_bytes:
            raise ValueError("terminal hidden row has the wrong size")
        self._normalize()
        arr, n = self._tokens(tokens)
        index, nbytes = ctypes.c_uint(0), ctypes.c_ulonglong(0)
        th = terminal_hidden.contiguous()
        _lib.call("qwen36_prefix_cache_capture", self._pool, arr, n, th.data_ptr(),
                  stream_handle(th.device), ctypes.byref(index), ctypes.byref(nbytes))
        self._keep = th   # keep a temporary alive until the copy is queued
        return index.value, nbytes.value

    def terminal_hidden(self, index: int, out: torch.Tensor) -> torch.Tensor:
        _lib.call("qwen36_prefix_cache_copy_terminal", self._pool, index, out.data_ptr(),
                  stream_handle(out.device))
        return out

    def close(self) -> None:
        if getattr(self, "_pool", None):
            self._lib.qwen36_prefix_cache_destroy(self._pool)
            self._pool = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass
