"""Tensor plumbing shared by the host-side ops: pointer/stream extraction,
shape and dtype checks, and per-device scratch buffers."""
from __future__ import annotations

import torch


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require(t: torch.Tensor, name: str, dtype: torch.dtype, shape=None,
            contiguous: bool = True) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor (got {t.device})")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype} (got {t.dtype})")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)} (got {tuple(t.shape)})")
    if contiguous and not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


_SCRATCH: dict[tuple[str, int], torch.Tensor] = {}


def scratch(tag: str, nbytes: int, device: torch.device) -> torch.Tensor:
    """A reusable uint8 device buffer of at least ``nbytes`` bytes (zeroed
    when first allocated; the kernels write every workspace byte they read, so
    no call depends on what an earlier call left there).  Calls that share a
    tag on one device share the buffer, so they are ordered by the stream they
    run on."""
    key = (tag, device.index if device.index is not None else torch.cuda.current_device())
    buf = _SCRATCH.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device=device)
        _SCRATCH[key] = buf
    return buf
