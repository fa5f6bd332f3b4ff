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
# Buffers replaced by a larger one stay allocated: a HIP graph captured
# earlier may still hold their addresses, and freeing them would let the
# allocator hand that memory to other tensors which a replay then overwrites.
# Growth is geometric (a power of two, at least twice the outgrown size), so
# the retired buffers of one tag add up to less than its live buffer.
_RETIRED: list[tuple[str, torch.Tensor]] = []


def _grown_size(nbytes: int, old: int) -> int:
    want = max(int(nbytes), 2 * old, 256)
    return 1 << (want - 1).bit_length()


def scratch(tag: str, nbytes: int, device: torch.device) -> torch.Tensor:
    """A reusable uint8 device buffer of at least ``nbytes`` bytes (zeroed
    when first allocated; the kernels write every workspace byte they read, so
    no call depends on what an earlier call left there).  Calls that share a
    tag on one device share the buffer, so they are ordered by the stream they
    run on.  A buffer is never freed once handed out; growing one during
    graph capture is refused (make one eager call of the same size before
    capturing, as warm-up).  Sizes round up to a power of two and at least
    double on growth, so a tag's dead buffers never exceed its live one."""
    if device.index is not None:
        index = device.index
    else:
        index = torch.cuda.current_device() if device.type == "cuda" else 0
    key = (tag, index)
    buf = _SCRATCH.get(key)
    if buf is None or buf.numel() < nbytes:
        if device.type == "cuda" and torch.cuda.is_current_stream_capturing():
            raise RuntimeError(
                f"scratch '{tag}' would grow to {int(nbytes)} bytes during graph capture; "
                "run the call once eagerly with the same sizes before capturing")
        old = 0
        if buf is not None:
            _RETIRED.append((tag, buf))
            old = buf.numel()
        buf = torch.zeros(_grown_size(nbytes, old), dtype=torch.uint8, device=device)
        _SCRATCH[key] = buf
    return buf


def retired_bytes(tag: str | None = None) -> int:
    """Bytes held by outgrown scratch buffers (of one tag, or of all)."""
    return sum(b.numel() for t, b in _RETIRED if tag is None or t == tag)
