"""MI355X-native (gfx950) attention hot path of the Qwen3.6-35B-A3B engine.

Gated GQA full attention (decode + causal/prefix-extending prefill) and
Gated-DeltaNet linear attention, as hand-written HIP kernels behind the C ABI
of ``libqwen36_attn.so``.  Host code here mirrors the reference's per-layer
call signatures.
"""
from . import _lib  # noqa: F401
from .build import LIB_PATH, build_library  # noqa: F401
