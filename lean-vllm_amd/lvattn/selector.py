"""Per-layer backend resolution with the reference's rules (``lean_vllm/attention/selector.py:19-39``): an
explicit name, then ``$LEAN_VLLM_ATTENTION_BACKEND``, then the first backend in priority order that is available
and validates. A named backend that cannot serve the layer raises instead of falling back."""

from __future__ import annotations

import os

from .abstract import AttentionBackend, LayerSpec
from .backend import MI355XAttention

# In a lean-vLLM checkout the MI355X backend goes first in BACKENDS, ahead of TorchAttention, which stays last
# and serves whatever nothing else does. This package ships only its own backend.
BACKENDS: tuple[type[AttentionBackend], ...] = (MI355XAttention,)


def _unsupported(backend: type[AttentionBackend], spec: LayerSpec) -> list[str]:
    if not backend.is_available():
        return ["not available on this machine"]
    return backend.validate(spec)


def get_attention_backend(spec: LayerSpec, name: str | None = None,
                          backends: tuple[type[AttentionBackend], ...] = BACKENDS) -> type[AttentionBackend]:
    name = name or os.getenv("LEAN_VLLM_ATTENTION_BACKEND") or None
    if name:
        by_name = {b.get_name(): b for b in backends}
        if name not in by_name:
            raise ValueError(f"unknown attention backend {name!r}, expected one of {sorted(by_name)}")
        reasons = _unsupported(by_name[name], spec)
        if reasons:
            raise RuntimeError(f"attention backend {name!r} was requested but cannot serve {spec}: {'; '.join(reasons)}")
        return by_name[name]
    for backend in backends:
        if not _unsupported(backend, spec):
            return backend
    raise RuntimeError(f"no attention backend serves {spec}")
