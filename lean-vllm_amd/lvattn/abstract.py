"""The per-layer attention backend interface.

This is the reference's ``AttentionBackend`` contract (``lean_vllm/attention/abstract.py:9-224``): the same
``LayerSpec``, capability flags, ``validate`` reasons, cache shape, and ``forward`` dispatch, restated so that
this package stands alone. In a lean-vLLM checkout the MI355X backend is registered against the reference's
own base class instead (the method set is identical).
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from dataclasses import dataclass

import torch

from .context import Context, split_decodes_and_prefills


@dataclass(frozen=True, slots=True)
class LayerSpec:
    """What one layer asks of a backend (``abstract.py:9-21``)."""

    head_size: int
    num_heads: int
    num_kv_heads: int
    dtype: torch.dtype
    latent_dim: int = 0  # an MLA layer's cached latent width; 0 for a layer caching keys and values

    @property
    def kind(self) -> str:
        return "mla" if self.latent_dim else "decoder"


def write_into(out: torch.Tensor | None, o: torch.Tensor) -> torch.Tensor:
    return o if out is None else out.copy_(o)


class AttentionBackend(ABC):
    supported_dtypes: tuple[torch.dtype, ...] = (torch.float16, torch.bfloat16)
    supported_kinds: tuple[str, ...] = ("decoder", "mla")

    def __init__(self, num_heads: int, head_dim: int, scale: float, num_kv_heads: int):
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads

    @staticmethod
    @abstractmethod
    def get_name() -> str: ...

    @staticmethod
    @abstractmethod
    def is_available() -> bool: ...

    @staticmethod
    def supports_cuda_graph() -> bool:
        return False

    @staticmethod
    def supports_full_cudagraph() -> bool:
        return True

    @staticmethod
    def split_decodes() -> bool:
        return False

    @staticmethod
    def supports_head_size(head_size: int) -> bool:
        return True

    @classmethod
    def validate(cls, spec: LayerSpec) -> list[str]:
        """Reasons this backend cannot serve ``spec`` (empty if it can), worded as ``abstract.py:72-84``."""
        reasons = []
        if spec.dtype not in cls.supported_dtypes:
            reasons.append(f"dtype {spec.dtype} is not one of {list(cls.supported_dtypes)}")
        if not cls.supports_head_size(spec.head_size):
            reasons.append(f"head size {spec.head_size} is not supported")
        if spec.num_heads % spec.num_kv_heads:
            reasons.append(f"{spec.num_heads} query heads do not group over {spec.num_kv_heads} key heads")
        if spec.kind not in cls.supported_kinds:
            reasons.append(f"{spec.kind} layers are not supported")
        return reasons

    @staticmethod
    def supports_mla_decode() -> bool:
        return False

    @staticmethod
    def supports_full_cudagraph_mla_decode() -> bool:
        return True

    @staticmethod
    def mla_block_size() -> int | None:
        return None

    @staticmethod
    def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int, head_dim: int) -> tuple[int, ...]:
        return (num_blocks, block_size, num_kv_heads, head_dim)

    @abstractmethod
    def store_kvcache(self, key, value, k_cache, v_cache, slot_mapping) -> None: ...

    def forward(self, q, k, v, k_cache, v_cache, context: Context, out=None):
        """Decode for a pure-decode step; otherwise prefill over the whole step, or -- for a splitting backend --
        decode over the leading one-query rows and prefill over the rest, each into its view of one output
        (``abstract.py:118-146``)."""
        if not context.is_prefill:
            return self.decode(q, k_cache, v_cache, context, out=out)
        if not self.split_decodes():
            return self.prefill(q, k, v, k_cache, v_cache, context, out=out)
        n, decodes, prefills = split_decodes_and_prefills(context)
        if decodes is None:
            return self.prefill(q, k, v, k_cache, v_cache, prefills, out=out)
        if prefills is None:
            return self.decode(q, k_cache, v_cache, decodes, out=out)
        if out is None:
            out = torch.empty_like(q)
        self.decode(q[:n], k_cache, v_cache, decodes, out=out[:n])
        self.prefill(q[n:], k[n:], v[n:], k_cache, v_cache, prefills, out=out[n:])
        return out

    @abstractmethod
    def prefill(self, q, k, v, k_cache, v_cache, context: Context, out=None): ...

    @abstractmethod
    def decode(self, q, k_cache, v_cache, context: Context, out=None): ...

    def store_latents(self, latent, latent_cache, slot_mapping) -> None:
        raise NotImplementedError(f"the {self.get_name()} backend stores no MLA latents")

    def varlen_with_lse(self, q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, causal,
                        host_cu_seqlens=None):
        raise NotImplementedError(f"the {self.get_name()} backend has no varlen_with_lse, so serves no MLA layer")

    def mla_decode(self, q, latent_cache, v_dim, context: Context):
        raise NotImplementedError(f"the {self.get_name()} backend has no MLA decode")

    @classmethod
    def before_full_graph_replay(cls, context: Context, batch_size: int) -> None:
        """Refresh what a captured full graph reads but cannot compute itself, before it replays."""
