"""lvattn: lean-vLLM's continuous-batching attention path, MI355X-native (gfx950 HIP kernels behind a C ABI).

- ``MI355XAttention``: the per-layer attention backend (store_kvcache, decode, prefill, mixed steps).
- ``Packer``: the ragged-batch packing of a step on the GPU.
- ``DecodeGraphs``: full-graph decode steps (pack, store and attention captured per batch size).
- ``merge_attention`` / ``merge_attention_``: the log-sum-exp merge of two partial attentions.
- ``whole_context``: a step's cached keys as one chunk, for MLA prefill in one call (``prefill_with_context``).
- ``Context``, ``LayerSpec``, ``AttentionBackend``, ``get_attention_backend``: the reference's interface.
"""

from .abstract import AttentionBackend, LayerSpec, write_into
from .backend import MI355XAttention
from .merge import merge_attention, merge_attention_
from .context import Context, get_context, reset_context, set_context, split_decodes_and_prefills, use_context
from .pack import Packer, StagingBuffers, decode_query_len
from .graphs import DecodeGraphs
from .mla import whole_context
from .selector import BACKENDS, get_attention_backend

__all__ = [
    "BACKENDS",
    "AttentionBackend",
    "Context",
    "DecodeGraphs",
    "LayerSpec",
    "MI355XAttention",
    "Packer",
    "StagingBuffers",
    "decode_query_len",
    "get_attention_backend",
    "get_context",
    "merge_attention",
    "merge_attention_",
    "reset_context",
    "set_context",
    "split_decodes_and_prefills",
    "use_context",
    "whole_context",
    "write_into",
]
