"""The per-step attention metadata every layer reads.

Field names and meanings are the reference's ``Context`` (``lean_vllm/utils/context.py:7-27``), so a step built
by lean-vLLM's ``ModelRunner`` reaches this backend unchanged and a step built by ``lvattn.pack`` reaches
lean-vLLM's other backends unchanged.
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass

import torch


@dataclass(slots=True)
class Context:
    is_prefill: bool = False
    cu_seqlens_q: torch.Tensor | None = None  # int32 [B+1], device
    cu_seqlens_k: torch.Tensor | None = None  # int32 [B+1], device
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None  # int32 [T], -1 = do not store
    context_lens: torch.Tensor | None = None  # int32 [B], keys per row including this step's
    block_tables: torch.Tensor | None = None  # int32 [B, W], -1 padded
    logits_indices: torch.Tensor | None = None
    cu_seqlens_q_host: list[int] | None = None  # host copies, so planning needs no device read
    cu_seqlens_k_host: list[int] | None = None
    context_chunks: list | None = None
    mla_decode_metadata: object | None = None
    decode_splits: dict | None = None  # cached split_decodes_and_prefills results, by query length
    decode_query_len: int = 1
    attn_metadata: dict | None = None  # per-step plans shared by every layer
    piecewise_size: int | None = None
    full_graph_size: int | None = None
    num_actual_tokens: int | None = None


def split_decodes_and_prefills(context, query_len: int = 1):
    """``(n, decode_context, prefill_context)``: the leading ``n`` rows of ``query_len`` queries, sliced off the
    rest. Semantics of ``lean_vllm/utils/context.py:30-78``: with no tables or no host lengths nothing splits;
    the prefill half is re-based to start at zero (its device ``cu_seqlens_k`` by a device-side offset); the
    result is cached on the context per query length."""
    if context.block_tables is None or context.cu_seqlens_q_host is None:
        return 0, None, context
    cache = context.decode_splits if context.decode_splits is not None else {}
    context.decode_splits = cache
    if query_len in cache:
        return cache[query_len]
    cu_q, cu_k = context.cu_seqlens_q_host, context.cu_seqlens_k_host
    rows = len(cu_q) - 1
    n = 0
    while n < rows and cu_q[n + 1] - cu_q[n] == query_len:
        n += 1
    decodes = None
    if n:
        decodes = Context(
            cu_seqlens_q=context.cu_seqlens_q[: n + 1],
            cu_seqlens_k=context.cu_seqlens_k[: n + 1],
            cu_seqlens_q_host=list(cu_q[: n + 1]),
            cu_seqlens_k_host=list(cu_k[: n + 1]),
            max_seqlen_q=query_len,
            max_seqlen_k=max(cu_k[i + 1] - cu_k[i] for i in range(n)),
            context_lens=context.context_lens[:n],
            block_tables=context.block_tables[:n],
        )
    if n == 0:
        prefills = context
    elif n == rows:
        prefills = None
    else:
        sub_q = [x - cu_q[n] for x in cu_q[n:]]
        sub_k = [x - cu_k[n] for x in cu_k[n:]]
        prefills = Context(
            is_prefill=True,
            cu_seqlens_q=context.cu_seqlens_q[n:] - cu_q[n],
            cu_seqlens_k=context.cu_seqlens_k[n:] - context.cu_seqlens_k[n],
            cu_seqlens_q_host=sub_q,
            cu_seqlens_k_host=sub_k,
            max_seqlen_q=max(b - a for a, b in zip(sub_q, sub_q[1:])),
            max_seqlen_k=max(b - a for a, b in zip(sub_k, sub_k[1:])),
            context_lens=context.context_lens[n:],
            block_tables=context.block_tables[n:],
        )
    cache[query_len] = (n, decodes, prefills)
    return cache[query_len]


_CONTEXT = Context()


def get_context():
    return _CONTEXT


@contextmanager
def use_context(context):
    """Make ``context`` current for one pass; the previous one comes back on exit, even on error."""
    global _CONTEXT
    saved = _CONTEXT
    _CONTEXT = context
    try:
        yield context
    finally:
        _CONTEXT = saved


@contextmanager
def set_context(is_prefill: bool, **fields):
    with use_context(Context(is_prefill, **fields)) as context:
        yield context


def reset_context():
    global _CONTEXT
    _CONTEXT = Context()
