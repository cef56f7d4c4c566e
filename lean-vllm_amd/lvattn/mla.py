"""MLA prefill over cached context: the step's cached keys as one chunk, for ``prefill_with_context``.

``MLAAttention._prefill`` (``lean_vllm/layers/attention.py:265-317``) expands the cached latents in chunks of at most
``max_context_chunk`` keys (``context_chunks``, ``:156-187``), attends each chunk unmasked and the new tokens
causally, and merges the partials by log-sum-exp. When a step's cached keys fit one chunk, ``whole_context`` gives
the cache slots of every row's cached keys in row order and their ``cu_seqlens``, so the layer expands them at once
and calls ``MI355XAttention.prefill_with_context`` -- one kernel, no partial outputs, no merges.
"""

from __future__ import annotations

import torch

from .context import Context


def whole_context(context: Context, block_size: int) -> tuple[torch.Tensor, torch.Tensor, int]:
    """``(slots, cu_seqlens_ctx, max_ctx)`` of the step's cached keys: ``slots`` int64 ``[Tc]`` (device) are the
    cache slots of row 0's cached keys in position order, then row 1's, ...; ``cu_seqlens_ctx`` int32 ``[B + 1]``
    (device) their row offsets (a row with no cached keys has none); ``max_ctx`` the longest row's count. A row's
    cached keys are its keys before this step's new tokens: ``(cu_k[i+1] - cu_k[i]) - (cu_q[i+1] - cu_q[i])``.
    Planned once per step and kept in ``context.attn_metadata``, from the host copies of ``cu_seqlens_q/k``."""
    meta = context.attn_metadata
    if meta is None:
        meta = context.attn_metadata = {}
    key = ("mla_whole_context", block_size)
    if key in meta:
        return meta[key]
    cu_q, cu_k = context.cu_seqlens_q_host, context.cu_seqlens_k_host
    if cu_k is None:  # kept drafts are known only on the device: read back (a sync), as the reference does
        assert context.cu_seqlens_k is not None
        cu_k = context.cu_seqlens_k.tolist()
    assert cu_q is not None and context.block_tables is not None
    rows = len(cu_q) - 1
    lens = [(cu_k[i + 1] - cu_k[i]) - (cu_q[i + 1] - cu_q[i]) for i in range(rows)]
    assert all(n >= 0 for n in lens), "a row has fewer keys than queries"
    starts = [0] * (rows + 1)
    for i, n in enumerate(lens):
        starts[i + 1] = starts[i] + n
    tables = context.block_tables
    device = tables.device
    total = starts[-1]
    lens_t = torch.tensor(lens, dtype=torch.int64, device=device)
    row_of = torch.repeat_interleave(torch.arange(rows, device=device), lens_t, output_size=total)
    pos = torch.arange(total, device=device) - torch.tensor(starts[:-1], dtype=torch.int64, device=device)[row_of]
    slots = tables[row_of, pos // block_size].long() * block_size + pos % block_size
    cu_ctx = torch.tensor(starts, dtype=torch.int32, device=device)
    meta[key] = (slots, cu_ctx, max(lens, default=0))
    return meta[key]
