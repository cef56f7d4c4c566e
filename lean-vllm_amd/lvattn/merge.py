"""Attention over two disjoint key sets from each one's output and natural log-sum-exp, on the GPU.

``merge_attention`` / ``merge_attention_`` keep the reference's signatures and semantics
(``lean_vllm/attention/merge.py:8-28``; the in-place form overwrites ``out`` -- or ``o_a`` -- and ``lse_a``):
``M = max(lse_a, lse_b)``, ``w = exp(lse - M)``, ``o = (w_a o_a + w_b o_b) / (w_a + w_b)``, ``lse = M + log(w_a + w_b)``
in fp32, one launch of ``lv_merge_attn_states``. A side whose lse is -inf weighs zero.
"""

from __future__ import annotations

import torch

from . import _capi


def merge_attention_(o_a, lse_a, o_b, lse_b, out=None) -> None:
    """Write the merged output to ``out`` (or ``o_a``) and the merged log-sum-exp to ``lse_a``. o ``[T, H, D]``
    and lse ``[T, H]`` (fp32) with any strides but a unit-stride head dim."""
    tokens, heads, dim = o_a.shape
    out = o_a if out is None else out
    assert o_b.shape == o_a.shape == out.shape and o_a.dtype == o_b.dtype == out.dtype
    assert o_a.stride(-1) == 1 and o_b.stride(-1) == 1 and out.stride(-1) == 1, "the head dim must be contiguous"
    assert lse_a.dtype == lse_b.dtype == torch.float32 and lse_a.shape == lse_b.shape == (tokens, heads)
    _capi.call("lv_merge_attn_states", out.data_ptr(), out.stride(0), out.stride(1), o_a.data_ptr(), o_a.stride(0),
               o_a.stride(1), lse_a.data_ptr(), lse_a.stride(0), lse_a.stride(1), o_b.data_ptr(), o_b.stride(0),
               o_b.stride(1), lse_b.data_ptr(), lse_b.stride(0), lse_b.stride(1), tokens, heads, dim,
               _capi.DTYPES[o_a.dtype], _capi.stream_of(o_a.device))


def merge_attention(o_a, lse_a, o_b, lse_b) -> tuple[torch.Tensor, torch.Tensor]:
    """The merged output and log-sum-exp as new tensors; the inputs are left as they are."""
    out = torch.empty_like(o_a)
    lse = lse_a.clone()
    merge_attention_(o_a, lse, o_b, lse_b, out)
    return out, lse
