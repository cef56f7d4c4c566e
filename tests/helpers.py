"""Shared builders for the tests: paged steps with known per-row keys, on any device."""

from __future__ import annotations

import torch

from oracle import attention as A


def slots_for(table, bs, start, end):
    return [table[p // bs] * bs + p % bs for p in range(start, end)]


def randn(*shape, gen, device, dtype):
    """N(0, 1) drawn in fp32 on the CPU from ``gen`` and cast: identical on every device."""
    return torch.randn(*shape, generator=gen).to(dtype).to(device)


def paged_step(num_cached, num_new, tables, nblocks, *, heads, kv_heads, dim, bs, device, dtype, seed=0,
               layout="NHD", fill=0.0, token_stride=None):
    """A step whose rows have ``num_cached`` keys already in the cache and ``num_new`` new ones.

    Returns (q_list, k_full, v_full, k_new, v_new, k_cache, v_cache, slot_mapping): the cache holds every prefix
    key; the new keys are NOT yet stored (``slot_mapping`` says where they go). ``token_stride`` (NHD only): the
    caches are views whose token rows lie that many elements apart.
    """
    gen = torch.Generator()
    gen.manual_seed(seed)
    if token_stride is not None:
        assert layout == "NHD" and token_stride >= kv_heads * dim
        k_cache, v_cache = (torch.full((nblocks * bs, token_stride), fill, dtype=dtype, device=device)
                            [:, :kv_heads * dim].view(nblocks, bs, kv_heads, dim) for _ in range(2))
    elif layout == "NHD":
        k_cache = torch.full((nblocks, bs, kv_heads, dim), fill, dtype=dtype, device=device)
        v_cache = torch.full((nblocks, bs, kv_heads, dim), fill, dtype=dtype, device=device)
    else:  # (block, head, token, dim) underneath, seen as (block, token, head, dim)
        k_cache = torch.full((nblocks, kv_heads, bs, dim), fill, dtype=dtype, device=device).transpose(1, 2)
        v_cache = torch.full((nblocks, kv_heads, bs, dim), fill, dtype=dtype, device=device).transpose(1, 2)
    qs, kf, vf, slots = [], [], [], []
    for c, n, t in zip(num_cached, num_new, tables):
        k = randn(c + n, kv_heads, dim, gen=gen, device=device, dtype=dtype)
        v = randn(c + n, kv_heads, dim, gen=gen, device=device, dtype=dtype)
        qs.append(randn(n, heads, dim, gen=gen, device=device, dtype=dtype))
        pre = torch.tensor(slots_for(t, bs, 0, c), dtype=torch.long, device=device)
        if c:
            k_cache[pre // bs, pre % bs] = k[:c]
            v_cache[pre // bs, pre % bs] = v[:c]
        kf.append(k)
        vf.append(v)
        slots += slots_for(t, bs, c, c + n)
    k_new = torch.cat([k[c:] for k, c in zip(kf, num_cached)])
    v_new = torch.cat([v[c:] for v, c in zip(vf, num_cached)])
    slot_mapping = torch.tensor(slots, dtype=torch.int32, device=device)
    return qs, kf, vf, k_new, v_new, k_cache, v_cache, slot_mapping


def context_for(num_cached, num_new, tables, device, is_prefill=True, host=True):
    from lvattn import Context

    totals = [c + n for c, n in zip(num_cached, num_new)]
    cu_q = [0, *torch.tensor(num_new).cumsum(0).tolist()]
    cu_k = [0, *torch.tensor(totals).cumsum(0).tolist()]
    return Context(
        is_prefill=is_prefill,
        cu_seqlens_q=torch.tensor(cu_q, dtype=torch.int32, device=device),
        cu_seqlens_k=torch.tensor(cu_k, dtype=torch.int32, device=device),
        max_seqlen_q=max(num_new),
        max_seqlen_k=max(totals),
        context_lens=torch.tensor(totals, dtype=torch.int32, device=device),
        block_tables=torch.tensor(tables, dtype=torch.int32, device=device),
        cu_seqlens_q_host=cu_q if host else None,
        cu_seqlens_k_host=cu_k if host else None,
    )


def dense_expected(qs, kf, vf, scale):
    """fp32 textbook attention per row (the reference test oracle), on the CPU."""
    return torch.cat([A.dense_attention(q.cpu().float(), k.cpu().float(), v.cpu().float(), scale)
                      for q, k, v in zip(qs, kf, vf)])
