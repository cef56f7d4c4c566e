"""Attention math on the CPU in fp32: the oracle for the paged-attention kernels. TEST INFRASTRUCTURE ONLY.

Three layers of oracle, each checking the next:
1. ``attention_loops``: pure-Python loops with ``math.exp``, for tiny inputs only (brute force).
2. ``dense_scores`` / ``dense_attention``: the reference's textbook test oracle, per head, no paging, no SDPA
   (``tests/test_attention_backends.py:93-116``), with the bottom-right causal mask.
3. ``TorchMath``: the reference PyTorch backend's algorithm (``lean_vllm/attention/torch_backend.py:62-181``):
   page gather with zeroed padding, row padding, bottom-right mask, GQA-folded SDPA, latent-as-one-head MLA.
   This is what the GPU kernels are compared with at test sizes and what the CPU baseline times.

Also ``merge_attention`` (``lean_vllm/attention/merge.py:8-15``) and ``paged_attention_with_lse``
(``tests/test_attention_backends.py:1052-1064``).

Pinned by (``tests/test_oracle_attention.py``): closed forms (one key returns its value; equal keys return the
mean of the values; a zero query averages), brute force against ``attention_loops``, the reference's invariants
(decode == one-token prefill, mixed == separate, bottom-right differs from top-left, NaN/inf in unused slots is
ignored, merge of a split == unsplit, rows with no keys give lse = -inf), and planted mistakes (dropped scale,
top-left mask, ``repeat`` for ``repeat_interleave``) that each check must reject. ``decode_in_row_chunks`` is
pinned against ``TorchMath.decode`` of the whole batch and the dense oracle, with a planted page-count floor and a
planted one-row table shift rejected.
"""

from __future__ import annotations

import math
from types import SimpleNamespace

import torch
import torch.nn.functional as F


# ----------------------------------------------------------------------------------------------------------
# 1. brute force


def attention_loops(q, k, v, scale: float, causal: bool = True):
    """Nested Python loops over one sequence. q [lq][H][D], k/v [lk][Hkv][D] as nested lists or tensors;
    query head h reads key head h // (H // Hkv); query j sees keys 0..lk-lq+j when causal."""
    q, k, v = (x.tolist() if isinstance(x, torch.Tensor) else x for x in (q, k, v))
    lq, lk = len(q), len(k)
    heads, kv_heads = len(q[0]), len(k[0])
    group = heads // kv_heads
    out = []
    for j in range(lq):
        row = []
        for h in range(heads):
            g = h // group
            last = lk - lq + j if causal else lk - 1
            logits = [scale * sum(a * b for a, b in zip(q[j][h], k[i][g])) for i in range(last + 1)]
            top = max(logits)
            weights = [math.exp(x - top) for x in logits]
            total = sum(weights)
            dim = len(v[0][g])
            row.append([sum(weights[i] * v[i][g][d] for i in range(last + 1)) / total for d in range(dim)])
        out.append(row)
    return out


# ----------------------------------------------------------------------------------------------------------
# 2. textbook dense oracle (tests/test_attention_backends.py:93-116)


def dense_scores(q, k, scale: float, compute_dtype=torch.float32, causal: bool = True):
    """Logits one head at a time, ``[H, lq, lk]``; q ``[lq, H, D]``, k ``[lk, Hkv, D]``; bottom-right causal."""
    lq, heads, _ = q.shape
    lk, kv_heads, _ = k.shape
    k = k.repeat_interleave(heads // kv_heads, dim=1)
    scores = torch.empty(heads, lq, lk, dtype=compute_dtype)
    for h in range(heads):
        scores[h] = (q[:, h, :].to(compute_dtype) @ k[:, h, :].to(compute_dtype).T) * scale
        if causal:
            for j in range(lq):
                scores[h, j, lk - lq + j + 1:] = float("-inf")
    return scores


def dense_attention(q, k, v, scale: float, compute_dtype=torch.float32, causal: bool = True):
    """Attention one head at a time; q ``[lq, H, D]``, k ``[lk, Hkv, D]``, v ``[lk, Hkv, Dv]`` -> ``[lq, H, Dv]``."""
    heads = q.size(1)
    v = v.repeat_interleave(heads // v.size(1), dim=1)
    scores = dense_scores(q, k, scale, compute_dtype, causal)
    out = torch.empty(q.size(0), heads, v.size(2), dtype=q.dtype)
    for h in range(heads):
        out[:, h, :] = (scores[h].softmax(dim=-1) @ v[:, h, :].to(compute_dtype)).to(q.dtype)
    return out


def dense_lse(q, k, scale: float, causal: bool = True):
    """Natural log-sum-exp of the logits, ``[lq, H]``."""
    return dense_scores(q, k, scale, causal=causal).logsumexp(-1).T


# ----------------------------------------------------------------------------------------------------------
# 3. TorchAttention's algorithm (lean_vllm/attention/torch_backend.py)


def context(**fields):
    """A per-step context with the reference ``Context`` field names (``lean_vllm/utils/context.py:7-27``)."""
    base = dict(is_prefill=False, cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=0, max_seqlen_k=0,
                slot_mapping=None, context_lens=None, block_tables=None)
    base.update(fields)
    return SimpleNamespace(**base)


class TorchMath:
    """fp32 restatement of ``TorchAttention`` (``torch_backend.py:9-181``). Inputs of any float dtype are
    evaluated in fp32; outputs are fp32."""

    def __init__(self, num_heads: int, head_dim: int, scale: float, num_kv_heads: int):
        self.num_heads, self.head_dim, self.scale, self.num_kv_heads = num_heads, head_dim, scale, num_kv_heads

    # -- helpers (torch_backend.py:121-181)
    @staticmethod
    def pad_rows(x, cu, max_len: int):
        """Packed ``[N, ...]`` -> ``[B, max_len, ...]``; past a row's end are other rows' tokens (masked later)."""
        index = cu[:-1].long().unsqueeze(1) + torch.arange(max_len)
        return x[index.clamp(max=x.size(0) - 1)]

    @staticmethod
    def unpad_rows(x, cu, num_tokens: int):
        tokens = torch.arange(num_tokens, dtype=cu.dtype)
        rows = torch.searchsorted(cu, tokens, right=True) - 1
        return x[rows, tokens - cu[rows]]

    @staticmethod
    def gather_pages(cache, block_tables, seqlen: int, seqlens):
        """Each row's cached tokens ``[B, seqlen, ...]``, with slots past its length overwritten by zero."""
        bs = cache.size(1)
        nblocks = -(-seqlen // bs)
        blocks = block_tables[:, :nblocks].long().clamp(min=0)
        got = cache[blocks].flatten(1, 2)[:, :seqlen].float()
        pad = torch.arange(got.size(1)) >= seqlens.long().unsqueeze(1)
        pad = pad.view(*pad.shape, *([1] * (got.ndim - 2)))
        return got.masked_fill(pad, 0.0)

    @staticmethod
    def key_mask(seqlens_k, max_k: int):
        return (torch.arange(max_k) < seqlens_k.long().unsqueeze(1)).view(-1, 1, 1, max_k)

    @classmethod
    def mask(cls, cu_q, cu_k, max_q: int, max_k: int, causal: bool):
        lens_q = (cu_q[1:] - cu_q[:-1]).long()
        lens_k = (cu_k[1:] - cu_k[:-1]).long()
        m = cls.key_mask(lens_k, max_k)
        if not causal:
            return m
        q_pos = (lens_k - lens_q).view(-1, 1, 1, 1) + torch.arange(max_q).view(-1, 1)
        return m & (torch.arange(max_k) <= q_pos)

    def sdpa(self, q, k, v, mask):
        """GQA fold: the ``g`` query heads sharing a key head become one longer query sequence (h -> h // g)."""
        b, lq, heads, d = q.shape
        g = heads // self.num_kv_heads
        qf = q.reshape(b, lq, self.num_kv_heads, g, d).permute(0, 2, 3, 1, 4).reshape(b, self.num_kv_heads, g * lq, d)
        mf = mask.expand(b, 1, lq, mask.size(-1)).unsqueeze(2).expand(b, 1, g, lq, mask.size(-1))
        mf = mf.reshape(b, 1, g * lq, mask.size(-1))
        o = F.scaled_dot_product_attention(qf.float(), k.transpose(1, 2).float(), v.transpose(1, 2).float(),
                                           attn_mask=mf, scale=self.scale)
        dv = o.size(-1)
        return o.reshape(b, self.num_kv_heads, g, lq, dv).permute(0, 3, 1, 2, 4).reshape(b, lq, heads, dv)

    # -- backend methods
    def prefill(self, q, k, v, k_cache, v_cache, ctx):
        cu_q, cu_k = ctx.cu_seqlens_q, ctx.cu_seqlens_k
        q_pad = self.pad_rows(q.float(), cu_q, ctx.max_seqlen_q)
        if ctx.block_tables is not None:  # every key from the pages (torch_backend.py:67-70)
            lens_k = cu_k[1:] - cu_k[:-1]
            k_pad = self.gather_pages(k_cache, ctx.block_tables, ctx.max_seqlen_k, lens_k)
            v_pad = self.gather_pages(v_cache, ctx.block_tables, ctx.max_seqlen_k, lens_k)
        else:
            k_pad = self.pad_rows(k.float(), cu_k, ctx.max_seqlen_k)
            v_pad = self.pad_rows(v.float(), cu_k, ctx.max_seqlen_k)
        m = self.mask(cu_q, cu_k, ctx.max_seqlen_q, ctx.max_seqlen_k, causal=True)
        return self.unpad_rows(self.sdpa(q_pad, k_pad, v_pad, m), cu_q, q.size(0))

    def decode(self, q, k_cache, v_cache, ctx):
        bt, lens = ctx.block_tables, ctx.context_lens
        max_k = bt.size(1) * k_cache.size(1)  # the table's width: no length is read back (torch_backend.py:98)
        k = self.gather_pages(k_cache, bt, max_k, lens)
        v = self.gather_pages(v_cache, bt, max_k, lens)
        m = self.key_mask(lens, max_k)
        return self.sdpa(q.float().unsqueeze(1), k, v, m).squeeze(1)

    def varlen_with_lse(self, q, k, v, cu_q, cu_k, max_q: int, max_k: int, causal: bool):
        """Unpaged varlen attention and its natural log-sum-exp ``[T, H]`` (``torch_backend.py:78-91``)."""
        g = self.num_heads // self.num_kv_heads
        qp = self.pad_rows(q.float(), cu_q, max_q).transpose(1, 2)
        kp = self.pad_rows(k.float(), cu_k, max_k).repeat_interleave(g, dim=2).transpose(1, 2)
        vp = self.pad_rows(v.float(), cu_k, max_k).repeat_interleave(g, dim=2).transpose(1, 2)
        s = qp @ kp.transpose(-1, -2) * self.scale
        s = s.masked_fill(~self.mask(cu_q, cu_k, max_q, max_k, causal), float("-inf"))
        o = (s.softmax(dim=-1) @ vp).transpose(1, 2)
        lse = s.logsumexp(dim=-1).transpose(1, 2)
        return self.unpad_rows(o, cu_q, q.size(0)), self.unpad_rows(lse, cu_q, q.size(0))

    def mla_decode(self, q, latent_cache, v_dim: int, ctx):
        """Latents read as one key head shared by all heads, values = their first ``v_dim`` entries; each row's
        ``lq`` queries are its last positions, causal (``torch_backend.py:105-119``)."""
        bt, lens = ctx.block_tables, ctx.context_lens
        lq = q.size(0) // lens.size(0)
        max_k = bt.size(1) * latent_cache.size(1)
        lat = self.gather_pages(latent_cache, bt, max_k, lens)  # [B, Lk, D]
        heads = q.size(1)
        kv = lat.unsqueeze(1).expand(-1, heads, -1, -1)
        q_pos = (lens.long() - lq).view(-1, 1, 1, 1) + torch.arange(lq).view(-1, 1)
        m = self.key_mask(lens, max_k) & (torch.arange(max_k) <= q_pos)
        qb = q.float().reshape(-1, lq, heads, q.size(-1)).transpose(1, 2)
        o = F.scaled_dot_product_attention(qb, kv, kv[..., :v_dim], attn_mask=m, scale=self.scale)
        return o.transpose(1, 2).reshape(-1, heads, v_dim)


def decode_in_row_chunks(math_: TorchMath, q, k_cache, v_cache, context_lens, block_tables, rows_per_chunk: int):
    """``TorchMath.decode`` over slices of rows, each gathering only its own table width: the same math with a
    bounded padded gather (the full padded gather of large batches does not fit host memory)."""
    outs = []
    bs = k_cache.size(1)
    for r0 in range(0, q.size(0), rows_per_chunk):
        lens = context_lens[r0:r0 + rows_per_chunk]
        width = -(-int(lens.max()) // bs)
        sub = context(context_lens=lens, block_tables=block_tables[r0:r0 + rows_per_chunk, :width])
        outs.append(math_.decode(q[r0:r0 + rows_per_chunk], k_cache, v_cache, sub))
    return torch.cat(outs)


# ----------------------------------------------------------------------------------------------------------
# merge and the paged LSE oracle


def merge_attention(o_a, lse_a, o_b, lse_b):
    """Attention over two disjoint key sets from each one's output and natural lse (``merge.py:8-15``):
    ``w_b = sigmoid(lse_b - lse_a)``, ``o = lerp(o_a, o_b, w_b)``, ``lse = logaddexp``."""
    w_b = torch.sigmoid(lse_b - lse_a).unsqueeze(-1)
    o = torch.lerp(o_a.float(), o_b.float(), w_b)
    return o, torch.logaddexp(lse_a, lse_b)


def paged_attention_with_lse(q, k_cache, v_cache, n: int, pages, scale: float, causal: bool):
    """One row against its first ``n`` cached keys: ``[lq, H, D]`` and lse ``[H, lq]``
    (``tests/test_attention_backends.py:1052-1064``)."""
    bs = k_cache.size(1)
    pages = torch.as_tensor(pages)[: -(-n // bs)].long()
    k, v = (c[pages].flatten(0, 1)[:n].float() for c in (k_cache, v_cache))
    g = q.size(1) // k.size(1)
    k, v = k.repeat_interleave(g, dim=1), v.repeat_interleave(g, dim=1)
    s = torch.einsum("qhd,khd->hqk", q.float(), k) * scale
    if causal:
        lq = q.size(0)
        seen = torch.arange(n) <= (n - lq + torch.arange(lq)).unsqueeze(1)
        s = s.masked_fill(~seen, float("-inf"))
    return torch.einsum("hqk,khd->qhd", s.softmax(-1), v), s.logsumexp(-1)


def mla_absorbed(q_nope, q_pe, w_uk_t, w_uv, latent_cache, ctx, scale: float):
    """Absorbed MLA decode as ``MLAAttention._decode_latents`` composes it (``lean_vllm/layers/attention.py:319-335``):
    ``q_lat = q_nope @ W_UK_T`` per head, attend latents, then ``o @ W_UV``. Shapes: q_nope ``[B, N, P]``,
    q_pe ``[B, N, R]``, w_uk_t ``[N, P, L]``, w_uv ``[N, L, V]``."""
    q_lat = torch.bmm(q_nope.float().transpose(0, 1), w_uk_t.float()).transpose(0, 1)
    q = torch.cat([q_lat, q_pe.float()], dim=-1)
    o = TorchMath(q.size(1), q.size(2), scale, 1).mla_decode(q, latent_cache, w_uk_t.size(2), ctx)
    return torch.bmm(o.transpose(0, 1), w_uv.float()).transpose(0, 1)
