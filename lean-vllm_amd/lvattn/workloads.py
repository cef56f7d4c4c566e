"""Synthetic continuous-batching steps of the shapes this path is measured on.

Each workload is a step's per-row scheduler state -- ``num_cached``, ``num_new`` and a block list per row, in
scheduler order -- plus the layer shape and the model's number of attention layers (Qwen3-0.6B 28, Qwen3-8B 36,
DeepSeek-V2-Lite 27), every one of which attends the same step. Lengths and block lists come from ``numpy.random.default_rng(seed)``
(identical on every machine); block lists are consecutive slices of a seeded permutation of the block pool, so
pages are scattered. Tensor values are drawn by ``materialize`` with a seeded torch generator on the target
device. Key lengths include the token(s) stored this step (``context_lens = num_cached + num_new``).

- ``qwen3_0_6b_mixed``: 16/8 heads, d128, bs 256, pool 512; chunks 0->512 and 256->384 new, plus 30 decode rows
  with context U[64, 2048].
- ``qwen3_8b_decode``: 32/8 heads, d128, bs 256, pool 12,000; 256 decode rows, context U[512, 8192].
- ``qwen3_8b_mixed``: 32/8 heads, d128, bs 256, pool 24,000; 4 chunks of 1536 new tokens on a cached prefix
  U[0, 6144], plus 2048 decode rows with context U[256, 4096] (8192 tokens).
- ``qwen3_8b_prefill``: the four prompt chunks of ``qwen3_8b_mixed`` alone (a step of prompts; MFMA-bound).
- ``qwen3_8b_long``: 32/8 heads, d128, bs 256, pool 10,000; 16 decode rows, context U[32768, 131072].
- ``qwen3_8b_prefix_chunk``: 32/8 heads, d128, bs 256, pool 1024; one prompt chunk of 1024 new tokens on a cached
  prefix of 30,720 (a step of prompts whose few query tiles each walk a long prefix: MFMA work split over keys).
- ``deepseek_v2_lite_mla``: 16 heads, latent 576 (512 + 64 rope), values 512, bs 64, pool 34,000; 128 decode
  rows, context U[1024, 16384]; values N(0, 0.5); scale 1/sqrt(192).
- ``qwen3_8b_decode_bs16``, ``deepseek_v2_lite_mla_bs16``: the same two decode steps (same lengths) on 16-token
  pages, lean-vLLM's default ``kvcache_block_size`` (``lean_vllm/config.py:46``; MLA layers keep it when the backend
  names no page size, ``:85-89``), over pools of the same bytes (192,000 and 136,000 pages).
- ``deepseek_v2_lite_mla_prefill``: the same layer's prompt chunks as ``MLAAttention._prefill`` runs them
  (``lean_vllm/layers/attention.py:265-317``) on expanded heads (q.k 192, values 128): 4 chunks of 1536 new tokens
  on a cached prefix U[0, 6144]; the new tokens attend the prefix unmasked and each other causally, in one
  ``prefill_with_context`` call. ``deepseek_v2_lite_mla_prefill_two_pass`` is the same step as the reference layer's
  calls: causal ``varlen_with_lse`` over the new tokens, unmasked over the prefix, merged by lse.
"""

from __future__ import annotations

import dataclasses
import functools
import math
from dataclasses import dataclass, field

import numpy as np
import torch


@dataclass
class Workload:
    name: str
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    pool: int
    num_cached: list[int]
    num_new: list[int]
    block_lists: list[list[int]]
    scale: float
    value_std: float = 1.0
    latent_dim: int = 0  # MLA: cached latent width
    v_dim: int = 0  # MLA: value width (leading entries of a latent)
    expanded: tuple = (0, 0)  # MLA prefill: (q.k width, value width) of the expanded heads
    num_layers: int = 1  # attention layers of the model the step belongs to (each attends the same step)
    two_pass: bool = False  # MLA prefill: the reference layer's calls (two varlen passes and a merge), not one call
    notes: dict = field(default_factory=dict)

    @property
    def rows(self) -> int:
        return len(self.num_new)

    @property
    def tokens(self) -> int:
        return int(sum(self.num_new))

    @property
    def context_lens(self) -> np.ndarray:
        return np.asarray(self.num_cached, np.int64) + np.asarray(self.num_new, np.int64)

    @property
    def is_mla(self) -> bool:
        return self.latent_dim > 0

    @property
    def is_mla_prefill(self) -> bool:
        return self.expanded[0] > 0

    def kv_bytes_per_token(self, elem_bytes: int = 2) -> int:
        """Cache bytes one attended key position costs: K and V of every kv head, or one MLA latent."""
        if self.is_mla:
            return self.latent_dim * elem_bytes
        return 2 * self.num_kv_heads * self.head_dim * elem_bytes


def _tables(rng, pool: int, ends, block_size: int) -> list[list[int]]:
    perm = rng.permutation(pool)
    need = [-(-int(e) // block_size) for e in ends]
    if sum(need) > pool:
        raise ValueError(f"pool of {pool} blocks is smaller than the {sum(need)} the step needs")
    out, at = [], 0
    for n in need:
        out.append([int(x) for x in perm[at:at + n]])
        at += n
    return out


def qwen3_0_6b_mixed(seed: int = 0) -> Workload:
    rng = np.random.default_rng(seed)
    dec = rng.integers(64, 2048 + 1, size=30)
    num_cached = [0, 256] + [int(c) - 1 for c in dec]
    num_new = [512, 384] + [1] * 30
    ends = [c + n for c, n in zip(num_cached, num_new)]
    return Workload("qwen3_0_6b_mixed", 16, 8, 128, 256, 512, num_cached, num_new, _tables(rng, 512, ends, 256),
                    1 / math.sqrt(128), num_layers=28)


def qwen3_8b_decode(seed: int = 0, batch: int = 256, block_size: int = 256) -> Workload:
    rng = np.random.default_rng(seed)
    ctx = rng.integers(512, 8192 + 1, size=batch)
    num_cached = [int(c) - 1 for c in ctx]
    num_new = [1] * batch
    pool = 12_000 * 256 // block_size
    name = "qwen3_8b_decode" if block_size == 256 else f"qwen3_8b_decode_bs{block_size}"
    return Workload(name, 32, 8, 128, block_size, pool, num_cached, num_new, _tables(rng, pool, ctx, block_size),
                    1 / math.sqrt(128), num_layers=36)


def qwen3_8b_mixed(seed: int = 0, block_size: int = 256) -> Workload:
    rng = np.random.default_rng(seed)
    prefix = rng.integers(0, 6144 + 1, size=4)
    dec = rng.integers(256, 4096 + 1, size=2048)
    # Scheduler order: the chunks first; packing moves the one-token rows to the front.
    num_cached = [int(p) for p in prefix] + [int(c) - 1 for c in dec]
    num_new = [1536] * 4 + [1] * 2048
    ends = [c + n for c, n in zip(num_cached, num_new)]
    pool = 24_000 * 256 // block_size
    name = "qwen3_8b_mixed" if block_size == 256 else f"qwen3_8b_mixed_bs{block_size}"
    return Workload(name, 32, 8, 128, block_size, pool, num_cached, num_new, _tables(rng, pool, ends, block_size),
                    1 / math.sqrt(128), num_layers=36)


def qwen3_8b_prefill(seed: int = 0, block_size: int = 256) -> Workload:
    """The Qwen3-8B mixed step's four prompt chunks alone (same draws): a step of prompts, MFMA-bound."""
    mixed = qwen3_8b_mixed(seed, block_size)
    rows = [i for i, n in enumerate(mixed.num_new) if n > 1]
    name = "qwen3_8b_prefill" if block_size == 256 else f"qwen3_8b_prefill_bs{block_size}"
    return Workload(name, 32, 8, 128, block_size, mixed.pool, [mixed.num_cached[i] for i in rows],
                    [mixed.num_new[i] for i in rows], [mixed.block_lists[i] for i in rows], 1 / math.sqrt(128),
                    num_layers=36)


def qwen3_8b_prefix_chunk(seed: int = 0, block_size: int = 256) -> Workload:
    """One prompt chunk of 1024 new tokens on a cached prefix of 30,720 (a long prompt's late chunk): 32 query tiles
    per kv head, each walking some 490 key tiles."""
    num_cached, num_new = [30_720], [1024]
    pool = 1024 * 256 // block_size
    rng = np.random.default_rng(seed)
    return Workload("qwen3_8b_prefix_chunk", 32, 8, 128, block_size, pool, num_cached, num_new,
                    _tables(rng, pool, [31_744], block_size), 1 / math.sqrt(128), num_layers=36)


def qwen3_8b_long(seed: int = 0) -> Workload:
    rng = np.random.default_rng(seed)
    ctx = rng.integers(32768, 131072 + 1, size=16)
    num_cached = [int(c) - 1 for c in ctx]
    return Workload("qwen3_8b_long", 32, 8, 128, 256, 10_000, num_cached, [1] * 16,
                    _tables(rng, 10_000, ctx, 256), 1 / math.sqrt(128), num_layers=36)


def deepseek_v2_lite_mla(seed: int = 0, block_size: int = 64) -> Workload:
    rng = np.random.default_rng(seed)
    ctx = rng.integers(1024, 16384 + 1, size=128)
    num_cached = [int(c) - 1 for c in ctx]
    pool = 34_000 * 64 // block_size
    name = "deepseek_v2_lite_mla" if block_size == 64 else f"deepseek_v2_lite_mla_bs{block_size}"
    return Workload(name, 16, 1, 576, block_size, pool, num_cached, [1] * 128, _tables(rng, pool, ctx, block_size),
                    1 / math.sqrt(192), value_std=0.5, latent_dim=576, v_dim=512, num_layers=27)


def deepseek_v2_lite_mla_prefill(seed: int = 0) -> Workload:
    rng = np.random.default_rng(seed)
    prefix = rng.integers(0, 6144 + 1, size=4)
    num_cached = [int(p) for p in prefix]
    num_new = [1536] * 4
    ends = [c + n for c, n in zip(num_cached, num_new)]
    return Workload("deepseek_v2_lite_mla_prefill", 16, 1, 576, 64, 1024, num_cached, num_new,
                    _tables(rng, 1024, ends, 64), 1 / math.sqrt(192), value_std=0.5, latent_dim=576, v_dim=512,
                    expanded=(192, 128), num_layers=27)


WORKLOADS = {
    "qwen3_0_6b_mixed": qwen3_0_6b_mixed,
    "qwen3_8b_decode": qwen3_8b_decode,
    "qwen3_8b_mixed": qwen3_8b_mixed,
    "qwen3_8b_prefill": qwen3_8b_prefill,
    "qwen3_8b_long": qwen3_8b_long,
    "qwen3_8b_prefix_chunk": qwen3_8b_prefix_chunk,
    "deepseek_v2_lite_mla": deepseek_v2_lite_mla,
    "deepseek_v2_lite_mla_prefill": deepseek_v2_lite_mla_prefill,
    "deepseek_v2_lite_mla_prefill_two_pass": lambda seed=0: dataclasses.replace(
        deepseek_v2_lite_mla_prefill(seed), name="deepseek_v2_lite_mla_prefill_two_pass", two_pass=True),
    "qwen3_8b_decode_bs16": lambda seed=0: qwen3_8b_decode(seed, block_size=16),
    "qwen3_8b_mixed_bs16": lambda seed=0: qwen3_8b_mixed(seed, block_size=16),
    "qwen3_8b_prefill_bs16": lambda seed=0: qwen3_8b_prefill(seed, block_size=16),
    "deepseek_v2_lite_mla_bs16": lambda seed=0: deepseek_v2_lite_mla(seed, block_size=16),
}


@dataclass
class Tensors:
    q: torch.Tensor  # [T, Hq, D] (MLA: [T, H, latent])
    k_new: torch.Tensor | None  # [T, Hkv, D] this step's keys (MLA: latents [T, latent])
    v_new: torch.Tensor | None
    k_cache: torch.Tensor  # [pool, bs, Hkv, D] (MLA: [pool, bs, latent])
    v_cache: torch.Tensor | None
    expanded: dict | None = None  # MLA prefill: q, k, v of the new tokens and k, v of the cached prefix


def _randn_into(shape, generator, device, dtype, std: float, chunk: int = 1 << 27, alloc=None):
    """N(0, std) drawn in fp32 (in chunks, so a multi-GB cache needs no multi-GB fp32 temporary), then cast, into
    ``alloc(shape, dtype)`` (default: a new device tensor)."""
    out = alloc(shape, dtype) if alloc is not None else torch.empty(shape, dtype=dtype, device=device)
    flat = out.view(-1)
    for at in range(0, flat.numel(), chunk):
        n = min(chunk, flat.numel() - at)
        flat[at:at + n] = (torch.randn(n, generator=generator, device=device) * std).to(dtype)
    return out


def materialize(wl: Workload, device, dtype=torch.bfloat16, seed: int = 0, alloc=None) -> Tensors:
    """Draw the step's q, new K/V and a whole cache pool of N(0, std) values (the cache is filled everywhere,
    so unwritten pages hold finite values too). ``alloc(shape, dtype)``, if given, provides the tensors' memory."""
    device = torch.device(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    std = wl.value_std
    _randn = functools.partial(_randn_into, alloc=alloc)
    if wl.is_mla_prefill:
        dqk, dv = wl.expanded
        lat = _randn((wl.tokens, wl.latent_dim), gen, device, dtype, std)
        cache = _randn((wl.pool, wl.block_size, wl.latent_dim), gen, device, dtype, std)
        prefix = int(sum(wl.num_cached))
        ex = dict(q=_randn((wl.tokens, wl.num_heads, dqk), gen, device, dtype, 1.0),
                  k=_randn((wl.tokens, wl.num_heads, dqk), gen, device, dtype, 1.0),
                  v=_randn((wl.tokens, wl.num_heads, dv), gen, device, dtype, std),
                  k_ctx=_randn((prefix, wl.num_heads, dqk), gen, device, dtype, 1.0),
                  v_ctx=_randn((prefix, wl.num_heads, dv), gen, device, dtype, std))
        return Tensors(ex["q"], lat, None, cache, None, ex)
    if wl.is_mla:
        q = _randn((wl.tokens, wl.num_heads, wl.latent_dim), gen, device, dtype, std)
        lat = _randn((wl.tokens, wl.latent_dim), gen, device, dtype, std)
        cache = _randn((wl.pool, wl.block_size, wl.latent_dim), gen, device, dtype, std)
        return Tensors(q, lat, None, cache, None)
    q = _randn((wl.tokens, wl.num_heads, wl.head_dim), gen, device, dtype, std)
    k = _randn((wl.tokens, wl.num_kv_heads, wl.head_dim), gen, device, dtype, std)
    v = _randn((wl.tokens, wl.num_kv_heads, wl.head_dim), gen, device, dtype, std)
    shape = (wl.pool, wl.block_size, wl.num_kv_heads, wl.head_dim)
    return Tensors(q, k, v, _randn(shape, gen, device, dtype, std), _randn(shape, gen, device, dtype, std))


def batch_order(wl: Workload) -> np.ndarray:
    """Scheduler row of each batch row: one-token rows first, scheduler order kept within each group."""
    return np.argsort(np.asarray(wl.num_new) != 1, kind="stable")


def algorithmic_bytes(wl: Workload, elem_bytes: int = 2) -> dict:
    """Bytes the step must move at least once, from the drawn lengths: every attended key position's cache
    bytes, q and out, the store of this step's new K/V, and the pack kernel's inputs and outputs."""
    ctx = wl.context_lens
    kv = int(ctx.sum()) * wl.kv_bytes_per_token(elem_bytes)
    if wl.is_mla_prefill:  # every expanded key and value once, q and out
        dqk, dv = wl.expanded
        kv = int(ctx.sum()) * wl.num_heads * (dqk + dv) * elem_bytes
        qo = wl.tokens * wl.num_heads * (dqk + dv) * elem_bytes
        store = 2 * wl.tokens * wl.latent_dim * elem_bytes
    elif wl.is_mla:
        qo = wl.tokens * wl.num_heads * (wl.latent_dim + wl.v_dim) * elem_bytes
        store = 2 * wl.tokens * wl.latent_dim * elem_bytes
    else:
        qo = 2 * wl.tokens * wl.num_heads * wl.head_dim * elem_bytes
        store = 2 * wl.tokens * wl.kv_bytes_per_token(elem_bytes)
    nblocks = sum(len(b) for b in wl.block_lists)
    width = max(len(b) for b in wl.block_lists)
    pack = 4 * (3 * wl.rows + 1 + nblocks) + 4 * (4 * wl.rows + 2) + 12 * wl.tokens + 4 * wl.rows * width
    return dict(kv=kv, qo=qo, store=store, pack=pack, attention=kv + qo, total=kv + qo + store + pack)


def algorithmic_flops(wl: Workload) -> int:
    """4 * heads * D * (keys each query sees), summed over queries (QK and PV, 2 flops per MAC)."""
    total = 0
    for c, n in zip(wl.num_cached, wl.num_new):
        seen = n * c + n * (n + 1) // 2  # query j of the row sees c + j + 1 keys
        total += seen
    if wl.is_mla_prefill:
        d = sum(wl.expanded) // 2
    else:
        d = (wl.latent_dim + wl.v_dim) // 2 if wl.is_mla else wl.head_dim
    return 4 * wl.num_heads * d * total
