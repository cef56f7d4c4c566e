"""store_kvcache / store_latents on the GPU: bit-exact against the oracle scatter, -1 skipped, HND == NHD, and at
full config sizes by the size-independent property (written rows equal the inputs, every other byte unchanged)."""

import pytest
import torch

from lvattn import MI355XAttention
from lvattn import workloads as W
from oracle import store as S

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("layout", ["NHD", "HND"])
def test_store_matches_the_oracle_bit_for_bit(cuda, dtype, layout):
    heads, dim, bs, blocks = 2, 64, 16, 6
    gen = torch.Generator().manual_seed(0)
    key = torch.randn(40, heads, dim, generator=gen).to(dtype)
    value = torch.randn(40, heads, dim, generator=gen).to(dtype)
    slots = torch.randperm(blocks * bs, generator=gen)[:40].to(torch.int32)
    slots[[3, 17, 39]] = -1
    if layout == "NHD":
        kc = torch.full((blocks, bs, heads, dim), 7.0, dtype=dtype)
    else:
        kc = torch.full((blocks, heads, bs, dim), 7.0, dtype=dtype).transpose(1, 2)
    vc = kc.clone() if layout == "NHD" else kc.transpose(1, 2).clone().transpose(1, 2)
    want_k, want_v = kc.clone(), vc.clone()
    S.store_kvcache(key, value, want_k, want_v, slots)
    dk, dv = kc.to(cuda), vc.to(cuda)
    if layout == "HND":  # keep the transposed storage on the device
        dk = kc.transpose(1, 2).contiguous().to(cuda).transpose(1, 2)
        dv = vc.transpose(1, 2).contiguous().to(cuda).transpose(1, 2)
    MI355XAttention(4, dim, 1.0, heads).store_kvcache(key.to(cuda), value.to(cuda), dk, dv, slots.to(cuda))
    torch.cuda.synchronize()
    assert torch.equal(dk.cpu(), want_k) and torch.equal(dv.cpu(), want_v)


@pytest.mark.parametrize("heads,dim,dtype", [(1, 2, torch.float16), (1, 4, torch.float16), (3, 64, torch.bfloat16),
                                             (16, 128, torch.bfloat16), (5, 24, torch.float32), (3, 7, torch.uint8),
                                             (3, 1, torch.float16)])
@pytest.mark.parametrize("tokens", [1, 2, 3, 5, 7, 41])
def test_store_row_widths_and_token_tails(cuda, heads, dim, dtype, tokens):
    """Rows of one or two pieces (fewer copying threads than a workgroup's four tokens), rows spread over two thread
    shares (16 x 128 bf16 = 4 KB per token), token counts that leave a last workgroup short, and rows whose widths
    allow only 1- or 2-byte pieces (7 one-byte elements per head; one fp16 element per head): bit-exact."""
    bs, blocks = 16, 4
    gen = torch.Generator().manual_seed(tokens * 100 + dim)
    key, value = ((torch.randn(tokens, heads, dim, generator=gen) * 3).to(dtype) if dtype.is_floating_point else
                  torch.randint(0, 256, (tokens, heads, dim), generator=gen).to(dtype) for _ in range(2))
    slots = torch.randperm(blocks * bs, generator=gen)[:tokens].to(torch.int32)
    if tokens > 2:
        slots[tokens // 2] = -1
    kc = torch.full((blocks, bs, heads, dim), 7, dtype=dtype)
    vc = torch.full((blocks, bs, heads, dim), 9 if dtype == torch.uint8 else -7, dtype=dtype)
    want_k, want_v = kc.clone(), vc.clone()
    S.store_kvcache(key, value, want_k, want_v, slots)
    dk, dv = kc.to(cuda), vc.to(cuda)
    MI355XAttention(heads, dim, 1.0, heads).store_kvcache(key.to(cuda), value.to(cuda), dk, dv, slots.to(cuda))
    torch.cuda.synchronize()
    assert torch.equal(dk.cpu(), want_k) and torch.equal(dv.cpu(), want_v)


@pytest.mark.parametrize("dim,dtype", [(576, torch.bfloat16), (4, torch.float16), (1152, torch.bfloat16),
                                       (5, torch.uint8), (1, torch.float16), (2, torch.float16)])
def test_store_latent_widths(cuda, dim, dtype):
    """Latents of 576 (one thread share), 4 (one piece) and 1152 elements (two shares of 128 threads), and rows of
    5, 2 and 4 bytes (1-, 2- and 4-byte pieces)."""
    gen = torch.Generator().manual_seed(dim)
    latent = (torch.randn(9, dim, generator=gen).to(dtype) if dtype.is_floating_point else
              torch.randint(0, 256, (9, dim), generator=gen).to(dtype))
    slots = torch.tensor([5, -1, 0, 63, 17, -1, 40, 2, 33], dtype=torch.int32)
    cache = torch.full((2, 32, dim), 7, dtype=dtype)
    want = cache.clone()
    S.store_latents(latent, want, slots.tolist())
    got = cache.to(cuda)
    MI355XAttention(16, 128, 1.0, 16).store_latents(latent.to(cuda), got, slots.to(cuda))
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), want)


def test_store_latents_skips_negative_slots(cuda):
    """tests/test_attention_backends.py:439-455."""
    b = MI355XAttention(16, 128, 1.0, 16)
    cache = torch.full((2, 64, 576), 7.0, dtype=torch.bfloat16, device=cuda)
    latent = torch.randn(3, 576, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    b.store_latents(latent.to(cuda), cache, torch.tensor([0, -1, 69], dtype=torch.int32, device=cuda))
    want = torch.full((2, 64, 576), 7.0, dtype=torch.bfloat16)
    S.store_latents(latent, want, [0, -1, 69])
    assert torch.equal(cache.cpu(), want)


@pytest.mark.parametrize("name", ["qwen3_0_6b_mixed", "qwen3_8b_decode"])
def test_store_at_config_size(cuda, name):
    """The step's new K/V into the full pool: written rows equal the inputs; the rest of the pool is untouched."""
    wl = W.WORKLOADS[name]()
    t = W.materialize(wl, cuda)
    ends = wl.context_lens
    slots = torch.tensor([wl.block_lists[i][(e - n + j) // wl.block_size] * wl.block_size + (e - n + j) % wl.block_size
                          for i, (e, n) in enumerate(zip(ends, wl.num_new)) for j in range(n)],
                         dtype=torch.int32, device=cuda)
    before_k = t.k_cache.view(-1, wl.num_kv_heads, wl.head_dim).sum(dtype=torch.float64, dim=(1, 2))
    before_v = t.v_cache.view(-1, wl.num_kv_heads, wl.head_dim).sum(dtype=torch.float64, dim=(1, 2))
    MI355XAttention(wl.num_heads, wl.head_dim, wl.scale, wl.num_kv_heads).store_kvcache(
        t.k_new, t.v_new, t.k_cache, t.v_cache, slots)
    torch.cuda.synchronize()
    flat_k = t.k_cache.view(-1, wl.num_kv_heads, wl.head_dim)
    flat_v = t.v_cache.view(-1, wl.num_kv_heads, wl.head_dim)
    assert torch.equal(flat_k[slots.long()], t.k_new) and torch.equal(flat_v[slots.long()], t.v_new)
    after_k = flat_k.sum(dtype=torch.float64, dim=(1, 2))
    after_v = flat_v.sum(dtype=torch.float64, dim=(1, 2))
    other = torch.ones(flat_k.size(0), dtype=torch.bool, device=cuda)
    other[slots.long()] = False
    assert torch.equal(after_k[other], before_k[other]) and torch.equal(after_v[other], before_v[other])


def _snapshot_check(cache_before, cache_after, pages, oracle_write):
    """The touched pages after the GPU store equal the oracle's scatter applied to their snapshot, bit for bit."""
    want = cache_before.clone()
    oracle_write(want)
    assert torch.equal(cache_after, want)


@pytest.mark.parametrize("name", ["qwen3_8b_mixed", "qwen3_0_6b_mixed"])
def test_store_of_a_mixed_step_matches_the_oracle_on_its_pages(cuda, name):
    """A mixed step's new K/V at full size (the Qwen3-8B step's 8,192 tokens: 2048 decode rows and four 1536-token
    chunks, 32 MiB each of K and V into a 24,000-page pool): the slots come from the packing oracle; every page the
    step touches is copied to the host before and after the GPU store, and the after-copy must equal the oracle's
    scatter (TorchAttention.store_kvcache, torch_backend.py:34-48) applied to the before-copy, bit for bit. The rest
    of the pool is checked unchanged by per-row checksums."""
    import numpy as np

    from oracle import pack as P

    wl = W.WORKLOADS[name]()
    t = W.materialize(wl, cuda)
    bs = wl.block_size
    packed = P.pack_numpy(wl.num_cached, wl.num_new, wl.block_lists, bs)
    slots = packed["slot_mapping"].astype(np.int64)
    order = packed["order"]
    # the step's new tokens in batch order (the pack kernel's token order), as the bench hands them over
    k_new, v_new = t.k_new, t.v_new
    pages = np.unique(slots // bs)
    remap = {int(p): i for i, p in enumerate(pages)}
    local = torch.tensor([remap[int(s // bs)] * bs + int(s % bs) for s in slots], dtype=torch.long)
    sel = torch.tensor(pages, dtype=torch.long, device=cuda)
    k_before, v_before = t.k_cache[sel].cpu(), t.v_cache[sel].cpu()
    others = torch.ones(wl.pool, dtype=torch.bool, device=cuda)
    others[sel] = False
    sum_k = t.k_cache[others].view(int(others.sum()), -1).sum(dim=1, dtype=torch.float64)
    sum_v = t.v_cache[others].view(int(others.sum()), -1).sum(dim=1, dtype=torch.float64)
    slot_dev = torch.tensor(slots, dtype=torch.int32, device=cuda)
    MI355XAttention(wl.num_heads, wl.head_dim, wl.scale, wl.num_kv_heads).store_kvcache(
        k_new, v_new, t.k_cache, t.v_cache, slot_dev)
    torch.cuda.synchronize()
    k_host, v_host = k_new.cpu(), v_new.cpu()
    _snapshot_check(k_before, t.k_cache[sel].cpu(), pages, lambda c: S.store_kvcache(k_host, v_host, c, c.clone(),
                                                                                      local.numpy()))
    _snapshot_check(v_before, t.v_cache[sel].cpu(), pages, lambda c: S.store_kvcache(v_host, k_host, c, c.clone(),
                                                                                      local.numpy()))
    assert torch.equal(t.k_cache[others].view(int(others.sum()), -1).sum(dim=1, dtype=torch.float64), sum_k)
    assert torch.equal(t.v_cache[others].view(int(others.sum()), -1).sum(dim=1, dtype=torch.float64), sum_v)
    assert len(order) == wl.rows and slots.size == wl.tokens


def test_store_latents_of_the_deepseek_v2_lite_step(cuda):
    """DeepSeek-V2-Lite's decode step at full size: 128 latents of 576 entries into a 34,000-page pool of 64-latent
    pages, plus a -1 slot; the touched pages after the GPU store equal the oracle's scatter
    (torch_backend.py:50-60) on their snapshot, bit for bit, and the rest of the pool is unchanged."""
    wl = W.deepseek_v2_lite_mla()
    t = W.materialize(wl, cuda)
    bs = wl.block_size
    ends = wl.context_lens
    slots = [wl.block_lists[r][(e - 1) // bs] * bs + (e - 1) % bs for r, e in enumerate(ends)]
    slots[5] = -1  # a padding token stores nothing
    pages = sorted({s // bs for s in slots if s >= 0})
    remap = {p: i for i, p in enumerate(pages)}
    local = [remap[s // bs] * bs + s % bs if s >= 0 else -1 for s in slots]
    sel = torch.tensor(pages, dtype=torch.long, device=cuda)
    before = t.k_cache[sel].cpu()
    others = torch.ones(wl.pool, dtype=torch.bool, device=cuda)
    others[sel] = False
    checksum = t.k_cache[others].view(int(others.sum()), -1).sum(dim=1, dtype=torch.float64)
    MI355XAttention(wl.num_heads, wl.latent_dim, wl.scale, wl.num_heads).store_latents(
        t.k_new, t.k_cache, torch.tensor(slots, dtype=torch.int32, device=cuda))
    torch.cuda.synchronize()
    latent = t.k_new.cpu()
    _snapshot_check(before, t.k_cache[sel].cpu(), pages, lambda c: S.store_latents(latent, c, local))
    assert torch.equal(t.k_cache[others].view(int(others.sum()), -1).sum(dim=1, dtype=torch.float64), checksum)
