"""Pins the store oracle: slot -1 untouched, exact round trip, NHD == HND, and a brute-force loop (CPU only)."""

import torch

from oracle import store as S


def _cache(blocks, bs, heads, dim, dtype=torch.float32, fill=7.0):
    return torch.full((blocks, bs, heads, dim), fill, dtype=dtype), torch.full((blocks, bs, heads, dim), fill, dtype=dtype)


def test_negative_slots_leave_rows_untouched():
    """tests/test_attention_backends.py:550-564."""
    k_cache, v_cache = _cache(2, 16, 2, 64)
    key, value = torch.randn(3, 2, 64), torch.randn(3, 2, 64)
    S.store_kvcache(key, value, k_cache, v_cache, [0, -1, 5])
    flat = k_cache.flatten(0, 1)
    assert torch.equal(flat[0], key[0]) and torch.equal(flat[5], key[2])
    assert (flat[1:5] == 7.0).all() and (flat[6:] == 7.0).all()


def test_bf16_round_trip_is_exact():
    """tests/test_attention_backends.py:756-769."""
    k_cache, v_cache = _cache(2, 16, 2, 64, torch.bfloat16, 0.0)
    key = torch.randn(32, 2, 64).to(torch.bfloat16)
    value = torch.randn(32, 2, 64).to(torch.bfloat16)
    slots = [0 * 16 + i for i in range(16)] + [1 * 16 + i for i in range(16)]
    S.store_kvcache(key, value, k_cache, v_cache, slots)
    assert torch.equal(k_cache.flatten(0, 1)[slots], key) and torch.equal(v_cache.flatten(0, 1)[slots], value)


def test_hnd_and_nhd_caches_end_equal():
    """tests/test_attention_backends.py:573-586: an HND cache seen through its transposed view."""
    nhd = _cache(4, 16, 2, 64, fill=0.0)
    hnd = tuple(torch.zeros(4, 2, 16, 64).transpose(1, 2) for _ in range(2))
    slots = list(range(16, 35)) + [0, 1, 2, 3, 4, -1]
    key, value = torch.randn(len(slots), 2, 64), torch.randn(len(slots), 2, 64)
    for kc, vc in (nhd, hnd):
        S.store_kvcache(key, value, kc, vc, slots)
    assert torch.equal(nhd[0], hnd[0]) and torch.equal(nhd[1], hnd[1])


def test_scatter_matches_the_element_loop():
    k_cache, v_cache = _cache(3, 4, 2, 3)
    loop_cache = k_cache.clone()
    key = torch.randn(5, 2, 3)
    slots = [11, -1, 0, 4, 7]
    S.store_kvcache(key, key, k_cache, v_cache, slots)
    S.store_loop(key, loop_cache, slots)
    assert torch.equal(k_cache, loop_cache)


def test_latents_scatter_by_flat_slot():
    """tests/test_attention_backends.py:439-455."""
    cache = torch.full((2, 64, 576), 7.0)
    latent = torch.randn(3, 576)
    S.store_latents(latent, cache, [0, -1, 64 + 5])
    flat = cache.flatten(0, 1)
    assert torch.equal(flat[0], latent[0]) and torch.equal(flat[69], latent[2])
    untouched = [i for i in range(128) if i not in (0, 69)]
    assert (flat[untouched] == 7.0).all()
