"""The paged-cache scatter on the CPU: the oracle for the store kernels. TEST INFRASTRUCTURE ONLY.

Restates ``TorchAttention.store_kvcache`` / ``store_latents`` (``lean_vllm/attention/torch_backend.py:34-60``)
with the stride semantics of the Triton kernels they stand beside (``lean_vllm/attention/triton_cache.py:9-55``):
the cache is addressed by (block, offset) through its own strides, so an HND cache seen through a transposed
view takes the same writes, and slot ``-1`` writes nothing.

Pinned by (``tests/test_oracle_store.py``): slot ``-1`` leaves rows untouched
(``tests/test_attention_backends.py:550-564``, ``:439-455``); exact round trip
(``:756-769``); NHD and HND caches end equal (``:573-586``); a pure-Python per-element loop on tiny inputs.
"""

from __future__ import annotations

import numpy as np
import torch


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  slot_mapping) -> None:
    """``k_cache[slot // bs, slot % bs] = key[t]`` (and V) for every ``slot >= 0``; caches are
    ``[num_blocks, block_size, heads, dim]`` views (any strides)."""
    slots = torch.as_tensor(np.asarray(slot_mapping), dtype=torch.long)
    assert slots.numel() == key.size(0)
    keep = slots >= 0
    slots = slots[keep]
    bs = k_cache.size(1)
    blocks, offsets = slots // bs, slots % bs
    k_cache[blocks, offsets] = key[keep]
    v_cache[blocks, offsets] = value[keep]


def store_latents(latent: torch.Tensor, latent_cache: torch.Tensor, slot_mapping) -> None:
    """``latent_cache.view(-1, dim)[slot] = latent[t]`` for every ``slot >= 0``."""
    slots = torch.as_tensor(np.asarray(slot_mapping), dtype=torch.long)
    assert slots.numel() == latent.size(0)
    keep = slots >= 0
    latent_cache.view(-1, latent_cache.size(-1))[slots[keep]] = latent[keep]


def store_loop(key: torch.Tensor, cache: torch.Tensor, slot_mapping) -> None:
    """The same scatter, one element at a time, for tiny inputs (the brute-force check of ``store_kvcache``)."""
    bs = cache.size(1)
    for t, slot in enumerate(list(np.asarray(slot_mapping).tolist())):
        if slot < 0:
            continue
        for h in range(key.size(1)):
            for d in range(key.size(2)):
                cache[slot // bs, slot % bs, h, d] = key[t, h, d]
