"""Opt-in index checks before any launch (``LVATTN_CHECK=1``): the debug mode of this path.

The kernels trust their index inputs -- slots, block tables, key lengths -- as the reference's kernels do. A
scheduler bug that hands over a slot past the pool, a table entry past the pool, or a key length that its table
does not cover would make a kernel read or write outside the caches. With ``LVATTN_CHECK`` set to anything but
``""`` or ``"0"`` when this module is imported (or when ``refresh()`` reads it again), the backend first copies those
inputs to the host (a synchronising copy: this is a debug mode) and raises ``ValueError`` naming the first bad entry.
Off by default: the checks read back device memory, which a captured graph cannot do.
"""

from __future__ import annotations

import os

import torch


def enabled() -> bool:
    """``LVATTN_CHECK`` as the environment holds it now."""
    return os.environ.get("LVATTN_CHECK", "") not in ("", "0")


ENABLED = enabled()  # read once: the backend tests this flag on every call


def refresh() -> bool:
    """Read ``LVATTN_CHECK`` again (after the environment changed)."""
    global ENABLED
    ENABLED = enabled()
    return ENABLED


def _host(t: torch.Tensor) -> torch.Tensor:
    return t.detach().to("cpu", torch.int64)


def _first(mask: torch.Tensor) -> int:
    return int(mask.nonzero()[0, 0])


def check_slots(slot_mapping: torch.Tensor, num_blocks: int, block_size: int, what: str = "slot_mapping") -> None:
    """Every slot is -1 (skip) or in ``[0, num_blocks * block_size)``."""
    s = _host(slot_mapping).reshape(-1)
    bad = (s < -1) | (s >= num_blocks * block_size)
    if bad.any():
        i = _first(bad)
        raise ValueError(f"{what}[{i}] = {int(s[i])} is outside [-1, {num_blocks * block_size}) "
                         f"({num_blocks} blocks of {block_size})")


def check_tables(block_tables: torch.Tensor, num_blocks: int) -> None:
    """Every table entry is -1 (padding) or a block of the pool, ``[0, num_blocks)``."""
    t = _host(block_tables)
    bad = (t < -1) | (t >= num_blocks)
    if bad.any():
        r, j = (int(x) for x in bad.nonzero()[0])
        raise ValueError(f"block_tables[{r}, {j}] = {int(t[r, j])} is outside [-1, {num_blocks})")


def check_key_lengths(lens: torch.Tensor, block_tables: torch.Tensor, block_size: int, what: str = "context_lens"
                      ) -> None:
    """Every row's key length is in ``[0, width * block_size]`` and each of its first ``ceil(len / block_size)``
    table entries names a block (not -1)."""
    lens = _host(lens).reshape(-1)
    t = _host(block_tables)
    if lens.numel() != t.size(0):
        raise ValueError(f"{what} has {lens.numel()} rows, block_tables {t.size(0)}")
    width = t.size(1)
    bad = (lens < 0) | (lens > width * block_size)
    if bad.any():
        i = _first(bad)
        raise ValueError(f"{what}[{i}] = {int(lens[i])} is outside [0, {width * block_size}] "
                         f"(a table of {width} blocks of {block_size})")
    need = (lens + block_size - 1) // block_size
    missing = (torch.arange(width).unsqueeze(0) < need.unsqueeze(1)) & (t < 0)
    if missing.any():
        r, j = (int(x) for x in missing.nonzero()[0])
        raise ValueError(f"row {r} needs {int(need[r])} blocks for its {int(lens[r])} keys but block_tables[{r}, {j}]"
                         f" is -1")


def check_query_rows(cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor, num_tokens: int) -> None:
    """``cu_seqlens_q/k`` start at 0 and never fall, ``cu_seqlens_q`` ends at the token count, and no row has more
    queries than keys."""
    cq, ck = _host(cu_seqlens_q).reshape(-1), _host(cu_seqlens_k).reshape(-1)
    if cq.numel() != ck.numel() or cq.numel() < 1 or int(cq[0]) != 0 or int(ck[0]) != 0:
        raise ValueError("cu_seqlens_q and cu_seqlens_k must have one entry per row plus one, starting at 0")
    lq, lk = cq[1:] - cq[:-1], ck[1:] - ck[:-1]
    if (lq < 0).any() or (lk < 0).any():
        raise ValueError(f"cu_seqlens fall at row {_first((lq < 0) | (lk < 0))}")
    if int(cq[-1]) != num_tokens:
        raise ValueError(f"cu_seqlens_q ends at {int(cq[-1])}, but there are {num_tokens} query tokens")
    if (lq > lk).any():
        i = _first(lq > lk)
        raise ValueError(f"row {i} has {int(lq[i])} queries but only {int(lk[i])} keys")
