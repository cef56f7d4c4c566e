"""Ragged-batch packing on the CPU: the oracle for the GPU pack kernel. TEST INFRASTRUCTURE ONLY.

Restates the integer part of ``ModelRunner.prepare_batch`` (``lean_vllm/engine/model_runner.py:349-464``) for
the fields the attention path consumes: the decode-first row order, ``cu_seqlens_q/k``, ``positions``,
``slot_mapping``, ``context_lens``, the ``-1``-padded ``block_tables``, the host maxima and ``logits_indices``
(given each row's count of sampled logits rows). Token ids and the sampling and speculative-decoding bookkeeping
that decide those counts are outside the path and are not restated.

Pinned by (``tests/test_oracle_pack.py``):
- known answers from ``tests/test_model_runner.py:29-52`` and ``:179-195`` (positions ``[0,1,2]``/``[3]``,
  decode-first positions ``[2,0,1,2]``, ``cu_seqlens_q_host == [0,1,4]``, ``logits_indices`` ``[2]`` and
  ``[3, 0]``), and ``:437-443`` (a chunk that does not sample gives ``[]``);
- ``pack_loops``, a per-token loop restatement of the reference's own test oracle ``reference_batch``
  (``tests/test_model_runner.py:509-533``) driven by a restatement of ``random_batch`` (``:536-554``), compared
  field by field as ``check_batch`` does (``:571-596``);
- closed-form invariants (``cu`` differences equal the lengths, every slot lies in its row's own pages, a row
  with d drafts samples the last d + 1 token rows of its chunk);
- for rows whose previous drafts were rejected (``num_back``): ``move_back``, a restatement of the reference's
  device-side correction ``ModelRunner._move_back`` (``model_runner.py:527-551``) applied to the uncorrected
  packing, must equal the host-side correction ``starts[moved] -= num_rejected`` (``:379-385``) that
  ``pack_numpy`` applies.
"""

from __future__ import annotations

import numpy as np


def decode_query_len(lens: np.ndarray, num_speculative_tokens: int = 0) -> int:
    """The query length that leads the batch (``model_runner.py:51-63``): the most common length not above
    ``1 + num_speculative_tokens``, shorter on ties, else 1."""
    lens = np.asarray(lens, dtype=np.int64)
    short = lens[lens <= 1 + num_speculative_tokens]
    if short.size == 0:
        return 1
    return int(np.argmax(np.bincount(short)))


def pack_numpy(
    num_cached,
    num_new,
    block_lists: list[list[int]],
    block_size: int,
    num_speculative_tokens: int = 0,
    num_logits=None,
    dense_slots: bool = False,
    num_back=None,
) -> dict:
    """Vectorised restatement of ``prepare_batch``'s packing (``model_runner.py:356-446``, ``:448-462``).

    Inputs are in scheduler order. Returns the batch-order fields plus ``order`` (batch row -> scheduler row).
    ``num_logits`` (scheduler order, optional): logits rows each row samples -- its drafts + 1, or 0 for a row
    that does not sample this step; then ``logits_indices`` follows ``model_runner.py:424-430``.
    ``dense_slots``: one slot per token, -1 for rows without a block list, as a captured graph's padded rows
    carry (``model_runner.py:597-602``), instead of the compacted eager form (``:442-445``).
    ``num_back`` (scheduler order, optional): drafts of the previous step that were rejected, per row; the row's
    tokens start that many positions earlier (``model_runner.py:379-385``). The host maxima and
    ``cu_seqlens_*_host`` keep the uncorrected lengths, upper bounds as in the reference's device-side path.
    """
    num_cached = np.asarray(num_cached, dtype=np.int64)
    num_new = np.asarray(num_new, dtype=np.int64)
    host_ends = None
    if num_back is not None:
        host_ends = (num_cached + num_new)
        num_cached = num_cached - np.asarray(num_back, dtype=np.int64)
    rows = num_new.size
    query_len = decode_query_len(num_new, num_speculative_tokens)
    # Stable: rows whose length equals query_len first, scheduler order kept in each group (:367-374).
    order = np.argsort(num_new != query_len, kind="stable")
    lens, starts = num_new[order], num_cached[order]
    ends = starts + lens
    cu_q = np.concatenate([[0], np.cumsum(lens)])
    cu_k = np.concatenate([[0], np.cumsum(ends)])
    token_rows = np.repeat(np.arange(rows), lens)
    positions = starts[token_rows] + np.arange(int(cu_q[-1])) - cu_q[token_rows]
    tables = [list(block_lists[i]) for i in order]
    block_tables = None
    slot_mapping = np.zeros(0, dtype=np.int32)
    width = max((len(t) for t in tables), default=0)
    if any(tables):
        block_tables = np.full((rows, width), -1, dtype=np.int32)
        for r, t in enumerate(tables):
            block_tables[r, : len(t)] = t
        has = np.array([bool(t) for t in tables])[token_rows]
        pos = positions[has]
        blocks = block_tables[token_rows[has], pos // block_size].astype(np.int64)
        slot_mapping = (blocks * block_size + pos % block_size).astype(np.int32)
        if dense_slots:
            dense = np.full(int(cu_q[-1]), -1, dtype=np.int32)
            dense[has] = slot_mapping
            slot_mapping = dense
    logits_indices = None
    if num_logits is not None:
        # model_runner.py:424-430: sampling rows in scheduler order, each the last num_logits token rows of its
        # chunk (its drafts, then the next token).
        n_all = np.asarray(num_logits, dtype=np.int64)
        row_of = np.empty(rows, dtype=np.int64)
        row_of[order] = np.arange(rows)
        sampling = np.flatnonzero(n_all > 0)
        n = n_all[sampling]
        last_index = cu_q[1:] - 1
        offsets = np.arange(int(n.sum())) - np.repeat(np.cumsum(n) - n, n)
        logits_indices = (np.repeat(last_index[row_of[sampling]] - (n - 1), n) + offsets).astype(np.int64)
    host_k = ends if host_ends is None else host_ends[order]
    return dict(
        logits_indices=logits_indices,
        order=order.astype(np.int32),
        cu_seqlens_q=cu_q.astype(np.int32),
        cu_seqlens_k=cu_k.astype(np.int32),
        positions=positions.astype(np.int64),
        slot_mapping=slot_mapping,
        context_lens=ends.astype(np.int32),
        block_tables=block_tables,
        max_seqlen_q=int(lens.max()) if rows else 0,
        max_seqlen_k=int(host_k.max()) if rows else 0,
        cu_seqlens_q_host=[int(x) for x in cu_q],
        cu_seqlens_k_host=[0, *np.cumsum(host_k).tolist()],
        decode_query_len=query_len,
    )


def move_back(packed: dict, num_back, block_size: int) -> dict:
    """``ModelRunner._move_back`` (``model_runner.py:527-551``) on an uncorrected packing: each moved row's tokens
    shift back by its rejected-draft count; positions, context lengths, ``cu_seqlens_k`` and the slots (looked up
    again in the padded block table) follow. ``num_back`` is in scheduler order; every row has a block list."""
    out = dict(packed)
    order = packed["order"].astype(np.int64)
    back = np.asarray(num_back, dtype=np.int64)[order]  # batch order
    cu_q = packed["cu_seqlens_q"].astype(np.int64)
    token_rows = np.repeat(np.arange(order.size), np.diff(cu_q))
    positions = packed["positions"] - back[token_rows]
    context_lens = packed["context_lens"].astype(np.int64) - back
    out["positions"] = positions
    out["context_lens"] = context_lens.astype(np.int32)
    out["cu_seqlens_k"] = np.concatenate([[0], np.cumsum(context_lens)]).astype(np.int32)
    blocks = packed["block_tables"][token_rows, positions // block_size].astype(np.int64)
    out["slot_mapping"] = (blocks * block_size + positions % block_size).astype(np.int32)
    return out


def pack_loops(num_cached, num_new, block_lists: list[list[int]], block_size: int, sampling=None) -> dict:
    """Per-token loops, restating the reference's test oracle ``reference_batch``
    (``tests/test_model_runner.py:509-533``) and its row order ``decodes_first`` (``:503-506``). ``sampling``
    (scheduler order) marks rows that sample their last token; ``logits_indices`` lists those tokens' rows in
    scheduler order (``:521-527``)."""
    lens = [int(x) for x in num_new]
    query_len = decode_query_len(np.array(lens))
    batch = sorted(range(len(lens)), key=lambda i: lens[i] != query_len)  # sorted() is stable
    out = dict(positions=[], slot_mapping=[], cu_seqlens_q=[0], cu_seqlens_k=[0], context_lens=[], order=batch)
    last_token = {}
    for i in batch:
        start = int(num_cached[i])
        end = start + lens[i]
        out["positions"] += list(range(start, end))
        out["cu_seqlens_q"].append(out["cu_seqlens_q"][-1] + lens[i])
        out["cu_seqlens_k"].append(out["cu_seqlens_k"][-1] + end)
        out["context_lens"].append(end)
        last_token[i] = out["cu_seqlens_q"][-1] - 1
        table = block_lists[i]
        if table:
            out["slot_mapping"] += [table[p // block_size] * block_size + p % block_size for p in range(start, end)]
    tables = [list(block_lists[i]) for i in batch]
    width = max((len(t) for t in tables), default=0)
    out["block_tables"] = [t + [-1] * (width - len(t)) for t in tables] if width else None
    if sampling is not None:
        out["logits_indices"] = [last_token[i] for i in range(len(lens)) if sampling[i]]
    return out


def random_rows(rng, block_size: int, with_tables: bool = True, max_rows: int = 24, pool: int = 10_000):
    """Decodes, cold prompts, resumed chunks and prefix hits in shuffled scheduler order; a restatement of
    ``random_batch`` (``tests/test_model_runner.py:536-554``) that returns the packing inputs only.

    ``rng`` is a ``random.Random``. Returns (num_cached, num_new, block_lists).
    """
    free = iter(rng.sample(range(pool), min(pool, max(2_000, 12 * max_rows))))  # scattered, so a wrong lookup shows
    num_cached, num_new, lists = [], [], []
    for _ in range(rng.randint(1, max_rows)):
        kind = rng.choice(["decode", "prompt", "chunk"])
        prompt = rng.randint(1, 90)
        if kind == "decode":
            cached, new = prompt, 1
        else:
            cached = rng.randrange(prompt) if kind == "chunk" else 0
            new = rng.randint(1, prompt - cached)
        end = cached + new
        table = [next(free) for _ in range(-(-end // block_size))] if with_tables else []
        num_cached.append(cached)
        num_new.append(new)
        lists.append(table)
    return num_cached, num_new, lists
