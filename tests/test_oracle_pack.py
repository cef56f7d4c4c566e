"""Pins the packing oracle: the reference's known answers, its per-token-loop oracle on random steps, and
closed-form invariants (CPU only)."""

import random

import numpy as np
import pytest

from oracle import pack as P


def test_known_answer_single_prompt_and_decode():
    """tests/test_model_runner.py:29-52: a 3-token prompt packs positions [0,1,2]; its next decode step [3]."""
    got = P.pack_numpy([0], [3], [[0]], block_size=8, num_logits=[1])
    assert got["positions"].tolist() == [0, 1, 2]
    assert got["logits_indices"].tolist() == [2]
    got = P.pack_numpy([3], [1], [[0]], block_size=8)
    assert got["positions"].tolist() == [3]
    assert got["cu_seqlens_q_host"] == [0, 1] and got["context_lens"].tolist() == [4]


def test_known_answer_one_query_rows_lead_the_batch():
    """tests/test_model_runner.py:179-195: a decoding row after a prompt in scheduler order leads the batch:
    positions [2, 0, 1, 2] and cu_seqlens_q_host [0, 1, 4]."""
    got = P.pack_numpy([0, 2], [3, 1], [[0], [0]], block_size=8, num_logits=[1, 1])
    assert got["positions"].tolist() == [2, 0, 1, 2]
    assert got["cu_seqlens_q_host"] == [0, 1, 4]
    assert got["logits_indices"].tolist() == [3, 0]  # scheduler order: the prompt's last row, then the decode
    assert got["order"].tolist() == [1, 0]
    # closed forms for the rest of the row: both rows end at 3 keys, all in page 0
    assert got["cu_seqlens_k_host"] == [0, 3, 6]
    assert got["slot_mapping"].tolist() == [2, 0, 1, 2]
    assert got["block_tables"].tolist() == [[0], [0]]


def test_known_answer_a_chunk_that_does_not_sample():
    """tests/test_model_runner.py:437-443: a recomputed chunk short of its planned end gathers no logits rows."""
    got = P.pack_numpy([2], [2], [[0]], block_size=8, num_logits=[0])
    assert got["logits_indices"].tolist() == []
    got = P.pack_numpy([8], [1], [[0, 1]], block_size=8, num_logits=[1])
    assert got["logits_indices"].tolist() == [0]


def test_rows_with_drafts_sample_their_last_token_rows():
    """Closed form (model_runner.py:424-430): a row verifying d drafts samples the last d + 1 token rows of its
    chunk, in order; rows keep scheduler order among themselves."""
    cached, new = [5, 0, 9, 4], [3, 7, 3, 2]
    n_log = [3, 1, 0, 2]
    got = P.pack_numpy(cached, new, [[0, 1]] * 4, block_size=8, num_speculative_tokens=2, num_logits=n_log)
    ends = dict(zip(got["order"].tolist(), got["cu_seqlens_q"][1:].tolist()))
    want = []
    for s, n in enumerate(n_log):
        want += list(range(ends[s] - n, ends[s]))
    assert got["logits_indices"].tolist() == want
    # a planted mistake (indices from the chunk's first row) is told apart
    firsts = dict(zip(got["order"].tolist(), got["cu_seqlens_q"][:-1].tolist()))
    assert want != [firsts[s] + j for s, n in enumerate(n_log) for j in range(n)]


def test_dense_slots_pad_rows_without_a_table_with_minus_one():
    """A captured graph's padding rows (model_runner.py:597-602): one slot per token, -1 where the row has no
    block list; the kept entries are the compacted eager slots, in order."""
    cached, new, lists = [4, -1, 9, -1], [1, 1, 1, 1], [[3], [], [5, 6], []]
    eager = P.pack_numpy(cached, new, lists, 8)
    dense = P.pack_numpy(cached, new, lists, 8, dense_slots=True)
    assert dense["slot_mapping"].tolist() == [28, -1, 49, -1]
    assert dense["slot_mapping"][dense["slot_mapping"] >= 0].tolist() == eager["slot_mapping"].tolist()
    assert dense["context_lens"].tolist() == [5, 0, 10, 0]


def test_query_len_is_the_most_common_short_length():
    """model_runner.py:51-63: most common length <= 1 + drafts, the shorter on ties, else 1."""
    assert P.decode_query_len(np.array([1, 1, 5, 3])) == 1
    assert P.decode_query_len(np.array([5, 7])) == 1
    assert P.decode_query_len(np.array([3, 3, 2, 1]), num_speculative_tokens=2) == 3
    assert P.decode_query_len(np.array([3, 2]), num_speculative_tokens=2) == 2


@pytest.mark.parametrize("seed", [0, 1])
def test_vectorised_packing_matches_the_per_token_loops(seed):
    """Twenty random steps of decodes, cold prompts, resumed chunks (every fifth without tables), as the
    reference checks prepare_batch against reference_batch (tests/test_model_runner.py:557-596)."""
    rng = random.Random(seed)
    bs = 8
    for step in range(20):
        cached, new, lists = P.random_rows(rng, bs, with_tables=step % 5 != 0)
        sampling = [rng.random() < 0.7 for _ in new]
        got = P.pack_numpy(cached, new, lists, bs, num_logits=[int(x) for x in sampling])
        want = P.pack_loops(cached, new, lists, bs, sampling=sampling)
        assert got["logits_indices"].tolist() == want["logits_indices"]
        assert got["order"].tolist() == want["order"]
        assert got["positions"].tolist() == want["positions"]
        assert got["slot_mapping"].tolist() == want["slot_mapping"]
        assert got["cu_seqlens_q"].tolist() == want["cu_seqlens_q"] == got["cu_seqlens_q_host"]
        assert got["cu_seqlens_k"].tolist() == want["cu_seqlens_k"] == got["cu_seqlens_k_host"]
        assert got["context_lens"].tolist() == want["context_lens"]
        assert got["max_seqlen_q"] == max(np.diff(want["cu_seqlens_q"]))
        assert got["max_seqlen_k"] == max(want["context_lens"])
        if want["block_tables"] is None:
            assert got["block_tables"] is None
        else:
            assert got["block_tables"].tolist() == want["block_tables"]


def test_invariants_on_a_large_random_step():
    """Each slot lies in its own row's pages at the right offset; cu differences are the lengths."""
    rng = random.Random(7)
    bs = 16
    cached, new, lists = P.random_rows(rng, bs, max_rows=200)
    got = P.pack_numpy(cached, new, lists, bs)
    order = got["order"]
    assert (np.diff(got["cu_seqlens_q"]) == np.asarray(new)[order]).all()
    assert (np.diff(got["cu_seqlens_k"]) == (np.asarray(cached) + np.asarray(new))[order]).all()
    t = 0
    for r, s in enumerate(order):
        for j in range(new[s]):
            pos = cached[s] + j
            assert got["positions"][t] == pos
            slot = got["slot_mapping"][t]
            assert slot // bs == lists[s][pos // bs] and slot % bs == pos % bs
            t += 1


def test_a_planted_off_by_one_is_caught():
    """The loop check discriminates: an oracle with slots one page off disagrees with the loops."""
    rng = random.Random(3)
    cached, new, lists = P.random_rows(rng, 8)
    got = P.pack_numpy(cached, new, lists, 8)
    want = P.pack_loops(cached, new, lists, 8)
    shifted = [lists[i][1:] + [0] for i in range(len(lists))]  # page index off by one
    bad = P.pack_numpy(cached, new, shifted, 8)
    assert got["slot_mapping"].tolist() == want["slot_mapping"]
    assert bad["slot_mapping"].tolist() != want["slot_mapping"]


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_rejected_drafts_move_rows_back_as_the_device_correction_does(seed):
    """Rows whose previous drafts were rejected: the host-side correction (``starts[moved] -= num_rejected``,
    model_runner.py:379-385) that ``pack_numpy(num_back=...)`` applies equals the device-side ``_move_back``
    (:527-551) applied to the uncorrected packing; host lengths stay the uncorrected upper bounds."""
    rng = random.Random(seed)
    bs = 8
    cached, new, lists = P.random_rows(rng, bs)
    k = 3
    new = [n if n > 1 else 1 + k for n in new]  # decode rows verify k drafts
    lists = [[*lst, *range(50_000 + 10 * i, 50_000 + 10 * i + 2)] for i, lst in enumerate(lists)]
    back = [rng.randint(0, min(k, c)) if n == 1 + k else 0 for c, n in zip(cached, new)]
    raw = P.pack_numpy(cached, new, lists, bs, num_speculative_tokens=k)
    got = P.pack_numpy(cached, new, lists, bs, num_speculative_tokens=k, num_back=back)
    want = P.move_back(raw, back, bs)
    for key in ("positions", "slot_mapping", "context_lens", "cu_seqlens_k", "cu_seqlens_q", "order"):
        assert got[key].tolist() == want[key].tolist(), key
    assert got["cu_seqlens_k_host"] == raw["cu_seqlens_k_host"] and got["max_seqlen_k"] == raw["max_seqlen_k"]
    host_fix = P.pack_numpy([c - b for c, b in zip(cached, back)], new, lists, bs, num_speculative_tokens=k)
    assert got["positions"].tolist() == host_fix["positions"].tolist()
    if any(back):  # a planted mistake (the counts taken in batch order instead of scheduler order) is told apart
        wrong = P.move_back(raw, [back[i] for i in raw["order"]], bs)
        assert wrong["positions"].tolist() != want["positions"].tolist() or raw["order"].tolist() == sorted(
            raw["order"].tolist())
