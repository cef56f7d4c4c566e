"""The pack kernel against the packing oracle, bit for bit: random steps (as the reference's
test_the_numpy_batch_matches_the_per_token_loops), the reference's known answers, and every config's step."""

import random

import numpy as np
import pytest
import torch

from lvattn import Packer
from lvattn import workloads as W
from oracle import pack as P

pytestmark = pytest.mark.gpu


def check(packer, cached, new, lists, bs, num_logits=None, drafts=0):
    positions, ctx = packer.pack(cached, new, lists, num_speculative_tokens=drafts, num_logits=num_logits)
    torch.cuda.synchronize()
    prefill = bool(np.any(np.asarray(new) > 1))
    want = P.pack_numpy(cached, new, lists, bs, drafts,
                        num_logits=(num_logits if num_logits is not None else [1] * len(new)) if prefill else None)
    if prefill:
        assert ctx["logits_indices"].dtype == torch.int64
        assert ctx["logits_indices"].tolist() == want["logits_indices"].tolist()
    else:
        assert ctx["logits_indices"] is None
    assert ctx["order"].tolist() == want["order"].tolist()
    assert positions.dtype == torch.int64 and positions.tolist() == want["positions"].tolist()
    for key in ("cu_seqlens_q", "cu_seqlens_k", "context_lens", "slot_mapping"):
        assert ctx[key].dtype == torch.int32
        assert ctx[key].tolist() == want[key].tolist(), key
    assert ctx["cu_seqlens_q_host"] == want["cu_seqlens_q_host"]
    assert ctx["cu_seqlens_k_host"] == want["cu_seqlens_k_host"]
    assert (ctx["max_seqlen_q"], ctx["max_seqlen_k"]) == (want["max_seqlen_q"], want["max_seqlen_k"])
    if want["block_tables"] is None:
        assert ctx["block_tables"] is None
    else:
        assert ctx["block_tables"].tolist() == want["block_tables"].tolist()


@pytest.mark.parametrize("seed", [0, 1])
def test_random_steps_match_the_oracle(cuda, seed):
    """Twenty steps through one packer, so each overwrites the last one's buffers; every fifth without tables."""
    rng = random.Random(seed)
    packer = Packer(cuda, 8)
    for step in range(20):
        cached, new, lists = P.random_rows(rng, 8, with_tables=step % 5 != 0)
        check(packer, cached, new, lists, 8)


@pytest.mark.parametrize("seed", [2, 3])
def test_random_steps_with_sampling_and_drafts_match_the_oracle(cuda, seed):
    """Rows that do or do not sample, and decode rows verifying up to 3 drafts (drafts + 1 logits rows each)."""
    rng = random.Random(seed)
    packer = Packer(cuda, 8)
    for _ in range(10):
        cached, new, lists = P.random_rows(rng, 8)
        drafts = rng.randint(0, 3)
        new = [n if n > 1 else 1 + rng.randint(0, drafts) for n in new]
        lists = [lst + [lst[-1]] * 2 if lst else lst for lst in lists]  # room for the drafts' pages
        n_log = [rng.choice([0, 1]) if n > 1 + drafts else rng.choice([0, n]) for n in new]
        check(packer, cached, new, lists, 8, num_logits=n_log, drafts=drafts)


def test_known_answers(cuda):
    """tests/test_model_runner.py:179-195 and :29-52."""
    packer = Packer(cuda, 8)
    positions, ctx = packer.pack([0, 2], [3, 1], [[0], [0]])
    assert positions.tolist() == [2, 0, 1, 2]
    assert ctx["cu_seqlens_q_host"] == [0, 1, 4] and ctx["is_prefill"]
    assert ctx["slot_mapping"].tolist() == [2, 0, 1, 2]
    assert ctx["logits_indices"].tolist() == [3, 0]
    positions, ctx = packer.pack([0], [3], [[0]])
    assert ctx["logits_indices"].tolist() == [2]
    positions, ctx = packer.pack([3], [1], [[0]])
    assert not ctx["is_prefill"] and ctx["logits_indices"] is None


def test_many_rows(cuda):
    rng = random.Random(11)
    packer = Packer(cuda, 16)
    cached, new, lists = P.random_rows(rng, 16, max_rows=4000, pool=400_000)
    check(packer, cached, new, lists, 16)


@pytest.mark.parametrize("name", list(W.WORKLOADS))
def test_config_steps(cuda, name):
    wl = W.WORKLOADS[name]()
    check(Packer(cuda, wl.block_size), wl.num_cached, wl.num_new, wl.block_lists, wl.block_size)


@pytest.mark.parametrize("seed", [4, 5])
def test_rows_moved_back_by_rejected_drafts_match_the_oracle(cuda, seed):
    """Per-row rejected-draft counts handed over on the device (num_back): positions, slots, context lengths and
    cu_seqlens_k follow the corrected starts (model_runner.py:379-385, 527-551); host lengths stay upper bounds."""
    rng = random.Random(seed)
    bs, k = 8, 3
    packer = Packer(cuda, bs)
    for _ in range(5):
        cached, new, lists = P.random_rows(rng, bs)
        new = [n if n > 1 else 1 + k for n in new]
        lists = [lst + [lst[-1]] * 2 if lst else lst for lst in lists]
        back = [rng.randint(0, min(k, c)) if n == 1 + k else 0 for c, n in zip(cached, new)]
        is_prompt = [n != 1 + k for n in new]
        positions, ctx = packer.pack(cached, new, lists, num_speculative_tokens=k, is_prompt=is_prompt,
                                     num_back=torch.tensor(back, dtype=torch.int32, device=cuda))
        torch.cuda.synchronize()
        want = P.pack_numpy(cached, new, lists, bs, k, num_back=back)
        assert positions.tolist() == want["positions"].tolist()
        for key in ("cu_seqlens_q", "cu_seqlens_k", "context_lens", "slot_mapping", "order"):
            assert ctx[key].tolist() == want[key].tolist(), key
        assert ctx["cu_seqlens_k_host"] == want["cu_seqlens_k_host"] and ctx["max_seqlen_k"] == want["max_seqlen_k"]


def test_a_page_past_a_short_block_list_stores_nothing(cuda):
    """Called through the C ABI with a block list shorter than its row (which Packer refuses on the host), the pack
    kernel gives the uncovered tokens slot -1 instead of reading the next row's blocks."""
    from lvattn import _capi

    i32 = dict(dtype=torch.int32, device=cuda)
    cached, new = torch.tensor([14, 0], **i32), torch.tensor([4, 2], **i32)
    indptr, ids = torch.tensor([0, 1, 2], **i32), torch.tensor([5, 9], **i32)  # row 0 needs 3 blocks of 8, has 1
    out = {n: torch.full((8,), -7, **i32) for n in ("order", "cu_q", "cu_k", "slots", "lens", "tables")}
    positions = torch.zeros(6, dtype=torch.int64, device=cuda)
    _capi.call("lv_pack", cached.data_ptr(), new.data_ptr(), indptr.data_ptr(), ids.data_ptr(), 2, 1, 8, 1, 6,
               out["order"].data_ptr(), out["cu_q"].data_ptr(), out["cu_k"].data_ptr(), positions.data_ptr(),
               out["slots"].data_ptr(), out["lens"].data_ptr(), out["tables"].data_ptr(), None, None, None, 0,
               _capi.stream_of(cuda))
    torch.cuda.synchronize()
    assert positions.tolist() == [14, 15, 16, 17, 0, 1]
    assert out["slots"][:6].tolist() == [-1, -1, -1, -1, 72, 73]  # row 0's page 1 and 2 are past its list
