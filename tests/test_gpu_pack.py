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
