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


def check(packer, cached, new, lists, bs):
    positions, ctx = packer.pack(cached, new, lists)
    torch.cuda.synchronize()
    want = P.pack_numpy(cached, new, lists, bs)
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


def test_known_answers(cuda):
    """tests/test_model_runner.py:179-195."""
    packer = Packer(cuda, 8)
    positions, ctx = packer.pack([0, 2], [3, 1], [[0], [0]])
    assert positions.tolist() == [2, 0, 1, 2]
    assert ctx["cu_seqlens_q_host"] == [0, 1, 4] and ctx["is_prefill"]
    assert ctx["slot_mapping"].tolist() == [2, 0, 1, 2]


def test_many_rows(cuda):
    rng = random.Random(11)
    packer = Packer(cuda, 16)
    cached, new, lists = P.random_rows(rng, 16, max_rows=4000, pool=400_000)
    check(packer, cached, new, lists, 16)


@pytest.mark.parametrize("name", list(W.WORKLOADS))
def test_config_steps(cuda, name):
    wl = W.WORKLOADS[name]()
    check(Packer(cuda, wl.block_size), wl.num_cached, wl.num_new, wl.block_lists, wl.block_size)
