"""Full-graph decode steps (pack, store and attention captured per batch size) against the oracle, as a
ModelRunner replays them (lean_vllm/engine/model_runner.py:585-607): fewer rows than the graph holds (its
padding rows must store and attend nothing), one query per row and rows verifying drafts, several replays of one
graph with new lengths and tables. The cache after each replay must equal the oracle's store bit for bit, over
the whole pool; attention within bf16 2e-2 / 1e-2 of the fp32 dense oracle."""

import math
import random

import pytest
import torch

from helpers import randn, slots_for
from lvattn import DecodeGraphs, MI355XAttention
from oracle import attention as A

pytestmark = pytest.mark.gpu

H, HKV, SCALE, BS, DIM = 8, 2, 0.137, 16, 128
TOL = dict(atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("query_len", [1, 3], ids=["decode", "drafts"])
def test_replayed_steps_match_the_oracle(cuda, query_len):
    dtype = torch.bfloat16
    backend = MI355XAttention(H, DIM, SCALE, HKV)
    nblocks, max_blocks = 64, 6
    gen = torch.Generator().manual_seed(0)
    k_cache = randn(nblocks, BS, HKV, DIM, gen=gen, device=cuda, dtype=dtype)
    v_cache = randn(nblocks, BS, HKV, DIM, gen=gen, device=cuda, dtype=dtype)
    graphs = DecodeGraphs(backend, k_cache, v_cache, [4, 8], max_blocks, query_len)
    graphs.capture()
    rng = random.Random(query_len)
    for rows in (3, 8, 5, 1, 4):
        pages = rng.sample(range(nblocks), rows * max_blocks)
        cached = [rng.randint(0, max_blocks * BS - query_len) for _ in range(rows)]
        cached[0] = 0  # a row whose first keys are this step's
        tables = [pages[i * max_blocks:(i + 1) * max_blocks][:math.ceil((c + query_len) / BS)]
                  for i, c in enumerate(cached)]
        t = rows * query_len
        q = randn(t, H, DIM, gen=gen, device=cuda, dtype=dtype)
        k = randn(t, HKV, DIM, gen=gen, device=cuda, dtype=dtype)
        v = randn(t, HKV, DIM, gen=gen, device=cuda, dtype=dtype)
        want_k, want_v = k_cache.cpu().clone(), v_cache.cpu().clone()
        out = graphs.replay(cached, tables, q, k, v).clone()
        torch.cuda.synchronize()
        for i, (c, table) in enumerate(zip(cached, tables)):
            s = torch.tensor(slots_for(table, BS, c, c + query_len))
            want_k[s // BS, s % BS] = k[i * query_len:(i + 1) * query_len].cpu()
            want_v[s // BS, s % BS] = v[i * query_len:(i + 1) * query_len].cpu()
        assert torch.equal(k_cache.cpu(), want_k) and torch.equal(v_cache.cpu(), want_v), rows
        want = []
        for i, (c, table) in enumerate(zip(cached, tables)):
            s = torch.tensor(slots_for(table, BS, 0, c + query_len))
            keys, vals = want_k[s // BS, s % BS].float(), want_v[s // BS, s % BS].float()
            want.append(A.dense_attention(q[i * query_len:(i + 1) * query_len].cpu().float(), keys, vals, SCALE))
        torch.testing.assert_close(out.float().cpu(), torch.cat(want), **TOL)


def test_a_step_larger_than_every_graph_is_refused(cuda):
    backend = MI355XAttention(H, DIM, SCALE, HKV)
    cache = torch.zeros(8, BS, HKV, DIM, dtype=torch.bfloat16, device=cuda)
    graphs = DecodeGraphs(backend, cache, cache.clone(), [2], 2)
    graphs.capture()
    q = torch.zeros(3, H, DIM, dtype=torch.bfloat16, device=cuda)
    kv = torch.zeros(3, HKV, DIM, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(ValueError, match="no captured graph"):
        graphs.replay([1, 1, 1], [[0], [1], [2]], q, kv, kv)
