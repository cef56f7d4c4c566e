"""MLA absorbed decode on the GPU against the oracle, through the C ABI.

Cases of the reference's check_mla_decode (tests/test_attention_backends.py:378-436): 8 heads, 576-wide latents
whose first 512 entries are the values, scale 0.137, pages of 16 and 64 tokens; mid-page, part-page and full rows;
rows long enough to be split over their latents beside a one-latent row; four queries per row (a row verifying
drafts). The expected output is the textbook dense attention of each row (fp32). Tolerances: fp16 6e-3 (the
reference's), bf16 2e-2 absolute / 1e-2 relative (the path's stated bar). DeepSeek-V2-Lite's full decode step is
checked row by row in test_gpu_fullsize.py.
"""

import math

import pytest
import torch

from helpers import slots_for
from lvattn import Context, MI355XAttention
from lvattn import workloads as W
from oracle import attention as A

pytestmark = pytest.mark.gpu

HEADS, LATENT, VDIM, SCALE = 8, 576, 512, 0.137
TOL = {torch.float16: dict(atol=6e-3, rtol=6e-3), torch.bfloat16: dict(atol=2e-2, rtol=1e-2)}


def check_mla(device, dtype, block_size, context_lens, tables, queries=1, heads=HEADS, seed=0):
    gen = torch.Generator().manual_seed(seed)
    nblocks = max(max(t) for t in tables) + 1
    cache = torch.zeros(nblocks, block_size, LATENT, dtype=dtype)
    latents = [torch.randn(n, LATENT, generator=gen).to(dtype) for n in context_lens]
    for lat, table in zip(latents, tables):
        slots = torch.tensor(slots_for(table, block_size, 0, lat.size(0)), dtype=torch.long)
        cache.view(-1, LATENT)[slots] = lat
    q = torch.randn(len(context_lens) * queries, heads, LATENT, generator=gen).to(dtype)
    ctx = Context(context_lens=torch.tensor(context_lens, dtype=torch.int32, device=device),
                  block_tables=torch.tensor(tables, dtype=torch.int32, device=device))
    out = MI355XAttention(heads, LATENT, SCALE, heads).mla_decode(q.to(device), cache.to(device), VDIM, ctx)
    torch.cuda.synchronize()
    want = torch.cat([
        (A.dense_scores(q[i * queries:(i + 1) * queries], lat.unsqueeze(1), SCALE).softmax(-1)
         @ lat[:, :VDIM].float()).transpose(0, 1)
        for i, lat in enumerate(latents)])
    assert out.shape == (len(context_lens) * queries, heads, VDIM) and out.dtype == dtype
    torch.testing.assert_close(out.float().cpu(), want, **TOL[dtype])


# Pages of 40 latents are not a multiple of 16: the kernel's split schedule instead of its balanced runs.
CASES = [(dtype, bs) for dtype in (torch.float16, torch.bfloat16) for bs in (16, 64)] + [(torch.bfloat16, 40)]
IDS = [f"{'fp16' if d == torch.float16 else 'bf16'}-bs{bs}" for d, bs in CASES]


@pytest.mark.parametrize("dtype, bs", CASES, ids=IDS)
def test_mla_decode(cuda, dtype, bs):
    check_mla(cuda, dtype, bs, [bs + 3, 3, 2 * bs], [[2, 0], [3, -1], [1, 4]])


@pytest.mark.parametrize("dtype, bs", CASES, ids=IDS)
def test_mla_decode_of_long_rows(cuda, dtype, bs):
    pages = torch.randperm(32, generator=torch.Generator().manual_seed(3)).tolist()
    check_mla(cuda, dtype, bs, [21 * bs - 5, 1, 9 * bs + 1],
              [pages[:21], pages[21:22] + [-1] * 20, pages[22:] + [-1] * 11])


@pytest.mark.parametrize("dtype, bs", CASES, ids=IDS)
def test_mla_decode_of_rows_verifying_drafts(cuda, dtype, bs):
    check_mla(cuda, dtype, bs, [bs + 3, 4, 2 * bs], [[2, 0], [3, -1], [1, 4]], queries=4)


@pytest.mark.parametrize("heads", [16, 20, 32])
def test_mla_decode_over_several_head_tiles(cuda, heads):
    """16 heads fill one MFMA tile; 20 and 32 take two, the last one partly empty for 20."""
    check_mla(cuda, torch.bfloat16, 64, [700, 65, 3000], [list(range(0, 11)) + [-1] * 36, [11, 12] + [-1] * 45,
                                                         list(range(13, 60))], heads=heads)


@pytest.mark.parametrize("queries", [1, 2])
def test_mla_decode_of_many_ragged_rows(cuda, queries):
    """64 rows of 0 to 600 latents: with runs of 256 latents most rows are cut over several runs and merged; a
    row without latents gives zeros, a row of `queries` latents lets its first query see one."""
    gen = torch.Generator().manual_seed(7)
    lens = torch.randint(queries, 601, (64,), generator=gen).tolist()
    lens[3], lens[10] = 0, queries
    need = [max(1, -(-n // 64)) for n in lens]
    perm = torch.randperm(sum(need), generator=gen).tolist()
    tables, at = [], 0
    for k in need:
        tables.append(perm[at:at + k] + [-1] * (max(need) - k))
        at += k
    check_mla(cuda, torch.bfloat16, 64, lens, tables, queries=queries, heads=16, seed=7)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_mla_decode_of_more_units_than_the_runs_hold(cuda, dtype):
    """8200 rows of one query and 16 heads: more (row, query, head tile) units than the balanced runs' in-kernel
    scan holds, so the split schedule (one workgroup per row and split, then the split merge) serves a page size
    that is a multiple of 16; rows of 1 to 300 latents, checked against TorchMath.mla_decode slice by slice."""
    gen = torch.Generator().manual_seed(21)
    rows, bs, heads = 8200, 64, 16
    lens = torch.randint(1, 301, (rows,), generator=gen)
    lens[0], lens[1] = 1, 300
    need = (lens + bs - 1) // bs
    width = int(need.max())
    perm = torch.randperm(int(need.sum()), generator=gen)
    bt = torch.full((rows, width), -1, dtype=torch.int32)
    at = 0
    for r in range(rows):
        n = int(need[r])
        bt[r, :n] = perm[at:at + n].to(torch.int32)
        at += n
    cache = (torch.randn(at, bs, LATENT, generator=gen) * 0.5).to(dtype)
    q = torch.randn(rows, heads, LATENT, generator=gen).to(dtype)
    ctx = Context(context_lens=lens.to(torch.int32).to(cuda), block_tables=bt.to(cuda))
    out = MI355XAttention(heads, LATENT, SCALE, heads).mla_decode(q.to(cuda), cache.to(cuda), VDIM, ctx)
    torch.cuda.synchronize()
    math_ = A.TorchMath(heads, LATENT, SCALE, 1)
    for r0 in range(0, rows, 1024):
        sl = slice(r0, min(r0 + 1024, rows))
        sub = A.context(context_lens=lens[sl].to(torch.int32), block_tables=bt[sl])
        want = math_.mla_decode(q[sl], cache, VDIM, sub)
        torch.testing.assert_close(out[sl].float().cpu(), want, **TOL[dtype])


def test_mla_rows_with_no_latents_give_zeros(cuda):
    b = MI355XAttention(16, LATENT, SCALE, 16)
    cache = torch.randn(2, 64, LATENT, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(cuda)
    q = torch.randn(2, 16, LATENT, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(cuda)
    ctx = Context(context_lens=torch.tensor([0, 5], dtype=torch.int32, device=cuda),
                  block_tables=torch.tensor([[0], [1]], dtype=torch.int32, device=cuda))
    out = b.mla_decode(q, cache, VDIM, ctx)
    assert torch.equal(out[0], torch.zeros_like(out[0]))
    want = A.TorchMath(16, LATENT, SCALE, 1).mla_decode(q[1:].cpu(), cache.cpu(), VDIM, A.context(
        context_lens=torch.tensor([5], dtype=torch.int32), block_tables=torch.tensor([[1]], dtype=torch.int32)))
    torch.testing.assert_close(out[1:].float().cpu(), want, **TOL[torch.bfloat16])


def test_mla_decode_replays_in_a_graph(cuda):
    """A captured MLA decode (split latents + merge) replays with new queries and lengths; each replay equals an
    eager call."""
    b = MI355XAttention(16, LATENT, SCALE, 16)
    gen = torch.Generator().manual_seed(8)
    cache = torch.randn(64, 64, LATENT, generator=gen).to(torch.bfloat16).to(cuda)
    lens = [3000, 65, 1]
    tables = torch.arange(3 * 20, dtype=torch.int32, device=cuda).view(3, 20)
    ctx = Context(context_lens=torch.tensor(lens, dtype=torch.int32, device=cuda), block_tables=tables)
    q = torch.randn(3, 16, LATENT, generator=gen).to(torch.bfloat16).to(cuda)
    out = torch.empty(3, 16, VDIM, dtype=torch.bfloat16, device=cuda)
    b.mla_decode(q, cache, VDIM, ctx, out=out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        b.mla_decode(q, cache, VDIM, ctx, out=out)
    for step in range(3):
        q.copy_(torch.randn(q.shape, generator=gen).to(q.dtype))
        ctx.context_lens.copy_(torch.tensor([max(n - 300 * step, 1) for n in lens], dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        eager = b.mla_decode(q, cache, VDIM, ctx)
        torch.cuda.synchronize()
        torch.testing.assert_close(out, eager, atol=0, rtol=0)
