"""The HIP backend against the oracle on the reference tests' cases (tests/test_attention_backends.py), through
the C ABI. Shapes: 8 query heads over 2 key heads, head dim 64 and 128, scale 0.137, 16-token pages.

Tolerances: fp16 6e-3 against fp32 (the reference's); bf16 2e-2 absolute / 1e-2 relative against an fp32
evaluation of the same math (the path's stated bar)."""

import math

import pytest
import torch

from helpers import context_for, dense_expected, paged_step, randn, slots_for
from lvattn import Context, MI355XAttention
from oracle import attention as A

pytestmark = pytest.mark.gpu

H, HKV, SCALE, BS = 8, 2, 0.137, 16
TOL = {torch.float16: dict(atol=6e-3, rtol=6e-3), torch.bfloat16: dict(atol=2e-2, rtol=1e-2)}


@pytest.fixture(params=[(torch.float16, 64), (torch.bfloat16, 64), (torch.bfloat16, 128)],
                ids=["fp16-d64", "bf16-d64", "bf16-d128"])
def case(request, cuda):
    dtype, dim = request.param
    return MI355XAttention(H, dim, SCALE, HKV), dtype, dim, cuda


def check(out, want, dtype):
    torch.testing.assert_close(out.float().cpu(), want.float(), **TOL[dtype])


def run_step(backend, dtype, dim, device, num_cached, num_new, tables, nblocks, layout="NHD", host=True):
    qs, kf, vf, kn, vn, kc, vc, slots = paged_step(num_cached, num_new, tables, nblocks, heads=H, kv_heads=HKV,
                                                   dim=dim, bs=BS, device=device, dtype=dtype, layout=layout)
    backend.store_kvcache(kn, vn, kc, vc, slots)
    ctx = context_for(num_cached, num_new, tables, device, host=host)
    out = backend.forward(torch.cat(qs), kn, vn, kc, vc, ctx)
    torch.cuda.synchronize()
    return out, dense_expected(qs, kf, vf, SCALE), (qs, kf, vf, kc, vc, ctx)


@pytest.mark.parametrize("bs", [16, 32, 48, 64, 256])
def test_prefill_through_the_lds_ring(case, bs):
    """Prompt tiles stream through the LDS ring for pages of a multiple of 64 keys (one page per tile) and of 16
    or 32 keys (four or two pages per tile, each lane loading from its key's page); 48-key pages take the register
    path. Prefixes of several tiles, tails that end mid-tile and mid-page, a decode row beside the chunks, pages
    scattered over the pool, and NaN in every unused cache slot (a tile's keys past the row's end must never bring
    one in)."""
    b, dtype, dim, dev = case
    cached, new = [3 * 64 + 5, 0, 70, bs - 1], [77, 130, 1, 9]
    need = [-(-(c + n) // bs) for c, n in zip(cached, new)]
    perm = torch.randperm(sum(need) + 3, generator=torch.Generator().manual_seed(bs)).tolist()
    width = max(need)
    tables, at = [], 0
    for k in need:
        tables.append(perm[at:at + k] + [-1] * (width - k))
        at += k
    qs, kf, vf, kn, vn, kc, vc, slots = paged_step(cached, new, tables, sum(need) + 3, heads=H, kv_heads=HKV,
                                                   dim=dim, bs=bs, device=dev, dtype=dtype, fill=float("nan"))
    b.store_kvcache(kn, vn, kc, vc, slots)
    out = b.forward(torch.cat(qs), kn, vn, kc, vc, context_for(cached, new, tables, dev))
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    check(out, dense_expected(qs, kf, vf, SCALE), dtype)


def test_prefill_of_a_cold_batch_with_pages(case):
    b, dtype, dim, dev = case
    out, want, _ = run_step(b, dtype, dim, dev, [0, 0], [5, BS + 3], [[0, 1, -1], [2, 3, 4]], 6)
    check(out, want, dtype)


def test_prefill_with_prefix_cache(case):
    b, dtype, dim, dev = case
    out, want, _ = run_step(b, dtype, dim, dev, [2 * BS + 2, 0], [6, 5],
                            [[0, 1, 2, 3, 4, 5], [6, 7, -1, -1, -1, -1]], 8)
    check(out, want, dtype)


def test_mixed_batch_of_chunks_and_decodes(case):
    b, dtype, dim, dev = case
    out, want, _ = run_step(b, dtype, dim, dev, [2 * BS + 5, BS + 1, 0], [1, 7, 4],
                            [[0, 1, 2], [3, 4, -1], [5, -1, -1]], 6)
    check(out, want, dtype)


@pytest.mark.parametrize("bs", [16, 32, 64])
@pytest.mark.parametrize("poison", [None, float("nan")], ids=["clean", "nan-slots"])
def test_both_launch_schedules_give_the_same_step(case, bs, poison, monkeypatch):
    """A mixed step (chunks on cached prefixes, decode rows, a cold prompt) under the serial schedule (prompt
    tiles on the whole GPU, then the decode rows) and the overlapped one (prompt tiles beside the decode rows):
    both match the oracle and each other bit for bit, since every item computes the same values either way (the
    decode items beside prompt tiles take their score maxima by IEEE maximum, which agrees with fmaxf on scores).
    With NaN in every unused cache slot, no NaN may reach a score under either schedule."""
    from lvattn import backend as B

    b, dtype, dim, dev = case
    cached, new = [2 * bs + 5, 0, 3 * bs, bs - 1, 7], [9, 70, 1, 1, 1]
    width = max(-(-(c + n) // bs) for c, n in zip(cached, new))
    tables, at = [], 0
    for c, n in zip(cached, new):
        k = -(-(c + n) // bs)
        tables.append(list(range(at, at + k)) + [-1] * (width - k))
        at += k
    fill = {} if poison is None else {"fill": poison}
    qs, kf, vf, kn, vn, kc, vc, slots = paged_step(cached, new, tables, at + 1, heads=H, kv_heads=HKV, dim=dim, bs=bs,
                                                   device=dev, dtype=dtype, **fill)
    b.store_kvcache(kn, vn, kc, vc, slots)
    want = dense_expected(qs, kf, vf, SCALE)
    outs = {}
    # serial; overlapped on the default share of the CUs; overlapped on as many as the library allows
    for name, sched, wgs in (("serial", B.SCHEDULE_SERIAL, 0), ("overlap", B.SCHEDULE_OVERLAP, 0),
                             ("overlap-wide", B.SCHEDULE_OVERLAP, 10_000)):
        monkeypatch.setattr(b, "_schedule", lambda context, elem_bytes, s=sched: s)
        monkeypatch.setattr(b, "_prompt_workgroups", lambda context, elem_bytes, n=wgs: n)
        out = b.forward(torch.cat(qs), kn, vn, kc, vc, context_for(cached, new, tables, dev))
        torch.cuda.synchronize()
        assert torch.isfinite(out).all()
        check(out, want, dtype)
        outs[name] = out
    assert torch.equal(outs["serial"], outs["overlap"])
    assert torch.equal(outs["serial"], outs["overlap-wide"])


def test_decode(case):
    b, dtype, dim, dev = case
    lens = [BS + 3, 3, 4 * BS]
    tables = [[0, 1, 2, 3], [4, 5, -1, -1], [6, 7, 8, 9]]
    qs, kf, vf, kn, vn, kc, vc, slots = paged_step([n - 1 for n in lens], [1, 1, 1], tables, 10, heads=H,
                                                   kv_heads=HKV, dim=dim, bs=BS, device=dev, dtype=dtype)
    b.store_kvcache(kn, vn, kc, vc, slots)
    ctx = Context(is_prefill=False, context_lens=torch.tensor(lens, dtype=torch.int32, device=dev),
                  block_tables=torch.tensor(tables, dtype=torch.int32, device=dev))
    out = b.forward(torch.cat(qs), kn, vn, kc, vc, ctx)
    check(out, dense_expected(qs, kf, vf, SCALE), dtype)


def test_decode_matches_equivalent_prefill(case):
    b, dtype, dim, dev = case
    n = 2 * BS + 1
    qs, kf, vf, kn, vn, kc, vc, slots = paged_step([n - 1], [1], [[0, 1, 2]], 3, heads=H, kv_heads=HKV, dim=dim,
                                                   bs=BS, device=dev, dtype=dtype)
    b.store_kvcache(kn, vn, kc, vc, slots)
    bt = torch.tensor([[0, 1, 2]], dtype=torch.int32, device=dev)
    dec = b.decode(qs[0], kc, vc, Context(context_lens=torch.tensor([n], dtype=torch.int32, device=dev), block_tables=bt))
    pre = b.prefill(qs[0], kn, vn, kc, vc, context_for([n - 1], [1], [[0, 1, 2]], dev))
    torch.testing.assert_close(dec, pre, **TOL[dtype])


def test_mixed_batch_matches_running_the_rows_separately(case):
    b, dtype, dim, dev = case
    num_cached, num_new = [BS + 1, 3 * BS], [6, 1]  # a chunk, then a decode row
    tables = [[0, 1, -1, -1], [2, 3, 4, 5]]
    out, _, (qs, kf, vf, kc, vc, ctx) = run_step(b, dtype, dim, dev, num_cached, num_new, tables, 6)
    chunk = b.prefill(qs[0], None, None, kc, vc, context_for([num_cached[0]], [6], [tables[0]], dev))
    dec = b.decode(qs[1], kc, vc, Context(context_lens=torch.tensor([3 * BS + 1], dtype=torch.int32, device=dev),
                                          block_tables=torch.tensor([tables[1]], dtype=torch.int32, device=dev)))
    torch.testing.assert_close(out, torch.cat([chunk, dec]), **TOL[dtype])


def test_top_left_causal_alignment_would_be_wrong(case):
    b, dtype, dim, dev = case
    lq, lk = 4, 2 * BS + 2
    out, want, (qs, kf, vf, *_ ) = run_step(b, dtype, dim, dev, [lk - lq], [lq], [[0, 1, 2]], 3)
    check(out, want, dtype)
    q, k, v = qs[0].float().cpu(), kf[0].float().cpu(), vf[0].float().cpu()
    top_left = torch.nn.functional.scaled_dot_product_attention(
        q.transpose(0, 1), k.repeat_interleave(H // HKV, 1).transpose(0, 1),
        v.repeat_interleave(H // HKV, 1).transpose(0, 1), is_causal=True, scale=SCALE).transpose(0, 1)
    assert not torch.allclose(out.float().cpu(), top_left, atol=5 * TOL[dtype]["atol"])


def test_an_hnd_cache_stores_and_attends_as_an_nhd_one(case):
    b, dtype, dim, dev = case
    args = ([BS + 3 - 1, 4], [1, 1], [[0, 3], [1, -1]], 4)
    nhd, _, _ = run_step(b, dtype, dim, dev, *args, layout="NHD")
    hnd, _, _ = run_step(b, dtype, dim, dev, *args, layout="HND")
    torch.testing.assert_close(hnd, nhd, atol=0, rtol=0)


# Token rows 2^23 - 8 elements (16 MiB) apart: a 64-key tile spans just under 2^30 bytes, the largest token stride
# the library accepts.
WIDE_STRIDE = (1 << 23) - 8


@pytest.mark.parametrize("bs", [16, 64])
def test_token_rows_at_the_largest_accepted_stride(cuda, bs):
    """Caches whose token rows lie 16 MiB apart: the prompt tiles' 24-bit row offsets and the decode tiles' 32-bit
    ones reach their largest values. A chunk on a prefix beside two decode rows gives the same bits as with packed
    caches and matches the dense oracle; pages of 16 keys take the swizzled stage, pages of 64 the padded one."""
    dtype, dim = torch.bfloat16, 128
    b = MI355XAttention(H, dim, SCALE, HKV)
    num_cached, num_new = [100, 70, 5], [40, 1, 1]
    per = [-(-(c + n) // bs) for c, n in zip(num_cached, num_new)]
    starts = [sum(per[:i]) for i in range(len(per))]
    tables = [list(range(s0, s0 + k)) + [-1] * (max(per) - k) for s0, k in zip(starts, per)]
    outs = []
    for stride in (None, WIDE_STRIDE):
        qs, kf, vf, kn, vn, kc, vc, slots = paged_step(num_cached, num_new, tables, sum(per), heads=H, kv_heads=HKV,
                                                       dim=dim, bs=bs, device=cuda, dtype=dtype, token_stride=stride)
        assert stride is None or kc.stride(1) == vc.stride(1) == stride
        b.store_kvcache(kn, vn, kc, vc, slots)
        outs.append(b.forward(torch.cat(qs), kn, vn, kc, vc, context_for(num_cached, num_new, tables, cuda)))
        torch.cuda.synchronize()
        del kc, vc
    assert torch.equal(outs[0], outs[1])
    check(outs[1], dense_expected(qs, kf, vf, SCALE), dtype)


def test_low_precision_no_worse_than_naive(cuda):
    """tests/test_attention_backends.py:705-753: bf16 error against fp32 at most twice naive bf16 arithmetic's."""
    b = MI355XAttention(H, 64, SCALE, HKV)
    num_cached, num_new = 2 * BS + 2, 6
    out, _, (qs, kf, vf, *_) = run_step(b, torch.bfloat16, 64, cuda, [num_cached], [num_new], [[0, 1, 2, 3]], 4)
    q, k, v = qs[0].cpu(), kf[0].cpu(), vf[0].cpu()
    ref = A.dense_attention(q.float(), k.float(), v.float(), SCALE)
    naive = A.dense_attention(q, k, v, SCALE, compute_dtype=torch.bfloat16).float()
    backend_err = (out.float().cpu() - ref).abs().max().item()
    naive_err = (naive - ref).abs().max().item()
    assert backend_err <= 2 * naive_err + 1e-6, (backend_err, naive_err)


@pytest.mark.parametrize("poison", [float("nan"), float("inf")], ids=["nan", "inf"])
def test_unwritten_cache_slots_are_ignored(cuda, poison):
    """tests/test_attention_backends.py:142-168, at kernel shapes: poison everywhere outside the rows' keys."""
    b = MI355XAttention(H, 64, SCALE, HKV)
    for num_cached, num_new, tables in (([20, 3], [1, 1], [[1, 2], [0, -1]]), ([20, 0], [5, 3], [[1, 2], [0, -1]])):
        qs, kf, vf, kn, vn, kc, vc, slots = paged_step(num_cached, num_new, tables, 3, heads=H, kv_heads=HKV, dim=64,
                                                       bs=BS, device=cuda, dtype=torch.float16, fill=poison)
        b.store_kvcache(kn, vn, kc, vc, slots)
        ctx = context_for(num_cached, num_new, tables, cuda, is_prefill=max(num_new) > 1)
        out = b.forward(torch.cat(qs), kn, vn, kc, vc, ctx)
        assert torch.isfinite(out).all()
        check(out, dense_expected(qs, kf, vf, SCALE), torch.float16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_long_rows_split_over_keys(cuda, dtype):
    """Rows long enough that decode splits them over keys, beside a one-key row and an empty-ish row."""
    bs = 256
    lens = [40_000, 1, 17, 9 * bs + 1, 5000]
    nblocks = sum(-(-n // bs) for n in lens)
    perm = torch.randperm(nblocks, generator=torch.Generator().manual_seed(1)).tolist()
    tables, at = [], 0
    width = max(-(-n // bs) for n in lens)
    for n in lens:
        k = -(-n // bs)
        tables.append(perm[at:at + k] + [-1] * (width - k))
        at += k
    b = MI355XAttention(32, 128, 1 / math.sqrt(128), 8)
    qs, kf, vf, kn, vn, kc, vc, slots = paged_step([n - 1 for n in lens], [1] * len(lens), tables, nblocks, heads=32,
                                                   kv_heads=8, dim=128, bs=bs, device=cuda, dtype=dtype)
    b.store_kvcache(kn, vn, kc, vc, slots)
    ctx = Context(context_lens=torch.tensor(lens, dtype=torch.int32, device=cuda),
                  block_tables=torch.tensor(tables, dtype=torch.int32, device=cuda))
    out = b.decode(torch.cat(qs), kc, vc, ctx)
    check(out, dense_expected(qs, kf, vf, 1 / math.sqrt(128)), dtype)


@pytest.mark.parametrize("lens, hp, shape, dtype", [
    ((300, 1500, 256), 2, (32, 8, 128), torch.bfloat16),
    ((30_000, 30_000, 2), 1, (32, 8, 128), torch.bfloat16),
    ((9_000, 12_000, 3), 1, (8, 2, 64), torch.float16),
    ((12_000, 12_000, 8), 2, (6, 2, 128), torch.bfloat16),
], ids=["pairs", "one-head", "one-head-d64-fp16", "pairs-group3"])
def test_split_rows_merge_the_same_bits_every_call(cuda, lens, hp, shape, dtype):
    """A split row is merged in the decode launch by whichever of its splits counts in last, from partials that the
    other splits, on any XCD, wrote through to memory. The merge reads them in split order, so every call gives the
    same bits whatever the order of arrival, and a stale partial would show as a difference. Eight calls on one
    step (256 rows of 300-1500 keys on pair items; two rows of 30,000 keys in 118 splits of 256 keys on one-head
    items, eight batches of the merge; three fp16 rows of 64-wide heads; eight rows whose kv pairs each serve three
    query-head groups of one head) must agree bit for bit, and the first with the fp32 oracle."""
    lo, hi, rows = lens
    heads, kv_heads, dim = shape
    bs = 16
    gen = torch.Generator().manual_seed(11)
    ctx_lens = torch.randint(lo, hi + 1, (rows,), generator=gen).tolist()
    tables, at = [], 0
    width = max(-(-n // bs) for n in ctx_lens)
    for n in ctx_lens:
        k = -(-n // bs)
        tables.append(list(range(at, at + k)) + [-1] * (width - k))
        at += k
    b = MI355XAttention(heads, dim, 1 / math.sqrt(dim), kv_heads)
    qs, kf, vf, kn, vn, kc, vc, slots = paged_step([n - 1 for n in ctx_lens], [1] * rows, tables, at, heads=heads,
                                                   kv_heads=kv_heads, dim=dim, bs=bs, device=cuda, dtype=dtype)
    b.store_kvcache(kn, vn, kc, vc, slots)
    ctx = Context(context_lens=torch.tensor(ctx_lens, dtype=torch.int32, device=cuda),
                  block_tables=torch.tensor(tables, dtype=torch.int32, device=cuda))
    q = torch.cat(qs)
    b.launch_trace = []
    outs = [b.decode(q, kc, vc, ctx).clone() for _ in range(8)]
    torch.cuda.synchronize()
    info = b.launch_trace[-1]
    print(f"{rows} rows: {info}", flush=True)
    assert info["kv_heads_per_item"] == hp and info["splitk_merge"] and info["max_splits"] > 1, info
    for i, o in enumerate(outs[1:], 1):
        assert torch.equal(o, outs[0]), f"call {i} differs from the first"
    check(outs[0], dense_expected(qs, kf, vf, 1 / math.sqrt(dim)), dtype)


def test_zero_length_rows_give_zeros(cuda):
    """Graph padding rows (context_len 0) produce a zero output and disturb no other row."""
    b = MI355XAttention(H, 64, SCALE, HKV)
    qs, kf, vf, kn, vn, kc, vc, slots = paged_step([9], [1], [[0]], 2, heads=H, kv_heads=HKV, dim=64, bs=BS,
                                                   device=cuda, dtype=torch.bfloat16)
    b.store_kvcache(kn, vn, kc, vc, slots)
    q = torch.cat([qs[0], torch.ones(1, H, 64, dtype=torch.bfloat16, device=cuda)])
    ctx = Context(context_lens=torch.tensor([10, 0], dtype=torch.int32, device=cuda),
                  block_tables=torch.tensor([[0], [1]], dtype=torch.int32, device=cuda))
    out = b.decode(q, kc, vc, ctx)
    assert torch.equal(out[1], torch.zeros_like(out[1]))
    check(out[:1], dense_expected(qs, kf, vf, SCALE), torch.bfloat16)


def test_out_is_written_in_place(cuda):
    b = MI355XAttention(H, 64, SCALE, HKV)
    out, want, (qs, kf, vf, kc, vc, ctx) = run_step(b, torch.float16, 64, cuda, [20, 0], [1, 7], [[0, 1], [2, -1]], 3)
    buf = torch.empty(10, H, 64, dtype=torch.float16, device=cuda)
    got = b.forward(torch.cat(qs), None, None, kc, vc, ctx, out=buf[2:10])
    assert got.data_ptr() == buf[2:].data_ptr()
    check(buf[2:10], want, torch.float16)


def test_decode_replays_in_a_graph(cuda):
    """A captured decode replays correctly with new queries and lengths written into its static inputs; each
    replay is checked against an eager call, with eager work between replays."""
    b = MI355XAttention(32, 128, 1 / math.sqrt(128), 8)
    bs, rows, width = 256, 4, 8
    lens = [300, 1500, 2047, 40]
    qs, kf, vf, kn, vn, kc, vc, slots = paged_step([n - 1 for n in lens], [1] * rows,
                                                   [[r * width + j for j in range(width)] for r in range(rows)],
                                                   rows * width, heads=32, kv_heads=8, dim=128, bs=bs, device=cuda,
                                                   dtype=torch.bfloat16)
    b.store_kvcache(kn, vn, kc, vc, slots)
    q = torch.cat(qs).clone()
    ctx = Context(context_lens=torch.tensor(lens, dtype=torch.int32, device=cuda),
                  block_tables=torch.arange(rows * width, dtype=torch.int32, device=cuda).view(rows, width))
    out = torch.empty_like(q)
    b.decode(q, kc, vc, ctx, out=out)  # warm: allocates the workspace outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        b.decode(q, kc, vc, ctx, out=out)
    gen = torch.Generator().manual_seed(5)
    for step in range(3):
        q.copy_(torch.randn(q.shape, generator=gen).to(q.dtype))
        ctx.context_lens.copy_(torch.tensor([max(l - 37 * step, 1) for l in lens], dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        eager = b.decode(q, kc, vc, ctx)
        torch.cuda.synchronize()
        torch.testing.assert_close(out, eager, atol=0, rtol=0)


@pytest.mark.parametrize("schedule", ["serial", "overlap"])
def test_mixed_step_replays_in_a_graph(cuda, schedule, monkeypatch):
    """A captured mixed step (work-list plan, prompt kernel, decode kernel, split-K merge) replays with new queries
    and cache contents; each replay equals an eager call, with eager work between replays. This step is small, so
    its overlapped schedule is the one-launch form; the two-stream form (decode items forked onto the library's
    second stream and joined back by events inside the capture) is captured in
    test_layers_of_one_step_share_one_plan's 600-row mixed step."""
    from lvattn import backend as B

    sched = B.SCHEDULE_OVERLAP if schedule == "overlap" else B.SCHEDULE_SERIAL
    b = MI355XAttention(32, 128, 1 / math.sqrt(128), 8)
    monkeypatch.setattr(b, "_schedule", lambda context, elem_bytes: sched)
    bs, width = 256, 24
    num_cached, num_new = [300, 5000, 0, 1999], [1, 1, 700, 64]
    tables = [[r * width + j for j in range(width)] for r in range(4)]
    qs, kf, vf, kn, vn, kc, vc, slots = paged_step(num_cached, num_new, tables, 4 * width, heads=32, kv_heads=8,
                                                   dim=128, bs=bs, device=cuda, dtype=torch.bfloat16)
    b.store_kvcache(kn, vn, kc, vc, slots)
    ctx = context_for(num_cached, num_new, tables, cuda)
    q = torch.cat(qs).clone()
    out = torch.empty_like(q)
    b.forward(q, kn, vn, kc, vc, ctx, out=out)  # warm: grows the workspace outside capture
    torch.cuda.synchronize()
    torch.testing.assert_close(out.float().cpu(), dense_expected(qs, kf, vf, 1 / math.sqrt(128)),
                               atol=2e-2, rtol=1e-2)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        b.forward(q, kn, vn, kc, vc, ctx, out=out)
    gen = torch.Generator().manual_seed(9)
    for _ in range(3):
        q.copy_(torch.randn(q.shape, generator=gen).to(q.dtype))
        kc.view(-1)[: 1 << 20].copy_(torch.randn(1 << 20, generator=gen).to(kc.dtype))
        graph.replay()
        torch.cuda.synchronize()
        eager = b.forward(q, kn, vn, kc, vc, ctx)
        torch.cuda.synchronize()
        torch.testing.assert_close(out, eager, atol=0, rtol=0)


def test_decode_of_more_rows_than_the_planner_holds(cuda):
    """A decode step of 5000 short rows (over the 4096 rows the device work list holds): one workgroup per (row,
    split, head group) without a plan, checked against the oracle, beside rows of 0 and 1 keys."""
    gen = torch.Generator().manual_seed(12)
    rows = 5000
    lens = torch.randint(1, 70, (rows,), generator=gen).tolist()
    lens[17], lens[4999] = 1, 69
    b = MI355XAttention(H, 64, SCALE, HKV)
    width = max(-(-n // BS) for n in lens)
    perm = torch.randperm(rows * width, generator=gen).tolist()
    tables = [perm[r * width:r * width + -(-n // BS)] + [-1] * (width - -(-n // BS)) for r, n in enumerate(lens)]
    qs, kf, vf, kn, vn, kc, vc, slots = paged_step([n - 1 for n in lens], [1] * rows, tables, rows * width, heads=H,
                                                   kv_heads=HKV, dim=64, bs=BS, device=cuda, dtype=torch.bfloat16)
    b.store_kvcache(kn, vn, kc, vc, slots)
    ctx = Context(context_lens=torch.tensor(lens, dtype=torch.int32, device=cuda),
                  block_tables=torch.tensor(tables, dtype=torch.int32, device=cuda))
    b.launch_trace = []
    out = b.decode(torch.cat(qs), kc, vc, ctx)
    torch.cuda.synchronize()
    info = b.launch_trace[-1]
    assert info["decode_kernel"] == "decode_grid" and info["max_splits"] == 1, info
    math_ = A.TorchMath(H, 64, SCALE, HKV)
    want = A.decode_in_row_chunks(math_, torch.cat(qs).cpu(), kc.cpu(), vc.cpu(), ctx.context_lens.cpu(),
                                  ctx.block_tables.cpu(), rows_per_chunk=500)
    check(out, want, torch.bfloat16)


def test_a_step_past_the_work_list_never_splits_its_rows():
    """Split rows are merged through the work list's counters, so a decode step of more rows than the list holds
    must not split them, whatever its contexts: the route of 5000 rows of up to 128K keys keeps one item per row
    (lv_paged_attention_launch_info, the call's own route)."""
    from lvattn import _capi

    for heads, kv_heads, dim in ((32, 8, 128), (8, 1, 64), (64, 4, 128)):
        info = _capi.launch_info(5000, 5000, heads, kv_heads, dim, 16, dim, 0, 1, 131072, 0, 0, 0,
                                 _capi.DTYPES[torch.bfloat16])
        assert info["decode_kernel"] == "decode_grid" and info["max_splits"] == 1, (heads, kv_heads, info)


def test_a_decoder_step_whose_rows_all_carry_drafts(cuda):
    """Rows verifying drafts (three queries each) in a decoder model: the packer marks the step is_prefill, as the
    reference does (model_runner.py:380-384), so the mixed kernel attends each row's queries causally over its
    keys; some rows also had drafts of the previous step rejected, and the pack kernel moves them back
    (_move_back, model_runner.py:527-551). Checked against the dense oracle on the keys each query sees."""
    from lvattn import Packer

    gen = torch.Generator().manual_seed(13)
    k = 2
    num_cached = [40, 7, 100, 63]
    back = [0, 2, 1, 0]  # drafts of the previous step rejected, per row
    num_new = [1 + k] * 4
    bs = BS
    lists, at = [], 0
    for c, n in zip(num_cached, num_new):
        need = -(-(c + n) // bs)
        lists.append(list(range(at, at + need)))
        at += need
    packer = Packer(cuda, bs)
    back_dev = torch.tensor(back, dtype=torch.int32, device=cuda)
    positions, fields = packer.pack(num_cached, num_new, lists, num_speculative_tokens=k, num_back=back_dev)
    assert fields["is_prefill"] and fields["logits_indices"].numel() == 4 * (k + 1)
    order = fields.pop("order").cpu().tolist()
    starts = [c - r for c, r in zip(num_cached, back)]  # where each row's tokens really start
    assert positions.cpu().tolist() == [starts[s] + j for s in order for j in range(num_new[s])]
    b = MI355XAttention(H, 64, SCALE, HKV)
    kc = torch.zeros(at, bs, HKV, 64, dtype=torch.bfloat16, device=cuda)
    vc = torch.zeros_like(kc)
    keys = [randn(starts[s] + num_new[s], HKV, 64, gen=gen, device=cuda, dtype=torch.bfloat16) for s in order]
    vals = [randn(starts[s] + num_new[s], HKV, 64, gen=gen, device=cuda, dtype=torch.bfloat16) for s in order]
    for r, s in enumerate(order):  # the prefix the previous steps stored
        pre = torch.tensor(slots_for(lists[s], bs, 0, starts[s]), dtype=torch.long, device=cuda)
        kc.view(-1, HKV, 64)[pre] = keys[r][:starts[s]]
        vc.view(-1, HKV, 64)[pre] = vals[r][:starts[s]]
    k_new = torch.cat([kk[starts[s]:] for kk, s in zip(keys, order)])
    v_new = torch.cat([vv[starts[s]:] for vv, s in zip(vals, order)])
    qs = [randn(num_new[s], H, 64, gen=gen, device=cuda, dtype=torch.bfloat16) for s in order]
    b.store_kvcache(k_new, v_new, kc, vc, fields["slot_mapping"])
    ctx = Context(**{kk: vv for kk, vv in fields.items() if kk in Context.__slots__})
    out = b.forward(torch.cat(qs), k_new, v_new, kc, vc, ctx)
    torch.cuda.synchronize()
    check(out, dense_expected(qs, keys, vals, SCALE), torch.bfloat16)


def _wide_step(cuda, num_cached, num_new, bs=16, seed=0):
    """Qwen3-8B head shapes (32/8, d128, bf16) over many rows: each row's pages are consecutive blocks."""
    width = max(-(-(c + n) // bs) for c, n in zip(num_cached, num_new))
    tables, at = [], 0
    for c, n in zip(num_cached, num_new):
        k = -(-(c + n) // bs)
        tables.append(list(range(at, at + k)) + [-1] * (width - k))
        at += k
    step = paged_step(num_cached, num_new, tables, at, heads=32, kv_heads=8, dim=128, bs=bs, device=cuda,
                      dtype=torch.bfloat16, seed=seed)
    return tables, step


def test_a_large_decode_batch_of_pair_items(cuda):
    """256 decode rows of up to 600 keys split over 512-key items: enough items that each takes a pair of adjacent
    kv heads, one workgroup per item. Checked against the oracle, then replayed from a captured graph with new
    queries and lengths (the plan kernel rebuilds the work list on every replay), each replay equal to an eager
    call."""
    gen = torch.Generator().manual_seed(3)
    lens = torch.randint(16, 601, (256,), generator=gen).tolist()
    tables, (qs, kf, vf, kn, vn, kc, vc, slots) = _wide_step(cuda, [n - 1 for n in lens], [1] * 256)
    b = MI355XAttention(32, 128, 1 / math.sqrt(128), 8)
    b.store_kvcache(kn, vn, kc, vc, slots)
    q = torch.cat(qs).clone()
    ctx = Context(context_lens=torch.tensor(lens, dtype=torch.int32, device=cuda),
                  block_tables=torch.tensor(tables, dtype=torch.int32, device=cuda))
    out = torch.empty_like(q)
    b.launch_trace = []
    b.decode(q, kc, vc, ctx, out=out)
    torch.cuda.synchronize()
    assert_route(b.launch_trace[-1], decode_kernel="decode_list", kv_heads_per_item=2, two_streams=False,
                 prompt_kernel="none")
    b.launch_trace = None
    torch.testing.assert_close(out.float().cpu(), dense_expected(qs, kf, vf, 1 / math.sqrt(128)), atol=2e-2, rtol=1e-2)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        b.decode(q, kc, vc, ctx, out=out)
    for step in range(3):
        q.copy_(torch.randn(q.shape, generator=gen).to(q.dtype))
        ctx.context_lens.copy_(torch.tensor([max(n - 53 * step, 1) for n in lens], dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        eager = b.decode(q, kc, vc, ctx)
        torch.cuda.synchronize()
        torch.testing.assert_close(out, eager, atol=0, rtol=0)


def test_a_mixed_step_of_many_decode_rows_under_both_schedules(cuda, monkeypatch):
    """Two prompt chunks beside 600 decode rows: under the overlapped schedule the decode items (2408 pair items,
    too few for the persistent grid) run one workgroup per item on the second stream beside the persistent prompt
    workgroups; under the serial one the prompt items run first on the whole GPU. Both match the oracle and each
    other bit for bit."""
    from lvattn import backend as B

    gen = torch.Generator().manual_seed(4)
    dec = torch.randint(16, 601, (600,), generator=gen).tolist()
    num_cached, num_new = [100, 0] + [n - 1 for n in dec], [40, 70] + [1] * 600
    tables, (qs, kf, vf, kn, vn, kc, vc, slots) = _wide_step(cuda, num_cached, num_new, seed=1)
    b = MI355XAttention(32, 128, 1 / math.sqrt(128), 8)
    b.store_kvcache(kn, vn, kc, vc, slots)
    want = dense_expected(qs, kf, vf, 1 / math.sqrt(128))
    outs = {}
    routes = {B.SCHEDULE_SERIAL: dict(prompt_kernel="prompt_list", decode_kernel="decode_list", two_streams=False),
              B.SCHEDULE_OVERLAP: dict(prompt_kernel="prompt_overlap", decode_kernel="decode_list", two_streams=True)}
    b.launch_trace = []
    for sched in (B.SCHEDULE_SERIAL, B.SCHEDULE_OVERLAP):
        monkeypatch.setattr(b, "_schedule", lambda context, elem_bytes, s=sched: s)
        out = b.forward(torch.cat(qs), kn, vn, kc, vc, context_for(num_cached, num_new, tables, cuda))
        torch.cuda.synchronize()
        assert_route(b.launch_trace[-1], kv_heads_per_item=2, **routes[sched])
        torch.testing.assert_close(out.float().cpu(), want, atol=2e-2, rtol=1e-2)
        outs[sched] = out
    assert torch.equal(outs[B.SCHEDULE_SERIAL], outs[B.SCHEDULE_OVERLAP])


# Steps whose layers share one plan, one per launch path of a step: (heads, kv heads, head dim), decode rows
# (count, key range), prompt rows (cached, new), the schedule, and the route the library takes for them.
PLAN_STEPS = {
    # split rows (the first three): each row's last split merges its partials and puts its counter back to zero,
    # which the two layers on the reused plan rely on
    "decode-pairs": ((32, 8, 128), (256, 16, 600), [], None,
                     dict(decode_kernel="decode_list", kv_heads_per_item=2, prompt_kernel="none", splitk_merge=True)),
    "decode-small": ((32, 8, 128), None, [], None,
                     dict(decode_kernel="decode_list", kv_heads_per_item=1, prompt_kernel="none", splitk_merge=True)),
    "mixed-one-launch": ((32, 8, 128), (30, 64, 2048), [(256, 384), (0, 512)], "overlap",
                         dict(decode_kernel="mixed_small", prompt_kernel="mixed_small", two_streams=False,
                              splitk_merge=True)),
    "mixed-serial": ((32, 8, 128), (600, 16, 600), [(100, 40), (0, 70)], "serial",
                     dict(decode_kernel="decode_list", prompt_kernel="prompt_list", two_streams=False)),
    "mixed-overlap-list": ((32, 8, 128), (600, 16, 600), [(100, 40), (0, 70)], "overlap",
                           dict(decode_kernel="decode_list", prompt_kernel="prompt_overlap", two_streams=True)),
    # the persistent ticket grid beside the prompt workgroups: pair items at d128 (the Qwen3-8B shape), one-head
    # items (odd kv heads), pair items at d64
    "beside-pairs-d128": ((32, 8, 128), (2048, 16, 256), [(100, 40), (0, 70)], "overlap",
                          dict(decode_kernel="decode_beside", kv_heads_per_item=2, prompt_kernel="prompt_overlap",
                               two_streams=True)),
    "beside-one-head-d128": ((12, 3, 128), (2100, 16, 256), [(100, 40), (0, 70)], "overlap",
                             dict(decode_kernel="decode_beside", kv_heads_per_item=1, prompt_kernel="prompt_overlap",
                                  two_streams=True)),
    "beside-pairs-d64": ((16, 4, 64), (3100, 16, 256), [(100, 40), (0, 70)], "overlap",
                         dict(decode_kernel="decode_beside", kv_heads_per_item=2, prompt_kernel="prompt_overlap",
                              two_streams=True)),
}


def assert_route(info, **want):
    got = {k: info[k] for k in want}
    assert got == want, f"launch route {info}, expected {want}"


@pytest.mark.parametrize("kind", list(PLAN_STEPS))
def test_layers_of_one_step_share_one_plan(cuda, kind, monkeypatch):
    """Three layers (each with its own cache) attend through one step's Context: the first plans the work list, the
    next two reuse it (LV_ATTN_REUSE_PLAN). On the persistent grid, the last workgroup of each layer must leave the
    ticket counters at zero for the next, and on split rows each row's last split its merge counter. Each case asserts the launch path it reaches (lv_paged_attention_launch_info
    on the call's arguments). Each layer equals the same call on a fresh Context (which plans again), bit for bit;
    the first matches the fp32 oracle; then the three layers are captured in one graph (one plan launch in it) and
    every replay equals the eager layers."""
    from lvattn import backend as B

    (heads, kv_heads, dim), dec, prompts, sched, route = PLAN_STEPS[kind]
    gen = torch.Generator().manual_seed(31)
    scale = 1 / math.sqrt(dim)
    b = MI355XAttention(heads, dim, scale, kv_heads)
    if dec is None:  # a few rows: one workgroup per one-head item
        num_cached, num_new = [300, 5000, 20], [1, 1, 1]
    else:
        n, lo, hi = dec
        lens = torch.randint(lo, hi + 1, (n,), generator=gen).tolist()
        num_cached = [c for c, _ in prompts] + [k - 1 for k in lens]
        num_new = [q for _, q in prompts] + [1] * n
        order = sorted(range(len(num_new)), key=lambda i: num_new[i] > 1)  # decode rows first
        num_cached, num_new = [num_cached[i] for i in order], [num_new[i] for i in order]
    if sched is not None:
        s_ = B.SCHEDULE_OVERLAP if sched == "overlap" else B.SCHEDULE_SERIAL
        monkeypatch.setattr(b, "_schedule", lambda context, elem_bytes: s_)
    tables, at = [], 0
    bs = 16
    width = max(-(-(c + q) // bs) for c, q in zip(num_cached, num_new))
    for c, q in zip(num_cached, num_new):
        k = -(-(c + q) // bs)
        tables.append(list(range(at, at + k)) + [-1] * (width - k))
        at += k
    step0 = paged_step(num_cached, num_new, tables, at, heads=heads, kv_heads=kv_heads, dim=dim, bs=bs, device=cuda,
                       dtype=torch.bfloat16, seed=2)
    print(f"{kind}: {len(num_new)} rows, {sum(num_new)} tokens", flush=True)
    q = torch.cat(step0[0])
    caches = [(step0[5], step0[6])]
    dgen = torch.Generator(device=cuda).manual_seed(32)
    for layer in range(2):  # two more layers: other keys and values in caches of the same shape
        caches.append(tuple(torch.randn(step0[5].shape, generator=dgen, device=cuda).to(torch.bfloat16)
                            for _ in range(2)))
    b.store_kvcache(step0[3], step0[4], *caches[0], step0[7])

    decode_only = all(x == 1 for x in num_new)
    template = (Context(context_lens=torch.tensor([c + x for c, x in zip(num_cached, num_new)], dtype=torch.int32,
                                                  device=cuda),
                        block_tables=torch.tensor(tables, dtype=torch.int32, device=cuda))
                if decode_only else context_for(num_cached, num_new, tables, cuda))

    def context():
        """A new step's Context over the same device tensors (no copies: it is also built inside the capture)."""
        skip = ("attn_metadata", "decode_splits")  # per-step caches
        return Context(**{k: getattr(template, k) for k in Context.__slots__ if k not in skip})

    b.launch_trace = []
    step = context()
    shared = [b.forward(q, None, None, kc, vc, step) for kc, vc in caches]
    torch.cuda.synchronize()
    assert sum(1 for k in step.attn_metadata if k[0] == "plan") == 1
    for info in b.launch_trace:
        assert_route(info, **route)
    b.launch_trace = None
    fresh = [b.forward(q, None, None, kc, vc, context()) for kc, vc in caches]
    torch.cuda.synchronize()
    for i, (x, y) in enumerate(zip(shared, fresh)):
        assert torch.equal(x, y), f"layer {i}"
    torch.testing.assert_close(shared[0].float().cpu(), dense_expected(step0[0], step0[1], step0[2], scale),
                               atol=2e-2, rtol=1e-2)
    outs = [torch.empty_like(q) for _ in caches]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_step = context()
        for (kc, vc), out in zip(caches, outs):
            b.forward(q, None, None, kc, vc, g_step, out=out)
    for rep in range(3):
        q.copy_(torch.randn(q.shape, generator=gen).to(q.dtype))
        graph.replay()
        torch.cuda.synchronize()
        eager = [b.forward(q, None, None, kc, vc, context()) for kc, vc in caches]
        torch.cuda.synchronize()
        for i, (x, y) in enumerate(zip(outs, eager)):
            assert torch.equal(x, y), f"replay {rep} layer {i}"


@pytest.mark.parametrize("factor", [6, 40])
@pytest.mark.parametrize("bs", [16, 64, 256])
def test_scores_far_above_the_first_tile(case, bs, factor, monkeypatch):
    """bf16 prompt tiles take a row's max from the item's first key tile and hold it; when later keys score far
    above it (keys 64 onward scaled 40x, some 200 log2 units higher), the item's row sums fail their check and the
    workgroup runs the item again with a running max. Scaled 6x (some 20-30 units higher) the held max stands: the
    probabilities reach 2^30, which bf16 P holds; fp16, whose P would overflow there, keeps the running max. Cold
    prompts whose queries past 64 see the scaled keys, next to a row whose keys stay unscaled, under both launch
    schedules, against the fp32 oracle."""
    from lvattn import backend as B

    b, dtype, dim, dev = case
    cached, new = [0, 0, 0], [200, 130, 70]
    need = [-(-(c + n) // bs) for c, n in zip(cached, new)]
    width = max(need)
    tables, at = [], 0
    for k in need:
        tables.append(list(range(at, at + k)) + [-1] * (width - k))
        at += k
    qs, kf, vf, kn, vn, kc, vc, slots = paged_step(cached, new, tables, at + 1, heads=H, kv_heads=HKV, dim=dim,
                                                   bs=bs, device=dev, dtype=dtype)
    for i in (0, 1):
        kf[i][64:] *= factor
    kn = torch.cat(kf)
    b.store_kvcache(kn, vn, kc, vc, slots)
    want = dense_expected(qs, kf, vf, SCALE)
    for sched in (B.SCHEDULE_SERIAL, B.SCHEDULE_OVERLAP):
        monkeypatch.setattr(b, "_schedule", lambda context, elem_bytes, s=sched: s)
        out = b.forward(torch.cat(qs), kn, vn, kc, vc, context_for(cached, new, tables, dev))
        torch.cuda.synchronize()
        assert torch.isfinite(out).all()
        check(out, want, dtype)


@pytest.mark.parametrize("dim", [64, 128])
def test_huge_values_with_scores_above_the_first_tile(cuda, dim):
    """bf16 values near 2^100 and keys from 64 onward scaled 9x (some 35-50 log2 units above the first tile): the held
    max's row sums stay below their bound, but its accumulators (probabilities near 2^45 times the values) overflow,
    where the fp32 oracle's do not. The accumulator check sends the item to the running max."""
    dtype, bs = torch.bfloat16, 64
    b = MI355XAttention(H, dim, SCALE, HKV)
    cached, new = [0, 0], [200, 130]
    need = [-(-(c + n) // bs) for c, n in zip(cached, new)]
    width = max(need)
    tables, at = [], 0
    for k in need:
        tables.append(list(range(at, at + k)) + [-1] * (width - k))
        at += k
    qs, kf, vf, kn, vn, kc, vc, slots = paged_step(cached, new, tables, at + 1, heads=H, kv_heads=HKV, dim=dim,
                                                   bs=bs, device=cuda, dtype=dtype)
    for i in (0, 1):
        kf[i][64:] *= 9
        vf[i] *= 2.0 ** 100
    kn, vn = torch.cat(kf), torch.cat(vf)
    b.store_kvcache(kn, vn, kc, vc, slots)
    want = dense_expected(qs, kf, vf, SCALE)
    assert torch.isfinite(want).all()
    out = b.forward(torch.cat(qs), kn, vn, kc, vc, context_for(cached, new, tables, cuda))
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    # The path's bf16 bar (2e-2 absolute, 1e-2 relative) at the values' scale.
    torch.testing.assert_close(out.float().cpu(), want.float(), atol=2e-2 * 2.0 ** 100, rtol=1e-2)
