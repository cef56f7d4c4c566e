"""Every launch route of paged attention, across the template axes a caller can reach, against the oracle.

The library picks its kernels from the step's shape (``lv_paged_attention_launch_info`` reports the choice):
- decode items one workgroup each (``decode_list``), with one kv head per item or a pair of adjacent kv heads (at
  least eight one-head items per CU, kv heads even);
- decode steps of more rows than the work list holds, one workgroup per (row, kv head, head group)
  (``decode_grid``);
- a small mixed step in one launch (``mixed_small``);
- prompt items on the whole GPU (``prompt_list``, the serial schedule) or on part of it beside the decode items
  (``prompt_overlap``), the decode items then one workgroup each or on the persistent ticket grid
  (``decode_beside``).
Each route is run for bf16 and fp16, head dims 64 and 128, GQA groups whose query heads go 1, 2 or 4 to a lane
group (groups 1, 2, 4, and 3, 6, 8 with several lane groups per kv head), and pages of 16, 32, 48 and 64 keys (the
prompt tile's swizzled, register-staged and padded stages). Each case asserts the route it reaches. Keys are few so
the CPU oracle (the textbook dense attention of each row, fp32) stays quick; steps of thousands of rows compare a
sample of their rows, chosen to include the first, the last and rows split over several items.

Tolerances: fp16 6e-3, bf16 2e-2 absolute / 1e-2 relative against the fp32 oracle.
"""

import math

import pytest
import torch

from helpers import context_for, dense_expected, paged_step
from lvattn import Context, MI355XAttention
from lvattn import backend as B

pytestmark = pytest.mark.gpu

TOL = {torch.float16: dict(atol=6e-3, rtol=6e-3), torch.bfloat16: dict(atol=2e-2, rtol=1e-2)}
DTYPES = [torch.bfloat16, torch.float16]
DT_IDS = ["bf16", "fp16"]
# (query heads, kv heads) by GQA group; the lane groups of 4, 2 or 1 query heads follow the group's factors.
GROUPS = {"g1": (8, 8), "g2": (16, 8), "g4": (32, 8), "g3": (12, 4), "g6": (24, 4), "g8": (16, 2)}
# Odd kv-head counts: decode items keep one kv head each whatever their number.
ODD_GROUPS = {"g1": (3, 3), "g2": (6, 3), "g4": (12, 3)}


def _tables(lens, bs):
    """Each row's pages as consecutive blocks, rows padded with -1 to the widest."""
    need = [-(-n // bs) for n in lens]
    width = max(need)
    tables, at = [], 0
    for k in need:
        tables.append(list(range(at, at + k)) + [-1] * (width - k))
        at += k
    return tables, at


def _step(cuda, dtype, dim, bs, heads, kv, num_cached, num_new, seed):
    tables, nblocks = _tables([c + n for c, n in zip(num_cached, num_new)], bs)
    step = paged_step(num_cached, num_new, tables, nblocks, heads=heads, kv_heads=kv, dim=dim, bs=bs, device=cuda,
                      dtype=dtype, seed=seed)
    return tables, step


def _run(cuda, dtype, dim, bs, heads, kv, num_cached, num_new, schedule=None, monkeypatch=None, seed=0):
    """One forward over the step; returns the output, the launch route and the step's rows."""
    tables, (qs, kf, vf, kn, vn, kc, vc, slots) = _step(cuda, dtype, dim, bs, heads, kv, num_cached, num_new, seed)
    b = MI355XAttention(heads, dim, 1 / math.sqrt(dim), kv)
    b.store_kvcache(kn, vn, kc, vc, slots)
    if schedule is not None:
        monkeypatch.setattr(b, "_schedule", lambda context, elem_bytes: schedule)
    b.launch_trace = []
    if all(n == 1 for n in num_new):
        lens = [c + 1 for c in num_cached]
        ctx = Context(context_lens=torch.tensor(lens, dtype=torch.int32, device=cuda),
                      block_tables=torch.tensor(tables, dtype=torch.int32, device=cuda))
        out = b.decode(torch.cat(qs), kc, vc, ctx)
    else:
        out = b.forward(torch.cat(qs), kn, vn, kc, vc, context_for(num_cached, num_new, tables, cuda))
    torch.cuda.synchronize()
    return out, b.launch_trace[-1], (qs, kf, vf, 1 / math.sqrt(dim))


def _check(out, rows, dtype, sample=None):
    """Compare the output rows of ``sample`` (all rows if None) with the dense oracle."""
    qs, kf, vf, scale = rows
    starts = [0]
    for q in qs:
        starts.append(starts[-1] + q.size(0))
    sel = range(len(qs)) if sample is None else sorted(set(sample))
    want = dense_expected([qs[r] for r in sel], [kf[r] for r in sel], [vf[r] for r in sel], scale)
    got = torch.cat([out[starts[r]:starts[r + 1]] for r in sel])
    torch.testing.assert_close(got.float().cpu(), want, **TOL[dtype])


def _route(info, **want):
    got = {k: info[k] for k in want}
    assert got == want, f"launch route {info}, expected {want}"


def _lens(n, lo, hi, seed, extra=()):
    gen = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (n,), generator=gen).tolist()
    for i, v in extra:
        lens[i] = v
    return lens


@pytest.mark.parametrize("group", list(GROUPS))
@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
def test_decode_items_of_one_kv_head(cuda, dtype, dim, group):
    """A few decode rows, one of them split over three items (700 keys on 256-key splits) beside rows of 1 key and of
    a page boundary: one workgroup per one-head item, the split row merged by its last split."""
    heads, kv = GROUPS[group]
    lens = [1, 17, 64, 255, 300, 700]
    out, info, rows = _run(cuda, dtype, dim, 16, heads, kv, [n - 1 for n in lens], [1] * len(lens))
    _route(info, decode_kernel="decode_list", kv_heads_per_item=1, prompt_kernel="none", splitk_merge=True)
    _check(out, rows, dtype)


@pytest.mark.parametrize("group", ["g1", "g2", "g4"])
@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
def test_decode_items_of_kv_head_pairs(cuda, dtype, dim, group):
    """256 decode rows over 8 kv heads: 2048 one-head items or more, so each item takes two adjacent kv heads."""
    heads, kv = GROUPS[group]
    lens = _lens(256, 16, 160, seed=1, extra=[(0, 1), (255, 160)])
    out, info, rows = _run(cuda, dtype, dim, 32, heads, kv, [n - 1 for n in lens], [1] * len(lens), seed=1)
    _route(info, decode_kernel="decode_list", kv_heads_per_item=2, prompt_kernel="none")
    _check(out, rows, dtype)


@pytest.mark.parametrize("group", ["g1", "g2", "g4", "odd-g1", "odd-g2", "odd-g4"])
@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
def test_decode_of_more_rows_than_the_work_list_holds(cuda, dtype, dim, group):
    """4100 short decode rows (past the 4096 rows of the device work list): one workgroup per (row, kv head, head
    group), unsplit, with kv-head pairs for an even kv-head count (2 here) and one kv head for an odd one."""
    odd = group.startswith("odd-")
    heads, kv = ODD_GROUPS[group[4:]] if odd else (GROUPS[group][0] // 4, 2)
    lens = _lens(4100, 1, 40, seed=2, extra=[(4099, 40)])
    out, info, rows = _run(cuda, dtype, dim, 16, heads, kv, [n - 1 for n in lens], [1] * len(lens), seed=2)
    _route(info, decode_kernel="decode_grid", kv_heads_per_item=1 if odd else 2, max_splits=1)
    _check(out, rows, dtype, sample=list(range(64)) + list(range(64, 4100, 97)) + [4099])


@pytest.mark.parametrize("bs", [16, 32, 48, 64])
@pytest.mark.parametrize("group", ["g1", "g2", "g4"])
@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
def test_a_small_mixed_step_in_one_launch(cuda, monkeypatch, dtype, dim, group, bs):
    """Two prompt chunks (one on a cached prefix) beside 20 decode rows, one of them split, under the overlapped
    schedule: prompt and decode items in one launch."""
    heads, kv = GROUPS[group]
    dec = _lens(20, 10, 300, seed=3, extra=[(7, 600)])
    num_cached, num_new = [0, 70] + [n - 1 for n in dec], [40, 33] + [1] * len(dec)
    out, info, rows = _run(cuda, dtype, dim, bs, heads, kv, num_cached, num_new, B.SCHEDULE_OVERLAP, monkeypatch,
                           seed=3)
    _route(info, decode_kernel="mixed_small", prompt_kernel="mixed_small", kv_heads_per_item=1, two_streams=False)
    _check(out, rows, dtype)


@pytest.mark.parametrize("bs", [16, 32, 48, 64])
@pytest.mark.parametrize("group", ["g1", "g2", "g4"])
@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
def test_a_small_mixed_step_of_kv_head_pairs_in_one_launch(cuda, monkeypatch, dtype, dim, group, bs):
    """The Qwen3-0.6B step's rows (30 decode rows of up to 2048 keys beside two chunks) over 8 kv heads: enough
    decode items for kv-head pairs, still one launch."""
    heads, kv = GROUPS[group]
    dec = _lens(30, 64, 2048, seed=4)
    num_cached, num_new = [0, 256] + [n - 1 for n in dec], [512, 384] + [1] * len(dec)
    out, info, rows = _run(cuda, dtype, dim, bs, heads, kv, num_cached, num_new, B.SCHEDULE_OVERLAP, monkeypatch,
                           seed=4)
    _route(info, decode_kernel="mixed_small", prompt_kernel="mixed_small", kv_heads_per_item=2)
    _check(out, rows, dtype)


@pytest.mark.parametrize("bs", [16, 32, 48, 64])
@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
def test_prompt_items_on_the_whole_gpu_then_decode_items(cuda, monkeypatch, dtype, dim, bs):
    """The serial schedule: a step's prompt items one workgroup each on the whole GPU, then its decode items."""
    heads, kv = GROUPS["g4"]
    dec = _lens(20, 10, 300, seed=5)
    num_cached, num_new = [0, 70] + [n - 1 for n in dec], [40, 33] + [1] * len(dec)
    out, info, rows = _run(cuda, dtype, dim, bs, heads, kv, num_cached, num_new, B.SCHEDULE_SERIAL, monkeypatch,
                           seed=5)
    _route(info, decode_kernel="decode_list", prompt_kernel="prompt_list", two_streams=False)
    _check(out, rows, dtype)


@pytest.mark.parametrize("bs", [16, 32, 48, 64])
@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
def test_prompt_items_beside_decode_items(cuda, monkeypatch, dtype, dim, bs):
    """Two chunks beside 600 decode rows under the overlapped schedule: persistent prompt workgroups on part of the
    CUs, the decode items (too few for the ticket grid) one workgroup each on the second stream."""
    heads, kv = GROUPS["g4"]
    dec = _lens(600, 16, 120, seed=6)
    num_cached, num_new = [100, 0] + [n - 1 for n in dec], [40, 70] + [1] * len(dec)
    out, info, rows = _run(cuda, dtype, dim, bs, heads, kv, num_cached, num_new, B.SCHEDULE_OVERLAP, monkeypatch,
                           seed=6)
    _route(info, decode_kernel="decode_list", prompt_kernel="prompt_overlap", two_streams=True)
    _check(out, rows, dtype, sample=[0, 1] + list(range(2, 602, 7)) + [601])


@pytest.mark.parametrize("group", ["g1", "g2", "g4", "odd-g1", "odd-g2", "odd-g4"])
@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
def test_decode_items_on_the_ticket_grid_beside_prompt_items(cuda, monkeypatch, dtype, dim, group):
    """Two chunks beside 2100 decode rows: enough decode items (8400 pair items over 8 kv heads, 6300 one-head
    items over 3) that persistent decode workgroups take them by ticket beside the prompt workgroups."""
    odd = group.startswith("odd-")
    heads, kv = ODD_GROUPS[group[4:]] if odd else GROUPS[group]
    dec = _lens(2100, 16, 48, seed=7)
    num_cached, num_new = [100, 0] + [n - 1 for n in dec], [40, 70] + [1] * len(dec)
    out, info, rows = _run(cuda, dtype, dim, 64, heads, kv, num_cached, num_new, B.SCHEDULE_OVERLAP, monkeypatch,
                           seed=7)
    _route(info, decode_kernel="decode_beside", prompt_kernel="prompt_overlap", two_streams=True,
           kv_heads_per_item=1 if odd else 2)
    _check(out, rows, dtype, sample=[0, 1] + list(range(2, 2102, 53)) + [2101])
