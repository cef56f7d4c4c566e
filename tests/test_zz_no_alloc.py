"""lv_paged_attention_static: the allocation-free variant of lv_paged_attention, through the C ABI.

Its work list, ticket and split-K partials live in the library's static device array instead of a caller's
workspace. Two calls in a row on one stream -- a mixed step whose decode rows are split over keys (plan, prompt
tiles beside the decode rows on the second stream, split-K merge), then a smaller decode step -- each give exactly
lv_paged_attention's output on the same inputs (the same kernels, so bit for bit), and the second call is not
disturbed by what the first left in the shared array. A step needing more workspace than the array holds is
refused with a message (that check runs before anything touches the GPU).
"""

import math

import pytest
import torch

from helpers import context_for, paged_step
from lvattn import MI355XAttention, _capi
from lvattn import backend as B

pytestmark = pytest.mark.gpu


def call(name, b, q, kc, vc, ctx, out, *, decode, schedule):
    """lv_paged_attention (with the backend's workspace) or lv_paged_attention_static on the same arguments."""
    rows = ctx.context_lens.numel() if decode else ctx.cu_seqlens_q.numel() - 1
    tokens, heads, dim = q.shape
    max_q = 1 if decode else ctx.max_seqlen_q
    max_k = ctx.block_tables.size(1) * kc.size(1)
    sb, st, sh, _ = kc.stride()
    args = [q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(), sb, st, sh, kc.size(1),
            ctx.block_tables.data_ptr(), ctx.block_tables.stride(0), None if decode else ctx.cu_seqlens_q.data_ptr(),
            ctx.context_lens.data_ptr() if decode else None, None if decode else ctx.cu_seqlens_k.data_ptr(), rows,
            tokens, heads, b.num_kv_heads, dim, float(b.scale), max_q, max_k, out.data_ptr(), out.stride(0),
            out.stride(1)]
    if name == "lv_paged_attention":
        nbytes = _capi.query("lv_paged_attention_workspace_bytes", rows, tokens, heads, b.num_kv_heads, dim, max_k,
                             int(decode))
        ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
        args += [ws.data_ptr(), ws.numel()]
    else:
        ws = None
    _capi.call(name, *args, schedule, 0, 0, _capi.DTYPES[q.dtype], _capi.stream_of(q.device))
    torch.cuda.synchronize()
    return ws


def test_the_static_workspace_gives_the_same_steps(cuda):
    b = MI355XAttention(32, 128, 1 / math.sqrt(128), 8)
    bs = 256
    # 1: a mixed step: decode rows long enough to be split over keys, beside two prompt chunks (overlapped)
    num_cached, num_new = [9000, 300, 0, 1999, 17000], [1, 1, 700, 64, 1]
    width = max(-(-(c + n) // bs) for c, n in zip(num_cached, num_new))
    tables = [[r * width + j for j in range(width)] for r in range(5)]
    qs, kf, vf, kn, vn, kc, vc, slots = paged_step(num_cached, num_new, tables, 5 * width, heads=32, kv_heads=8,
                                                   dim=128, bs=bs, device=cuda, dtype=torch.bfloat16)
    b.store_kvcache(kn, vn, kc, vc, slots)
    ctx = context_for(num_cached, num_new, tables, cuda)
    q = torch.cat(qs)
    want = torch.full_like(q, float("nan"))
    got = torch.full_like(q, float("nan"))
    call("lv_paged_attention", b, q, kc, vc, ctx, want, decode=False, schedule=B.SCHEDULE_OVERLAP)
    call("lv_paged_attention_static", b, q, kc, vc, ctx, got, decode=False, schedule=B.SCHEDULE_OVERLAP)
    assert torch.isfinite(want).all()
    assert torch.equal(got, want)

    # 2: a smaller decode step right after, on the same static array
    lens = [40, 4097, 700]
    tables2 = [t[:-(-n // bs)] + [-1] * (width - -(-n // bs)) for t, n in zip(tables, lens)]
    from lvattn import Context

    ctx2 = Context(context_lens=torch.tensor(lens, dtype=torch.int32, device=cuda),
                   block_tables=torch.tensor(tables2, dtype=torch.int32, device=cuda))
    q2 = torch.randn(3, 32, 128, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(cuda)
    want2 = torch.full_like(q2, float("nan"))
    got2 = torch.full_like(q2, float("nan"))
    call("lv_paged_attention", b, q2, kc, vc, ctx2, want2, decode=True, schedule=B.SCHEDULE_AUTO)
    call("lv_paged_attention_static", b, q2, kc, vc, ctx2, got2, decode=True, schedule=B.SCHEDULE_AUTO)
    assert torch.isfinite(want2).all()
    assert torch.equal(got2, want2)
