"""lv_paged_attention_static: the allocation-free variant of lv_paged_attention, through the C ABI.

Its work list, ticket and split-K partials live in the library's static device array instead of a caller's
workspace. Calls in a row on one stream, each smaller than the one before -- a mixed step of 1100 decode rows beside
two prompt chunks (plan, prompt workgroups on part of the CUs, the persistent decode grid on the second stream,
joined back by events), a small mixed step whose decode rows are split over keys (one launch, split-K merge), then a
small decode step -- each give exactly lv_paged_attention's output on the same inputs (the same kernels, so bit for
bit), and no call is disturbed by what the one before left in the shared array. A step needing more workspace than
the array holds is refused with a message (that check runs before anything touches the GPU).
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


def route(b, q, kc, ctx, *, decode, schedule):
    """The launches either entry point makes for these arguments (lv_paged_attention_launch_info)."""
    rows = ctx.context_lens.numel() if decode else ctx.cu_seqlens_q.numel() - 1
    tokens, heads, dim = q.shape
    return _capi.launch_info(rows, tokens, heads, b.num_kv_heads, dim, kc.size(1), kc.stride(2), int(not decode),
                             1 if decode else ctx.max_seqlen_q, ctx.block_tables.size(1) * kc.size(1), schedule, 0, 0,
                             _capi.DTYPES[q.dtype])


def test_the_static_workspace_gives_the_same_steps(cuda):
    b = MI355XAttention(32, 128, 1 / math.sqrt(128), 8)
    bs = 256
    # 0: a mixed step large enough to fork: 1100 one-page decode rows beside two prompt chunks
    gen = torch.Generator().manual_seed(5)
    lens = torch.randint(16, bs + 1, (1100,), generator=gen).tolist()
    num_cached0, num_new0 = [n - 1 for n in lens] + [100, 0], [1] * 1100 + [40, 150]
    tables0 = [[r] for r in range(len(num_new0))]
    qs, kf, vf, kn, vn, kc0, vc0, slots = paged_step(num_cached0, num_new0, tables0, len(num_new0), heads=32,
                                                     kv_heads=8, dim=128, bs=bs, device=cuda, dtype=torch.bfloat16)
    b.store_kvcache(kn, vn, kc0, vc0, slots)
    ctx0 = context_for(num_cached0, num_new0, tables0, cuda)
    info = route(b, torch.cat(qs), kc0, ctx0, decode=False, schedule=B.SCHEDULE_OVERLAP)
    assert info["two_streams"] and info["decode_kernel"] == "decode_beside", info
    q0 = torch.cat(qs)
    want0 = torch.full_like(q0, float("nan"))
    got0 = torch.full_like(q0, float("nan"))
    call("lv_paged_attention", b, q0, kc0, vc0, ctx0, want0, decode=False, schedule=B.SCHEDULE_OVERLAP)
    call("lv_paged_attention_static", b, q0, kc0, vc0, ctx0, got0, decode=False, schedule=B.SCHEDULE_OVERLAP)
    assert torch.isfinite(want0).all()
    assert torch.equal(got0, want0)
    del kc0, vc0

    # 1: a small mixed step: decode rows long enough to be split over keys, beside two prompt chunks
    num_cached, num_new = [9000, 300, 0, 1999, 17000], [1, 1, 700, 64, 1]
    width = max(-(-(c + n) // bs) for c, n in zip(num_cached, num_new))
    tables = [[r * width + j for j in range(width)] for r in range(5)]
    qs, kf, vf, kn, vn, kc, vc, slots = paged_step(num_cached, num_new, tables, 5 * width, heads=32, kv_heads=8,
                                                   dim=128, bs=bs, device=cuda, dtype=torch.bfloat16)
    b.store_kvcache(kn, vn, kc, vc, slots)
    ctx = context_for(num_cached, num_new, tables, cuda)
    q = torch.cat(qs)
    info = route(b, q, kc, ctx, decode=False, schedule=B.SCHEDULE_OVERLAP)
    assert info["decode_kernel"] == "mixed_small" and info["splitk_merge"], info
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
