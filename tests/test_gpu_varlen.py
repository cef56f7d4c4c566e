"""Attention over packed keys (prefill without block tables, varlen_with_lse) and the log-sum-exp merge on the GPU.

Cases of the reference's tests (tests/test_attention_backends.py:171-263, 266-287): rows of 5, 1 and 12 queries;
causal and unmasked chunks that hold more keys than queries; MLA prefill's 192-wide q.k with 128-wide values
handed over as a view of a wider tensor; the merge in place and into a strided output with lse in a transposed
layout and a row with no keys. Expected values: the textbook dense oracle in fp32 (outputs and natural lse).
Tolerances: fp16 6e-3, bf16 2e-2 / 1e-2.
"""

import pytest
import torch

from lvattn import Context, MI355XAttention, merge_attention, merge_attention_
from oracle import attention as A

pytestmark = pytest.mark.gpu

H, HKV, SCALE = 8, 2, 0.137
TOL = {torch.float16: dict(atol=6e-3, rtol=6e-3), torch.bfloat16: dict(atol=2e-2, rtol=1e-2)}
CASES = [(torch.float16, 64), (torch.bfloat16, 64), (torch.bfloat16, 128)]
IDS = ["fp16-d64", "bf16-d64", "bf16-d128"]


def rnd(*shape, gen, dtype, device):
    return torch.randn(*shape, generator=gen).to(dtype).to(device)


def cumulative(lens, device):
    return torch.tensor([0, *torch.tensor(lens).cumsum(0).tolist()], dtype=torch.int32, device=device)


def dense_rows(qs, ks, vs, causal, scale=SCALE):
    out = torch.cat([A.dense_attention(q.cpu().float(), k.cpu().float(), v.cpu().float(), scale, causal=causal)
                     for q, k, v in zip(qs, ks, vs)])
    lse = torch.cat([A.dense_scores(q.cpu().float(), k.cpu().float(), scale, causal=causal).logsumexp(-1).T
                     for q, k in zip(qs, ks)])
    return out, lse


@pytest.mark.parametrize("dtype, dim", CASES, ids=IDS)
def test_prefill_without_cache(cuda, dtype, dim):
    gen = torch.Generator().manual_seed(0)
    lens = [5, 1, 12]
    qs = [rnd(n, H, dim, gen=gen, dtype=dtype, device=cuda) for n in lens]
    ks = [rnd(n, HKV, dim, gen=gen, dtype=dtype, device=cuda) for n in lens]
    vs = [rnd(n, HKV, dim, gen=gen, dtype=dtype, device=cuda) for n in lens]
    cu = cumulative(lens, cuda)
    ctx = Context(is_prefill=True, cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=max(lens), max_seqlen_k=max(lens))
    empty = torch.tensor([], dtype=dtype, device=cuda)
    b = MI355XAttention(H, dim, SCALE, HKV)
    out = b.forward(torch.cat(qs), torch.cat(ks), torch.cat(vs), empty, empty, ctx)
    torch.testing.assert_close(out.float().cpu(), dense_rows(qs, ks, vs, True)[0], **TOL[dtype])


@pytest.mark.parametrize("causal", [True, False], ids=["causal", "unmasked"])
@pytest.mark.parametrize("dtype, dim", CASES, ids=IDS)
def test_varlen_with_lse(cuda, dtype, dim, causal):
    gen = torch.Generator().manual_seed(1)
    lens_q = [5, 1, 12]
    lens_k = lens_q if causal else [7, 4, 16]
    qs = [rnd(n, H, dim, gen=gen, dtype=dtype, device=cuda) for n in lens_q]
    ks = [rnd(n, HKV, dim, gen=gen, dtype=dtype, device=cuda) for n in lens_k]
    vs = [rnd(n, HKV, dim, gen=gen, dtype=dtype, device=cuda) for n in lens_k]
    out, lse = MI355XAttention(H, dim, SCALE, HKV).varlen_with_lse(
        torch.cat(qs), torch.cat(ks), torch.cat(vs), cumulative(lens_q, cuda), cumulative(lens_k, cuda),
        max(lens_q), max(lens_k), causal)
    want, want_lse = dense_rows(qs, ks, vs, causal)
    assert lse.dtype == torch.float32 and lse.shape == (sum(lens_q), H)
    torch.testing.assert_close(out.float().cpu(), want, **TOL[dtype])
    torch.testing.assert_close(lse.cpu(), want_lse, **TOL[dtype])


@pytest.mark.parametrize("causal", [True, False], ids=["causal", "unmasked"])
def test_narrow_values_match_padded_ones(cuda, causal):
    """192-wide q.k with 128-wide values given as a view of a wider tensor, as MLA prefill hands them over."""
    dtype, heads, qk, vd = torch.bfloat16, 16, 192, 128
    gen = torch.Generator().manual_seed(2)
    lens_q = [5, 1, 12, 200]
    lens_k = lens_q if causal else [7, 4, 16, 333]
    q = rnd(sum(lens_q), heads, qk, gen=gen, dtype=dtype, device=cuda)
    k = rnd(sum(lens_k), heads, qk, gen=gen, dtype=dtype, device=cuda)
    v = rnd(sum(lens_k), heads, qk, gen=gen, dtype=dtype, device=cuda)[..., :vd]
    padded = torch.nn.functional.pad(v, (0, qk - vd))
    b = MI355XAttention(heads, qk, SCALE, heads)
    args = (cumulative(lens_q, cuda), cumulative(lens_k, cuda), max(lens_q), max(lens_k), causal)
    out, lse = b.varlen_with_lse(q, k, v, *args)
    wide, wide_lse = b.varlen_with_lse(q, k, padded, *args)
    assert out.shape[-1] == vd
    torch.testing.assert_close(out, wide[..., :vd], **TOL[dtype])
    torch.testing.assert_close(lse, wide_lse, **TOL[dtype])
    split = lambda x, lens: list(torch.split(x, lens))  # noqa: E731
    want, want_lse = dense_rows(split(q, lens_q), split(k, lens_k), split(v, lens_k), causal)
    torch.testing.assert_close(out.float().cpu(), want, **TOL[dtype])
    torch.testing.assert_close(lse.cpu(), want_lse, **TOL[dtype])
    if causal:
        ctx = Context(is_prefill=True, cu_seqlens_q=args[0], cu_seqlens_k=args[1], max_seqlen_q=args[2],
                      max_seqlen_k=args[3])
        empty = torch.tensor([], dtype=dtype, device=cuda)
        torch.testing.assert_close(b.prefill(q, k, v, empty, empty, ctx), out, atol=0, rtol=0)


def test_mla_prefill_shape_against_the_torch_restatement(cuda):
    """DeepSeek-V2-Lite's expanded prefill (16 heads, 192/128) on a 1536-token chunk beside short rows."""
    dtype, heads, qk, vd = torch.bfloat16, 16, 192, 128
    gen = torch.Generator().manual_seed(3)
    lens = [1536, 3, 400]
    q = rnd(sum(lens), heads, qk, gen=gen, dtype=dtype, device=cuda)
    k = rnd(sum(lens), heads, qk, gen=gen, dtype=dtype, device=cuda)
    v = rnd(sum(lens), heads, vd, gen=gen, dtype=dtype, device=cuda)
    cu = cumulative(lens, cuda)
    out, lse = MI355XAttention(heads, qk, 1 / 192 ** 0.5, heads).varlen_with_lse(q, k, v, cu, cu, max(lens),
                                                                                 max(lens), True)
    m = A.TorchMath(heads, qk, 1 / 192 ** 0.5, heads)
    want, want_lse = m.varlen_with_lse(q.cpu(), k.cpu(), v.cpu(), cu.cpu(), cu.cpu(), max(lens), max(lens), True)
    torch.testing.assert_close(out.float().cpu(), want, **TOL[dtype])
    torch.testing.assert_close(lse.cpu(), want_lse, **TOL[dtype])


def test_rows_without_keys_give_zero_and_minus_infinity(cuda):
    gen = torch.Generator().manual_seed(4)
    q = rnd(4, H, 64, gen=gen, dtype=torch.bfloat16, device=cuda)
    k = rnd(3, HKV, 64, gen=gen, dtype=torch.bfloat16, device=cuda)
    v = rnd(3, HKV, 64, gen=gen, dtype=torch.bfloat16, device=cuda)
    out, lse = MI355XAttention(H, 64, SCALE, HKV).varlen_with_lse(
        q, k, v, cumulative([2, 2], cuda), cumulative([0, 3], cuda), 2, 3, False)
    assert torch.equal(out[:2], torch.zeros_like(out[:2]))
    assert torch.isneginf(lse[:2]).all() and torch.isfinite(lse[2:]).all()


def test_merge_of_a_split_equals_the_whole(cuda):
    """Unmasked attention over a row's keys == the merge of attention over its two halves."""
    gen = torch.Generator().manual_seed(5)
    q = rnd(6, H, 128, gen=gen, dtype=torch.bfloat16, device=cuda)
    k = rnd(40, HKV, 128, gen=gen, dtype=torch.bfloat16, device=cuda)
    v = rnd(40, HKV, 128, gen=gen, dtype=torch.bfloat16, device=cuda)
    b = MI355XAttention(H, 128, SCALE, HKV)
    cq = cumulative([6], cuda)
    whole, whole_lse = b.varlen_with_lse(q, k, v, cq, cumulative([40], cuda), 6, 40, False)
    o_a, lse_a = b.varlen_with_lse(q, k[:17], v[:17], cq, cumulative([17], cuda), 6, 17, False)
    o_b, lse_b = b.varlen_with_lse(q, k[17:], v[17:], cq, cumulative([23], cuda), 6, 23, False)
    merge_attention_(o_a, lse_a, o_b, lse_b)
    torch.testing.assert_close(o_a, whole, **TOL[torch.bfloat16])
    torch.testing.assert_close(lse_a, whole_lse, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("dim", [128, 192, 100], ids=["d128", "d192", "d100-scalar"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("into", [False, True], ids=["in_place", "into_out"])
def test_merge_matches_the_oracle(cuda, dtype, into, dim):
    """In place or into an output strided as a split's rows, with lse in a transposed layout and a row whose lse
    is -inf (no cached keys), as tests/test_attention_backends.py:266-287. Widths that are multiples of 8 take
    16-byte lanes (192: rows of 24 lanes, 10 to a workgroup); 100 takes the element-wise kernel."""
    gen = torch.Generator().manual_seed(6)
    tokens, heads = 37, 16
    o_a = rnd(tokens, heads, dim, gen=gen, dtype=dtype, device=cuda)
    o_b = rnd(tokens, heads, dim, gen=gen, dtype=dtype, device=cuda)
    lse_a = (torch.randn(heads, tokens, generator=gen) * 3).to(cuda).T
    lse_b = (torch.randn(heads, tokens, generator=gen) * 3).to(cuda).T
    lse_a[0] = float("-inf")
    want_o, want_lse = A.merge_attention(o_a.cpu(), lse_a.cpu(), o_b.cpu(), lse_b.cpu())
    got_o, got_lse = merge_attention(o_a, lse_a, o_b, lse_b)
    torch.testing.assert_close(got_o.float().cpu(), want_o, atol=1e-2, rtol=1e-2)
    torch.testing.assert_close(got_lse.cpu(), want_lse)
    before = o_a.clone()
    out = torch.empty(tokens + 3, heads, dim, dtype=dtype, device=cuda)[3:] if into else None
    merge_attention_(o_a, lse_a, o_b, lse_b, out)
    torch.testing.assert_close((o_a if out is None else out).float().cpu(), want_o, atol=1e-2, rtol=1e-2)
    torch.testing.assert_close(lse_a.cpu(), want_lse)
    if into:
        assert torch.equal(o_a, before)


@pytest.mark.parametrize("path", ["two_pass_and_merge", "one_call"])
def test_full_size_mla_prefill_step(cuda, path):
    """The measured DeepSeek-V2-Lite prefill step at full size (4 chunks of 1536 new tokens on prefixes up to 6144,
    192-wide q.k and 128-wide values), either as the reference's layer runs it (causal attention over each chunk,
    unmasked attention over its prefix, the LSE merge) or in one ``prefill_with_context`` call, as the bench runs
    it. Every 64th query of every chunk and its last query are checked against the fp32 oracle over the prefix keys
    followed by the chunk's keys up to the query."""
    import numpy as np

    from lvattn import workloads as W

    wl = W.deepseek_v2_lite_mla_prefill()
    ex = W.materialize(wl, cuda).expanded
    b = MI355XAttention(wl.num_heads, wl.expanded[0], wl.scale, wl.num_heads)
    cu_q_host = [0, *np.cumsum(wl.num_new).tolist()]
    cu_c_host = [0, *np.cumsum(wl.num_cached).tolist()]
    cu_q = torch.tensor(cu_q_host, dtype=torch.int32, device=cuda)
    cu_c = torch.tensor(cu_c_host, dtype=torch.int32, device=cuda)
    max_q, max_c = max(wl.num_new), max(max(wl.num_cached), 1)
    if path == "one_call":
        out = b.prefill_with_context(ex["q"], ex["k"], ex["v"], ex["k_ctx"], ex["v_ctx"], cu_q, cu_c, max_q)
    else:
        o, lse = b.varlen_with_lse(ex["q"], ex["k"], ex["v"], cu_q, cu_q, max_q, max_q, True)
        co, clse = b.varlen_with_lse(ex["q"], ex["k_ctx"], ex["v_ctx"], cu_q, cu_c, max_q, max_c, False)
        out = torch.empty_like(o)
        merge_attention_(co, clse, o, lse, out)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    for r in range(len(wl.num_new)):
        k_row = torch.cat([ex["k_ctx"][cu_c_host[r]:cu_c_host[r + 1]], ex["k"][cu_q_host[r]:cu_q_host[r + 1]]])
        v_row = torch.cat([ex["v_ctx"][cu_c_host[r]:cu_c_host[r + 1]], ex["v"][cu_q_host[r]:cu_q_host[r + 1]]])
        k_row, v_row = k_row.cpu().float(), v_row.cpu().float()
        prefix = wl.num_cached[r]
        for j in sorted(set(range(0, wl.num_new[r], 64)) | {wl.num_new[r] - 1}):
            t = cu_q_host[r] + j
            k, v = k_row[:prefix + j + 1], v_row[:prefix + j + 1]
            want = A.dense_attention(ex["q"][t:t + 1].cpu().float(), k, v, wl.scale, causal=False)
            torch.testing.assert_close(out[t:t + 1].float().cpu(), want, **TOL[torch.bfloat16],
                                       msg=lambda m: f"chunk {r} query {j}: {m}")


CTX_CASES = [(torch.bfloat16, 16, 16, 192, 128), (torch.bfloat16, 8, 2, 128, 128), (torch.float16, 8, 2, 64, 64),
             (torch.bfloat16, 4, 4, 192, 192)]


@pytest.mark.parametrize("dtype, heads, kv_heads, qk, vd", CTX_CASES, ids=["mla-192-128", "gqa-128", "fp16-64",
                                                                            "192-192"])
def test_prefill_with_context(cuda, dtype, heads, kv_heads, qk, vd):
    """One call over context keys then causal new keys equals the dense oracle over each row's [context; new] keys
    with the causal mask aligned to the end: rows with no context, with context a multiple of the 64-key tile and
    not, with one query, and with more queries than one item holds; lse included. The two-pass path (causal and
    unmasked varlen_with_lse, then the merge) agrees within the same tolerance."""
    gen = torch.Generator().manual_seed(5)
    lens_q = [5, 1, 12, 300, 70, 64]
    lens_c = [0, 7, 64, 333, 1, 128]
    q = rnd(sum(lens_q), heads, qk, gen=gen, dtype=dtype, device=cuda)
    k = rnd(sum(lens_q), kv_heads, qk, gen=gen, dtype=dtype, device=cuda)
    v = rnd(sum(lens_q), kv_heads, vd, gen=gen, dtype=dtype, device=cuda)
    kc = rnd(sum(lens_c), kv_heads, qk, gen=gen, dtype=dtype, device=cuda)
    vc = rnd(sum(lens_c), kv_heads, vd, gen=gen, dtype=dtype, device=cuda)
    cu_q, cu_c = cumulative(lens_q, cuda), cumulative(lens_c, cuda)
    b = MI355XAttention(heads, qk, SCALE, kv_heads)
    out, lse = b.prefill_with_context(q, k, v, kc, vc, cu_q, cu_c, max(lens_q), want_lse=True)
    torch.cuda.synchronize()
    qs, ks, vs = [], [], []
    oq = oc = 0
    for nq, nc in zip(lens_q, lens_c):
        qs.append(q[oq:oq + nq])
        ks.append(torch.cat([kc[oc:oc + nc], k[oq:oq + nq]]))
        vs.append(torch.cat([vc[oc:oc + nc], v[oq:oq + nq]]))
        oq, oc = oq + nq, oc + nc
    want, want_lse = dense_rows(qs, ks, vs, True)
    torch.testing.assert_close(out.float().cpu(), want, **TOL[dtype])
    torch.testing.assert_close(lse.cpu(), want_lse, **TOL[dtype])
    o1, l1 = b.varlen_with_lse(q, k, v, cu_q, cu_q, max(lens_q), max(lens_q), True)
    o2, l2 = b.varlen_with_lse(q, kc, vc, cu_q, cu_c, max(lens_q), max(lens_c), False)
    two = torch.empty_like(o1)
    merge_attention_(o2, l2, o1, l1, two)
    torch.testing.assert_close(out.float().cpu(), two.float().cpu(), **TOL[dtype])


def test_prefill_with_context_writes_into_a_strided_out(cuda):
    """``out`` as a view of a wider buffer (the layer's output slice): only its columns change."""
    dtype, heads, qk, vd = torch.bfloat16, 16, 192, 128
    gen = torch.Generator().manual_seed(6)
    lens_q, lens_c = [9, 130], [65, 0]
    q = rnd(sum(lens_q), heads, qk, gen=gen, dtype=dtype, device=cuda)
    k = rnd(sum(lens_q), heads, qk, gen=gen, dtype=dtype, device=cuda)
    v = rnd(sum(lens_q), heads, vd, gen=gen, dtype=dtype, device=cuda)
    kc = rnd(sum(lens_c), heads, qk, gen=gen, dtype=dtype, device=cuda)
    vc = rnd(sum(lens_c), heads, vd, gen=gen, dtype=dtype, device=cuda)
    cu_q, cu_c = cumulative(lens_q, cuda), cumulative(lens_c, cuda)
    b = MI355XAttention(heads, qk, SCALE, heads)
    wide = torch.full((sum(lens_q), heads, vd + 64), 3.0, dtype=dtype, device=cuda)
    b.prefill_with_context(q, k, v, kc, vc, cu_q, cu_c, max(lens_q), out=wide[..., :vd])
    want = b.prefill_with_context(q, k, v, kc, vc, cu_q, cu_c, max(lens_q))
    torch.cuda.synchronize()
    assert torch.equal(wide[..., :vd], want) and (wide[..., vd:] == 3.0).all()


# Token rows 2^23 - 8 elements (16 MiB) apart: a 64-key tile spans just under 2^30 bytes, the largest token stride
# the library accepts.
WIDE_STRIDE = (1 << 23) - 8


def widen(x):
    """The same values with token rows WIDE_STRIDE elements apart."""
    t, h, d = x.shape
    w = torch.empty(t, WIDE_STRIDE, dtype=x.dtype, device=x.device)[:, :h * d].view(t, h, d)
    w.copy_(x)
    assert w.stride(0) == WIDE_STRIDE
    return w


def test_packed_keys_at_the_largest_accepted_stride(cuda):
    """Keys, values and context keys whose token rows lie 16 MiB apart: the 24-bit row offsets of the tiles reach
    their largest values. MLA prefill's widths over context keys, and causal varlen_with_lse, give the same bits as
    with packed tensors; the context call also matches the dense oracle."""
    dtype, heads, qk, vd = torch.bfloat16, 16, 192, 128
    gen = torch.Generator().manual_seed(7)
    lens_q, lens_c = [70, 5], [65, 3]
    q = rnd(sum(lens_q), heads, qk, gen=gen, dtype=dtype, device=cuda)
    k = rnd(sum(lens_q), heads, qk, gen=gen, dtype=dtype, device=cuda)
    v = rnd(sum(lens_q), heads, vd, gen=gen, dtype=dtype, device=cuda)
    kc = rnd(sum(lens_c), heads, qk, gen=gen, dtype=dtype, device=cuda)
    vc = rnd(sum(lens_c), heads, vd, gen=gen, dtype=dtype, device=cuda)
    cu_q, cu_c = cumulative(lens_q, cuda), cumulative(lens_c, cuda)
    b = MI355XAttention(heads, qk, SCALE, heads)
    wk, wv, wkc, wvc = widen(k), widen(v), widen(kc), widen(vc)
    out, lse = b.prefill_with_context(q, k, v, kc, vc, cu_q, cu_c, max(lens_q), want_lse=True)
    w_out, w_lse = b.prefill_with_context(q, wk, wv, wkc, wvc, cu_q, cu_c, max(lens_q), want_lse=True)
    o, ls = b.varlen_with_lse(q, k, v, cu_q, cu_q, max(lens_q), max(lens_q), True)
    w_o, w_ls = b.varlen_with_lse(q, wk, wv, cu_q, cu_q, max(lens_q), max(lens_q), True)
    torch.cuda.synchronize()
    assert torch.equal(w_out, out) and torch.equal(w_lse, lse)
    assert torch.equal(w_o, o) and torch.equal(w_ls, ls)
    qs, ks, vs = [], [], []
    oq = oc = 0
    for nq, nc in zip(lens_q, lens_c):
        qs.append(q[oq:oq + nq])
        ks.append(torch.cat([kc[oc:oc + nc], k[oq:oq + nq]]))
        vs.append(torch.cat([vc[oc:oc + nc], v[oq:oq + nq]]))
        oq, oc = oq + nq, oc + nc
    want, want_lse = dense_rows(qs, ks, vs, True)
    torch.testing.assert_close(w_out.float().cpu(), want, **TOL[dtype])
    torch.testing.assert_close(w_lse.cpu(), want_lse, **TOL[dtype])


@pytest.mark.parametrize("factor", [6, 40])
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "unmasked"])
@pytest.mark.parametrize("dtype, dim", CASES, ids=IDS)
def test_scores_far_above_the_first_tile(cuda, dtype, dim, causal, factor):
    """Keys from 64 onward scaled 40x: the held max of the item's first tile fails its check and the item runs
    again with a running max. Scaled 6x, some 20-30 log2 units higher: the held max stands in bf16 (P up to 2^30)
    and fp16 keeps the running max (its P would overflow). Output and log-sum-exp against the fp32 oracle."""
    gen = torch.Generator().manual_seed(2)
    lens_q = [150, 3, 90]
    lens_k = lens_q if causal else [170, 80, 200]
    qs = [rnd(n, H, dim, gen=gen, dtype=dtype, device=cuda) for n in lens_q]
    ks = [rnd(n, HKV, dim, gen=gen, dtype=dtype, device=cuda) for n in lens_k]
    vs = [rnd(n, HKV, dim, gen=gen, dtype=dtype, device=cuda) for n in lens_k]
    for k in ks:
        k[64:] *= factor
    out, lse = MI355XAttention(H, dim, SCALE, HKV).varlen_with_lse(
        torch.cat(qs), torch.cat(ks), torch.cat(vs), cumulative(lens_q, cuda), cumulative(lens_k, cuda),
        max(lens_q), max(lens_k), causal)
    want, want_lse = dense_rows(qs, ks, vs, causal)
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    torch.testing.assert_close(out.float().cpu(), want, **TOL[dtype])
    torch.testing.assert_close(lse.cpu(), want_lse, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("factor", [6, 40])
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "unmasked"])
def test_scores_far_above_the_first_tile_mla_widths(cuda, causal, factor):
    """The same for MLA prefill's expanded heads (q.k 192, values 128 as a view), which run 8-wave items: keys from 64
    onward scaled 40x, so the held max fails its check and the item runs again with a running max, or 6x, so that
    the held max stands with probabilities up to about 2^30."""
    dtype, heads, qk, vd = torch.bfloat16, 16, 192, 128
    gen = torch.Generator().manual_seed(3)
    lens_q = [300, 5, 140]
    lens_k = lens_q if causal else [310, 90, 150]
    q = rnd(sum(lens_q), heads, qk, gen=gen, dtype=dtype, device=cuda)
    k = rnd(sum(lens_k), heads, qk, gen=gen, dtype=dtype, device=cuda)
    v = rnd(sum(lens_k), heads, qk, gen=gen, dtype=dtype, device=cuda)[..., :vd]
    ks = list(torch.split(k, lens_k))
    for kr in ks:
        kr[64:] *= factor
    out, lse = MI355XAttention(heads, qk, SCALE, heads).varlen_with_lse(
        q, k, v, cumulative(lens_q, cuda), cumulative(lens_k, cuda), max(lens_q), max(lens_k), causal)
    want, want_lse = dense_rows(list(torch.split(q, lens_q)), ks, list(torch.split(v, lens_k)), causal)
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    torch.testing.assert_close(out.float().cpu(), want, **TOL[dtype])
    torch.testing.assert_close(lse.cpu(), want_lse, rtol=1e-4, atol=1e-4)
