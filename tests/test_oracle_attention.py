"""Pins the attention oracle (CPU only): brute-force loops, closed forms, the reference's invariants and known
answers, and planted mistakes that each check must reject."""

import math

import pytest
import torch

from oracle import attention as A
from oracle import store as S

H, HKV, D, SCALE, BS = 8, 2, 64, 0.137, 16  # the reference tests' shapes (tests/test_attention_backends.py:23-29)
TOL = 2e-3


def randn(*shape, gen):
    return torch.randn(*shape, generator=gen)


@pytest.fixture
def gen():
    g = torch.Generator()
    g.manual_seed(0)
    return g


def slots_for(table, bs, start, end):
    return [table[p // bs] * bs + p % bs for p in range(start, end)]


def paged_step(gen, num_cached, num_new, tables, nblocks, bs=BS, heads=H, kv_heads=HKV, dim=D):
    """Rows with cached prefixes and new tokens; the cache holds every key (prefix written earlier, new stored)."""
    kc = torch.zeros(nblocks, bs, kv_heads, dim)
    vc = torch.zeros(nblocks, bs, kv_heads, dim)
    qs, ks, vs = [], [], []
    for c, n, t in zip(num_cached, num_new, tables):
        k, v = randn(c + n, kv_heads, dim, gen=gen), randn(c + n, kv_heads, dim, gen=gen)
        S.store_kvcache(k, v, kc, vc, slots_for(t, bs, 0, c + n))
        qs.append(randn(n, heads, dim, gen=gen))
        ks.append(k)
        vs.append(v)
    totals = [c + n for c, n in zip(num_cached, num_new)]
    ctx = A.context(
        is_prefill=True,
        cu_seqlens_q=torch.tensor([0, *torch.tensor(num_new).cumsum(0).tolist()], dtype=torch.int32),
        cu_seqlens_k=torch.tensor([0, *torch.tensor(totals).cumsum(0).tolist()], dtype=torch.int32),
        max_seqlen_q=max(num_new),
        max_seqlen_k=max(totals),
        context_lens=torch.tensor(totals, dtype=torch.int32),
        block_tables=torch.tensor(tables, dtype=torch.int32),
    )
    return qs, ks, vs, kc, vc, ctx


# ------------------------------------------------------------------------------------------------ brute force

@pytest.mark.parametrize("lq, lk, causal", [(1, 7, True), (4, 9, True), (3, 3, True), (5, 6, False)])
def test_dense_matches_brute_force_loops(gen, lq, lk, causal):
    q, k, v = randn(lq, 4, 5, gen=gen), randn(lk, 2, 5, gen=gen), randn(lk, 2, 5, gen=gen)
    want = torch.tensor(A.attention_loops(q, k, v, 0.3, causal))
    torch.testing.assert_close(A.dense_attention(q, k, v, 0.3, causal=causal), want, atol=1e-5, rtol=1e-5)


def test_closed_forms(gen):
    k, v = randn(1, 2, 5, gen=gen), randn(1, 2, 5, gen=gen)
    q = randn(1, 4, 5, gen=gen)
    # one key: the output is its value, whatever the query
    torch.testing.assert_close(A.dense_attention(q, k, v, 0.5), v.repeat_interleave(2, dim=1))
    # equal keys: uniform weights, the mean of the values
    k = randn(1, 2, 5, gen=gen).expand(6, 2, 5).contiguous()
    v = randn(6, 2, 5, gen=gen)
    torch.testing.assert_close(A.dense_attention(q, k, v, 0.5), v.mean(0, keepdim=True).repeat_interleave(2, dim=1))
    # zero query, causal with lq < lk: query j averages the first lk - lq + j + 1 values
    q0 = torch.zeros(3, 4, 5)
    k, v = randn(8, 2, 5, gen=gen), randn(8, 2, 5, gen=gen)
    out = A.dense_attention(q0, k, v, 0.5)
    for j in range(3):
        torch.testing.assert_close(out[j], v[: 8 - 3 + j + 1].mean(0).repeat_interleave(2, dim=0))
    # lse of a zero query over n keys is log n
    torch.testing.assert_close(A.dense_lse(torch.zeros(1, 4, 5), k, 0.5, causal=False),
                               torch.full((1, 4), math.log(8.0)))


# ----------------------------------------------------------------------------- TorchMath vs the dense oracle

def expected(qs, ks, vs, scale=SCALE):
    return torch.cat([A.dense_attention(q, k, v, scale) for q, k, v in zip(qs, ks, vs)])


def test_prefill_without_cache(gen):
    """tests/test_attention_backends.py:171-190: keys from k/v, no pages."""
    seqlens = [5, 1, 12]
    qs = [randn(n, H, D, gen=gen) for n in seqlens]
    ks = [randn(n, HKV, D, gen=gen) for n in seqlens]
    vs = [randn(n, HKV, D, gen=gen) for n in seqlens]
    cu = torch.tensor([0, 5, 6, 18], dtype=torch.int32)
    ctx = A.context(is_prefill=True, cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=12, max_seqlen_k=12)
    out = A.TorchMath(H, D, SCALE, HKV).prefill(torch.cat(qs), torch.cat(ks), torch.cat(vs), None, None, ctx)
    torch.testing.assert_close(out, expected(qs, ks, vs), atol=TOL, rtol=TOL)


@pytest.mark.parametrize("num_cached, num_new, tables, nblocks", [
    ([0, 0], [5, BS + 3], [[0, 1, -1], [2, 3, 4]], 6),                              # cold pages :290-325
    ([2 * BS + 2, 0], [6, 5], [[0, 1, 2, 3, 4, 5], [6, 7, -1, -1, -1, -1]], 8),       # prefix cache :328-368
    ([2 * BS + 5, BS + 1, 0], [1, 7, 4], [[0, 1, 2], [3, 4, -1], [5, -1, -1]], 6),    # mixed :800-814
])
def test_paged_prefill(gen, num_cached, num_new, tables, nblocks):
    qs, ks, vs, kc, vc, ctx = paged_step(gen, num_cached, num_new, tables, nblocks)
    out = A.TorchMath(H, D, SCALE, HKV).prefill(torch.cat(qs), None, None, kc, vc, ctx)
    torch.testing.assert_close(out, expected(qs, ks, vs), atol=TOL, rtol=TOL)


def test_decode(gen):
    """tests/test_attention_backends.py:526-547: mid-page, part-page and full rows."""
    lens = [BS + 3, 3, 4 * BS]
    tables = [[0, 1, 2, 3], [4, 5, -1, -1], [6, 7, 8, 9]]
    qs, ks, vs, kc, vc, _ = paged_step(gen, [n - 1 for n in lens], [1, 1, 1], tables, 10)
    ctx = A.context(context_lens=torch.tensor(lens, dtype=torch.int32), block_tables=torch.tensor(tables, dtype=torch.int32))
    out = A.TorchMath(H, D, SCALE, HKV).decode(torch.cat(qs), kc, vc, ctx)
    torch.testing.assert_close(out, expected(qs, ks, vs), atol=TOL, rtol=TOL)


def test_decode_equals_one_token_prefill(gen):
    """tests/test_attention_backends.py:623-660."""
    n = 2 * BS + 1
    qs, ks, vs, kc, vc, ctx = paged_step(gen, [n - 1], [1], [[0, 1, 2]], 3)
    m = A.TorchMath(H, D, SCALE, HKV)
    dec = m.decode(qs[0], kc, vc, A.context(context_lens=ctx.context_lens, block_tables=ctx.block_tables))
    torch.testing.assert_close(dec, m.prefill(qs[0], None, None, kc, vc, ctx), atol=TOL, rtol=TOL)


def test_bottom_right_is_not_top_left(gen):
    """tests/test_attention_backends.py:663-702: with lq < lk the top-left mask gives a different answer."""
    lq, lk = 4, 2 * BS + 2
    qs, ks, vs, kc, vc, ctx = paged_step(gen, [lk - lq], [lq], [[0, 1, 2]], 3)
    out = A.TorchMath(H, D, SCALE, HKV).prefill(qs[0], None, None, kc, vc, ctx)
    torch.testing.assert_close(out, A.dense_attention(qs[0], ks[0], vs[0], SCALE), atol=TOL, rtol=TOL)
    top_left = torch.nn.functional.scaled_dot_product_attention(
        qs[0].transpose(0, 1), ks[0].repeat_interleave(4, 1).transpose(0, 1), vs[0].repeat_interleave(4, 1).transpose(0, 1),
        is_causal=True, scale=SCALE).transpose(0, 1)
    assert not torch.allclose(out, top_left, atol=5 * TOL)


@pytest.mark.parametrize("mode", ["decode", "prefill", "mla_decode"])
@pytest.mark.parametrize("poison", [float("nan"), float("inf")])
def test_unwritten_slots_are_ignored(mode, poison):
    """tests/test_attention_backends.py:142-168: NaN/inf in unused slots and padding pages never leak."""
    m = A.TorchMath(2, 4, 0.5, 1)
    cache = torch.full((3, 2, 1, 4), poison)
    cache[1, 0] = 1
    cache[2] = 1
    cache[0, 0] = 1
    ctx = A.context(is_prefill=mode == "prefill", block_tables=torch.tensor([[1, -1], [2, 0]], dtype=torch.int32),
                    context_lens=torch.tensor([1, 3], dtype=torch.int32),
                    cu_seqlens_q=torch.tensor([0, 1, 2], dtype=torch.int32),
                    cu_seqlens_k=torch.tensor([0, 1, 4], dtype=torch.int32), max_seqlen_q=1, max_seqlen_k=3)
    q = torch.ones(2, 2, 4)
    if mode == "mla_decode":
        out = m.mla_decode(q, cache.squeeze(2), 2, ctx)
    elif mode == "prefill":
        out = m.prefill(q, None, None, cache, cache, ctx)
    else:
        out = m.decode(q, cache, cache, ctx)
    torch.testing.assert_close(out, torch.ones_like(out))


@pytest.mark.parametrize("causal", [True, False])
def test_varlen_with_lse(gen, causal):
    """tests/test_attention_backends.py:194-222, with 192-wide keys and 128-wide values as well."""
    for dq, dv in ((D, D), (192, 128)):
        lq = [5, 1, 12]
        lk = lq if causal else [7, 4, 16]
        qs = [randn(n, H, dq, gen=gen) for n in lq]
        ks = [randn(n, HKV, dq, gen=gen) for n in lk]
        vs = [randn(n, HKV, dv, gen=gen) for n in lk]
        cu = lambda ls: torch.tensor([0, *torch.tensor(ls).cumsum(0).tolist()], dtype=torch.int32)  # noqa: E731
        o, lse = A.TorchMath(H, dq, SCALE, HKV).varlen_with_lse(torch.cat(qs), torch.cat(ks), torch.cat(vs), cu(lq),
                                                                 cu(lk), max(lq), max(lk), causal)
        want = torch.cat([A.dense_attention(q, k, v, SCALE, causal=causal) for q, k, v in zip(qs, ks, vs)])
        want_lse = torch.cat([A.dense_lse(q, k, SCALE, causal) for q, k in zip(qs, ks)])
        torch.testing.assert_close(o, want, atol=TOL, rtol=TOL)
        torch.testing.assert_close(lse, want_lse, atol=TOL, rtol=TOL)


def test_merge_of_a_split_equals_the_whole(gen):
    """merge.py:8-15: attention over keys [0, a) and [a, n), merged by lse, equals attention over [0, n)."""
    n, a = 40, 17
    kc = torch.zeros(3, BS, HKV, D)
    vc = torch.zeros(3, BS, HKV, D)
    k, v = randn(n, HKV, D, gen=gen), randn(n, HKV, D, gen=gen)
    pages = [2, 0, 1]
    S.store_kvcache(k, v, kc, vc, slots_for(pages, BS, 0, n))
    q = randn(3, H, D, gen=gen)
    whole, whole_lse = A.paged_attention_with_lse(q, kc, vc, n, pages, SCALE, causal=False)
    qa = A.dense_attention(q, k[:a], v[:a], SCALE, causal=False)
    qb = A.dense_attention(q, k[a:], v[a:], SCALE, causal=False)
    la = A.dense_lse(q, k[:a], SCALE, causal=False)
    lb = A.dense_lse(q, k[a:], SCALE, causal=False)
    o, lse = A.merge_attention(qa, la, qb, lb)
    torch.testing.assert_close(o, whole, atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(lse, whole_lse.T, atol=1e-4, rtol=1e-4)
    # a side with no keys (lse = -inf) leaves the other unchanged
    o2, lse2 = A.merge_attention(qa, torch.full_like(la, -math.inf), qb, lb)
    torch.testing.assert_close(o2, qb.float())
    torch.testing.assert_close(lse2, lb)


@pytest.mark.parametrize("queries", [1, 4])
def test_mla_decode_against_dense(gen, queries):
    """tests/test_attention_backends.py:381-436: latents as one shared key head, values = the first 512."""
    bs, lat, vdim = 16, 576, 512
    lens = [bs + 3, 4 if queries > 1 else 3, 2 * bs]
    tables = [[2, 0], [3, -1], [1, 4]]
    cache = torch.zeros(5, bs, lat)
    lats = [randn(n, lat, gen=gen) for n in lens]
    for x, t in zip(lats, tables):
        S.store_latents(x, cache, slots_for(t, bs, 0, x.size(0)))
    q = randn(len(lens) * queries, H, lat, gen=gen)
    ctx = A.context(context_lens=torch.tensor(lens, dtype=torch.int32), block_tables=torch.tensor(tables, dtype=torch.int32))
    out = A.TorchMath(H, lat, SCALE, H).mla_decode(q, cache, vdim, ctx)
    want = torch.cat([
        (A.dense_scores(q[i * queries:(i + 1) * queries], x.unsqueeze(1), SCALE).softmax(-1) @ x[:, :vdim]).transpose(0, 1)
        for i, x in enumerate(lats)])
    torch.testing.assert_close(out, want, atol=TOL, rtol=TOL)


def test_absorbed_mla_equals_expanded_attention(gen):
    """docs/deepseek-v2.md:146-152: q.(W_UK c) = (W_UK^T q).c, and W_UV applies after attention."""
    n_heads, p_dim, r_dim, l_dim, v_dim, bs = 4, 8, 4, 16, 6, 16
    lens = [21, 5]
    tables = [[1, 0], [2, -1]]
    c = [randn(n, l_dim, gen=gen) for n in lens]
    pe = [randn(n, r_dim, gen=gen) for n in lens]
    cache = torch.zeros(3, bs, l_dim + r_dim)
    for ci, pi, t in zip(c, pe, tables):
        S.store_latents(torch.cat([ci, pi], -1), cache, slots_for(t, bs, 0, ci.size(0)))
    w_uk = randn(n_heads, l_dim, p_dim, gen=gen)  # k_nope = c @ W_UK
    w_uv = randn(n_heads, l_dim, v_dim, gen=gen)  # v = c @ W_UV
    q_nope, q_pe = randn(2, n_heads, p_dim, gen=gen), randn(2, n_heads, r_dim, gen=gen)
    ctx = A.context(context_lens=torch.tensor(lens, dtype=torch.int32), block_tables=torch.tensor(tables, dtype=torch.int32))
    got = A.mla_absorbed(q_nope, q_pe, w_uk.transpose(1, 2), w_uv, cache, ctx, 0.3)  # W_UK_T = W_UK^T per head
    for b in range(2):
        k = torch.cat([torch.einsum("nl,hlp->nhp", c[b], w_uk), pe[b].unsqueeze(1).expand(-1, n_heads, -1)], -1)
        v = torch.einsum("nl,hlv->nhv", c[b], w_uv)
        q = torch.cat([q_nope[b:b + 1], q_pe[b:b + 1]], -1)
        torch.testing.assert_close(got[b:b + 1], A.dense_attention(q, k, v, 0.3), atol=1e-4, rtol=1e-4)


# ------------------------------------------------------------------------------------------ planted mistakes

class _DroppedScale(A.TorchMath):
    def __init__(self, *a):
        super().__init__(*a)
        self.scale = 1.0


class _TopLeft(A.TorchMath):
    @classmethod
    def mask(cls, cu_q, cu_k, max_q, max_k, causal):
        m = cls.key_mask(cu_k[1:] - cu_k[:-1], max_k)
        return m & (torch.arange(max_k) <= torch.arange(max_q).view(-1, 1)) if causal else m


class _TiledGroups(A.TorchMath):
    def sdpa(self, q, k, v, mask):  # query head h reads key head h % Hkv (repeat) instead of h // g
        g = self.num_heads // self.num_kv_heads
        k = k.repeat(1, 1, g, 1)
        v = v.repeat(1, 1, g, 1)
        o = torch.nn.functional.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                                             attn_mask=mask, scale=self.scale)
        return o.transpose(1, 2)


@pytest.mark.parametrize("mutant", [_DroppedScale, _TopLeft, _TiledGroups])
def test_planted_mistakes_are_rejected(gen, mutant):
    num_cached, num_new, tables = [2 * BS + 2, 0], [6, 5], [[0, 1, 2, 3, 4, 5], [6, 7, -1, -1, -1, -1]]
    qs, ks, vs, kc, vc, ctx = paged_step(gen, num_cached, num_new, tables, 8)
    good = A.TorchMath(H, D, SCALE, HKV).prefill(torch.cat(qs), None, None, kc, vc, ctx)
    bad = mutant(H, D, SCALE, HKV).prefill(torch.cat(qs), None, None, kc, vc, ctx)
    want = expected(qs, ks, vs)
    torch.testing.assert_close(good, want, atol=TOL, rtol=TOL)
    assert not torch.allclose(bad, want, atol=5 * TOL)


# ------------------------------------------------------------------------------ decode over slices of rows

def _chunked_width_floor(math_, q, k_cache, v_cache, context_lens, block_tables, rows_per_chunk):
    """A planted mistake: each slice's table narrowed to floor(longest / bs) pages (at least one) instead of ceil."""
    outs, bs = [], k_cache.size(1)
    for r0 in range(0, q.size(0), rows_per_chunk):
        lens = context_lens[r0:r0 + rows_per_chunk]
        sub = A.context(context_lens=lens, block_tables=block_tables[r0:r0 + rows_per_chunk, :max(1, int(lens.max()) // bs)])
        outs.append(math_.decode(q[r0:r0 + rows_per_chunk], k_cache, v_cache, sub))
    return torch.cat(outs)


def _chunked_tables_shifted(math_, q, k_cache, v_cache, context_lens, block_tables, rows_per_chunk):
    """A planted mistake: each slice reads the table rows of the slice one row later."""
    outs, bs = [], k_cache.size(1)
    for r0 in range(0, q.size(0), rows_per_chunk):
        lens = context_lens[r0:r0 + rows_per_chunk]
        width = -(-int(lens.max()) // bs)
        rows = torch.arange(r0 + 1, r0 + 1 + lens.numel()).clamp(max=block_tables.size(0) - 1)
        sub = A.context(context_lens=lens, block_tables=block_tables[rows, :width])
        outs.append(math_.decode(q[r0:r0 + rows_per_chunk], k_cache, v_cache, sub))
    return torch.cat(outs)


@pytest.mark.parametrize("rows_per_chunk", [1, 3, 7, 10])
def test_decode_in_row_chunks_equals_decode_of_the_whole_batch(gen, rows_per_chunk):
    """``decode_in_row_chunks`` (the CPU baseline's decode) against ``TorchMath.decode`` of the whole batch and the
    dense oracle: seven rows whose lengths end mid-page, on a page boundary and in the table's last page, sliced
    into chunks of 1, 3, 7 and 10 rows. Each slice's table is narrowed to its own longest row, so slices whose
    longest row ends mid-page (3 BS + 5 in the first chunk of three) and slices that end on a page boundary are both
    exercised; two planted mistakes (a floor for the slice's page count, table rows shifted by one) are rejected."""
    lens = [3 * BS + 5, 2, BS, 6 * BS, BS + 1, 4 * BS - 1, 5]
    width = 6
    pages = torch.randperm(len(lens) * width, generator=gen).tolist()
    tables = [pages[r * width:r * width + -(-n // BS)] + [-1] * (width - -(-n // BS)) for r, n in enumerate(lens)]
    qs, ks, vs, kc, vc, _ = paged_step(gen, [n - 1 for n in lens], [1] * len(lens), tables, len(lens) * width)
    q = torch.cat(qs)
    cl, bt = torch.tensor(lens, dtype=torch.int32), torch.tensor(tables, dtype=torch.int32)
    m = A.TorchMath(H, D, SCALE, HKV)
    whole = m.decode(q, kc, vc, A.context(context_lens=cl, block_tables=bt))
    torch.testing.assert_close(whole, expected(qs, ks, vs), atol=TOL, rtol=TOL)
    got = A.decode_in_row_chunks(m, q, kc, vc, cl, bt, rows_per_chunk)
    torch.testing.assert_close(got, whole, atol=1e-5, rtol=1e-5)
    if rows_per_chunk < len(lens):  # slices narrower than the batch: the mistakes change what a slice reads
        for mutant in (_chunked_width_floor, _chunked_tables_shifted):
            bad = mutant(m, q, kc, vc, cl, bt, rows_per_chunk)
            assert not torch.allclose(bad, whole, atol=5 * TOL), mutant.__name__
