"""Seeded random steps through the HIP backend against the fp32 oracle.

Each paged case draws:
- a head grouping, odd ones included (query groups of 1, 3, 4, 8, and 6 over 2 key heads);
- the head width (64 or 128) and the dtype;
- a page size: one-page ring tiles (64, 128, 256), multi-page ring tiles (16, 32), or register-staged tiles (48);
- an NHD or HND cache;
- the launch schedule (serial or overlapped) for a step with prompts;
- 1-9 rows, each a decode row, a cold prompt or a chunk on a cached prefix, in scheduler order (decode rows first).

Block lists are scattered slices of a shuffled pool. Packed-key rows (all four width pairs, causal or not, with
context keys) and MLA decode rows (part-filled and several head tiles, drafts, split-schedule page sizes) are
drawn the same way. Tolerances are those of the other attention tests: fp16 6e-3 against fp32 (the reference's),
bf16 2e-2 absolute / 1e-2 relative."""

import numpy as np
import pytest
import torch

from helpers import context_for, dense_expected, paged_step
from lvattn import MI355XAttention
from lvattn import backend as B

pytestmark = pytest.mark.gpu

TOL = {torch.float16: dict(atol=6e-3, rtol=6e-3), torch.bfloat16: dict(atol=2e-2, rtol=1e-2)}
HEADS = [(4, 4), (8, 1), (6, 2), (12, 4), (16, 2), (32, 8), (24, 8)]
BLOCK_SIZES = [16, 32, 48, 64, 128, 256]


def draw_step(rng):
    hq, hkv = HEADS[rng.integers(len(HEADS))]
    dim = int(rng.choice([64, 128]))
    dtype = (torch.bfloat16, torch.float16)[int(rng.integers(2))]
    bs = int(rng.choice(BLOCK_SIZES))
    layout = ("NHD", "HND")[int(rng.integers(2))]
    rows = []
    for kind in rng.integers(0, 3, size=int(rng.integers(1, 10))):
        if kind == 0:
            rows.append((int(rng.integers(0, 1500)), 1))  # decode: the key stored this step and its cached prefix
        elif kind == 1:
            rows.append((0, int(rng.integers(2, 200))))  # cold prompt
        else:
            rows.append((int(rng.integers(1, 600)), int(rng.integers(2, 200))))  # chunk on a cached prefix
    rows.sort(key=lambda r: r[1] > 1)  # decode rows first
    cached, new = [r[0] for r in rows], [r[1] for r in rows]
    need = [-(-(c + n) // bs) for c, n in zip(cached, new)]
    pool = sum(need) + int(rng.integers(1, 8))
    perm = rng.permutation(pool).tolist()
    width = max(need) + int(rng.integers(0, 3))
    tables, at = [], 0
    for k in need:
        tables.append(perm[at:at + k] + [-1] * (width - k))
        at += k
    return hq, hkv, dim, dtype, bs, layout, cached, new, tables, pool


@pytest.mark.parametrize("seed", range(24))
def test_random_step_matches_the_oracle(cuda, seed, monkeypatch):
    rng = np.random.default_rng(7000 + seed)
    hq, hkv, dim, dtype, bs, layout, cached, new, tables, pool = draw_step(rng)
    scale = float(rng.uniform(0.05, 0.2))
    label = (f"seed {seed}: heads {hq}/{hkv} dim {dim} {dtype} bs {bs} {layout} "
             f"rows {list(zip(cached, new))}")
    backend = MI355XAttention(hq, dim, scale, hkv)
    qs, kf, vf, kn, vn, kc, vc, slots = paged_step(cached, new, tables, pool, heads=hq, kv_heads=hkv, dim=dim,
                                                   bs=bs, device=cuda, dtype=dtype, seed=seed, layout=layout)
    backend.store_kvcache(kn, vn, kc, vc, slots)
    decode_only = all(n == 1 for n in new)
    if not decode_only:
        sched = (B.SCHEDULE_SERIAL, B.SCHEDULE_OVERLAP)[int(rng.integers(2))]
        monkeypatch.setattr(backend, "_schedule", lambda context, elem_bytes, s=sched: s)
        label += f" schedule {'serial' if sched == B.SCHEDULE_SERIAL else 'overlap'}"
    ctx = context_for(cached, new, tables, cuda, is_prefill=not decode_only or bool(rng.integers(2)))
    out = backend.forward(torch.cat(qs), kn, vn, kc, vc, ctx)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all(), label
    want = dense_expected(qs, kf, vf, scale)
    torch.testing.assert_close(out.float().cpu(), want.float(), **TOL[dtype], msg=lambda m: f"{label}: {m}")


WIDTHS = [(64, 64), (128, 128), (192, 128), (192, 192)]


@pytest.mark.parametrize("seed", range(12))
def test_random_packed_rows_match_the_oracle(cuda, seed):
    """Attention over packed keys (``varlen_with_lse``), and one call over context keys then causal new keys
    (``prefill_with_context``), on random rows, widths and head groupings, outputs and natural lse."""
    from test_gpu_varlen import cumulative, dense_rows, rnd

    rng = np.random.default_rng(8000 + seed)
    hq, hkv = HEADS[rng.integers(len(HEADS))]
    qk, vd = WIDTHS[rng.integers(len(WIDTHS))]
    dtype = (torch.bfloat16, torch.float16)[int(rng.integers(2))]
    scale = float(rng.uniform(0.05, 0.2))
    causal = bool(rng.integers(2))
    rows = int(rng.integers(1, 7))
    lens_q = [int(rng.integers(1, 300)) for _ in range(rows)]
    lens_k = [n + int(rng.integers(0, 200)) if causal else int(rng.integers(1, 400)) for n in lens_q]
    lens_c = [int(rng.integers(0, 400)) for _ in range(rows)]
    label = (f"seed {seed}: heads {hq}/{hkv} widths {qk}/{vd} {dtype} causal {causal} q {lens_q} k {lens_k} "
             f"ctx {lens_c}")
    gen = torch.Generator().manual_seed(seed)
    b = MI355XAttention(hq, qk, scale, hkv)

    qs = [rnd(n, hq, qk, gen=gen, dtype=dtype, device=cuda) for n in lens_q]
    ks = [rnd(n, hkv, qk, gen=gen, dtype=dtype, device=cuda) for n in lens_k]
    vs = [rnd(n, hkv, vd, gen=gen, dtype=dtype, device=cuda) for n in lens_k]
    out, lse = b.varlen_with_lse(torch.cat(qs), torch.cat(ks), torch.cat(vs), cumulative(lens_q, cuda),
                                 cumulative(lens_k, cuda), max(lens_q), max(lens_k), causal)
    torch.cuda.synchronize()
    want, want_lse = dense_rows(qs, ks, vs, causal, scale)
    torch.testing.assert_close(out.float().cpu(), want, **TOL[dtype], msg=lambda m: f"varlen {label}: {m}")
    torch.testing.assert_close(lse.cpu(), want_lse, **TOL[dtype], msg=lambda m: f"varlen lse {label}: {m}")

    # Context keys, then each row's own keys (as many as its queries) under the causal mask.
    k = rnd(sum(lens_q), hkv, qk, gen=gen, dtype=dtype, device=cuda)
    v = rnd(sum(lens_q), hkv, vd, gen=gen, dtype=dtype, device=cuda)
    kc = rnd(max(sum(lens_c), 1), hkv, qk, gen=gen, dtype=dtype, device=cuda)
    vc = rnd(max(sum(lens_c), 1), hkv, vd, gen=gen, dtype=dtype, device=cuda)
    q = torch.cat(qs)
    out, lse = b.prefill_with_context(q, k, v, kc, vc, cumulative(lens_q, cuda), cumulative(lens_c, cuda),
                                      max(lens_q), want_lse=True)
    torch.cuda.synchronize()
    rq, rk, rv = [], [], []
    oq = oc = 0
    for nq, nc in zip(lens_q, lens_c):
        rq.append(q[oq:oq + nq])
        rk.append(torch.cat([kc[oc:oc + nc], k[oq:oq + nq]]))
        rv.append(torch.cat([vc[oc:oc + nc], v[oq:oq + nq]]))
        oq, oc = oq + nq, oc + nc
    want, want_lse = dense_rows(rq, rk, rv, True, scale)
    torch.testing.assert_close(out.float().cpu(), want, **TOL[dtype], msg=lambda m: f"context {label}: {m}")
    torch.testing.assert_close(lse.cpu(), want_lse, **TOL[dtype], msg=lambda m: f"context lse {label}: {m}")


@pytest.mark.parametrize("seed", range(12))
def test_random_mla_decode_matches_the_oracle(cuda, seed):
    """MLA absorbed decode on random rows: head counts that fill part of a 16-head tile or several, 1, 2 or 4
    queries per row, and page sizes that take the balanced runs (multiples of 16) or the split schedule."""
    from test_gpu_mla import check_mla

    rng = np.random.default_rng(9000 + seed)
    heads = int(rng.choice([8, 16, 24, 32, 64]))
    queries = int(rng.choice([1, 2, 4]))
    bs = int(rng.choice([16, 32, 40, 48, 64, 128]))
    dtype = (torch.bfloat16, torch.float16)[int(rng.integers(2))]
    lens = [int(rng.integers(queries, 2500)) for _ in range(int(rng.integers(1, 9)))]
    need = [-(-n // bs) for n in lens]
    perm = rng.permutation(sum(need) + 3).tolist()
    width = max(need)
    tables, at = [], 0
    for k in need:
        tables.append(perm[at:at + k] + [-1] * (width - k))
        at += k
    check_mla(cuda, dtype, bs, lens, tables, queries=queries, heads=heads, seed=seed)


WIDE_HEADS = [(8, 2), (16, 4), (32, 8), (12, 4), (24, 8), (6, 2), (64, 8), (8, 1)]


@pytest.mark.parametrize("seed", range(8))
def test_random_wide_decode_steps_match_the_oracle(cuda, seed, monkeypatch):
    """Steps of 300-1200 decode rows (some with one or two prompt chunks too): enough items that decode items take
    a pair of kv heads where the kv heads are even (16-token wave tiles at d128, 8-token ones at d64), and one head
    where they are odd; one workgroup per item, alone or beside the prompt workgroups. (The persistent grid beside
    prompt workgroups needs more items: test_gpu_attention.py's plan-sharing steps reach it.) The launch route each
    case takes is printed with its label."""
    rng = np.random.default_rng(9500 + seed)
    hq, hkv = WIDE_HEADS[seed % len(WIDE_HEADS)]
    dim = int(rng.choice([64, 128]))
    dtype = (torch.bfloat16, torch.float16)[int(rng.integers(2))]
    bs = int(rng.choice([16, 64, 256]))
    layout = ("NHD", "HND")[int(rng.integers(2))]
    n_dec = int(rng.integers(300, 1200))
    cached = [int(rng.integers(0, 2500)) for _ in range(n_dec)]
    new = [1] * n_dec
    for _ in range(int(rng.integers(0, 3))):
        cached.append(int(rng.integers(0, 500)))
        new.append(int(rng.integers(2, 300)))
    need = [-(-(c + n) // bs) for c, n in zip(cached, new)]
    pool = sum(need) + 3
    perm = rng.permutation(pool).tolist()
    width = max(need)
    tables, at = [], 0
    for k in need:
        tables.append(perm[at:at + k] + [-1] * (width - k))
        at += k
    scale = float(rng.uniform(0.05, 0.2))
    label = (f"seed {seed}: heads {hq}/{hkv} dim {dim} {dtype} bs {bs} {layout} decode rows {n_dec} "
             f"prompts {list(zip(cached[n_dec:], new[n_dec:]))}")
    print(label, flush=True)
    backend = MI355XAttention(hq, dim, scale, hkv)
    qs, kf, vf, kn, vn, kc, vc, slots = paged_step(cached, new, tables, pool, heads=hq, kv_heads=hkv, dim=dim,
                                                   bs=bs, device=cuda, dtype=dtype, seed=seed, layout=layout)
    backend.store_kvcache(kn, vn, kc, vc, slots)
    decode_only = len(new) == n_dec
    if not decode_only:
        sched = (B.SCHEDULE_SERIAL, B.SCHEDULE_OVERLAP)[seed % 2]
        monkeypatch.setattr(backend, "_schedule", lambda context, elem_bytes, s=sched: s)
        label += f" schedule {'serial' if sched == B.SCHEDULE_SERIAL else 'overlap'}"
    ctx = context_for(cached, new, tables, cuda, is_prefill=not decode_only)
    backend.launch_trace = []
    out = backend.forward(torch.cat(qs), kn, vn, kc, vc, ctx)
    torch.cuda.synchronize()
    info = backend.launch_trace[-1]
    label += f" route {info}"
    print(label, flush=True)
    if hkv % 2:
        assert info["kv_heads_per_item"] == 1, label
    assert torch.isfinite(out).all(), label
    want = dense_expected(qs, kf, vf, scale)
    torch.testing.assert_close(out.float().cpu(), want.float(), **TOL[dtype], msg=lambda m: f"{label}: {m}")
