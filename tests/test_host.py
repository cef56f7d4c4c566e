"""Host logic of the boundary (CPU only): the per-step Context split, backend selection, capability flags."""

import pytest
import torch

from lvattn import Context, LayerSpec, MI355XAttention, get_attention_backend, split_decodes_and_prefills
from lvattn.context import get_context, set_context, use_context

BS = 16


def host_context(num_cached, num_new, tables):
    totals = [c + n for c, n in zip(num_cached, num_new)]
    cu_q = [0, *torch.tensor(num_new).cumsum(0).tolist()]
    cu_k = [0, *torch.tensor(totals).cumsum(0).tolist()]
    return Context(
        is_prefill=True,
        cu_seqlens_q=torch.tensor(cu_q, dtype=torch.int32),
        cu_seqlens_k=torch.tensor(cu_k, dtype=torch.int32),
        max_seqlen_q=max(num_new),
        max_seqlen_k=max(totals),
        block_tables=torch.tensor(tables, dtype=torch.int32),
        cu_seqlens_q_host=cu_q,
        cu_seqlens_k_host=cu_k,
        context_lens=torch.tensor(totals, dtype=torch.int32),
    )


def test_the_split_slices_the_leading_one_query_rows():
    """Known answer of tests/test_attention_backends.py:874-889."""
    context = host_context([9, 0, 4, 2 * BS], [1, 1, 5, 3], [[0, -1, -1], [1, -1, -1], [2, -1, -1], [3, 4, 5]])
    n, decodes, prefills = split_decodes_and_prefills(context)
    assert n == 2
    assert decodes.context_lens.tolist() == [10, 1]
    assert decodes.block_tables.tolist() == [[0, -1, -1], [1, -1, -1]]
    assert prefills.cu_seqlens_q.tolist() == prefills.cu_seqlens_q_host == [0, 5, 8]
    assert prefills.cu_seqlens_k.tolist() == prefills.cu_seqlens_k_host == [0, 9, 12 + 2 * BS]
    assert (prefills.max_seqlen_q, prefills.max_seqlen_k) == (5, 3 + 2 * BS)
    assert prefills.block_tables.tolist() == [[2, -1, -1], [3, 4, 5]]
    assert split_decodes_and_prefills(context)[1] is decodes  # cached for every layer


def test_a_step_split_at_no_row_is_left_whole():
    """tests/test_attention_backends.py:892-894."""
    context = host_context([0, 3], [4, 1], [[0], [1]])
    assert split_decodes_and_prefills(context) == (0, None, context)


def test_context_nesting_restores_the_previous_one():
    outer = get_context()
    with set_context(True, max_seqlen_q=3) as ctx:
        assert get_context() is ctx and ctx.is_prefill and ctx.max_seqlen_q == 3
        inner = Context()
        with pytest.raises(ValueError):
            with use_context(inner):
                assert get_context() is inner
                raise ValueError
        assert get_context() is ctx
    assert get_context() is outer


def test_capabilities():
    b = MI355XAttention
    assert b.get_name() == "mi355x"
    assert b.supports_cuda_graph() and b.supports_full_cudagraph() and not b.split_decodes()
    assert b.get_kv_cache_shape(10, 256, 8, 128) == (10, 256, 8, 128)
    assert b.validate(LayerSpec(128, 32, 8, torch.bfloat16)) == []
    assert b.validate(LayerSpec(64, 8, 2, torch.float16)) == []
    assert "dtype torch.float32" in b.validate(LayerSpec(128, 32, 8, torch.float32))[0]
    assert "6 query heads do not group over 4 key heads" in b.validate(LayerSpec(128, 6, 4, torch.bfloat16))
    assert "head size 96 is not supported" in b.validate(LayerSpec(96, 32, 8, torch.bfloat16))


def test_selection_rules(monkeypatch):
    """selector.py:19-39: unknown names raise ValueError; a named backend that cannot serve raises RuntimeError."""
    monkeypatch.setattr(MI355XAttention, "is_available", staticmethod(lambda: True))
    monkeypatch.delenv("LEAN_VLLM_ATTENTION_BACKEND", raising=False)
    assert get_attention_backend(LayerSpec(128, 32, 8, torch.bfloat16)) is MI355XAttention
    with pytest.raises(ValueError, match="unknown attention backend"):
        get_attention_backend(LayerSpec(128, 32, 8, torch.bfloat16), name="nope")
    monkeypatch.setenv("LEAN_VLLM_ATTENTION_BACKEND", "mi355x")
    with pytest.raises(RuntimeError, match="dtype torch.float32"):
        get_attention_backend(LayerSpec(128, 32, 8, torch.float32))


def test_prompt_tiles_overlap_decode_rows_only_when_the_decode_bytes_cover_them():
    """The launch schedule of a step with prompts, from the context's host lengths, cached for every layer."""
    from lvattn import backend as B
    from lvattn import workloads as W

    attn = MI355XAttention(32, 128, 128 ** -0.5, 8)
    mixed = W.qwen3_8b_mixed(0)
    order = W.batch_order(mixed)
    new = [mixed.num_new[i] for i in order]
    ends = [mixed.num_cached[i] + mixed.num_new[i] for i in order]
    cu_q = [0, *torch.tensor(new).cumsum(0).tolist()]
    cu_k = [0, *torch.tensor(ends).cumsum(0).tolist()]
    ctx = Context(cu_seqlens_q_host=cu_q, cu_seqlens_k_host=cu_k)
    assert attn._schedule(ctx, 2) == B.SCHEDULE_OVERLAP  # 18.7 GB of decode rows hide 428 GFLOP of prompt tiles
    # The same decode rows beside 6 and 12 prompt chunks of 1536 tokens on 3000-token prefixes (569 and 1138
    # GFLOP): overlapped, the first still wins; the second ran 35% slower overlapped than serially.
    dec_new, dec_ends = [n for n in new if n == 1], [e for n, e in zip(new, ends) if n == 1]
    for chunks, want in ((6, B.SCHEDULE_OVERLAP), (12, B.SCHEDULE_SERIAL)):
        q = dec_new + [1536] * chunks
        k = dec_ends + [3000 + 1536] * chunks
        step = Context(cu_seqlens_q_host=[0, *torch.tensor(q).cumsum(0).tolist()],
                       cu_seqlens_k_host=[0, *torch.tensor(k).cumsum(0).tolist()])
        assert attn._schedule(step, 2) == want, chunks
        if want == B.SCHEDULE_OVERLAP:  # more prompt work than the mixed step: more than half the CUs asked for
            assert attn._prompt_workgroups(step, 2) > attn._prompt_workgroups(ctx, 2) > 100
    assert ctx.attn_metadata  # cached on the step's context
    prompts = Context(cu_seqlens_q_host=[0, 1536, 3072], cu_seqlens_k_host=[0, 2000, 5000])
    assert attn._schedule(prompts, 2) == B.SCHEDULE_SERIAL  # no decode rows: the prompt tiles take the whole GPU
    few = Context(cu_seqlens_q_host=[0, 1, 2, 1538], cu_seqlens_k_host=[0, 300, 600, 4000])
    assert attn._schedule(few, 2) == B.SCHEDULE_SERIAL
    assert attn._schedule(Context(), 2) == B.SCHEDULE_AUTO  # no host lengths: the library default


def test_the_schedule_choice_matches_a_per_row_count_in_any_row_order():
    """The bisection over leading one-query rows plus the walk over the rest equals a plain per-row count, for
    decode-first steps and for rows in any order."""
    import random

    from lvattn import backend as B

    attn = MI355XAttention(16, 128, 0.1, 8)
    rng = random.Random(0)
    for trial in range(200):
        rows = rng.randint(1, 40)
        lq = [1 if rng.random() < 0.7 else rng.randint(2, 3000) for _ in range(rows)]
        lk = [q + rng.randint(0, 20000 if q == 1 else 4000) for q in lq]
        if trial % 2 == 0:  # decode-first, as prepare_batch orders rows
            order = sorted(range(rows), key=lambda r: lq[r] != 1)
            lq, lk = [lq[r] for r in order], [lk[r] for r in order]
        cu_q = [0, *torch.tensor(lq).cumsum(0).tolist()]
        cu_k = [0, *torch.tensor(lk).cumsum(0).tolist()]
        dec = sum(k for q, k in zip(lq, lk) if q == 1) * 2 * 8 * 128 * 2
        flops = sum(4 * 16 * 128 * sum(k - q + j + 1 for j in range(q)) for q, k in zip(lq, lk) if q > 1)
        want = B.SCHEDULE_OVERLAP if dec / B.DECODE_BYTES_PER_S >= flops / B.PROMPT_FLOPS_PER_S else B.SCHEDULE_SERIAL
        assert attn._schedule(Context(cu_seqlens_q_host=cu_q, cu_seqlens_k_host=cu_k), 2) == want


def test_host_staging_lays_out_the_rows_as_the_pack_kernel_reads_them():
    """num_cached | num_new | block-list offsets | block ids, from lists, tuples or numpy rows, as the numpy
    restatement lays them out; mismatched row counts, a short buffer and ids past int32 are refused."""
    import numpy as np

    from lvattn import _hoststage

    rng = np.random.default_rng(3)
    rows = 300
    cached = rng.integers(0, 5000, rows).tolist()
    new = rng.integers(1, 4, rows).tolist()
    lists = [rng.integers(0, 10_000, rng.integers(0, 9)).tolist() for _ in range(rows)]
    lists[7] = tuple(lists[7])
    lists[8] = np.asarray(lists[8], dtype=np.int64)
    n = sum(len(x) for x in lists)
    assert _hoststage.count_ids(lists) == n
    buf = np.full(3 * rows + 1 + n + 5, -7, np.int32)
    got = _hoststage.stage_rows(cached, np.asarray(new), lists, buf.ctypes.data, 3 * rows + 1 + n)
    assert got == (rows, n, max(len(x) for x in lists))
    lengths = np.array([len(x) for x in lists])
    want = np.concatenate([cached, new, [0], np.cumsum(lengths), np.concatenate([np.asarray(x) for x in lists])])
    assert np.array_equal(buf[:3 * rows + 1 + n], want.astype(np.int32))
    assert (buf[3 * rows + 1 + n:] == -7).all()  # nothing written past the capacity given
    with pytest.raises(ValueError, match="one entry per row"):
        _hoststage.stage_rows(cached[:-1], new, lists, buf.ctypes.data, buf.size)
    with pytest.raises(ValueError, match="too small"):
        _hoststage.stage_rows(cached, new, lists, buf.ctypes.data, 3 * rows + n)
    with pytest.raises(OverflowError):
        _hoststage.stage_rows([0], [1], [[2 ** 31]], buf.ctypes.data, buf.size)


def test_graph_staging_pads_rows_with_no_context():
    """A captured step of bs rows: real rows first, then padding rows with num_cached -q (context length 0) and no
    blocks; every row has q new tokens."""
    import numpy as np

    from lvattn import _hoststage

    bs, q = 8, 3
    cached, lists = [4, 0, 9], [[5, 6], [7], [1, 2, 3]]
    buf = np.full(3 * bs + 1 + 6 + 2, -9, np.int32)
    assert _hoststage.stage_graph_rows(cached, lists, buf.ctypes.data, 3 * bs + 1 + 6, bs, q) == (3, 6, 3)
    assert buf[:bs].tolist() == [4, 0, 9] + [-q] * 5
    assert buf[bs:2 * bs].tolist() == [q] * bs
    assert buf[2 * bs:3 * bs + 1].tolist() == [0, 2, 3, 6, 6, 6, 6, 6, 6]
    assert buf[3 * bs + 1:3 * bs + 7].tolist() == [5, 6, 7, 1, 2, 3]
    assert (buf[3 * bs + 7:] == -9).all()
    with pytest.raises(ValueError, match="at most bs rows"):
        _hoststage.stage_graph_rows([0] * 9, [[]] * 9, buf.ctypes.data, buf.size, bs, q)


class _HostBuffers:
    """StagingBuffers on plain host memory (no pinned memory, no device): Packer.stage's host logic on a CPU."""

    def __init__(self):
        self._host = {}

    def host_view(self, name, n, dtype):
        buf = self._host.get(name)
        if buf is None or buf.numel() < n:
            buf = self._host[name] = torch.empty(max(n, 256), dtype=dtype)
        return buf[:n].numpy()

    def upload(self, name, n, dtype):
        return self._host[name][:n].clone()


def host_packer(block_size, decodes_latents=False):
    from lvattn import Packer

    packer = Packer.__new__(Packer)
    packer.block_size, packer.decodes_latents, packer.buffers = block_size, decodes_latents, _HostBuffers()
    return packer


def test_a_block_list_that_does_not_cover_its_row_is_refused():
    """A row whose block list is shorter than its num_cached + num_new tokens need would make the pack kernel read
    another row's blocks; the packer refuses it on the host (rows without a list, as in warmup, are fine)."""
    packer = host_packer(16)
    plan = packer.stage([0, 31, 5], [16, 1, 3], [[4], [7, 8], []])
    assert plan.rows == 3 and plan.slot_count == 17
    with pytest.raises(ValueError, match="row 1's block list holds 1 blocks; its 31 \\+ 2 tokens need 3"):
        packer.stage([0, 31, 5], [16, 2, 3], [[4], [7, 8][:1], []])
    with pytest.raises(ValueError, match="row 0's block list holds 1 blocks; its 0 \\+ 17 tokens need 2"):
        packer.stage([0], [17], [[4]])
    with pytest.raises(ValueError, match="row 1 has num_cached -1"):
        packer.stage([0, -1], [1, 1], [[4], [5]])


def test_the_step_kind_follows_the_reference_rule_for_drafts():
    """model_runner.py:380-384: a step is is_prefill with any prompt row, or with drafts unless the model decodes
    latents and every row has the same query length. Draft rows sample drafts + 1 logits rows by default."""
    k = 2
    packer = host_packer(16)
    plan = packer.stage([10, 20], [3, 3], [[0], [1, 2]], num_speculative_tokens=k)  # both rows verify 2 drafts
    assert plan.host["is_prefill"] and plan.logits == 6  # a decoder model: drafts go to the prefill path
    plan = packer.stage([10, 20], [1, 1], [[0], [1, 2]], num_speculative_tokens=k)
    assert not plan.host["is_prefill"] and plan.logits == -1
    plan = packer.stage([10, 0], [3, 3], [[0], [1]], num_speculative_tokens=k, is_prompt=[False, True])
    assert plan.host["is_prefill"] and plan.logits == 4  # the prompt samples one row, the draft row three
    mla = host_packer(16, decodes_latents=True)
    plan = mla.stage([10, 20], [3, 3], [[0], [1, 2]], num_speculative_tokens=k)
    assert not plan.host["is_prefill"]  # uniform drafts: latent decode with 3 queries per row
    plan = mla.stage([10, 20], [3, 2], [[0], [1, 2]], num_speculative_tokens=k)
    assert plan.host["is_prefill"]  # ragged drafts: the prefill path


def test_the_opt_in_index_checks(monkeypatch):
    """LVATTN_CHECK=1: slots past the pool, table entries past the pool, key lengths a table does not cover and
    inconsistent cu_seqlens raise ValueError before any launch (CPU tensors; nothing reaches the library)."""
    from lvattn import checks

    i32 = dict(dtype=torch.int32)
    checks.check_slots(torch.tensor([-1, 0, 63], **i32), 4, 16)
    with pytest.raises(ValueError, match=r"slot_mapping\[2\] = 64 is outside \[-1, 64\)"):
        checks.check_slots(torch.tensor([-1, 0, 64], **i32), 4, 16)
    with pytest.raises(ValueError, match=r"slot_mapping\[0\] = -2"):
        checks.check_slots(torch.tensor([-2], **i32), 4, 16)
    checks.check_tables(torch.tensor([[0, 3], [2, -1]], **i32), 4)
    with pytest.raises(ValueError, match=r"block_tables\[1, 1\] = 4 is outside \[-1, 4\)"):
        checks.check_tables(torch.tensor([[0, 3], [2, 4]], **i32), 4)
    bt = torch.tensor([[0, 3], [2, -1]], **i32)
    checks.check_key_lengths(torch.tensor([32, 16], **i32), bt, 16)
    with pytest.raises(ValueError, match=r"row 1 needs 2 blocks for its 17 keys but block_tables\[1, 1\] is -1"):
        checks.check_key_lengths(torch.tensor([32, 17], **i32), bt, 16)
    with pytest.raises(ValueError, match=r"context_lens\[0\] = 33 is outside \[0, 32\]"):
        checks.check_key_lengths(torch.tensor([33, 1], **i32), bt, 16)
    checks.check_query_rows(torch.tensor([0, 1, 4], **i32), torch.tensor([0, 9, 13], **i32), 4)
    with pytest.raises(ValueError, match="row 1 has 3 queries but only 2 keys"):
        checks.check_query_rows(torch.tensor([0, 1, 4], **i32), torch.tensor([0, 9, 11], **i32), 4)
    with pytest.raises(ValueError, match="ends at 4, but there are 5"):
        checks.check_query_rows(torch.tensor([0, 1, 4], **i32), torch.tensor([0, 9, 13], **i32), 5)

    monkeypatch.setenv("LVATTN_CHECK", "1")
    monkeypatch.setattr(checks, "ENABLED", True)
    b = MI355XAttention(8, 64, 0.1, 2)
    k_cache = torch.zeros(4, 16, 2, 64, dtype=torch.bfloat16)
    key = torch.zeros(2, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="outside"):
        b.store_kvcache(key, key, k_cache, k_cache.clone(), torch.tensor([5, 70], **i32))
    ctx = Context(context_lens=torch.tensor([40], **i32), block_tables=torch.tensor([[0, 1]], **i32))
    with pytest.raises(ValueError, match="outside"):
        b.decode(torch.zeros(1, 8, 64, dtype=torch.bfloat16), k_cache, k_cache.clone(), ctx)
    ctx = Context(cu_seqlens_q=torch.tensor([0, 3], **i32), cu_seqlens_k=torch.tensor([0, 2], **i32),
                  block_tables=torch.tensor([[0]], **i32), max_seqlen_q=3, max_seqlen_k=2)
    with pytest.raises(ValueError, match="3 queries but only 2 keys"):
        b.prefill(torch.zeros(3, 8, 64, dtype=torch.bfloat16), None, None, k_cache, k_cache.clone(), ctx)
    lat = torch.zeros(2, 16, 576, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="outside"):
        MI355XAttention(16, 576, 0.1, 16).store_latents(torch.zeros(1, 576, dtype=torch.bfloat16), lat,
                                                         torch.tensor([32], **i32))


def test_decode_refuses_rows_that_carry_drafts():
    """decode takes one query per row; a step with drafts is is_prefill (the reference sends it to prefill)."""
    b = MI355XAttention(8, 64, 0.1, 2)
    ctx = Context(context_lens=torch.tensor([5, 6], dtype=torch.int32),
                  block_tables=torch.tensor([[0], [1]], dtype=torch.int32))
    cache = torch.zeros(2, 16, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="one query per row"):
        b.decode(torch.zeros(6, 8, 64, dtype=torch.bfloat16), cache, cache, ctx)


def test_the_merge_keeps_the_reference_signature():
    """lvattn.merge_attention_ / merge_attention replace lean_vllm.attention.merge's (merge.py:8,18): same
    parameters, same defaults, same return convention (None for the in-place form)."""
    import inspect

    from lvattn import merge_attention, merge_attention_

    sig = inspect.signature(merge_attention_)
    assert list(sig.parameters) == ["o_a", "lse_a", "o_b", "lse_b", "out"]
    assert sig.parameters["out"].default is None
    assert list(inspect.signature(merge_attention).parameters) == ["o_a", "lse_a", "o_b", "lse_b"]


def test_layers_of_one_step_plan_once(monkeypatch):
    """The work list is planned once per step: the first layer's call plans, every later layer with the same
    Context passes LV_ATTN_REUSE_PLAN (the reference caches per-step plans in context.attn_metadata,
    flash_backend.py:16-20,157-160). A new step's Context plans again, and so does a layer of another shape."""
    from lvattn import _capi
    from lvattn import backend as B

    calls = []
    monkeypatch.setattr(_capi, "call", lambda name, *args: calls.append((name, args)))
    monkeypatch.setattr(_capi, "stream_of", lambda device: 0)
    i32 = dict(dtype=torch.int32)

    def flags_of(call):
        name, args = call
        assert name == "lv_paged_attention"
        return args[-3]

    cache = torch.zeros(8, 16, 2, 64, dtype=torch.bfloat16)
    step = Context(context_lens=torch.tensor([40, 7], **i32), block_tables=torch.tensor([[0, 1, 2], [3, -1, -1]], **i32))
    layer = MI355XAttention(8, 64, 0.1, 2)
    q = torch.zeros(2, 8, 64, dtype=torch.bfloat16)
    for _ in range(3):  # three layers of one step
        layer.decode(q, cache, cache, step)
    assert [flags_of(c) for c in calls] == [0, B.LV_ATTN_REUSE_PLAN, B.LV_ATTN_REUSE_PLAN]
    calls.clear()
    other = MI355XAttention(16, 64, 0.1, 2)  # another layer shape: its own plan
    other.decode(torch.zeros(2, 16, 64, dtype=torch.bfloat16), cache, cache, step)
    layer.decode(q, cache, cache, step)
    assert [flags_of(c) for c in calls] == [0, B.LV_ATTN_REUSE_PLAN]
    calls.clear()
    nxt = Context(context_lens=step.context_lens.clone(), block_tables=step.block_tables.clone())
    layer.decode(q, cache, cache, nxt)  # the next step
    assert [flags_of(c) for c in calls] == [0]
    calls.clear()
    mixed = host_context([20, 0], [1, 9], [[0, 1], [2, -1]])  # a step with prompts: the same rule
    for _ in range(2):
        layer.prefill(torch.zeros(10, 8, 64, dtype=torch.bfloat16), None, None, cache, cache, mixed)
    assert [flags_of(c) for c in calls] == [0, B.LV_ATTN_REUSE_PLAN]


def test_a_step_of_prompts_says_so(monkeypatch):
    """A step whose rows all have several queries passes LV_ATTN_PROMPTS_ONLY (no decode launch, no merge); a step
    with one decode row among its chunks does not."""
    from lvattn import _capi
    from lvattn import backend as B

    calls = []
    monkeypatch.setattr(_capi, "call", lambda name, *args: calls.append(args[-3]))
    monkeypatch.setattr(_capi, "stream_of", lambda device: 0)
    layer = MI355XAttention(8, 64, 0.1, 2)
    cache = torch.zeros(8, 16, 2, 64, dtype=torch.bfloat16)
    prompts = host_context([20, 0], [3, 9], [[0, 1], [2, -1]])
    layer.prefill(torch.zeros(12, 8, 64, dtype=torch.bfloat16), None, None, cache, cache, prompts)
    mixed = host_context([20, 0], [1, 9], [[0, 1], [2, -1]])
    layer.prefill(torch.zeros(10, 8, 64, dtype=torch.bfloat16), None, None, cache, cache, mixed)
    assert [bool(f & B.LV_ATTN_PROMPTS_ONLY) for f in calls] == [True, False]


def test_whole_context_slots_and_offsets():
    """``whole_context``: every row's cached keys in position order (rows with none included), their cache slots
    through the row's table, and the per-step cache in ``attn_metadata``."""
    from lvattn import Context, whole_context

    bs = 4
    cu_q = [0, 3, 4, 4, 9]          # new tokens per row: 3, 1, 0, 5
    cu_k = [0, 10, 11, 17, 30]      # keys per row: 10, 1, 6, 13 -> cached 7, 0, 6, 8
    tables = torch.tensor([[5, 2, 9, -1], [4, -1, -1, -1], [1, 0, -1, -1], [3, 8, 6, 7]], dtype=torch.int32)
    ctx = Context(is_prefill=True, cu_seqlens_q_host=cu_q, cu_seqlens_k_host=cu_k, block_tables=tables)
    slots, cu_ctx, max_ctx = whole_context(ctx, bs)
    want = []
    for r in range(4):
        cached = (cu_k[r + 1] - cu_k[r]) - (cu_q[r + 1] - cu_q[r])
        want += [int(tables[r, p // bs]) * bs + p % bs for p in range(cached)]
    assert slots.tolist() == want and slots.dtype == torch.int64
    assert cu_ctx.tolist() == [0, 7, 7, 13, 21] and cu_ctx.dtype == torch.int32 and max_ctx == 8
    assert whole_context(ctx, bs)[0] is slots  # planned once per step
