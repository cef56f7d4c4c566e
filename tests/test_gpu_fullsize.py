"""The measured steps at full size, packed, stored and attended as the bench runs them, against the fp32 oracle:
every decode row of every step (the Qwen3-8B mixed step's 2048, batch-256 decode, the 16 long-context rows, the
Qwen3-0.6B step's 30), one query in every prompt item of every chunk (at an offset that moves from item to item)
plus each chunk's last query (every query of the Qwen3-0.6B chunks), and every row of DeepSeek-V2-Lite's MLA decode
step.

Decode rows go through the oracle's restatement of the reference backend (``TorchMath.decode`` over slices of
rows, ``decode_in_row_chunks``) on the rows' pages copied to the host, so the persistent ticket grid, the
length-bucketed work list, the split-K merge and the overlapped prompt tiles are all checked on every item they
produce; each step asserts the launch route it takes (``lv_paged_attention_launch_info``). Prompt queries go
through the textbook dense oracle on the keys the query sees. Tolerance: max-abs 2e-2 / rel 1e-2 against fp32
(bf16).
"""

import pytest
import torch

from lvattn import Context, MI355XAttention, Packer
from lvattn import workloads as W
from oracle import attention as A

pytestmark = pytest.mark.gpu

TOL = dict(atol=2e-2, rtol=1e-2)


def compact_pages(cache, lists):
    """The given rows' pages copied to the host (cache dtype), renumbered 0..n-1, and the rows' tables over them."""
    pages = sorted({p for lst in lists for p in lst})
    index = {p: i for i, p in enumerate(pages)}
    host = cache[torch.tensor(pages, dtype=torch.long, device=cache.device)].cpu()
    width = max(len(lst) for lst in lists)
    bt = torch.full((len(lists), width), -1, dtype=torch.int32)
    for j, lst in enumerate(lists):
        bt[j, :len(lst)] = torch.tensor([index[p] for p in lst], dtype=torch.int32)
    return host, bt


# The launch route each measured paged step takes on an MI355X (256 CUs).
OVERLAP = dict(prompt_kernel="prompt_overlap", decode_kernel="decode_beside", two_streams=True, kv_heads_per_item=2)
PROMPTS = dict(prompt_kernel="prompt_list", decode_kernel="none", two_streams=False)
DECODE = dict(prompt_kernel="none", decode_kernel="decode_list", kv_heads_per_item=2)
ROUTES = {
    "qwen3_8b_mixed": OVERLAP, "qwen3_8b_mixed_bs16": OVERLAP,
    "qwen3_8b_prefill": PROMPTS, "qwen3_8b_prefill_bs16": PROMPTS, "qwen3_8b_prefix_chunk": PROMPTS,
    "qwen3_8b_decode": dict(DECODE, splitk_merge=True), "qwen3_8b_long": dict(DECODE, splitk_merge=True),
    "qwen3_0_6b_mixed": dict(prompt_kernel="mixed_small", decode_kernel="mixed_small", kv_heads_per_item=2,
                             splitk_merge=True),
}


def run_step(name, cuda):
    """Pack, store and attend one workload's step on the GPU; asserts the launch route; returns what the checks
    need."""
    wl = W.WORKLOADS[name]()
    t = W.materialize(wl, cuda)
    b = MI355XAttention(wl.num_heads, wl.head_dim, wl.scale, wl.num_kv_heads)
    _, fields = Packer(cuda, wl.block_size).pack(wl.num_cached, wl.num_new, wl.block_lists)
    order = fields.pop("order").cpu().tolist()
    b.store_kvcache(t.k_new, t.v_new, t.k_cache, t.v_cache, fields["slot_mapping"])
    ctx = Context(**{k: v for k, v in fields.items() if k in Context.__slots__})
    b.launch_trace = []
    out = b.forward(t.q, t.k_new, t.v_new, t.k_cache, t.v_cache, ctx)
    torch.cuda.synchronize()
    info = b.launch_trace[-1]
    print(f"{name}: {info}", flush=True)
    want = ROUTES[name]
    assert {k: info[k] for k in want} == want, f"{name}: route {info}, expected {want}"
    assert torch.isfinite(out).all()
    return wl, t, out, order, fields["cu_seqlens_q"].cpu().tolist()


def check_decode_rows(wl, t, out, order, cu_q, rows_per_slice=128, rows_per_chunk=8):
    """Every decode row (one query) against TorchMath.decode on its pages, ``rows_per_slice`` rows' pages on the
    host at a time, ``rows_per_chunk`` rows per padded gather; returns the number of rows checked."""
    math_ = A.TorchMath(wl.num_heads, wl.head_dim, wl.scale, wl.num_kv_heads)
    rows = [i for i in range(len(order)) if wl.num_new[order[i]] == 1]
    for r0 in range(0, len(rows), rows_per_slice):
        sl = rows[r0:r0 + rows_per_slice]
        lists = [wl.block_lists[order[i]] for i in sl]
        kc, bt = compact_pages(t.k_cache, lists)
        vc, _ = compact_pages(t.v_cache, lists)
        lens = torch.tensor([wl.num_cached[order[i]] + 1 for i in sl], dtype=torch.int32)
        q = t.q[[cu_q[i] for i in sl]].cpu()
        want = A.decode_in_row_chunks(math_, q, kc, vc, lens, bt, rows_per_chunk=rows_per_chunk)
        got = out[[cu_q[i] for i in sl]].float().cpu()
        for j in range(len(sl)):
            torch.testing.assert_close(got[j], want[j], **TOL,
                                       msg=lambda m: f"{wl.name}: decode row {sl[j]} (batch order): {m}")
        del kc, vc
    return len(rows)


def item_queries(lq, per_item):
    """One query position in every prompt item of a chunk of ``lq`` queries (an item spans ``per_item`` positions:
    128 (position, head) query rows over the GQA group), at an offset that moves from item to item, plus the chunk's
    last query."""
    return sorted({per_item * i + (7 * i) % per_item for i in range(-(-lq // per_item))} | {lq - 1})


def check_prompt_queries(wl, t, out, order, cu_q, every=None):
    """Each prompt chunk's queries -- every ``every``-th one, or by default one in every prompt item
    (``item_queries``) -- against the dense oracle over the row's keys up to its own position; returns the number
    of queries checked."""
    bs, n = wl.block_size, 0
    per_item = 128 // (wl.num_heads // wl.num_kv_heads)
    for i in range(len(order)):
        s = order[i]
        lq = wl.num_new[s]
        if lq == 1:
            continue
        lk = wl.num_cached[s] + lq
        pos = torch.arange(lk, device=t.k_cache.device)
        pages = torch.tensor(wl.block_lists[s], dtype=torch.long, device=t.k_cache.device)[pos // bs]
        k = t.k_cache[pages, pos % bs].cpu().float()
        v = t.v_cache[pages, pos % bs].cpu().float()
        picks = item_queries(lq, per_item) if every is None else sorted(set(range(0, lq, every)) | {lq - 1})
        for j in [j for j in picks if j < lq]:
            seen = lk - lq + j + 1
            q = t.q[cu_q[i] + j:cu_q[i] + j + 1].cpu().float()
            want = A.dense_attention(q, k[:seen], v[:seen], wl.scale, causal=False)
            got = out[cu_q[i] + j:cu_q[i] + j + 1].float().cpu()
            torch.testing.assert_close(got, want, **TOL, msg=lambda m: f"{wl.name}: chunk row {i} query {j}: {m}")
            n += 1
    return n


def test_qwen3_8b_mixed_step_every_decode_row(cuda):
    """The bench's primary step: all 2048 decode rows (the persistent grid of pair items beside the prompt
    workgroups)."""
    wl, t, out, order, cu_q = run_step("qwen3_8b_mixed", cuda)
    assert check_decode_rows(wl, t, out, order, cu_q) == 2048


def test_qwen3_8b_mixed_step_prompt_queries(cuda):
    """The same step's four 1536-token chunks, on cached prefixes up to 6144: one query in each of every chunk's 48
    prompt items (32 positions each) and the last query."""
    wl, t, out, order, cu_q = run_step("qwen3_8b_mixed", cuda)
    assert check_prompt_queries(wl, t, out, order, cu_q) == 4 * 49


def test_qwen3_8b_prompt_chunks_alone(cuda):
    """The four chunks as a step of prompts (prompt tiles on the whole GPU): one query per prompt item and the
    last."""
    wl, t, out, order, cu_q = run_step("qwen3_8b_prefill", cuda)
    assert check_prompt_queries(wl, t, out, order, cu_q) == 4 * 49


def test_qwen3_8b_mixed_step_on_16_token_pages(cuda):
    """The mixed step on lean-vLLM's default page size (16 keys: four pages per prompt tile): one query per prompt
    item of the chunks and their last, and every decode row."""
    wl, t, out, order, cu_q = run_step("qwen3_8b_mixed_bs16", cuda)
    assert check_prompt_queries(wl, t, out, order, cu_q) == 4 * 49
    assert check_decode_rows(wl, t, out, order, cu_q) == 2048


def test_qwen3_8b_chunk_on_a_long_prefix(cuda):
    """One 1024-token chunk on a 30,720-token prefix (32 prompt items per kv head, each walking some 490 key tiles):
    one query per prompt item and the last."""
    wl, t, out, order, cu_q = run_step("qwen3_8b_prefix_chunk", cuda)
    assert check_prompt_queries(wl, t, out, order, cu_q) == 33


def test_qwen3_8b_prompt_chunks_alone_on_16_token_pages(cuda):
    wl, t, out, order, cu_q = run_step("qwen3_8b_prefill_bs16", cuda)
    assert check_prompt_queries(wl, t, out, order, cu_q) == 4 * 49


@pytest.mark.parametrize("name, rows", [("qwen3_8b_decode", 256), ("qwen3_8b_long", 16)])
def test_decode_steps_every_row(cuda, name, rows):
    """Batch-256 decode (contexts 512-8192, split into two 4096-key items) and the long-context step (contexts
    32K-128K, split-K over up to 16 items per row): every row."""
    wl, t, out, order, cu_q = run_step(name, cuda)
    long = name == "qwen3_8b_long"
    assert check_decode_rows(wl, t, out, order, cu_q, rows_per_slice=16 if long else 64,
                             rows_per_chunk=2 if long else 8) == rows


def test_qwen3_0_6b_mixed_step_every_row_and_query(cuda):
    """The CPU-runnable step: its 30 decode rows and every query of its two chunks."""
    wl, t, out, order, cu_q = run_step("qwen3_0_6b_mixed", cuda)
    assert check_decode_rows(wl, t, out, order, cu_q) == 30
    assert check_prompt_queries(wl, t, out, order, cu_q, every=1) == 512 + 384


def test_deepseek_v2_lite_mla_decode_every_row(cuda):
    """DeepSeek-V2-Lite's MLA decode step (128 rows, contexts 1024-16384, 64-latent pages over a 34,000-page pool,
    balanced runs): every row against TorchMath.mla_decode on its pages."""
    wl = W.deepseek_v2_lite_mla()
    t = W.materialize(wl, cuda)
    b = MI355XAttention(wl.num_heads, wl.latent_dim, wl.scale, wl.num_heads)
    width = max(len(x) for x in wl.block_lists)
    bt = torch.full((wl.rows, width), -1, dtype=torch.int32)
    for r, lst in enumerate(wl.block_lists):
        bt[r, :len(lst)] = torch.tensor(lst, dtype=torch.int32)
    lens = torch.tensor(wl.context_lens, dtype=torch.int32)
    out = b.mla_decode(t.q, t.k_cache, wl.v_dim, Context(context_lens=lens.to(cuda), block_tables=bt.to(cuda)))
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    math_ = A.TorchMath(wl.num_heads, wl.latent_dim, wl.scale, 1)
    for r0 in range(0, wl.rows, 8):
        rows = list(range(r0, min(r0 + 8, wl.rows)))
        cache, cbt = compact_pages(t.k_cache, [wl.block_lists[r] for r in rows])
        ctx = A.context(context_lens=lens[rows], block_tables=cbt)
        want = math_.mla_decode(t.q[rows].cpu(), cache, wl.v_dim, ctx)
        got = out[rows].float().cpu()
        for j, r in enumerate(rows):
            torch.testing.assert_close(got[j], want[j], **TOL, msg=lambda m: f"MLA row {r}: {m}")
