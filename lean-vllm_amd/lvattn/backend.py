"""The MI355X attention backend: lean-vLLM's per-layer backend contract on hand-written gfx950 kernels.

Drop-in for ``lean_vllm/attention/abstract.py:29-224``: same constructor, capability flags, cache shape and
methods; registered ahead of ``TorchAttention`` in the selector's ``BACKENDS``. Differences in behaviour, all
allowed by the contract:
- ``split_decodes()`` is False: a step with prompts goes to ``prefill`` whole, and one kernel launch serves its
  decode rows (streaming) and prompt chunks (MFMA tiles) together, as the FA3 backend's single call does
  (``lean_vllm/attention/flash_backend.py:75-89``).
- Nothing syncs the host: slot -1 is skipped on the device, no length is read back, and split-K is sized from
  host bounds (``max_seqlen_k`` or the block-table width), so decode can be captured in a full graph.
- A row with no keys returns zeros (the torch backend returns NaN there; such rows are graph padding).
"""

from __future__ import annotations

import torch

from . import _capi, checks
from .abstract import AttentionBackend
from .context import Context


def _arch_ok() -> bool:
    if not torch.cuda.is_available():
        return False
    try:
        return torch.cuda.get_device_properties(0).gcnArchName.split(":")[0] == "gfx950"
    except Exception:
        return False


class _Workspace:
    """One growing device buffer per device for split-K partials and work lists. Its contents need no
    initialisation, so a captured graph replays with whatever the last call left. A buffer outgrown by a later
    call is kept, not freed: a graph captured earlier still addresses it. Calls that share it are ordered on one
    stream per device (as the engine's step loop issues them)."""

    def __init__(self):
        self._buf: dict[torch.device, torch.Tensor] = {}
        self._retired: list[torch.Tensor] = []

    def get(self, device: torch.device, nbytes: int) -> torch.Tensor | None:
        if nbytes == 0:
            return None
        buf = self._buf.get(device)
        if buf is None or buf.numel() < nbytes:
            size = max(nbytes, 2 * (buf.numel() if buf is not None else 0), 1 << 20)
            if buf is not None:
                self._retired.append(buf)
            buf = torch.empty(size, dtype=torch.uint8, device=device)
            self._buf[device] = buf
        return buf


_WORKSPACE = _Workspace()

# Launch schedules of a step with prompt rows (LV_SCHEDULE_* of lvattn.h).
SCHEDULE_AUTO, SCHEDULE_SERIAL, SCHEDULE_OVERLAP = 0, 1, 2
LV_ATTN_REUSE_PLAN, LV_ATTN_PROMPTS_ONLY = 1, 2  # flags of lv_paged_attention
# Measured MI355X rates the schedule choice compares (bf16, head_dim 128). Overlapped, the prompt tiles run at
# about 0.18 PFLOP/s (one workgroup on half the CUs, beside the decode rows) against 0.84 PFLOP/s alone on the whole
# GPU, and the decode rows stream about 6.6 TB/s. Overlap wins while the prompt tiles' extra time beside the decode
# rows, flops x (1/0.18 - 1/0.84 per PFLOP/s), fits in the decode rows' own time: steps of 2048 decode rows with 2
# to 8 prompt chunks of 1536 tokens ran 6-9% faster overlapped, with 12 and 16 chunks 35% and 65% slower.
DECODE_BYTES_PER_S = 6.6e12
PROMPT_FLOPS_PER_S = 1 / (1 / 1.8e14 - 1 / 8.4e14)  # 2.3e14
# One overlapped prompt workgroup (one per CU) runs about 1.3-1.4 TFLOP/s of prompt tiles beside the decode rows. An
# overlapped step asks for enough of them that the prompt tiles end with the decode rows; the library keeps the
# count between 44% and three quarters of the CUs.
PROMPT_WORKGROUP_FLOPS_PER_S = 1.3e12


class MI355XAttention(AttentionBackend):
    """Paged attention, cache stores and MLA latent decode on MI355X (gfx950) HIP kernels.

    ``launch_trace``: None, or a list to which every paged-attention call appends the launches the library made for
    it (``lv_paged_attention_launch_info`` on the call's own arguments), for callers and tests that check which path
    a step takes."""

    supported_dtypes = (torch.float16, torch.bfloat16)
    supported_kinds = ("decoder", "mla")
    launch_trace: list | None = None

    @staticmethod
    def get_name() -> str:
        return "mi355x"

    @staticmethod
    def is_available() -> bool:
        return _arch_ok() and _capi.LIBRARY.exists()

    @staticmethod
    def supports_cuda_graph() -> bool:
        return True

    @staticmethod
    def supports_full_cudagraph() -> bool:
        return True

    @staticmethod
    def split_decodes() -> bool:
        return False

    @staticmethod
    def supports_head_size(head_size: int) -> bool:
        return head_size in (64, 128, 192)

    @classmethod
    def validate(cls, spec) -> list[str]:
        reasons = super().validate(spec)
        if spec.kind == "decoder":
            if spec.head_size == 192:
                reasons.append("head size 192 is served for MLA layers (192-wide q.k, 128-wide values) only")
            if spec.num_kv_heads and spec.num_heads // max(spec.num_kv_heads, 1) > 64:
                reasons.append(f"{spec.num_heads // spec.num_kv_heads} query heads per key head exceed 64")
        elif spec.kind == "mla" and spec.latent_dim != 576:
            reasons.append(f"MLA latent width {spec.latent_dim} is not 576 (kv_lora_rank 512 + rope 64)")
        return reasons

    @staticmethod
    def supports_mla_decode() -> bool:
        return True

    @staticmethod
    def mla_block_size() -> int | None:
        return None

    # -- cache writes --------------------------------------------------------------------------------------
    def store_kvcache(self, key, value, k_cache, v_cache, slot_mapping) -> None:
        num_tokens, heads, dim = key.shape
        ks, vs, cs = key.stride(), value.stride(), k_cache.stride()
        assert ks[2] == 1 and vs[2] == 1, "unit dim stride"
        assert ks[1] == dim and vs[1] == dim, "head stride must equal head_dim"
        assert cs == v_cache.stride() and cs[3] == 1
        assert slot_mapping.numel() == num_tokens
        assert key.dtype == value.dtype == k_cache.dtype == v_cache.dtype
        if checks.ENABLED:
            checks.check_slots(slot_mapping, k_cache.size(0), k_cache.size(1))
        if slot_mapping.dtype != torch.int32:
            slot_mapping = slot_mapping.to(torch.int32)
        _capi.call("lv_store_kvcache", key.data_ptr(), value.data_ptr(), ks[0], vs[0], num_tokens, heads, dim,
                   k_cache.data_ptr(), v_cache.data_ptr(), cs[0], cs[1], cs[2], k_cache.size(1),
                   slot_mapping.data_ptr(), key.element_size(), _capi.stream_of(key.device))

    def store_latents(self, latent, latent_cache, slot_mapping) -> None:
        num_tokens, dim = latent.shape
        assert latent.stride(-1) == 1 and latent_cache.stride(-2) == dim and latent_cache.stride(-1) == 1
        assert slot_mapping.numel() == num_tokens and latent.dtype == latent_cache.dtype
        if checks.ENABLED:
            checks.check_slots(slot_mapping, latent_cache.numel() // dim, 1)
        slot_mapping = slot_mapping if slot_mapping.dtype == torch.int32 else slot_mapping.to(torch.int32)
        _capi.call("lv_store_latents", latent.data_ptr(), latent.stride(0), num_tokens, dim, latent_cache.data_ptr(),
                   slot_mapping.data_ptr(), latent.element_size(), _capi.stream_of(latent.device))

    # -- attention -----------------------------------------------------------------------------------------
    def _attend(self, q, k_cache, v_cache, out, *, context, block_tables, cu_seqlens_q, seqlens_k, cu_seqlens_k,
                rows, max_seqlen_q, max_seqlen_k, schedule=SCHEDULE_AUTO, prompt_workgroups=0, prompts_only=False):
        qs, cs = q.stride(), k_cache.stride()
        assert q.dtype in _capi.DTYPES and k_cache.dtype == q.dtype == v_cache.dtype
        assert qs[2] == 1 and cs == v_cache.stride() and cs[3] == 1
        assert block_tables is not None and block_tables.dtype == torch.int32
        if out is None:
            out = torch.empty_like(q)
        os_ = out.stride()
        assert out.shape == q.shape and os_[2] == 1 and out.dtype == q.dtype
        tokens, heads, dim = q.shape
        # The work list is planned once per step and every later layer reuses it, as the reference's backends cache
        # per-step plans in context.attn_metadata (flash_backend.py:16-20,157-160). The plan depends on the rows'
        # lengths (read through these tensors, which the step's context holds), the shape and the bound on key
        # lengths; the step's workspace size is kept with it.
        meta = context.attn_metadata
        if meta is None:
            meta = context.attn_metadata = {}
        key = ("plan", heads, self.num_kv_heads, dim, rows, tokens, max_seqlen_q, max_seqlen_k,
               id(cu_seqlens_q), id(seqlens_k), id(cu_seqlens_k))
        planned = meta.get(key)
        if planned is None:
            decode_only = cu_seqlens_q is None or max_seqlen_q == 1
            nbytes = _capi.query("lv_paged_attention_workspace_bytes", rows, tokens, heads, self.num_kv_heads, dim,
                                 max_seqlen_k, int(decode_only))
            planned = meta[key] = [nbytes, None, (cu_seqlens_q, seqlens_k, cu_seqlens_k)]  # holds the tensors
        ws = _WORKSPACE.get(q.device, planned[0])
        flags = LV_ATTN_REUSE_PLAN if ws is not None and planned[1] is ws else 0
        if prompts_only:
            flags |= LV_ATTN_PROMPTS_ONLY
        planned[1] = ws
        bt = block_tables
        _capi.call("lv_paged_attention", q.data_ptr(), qs[0], qs[1], k_cache.data_ptr(), v_cache.data_ptr(), cs[0],
                   cs[1], cs[2], k_cache.size(1), bt.data_ptr(), bt.stride(0), _capi.ptr(cu_seqlens_q),
                   _capi.ptr(seqlens_k), _capi.ptr(cu_seqlens_k), rows, tokens, heads, self.num_kv_heads, dim,
                   float(self.scale), max_seqlen_q, max_seqlen_k, out.data_ptr(), os_[0], os_[1], _capi.ptr(ws),
                   0 if ws is None else ws.numel(), schedule, prompt_workgroups, flags, _capi.DTYPES[q.dtype],
                   _capi.stream_of(q.device))
        if self.launch_trace is not None:
            self.launch_trace.append(_capi.launch_info(rows, tokens, heads, self.num_kv_heads, dim, k_cache.size(1),
                                                       cs[2], int(cu_seqlens_q is not None), max_seqlen_q,
                                                       max_seqlen_k, schedule, prompt_workgroups, flags,
                                                       _capi.DTYPES[q.dtype]))
        return out

    def _schedule(self, context: Context, elem_bytes: int) -> int:
        """Overlap a step's prompt tiles with its decode rows only when the decode rows' bytes take at least as
        long as the prompt tiles' MFMA work; otherwise (a step of prompts, or prompts with a few short decode rows)
        the prompt tiles run on the whole GPU first. Decided from the host lengths the context carries
        (``cu_seqlens_*_host``); without them the library's default (overlap) stands."""
        cu_q, cu_k = context.cu_seqlens_q_host, context.cu_seqlens_k_host
        if cu_q is None or cu_k is None:
            return SCHEDULE_AUTO
        key = ("schedule", self.num_heads, self.num_kv_heads, self.head_dim, elem_bytes)
        cache = context.attn_metadata if context.attn_metadata is not None else {}
        context.attn_metadata = cache  # per-step plans shared by every layer
        if key not in cache:
            # Rows come decode-first (prepare_batch's order): the leading one-query rows are those with
            # cu_q[i] == i, found by bisection, and their keys sum to cu_k[n]. The rest are walked one by one.
            rows = len(cu_q) - 1
            lo, hi = 0, rows
            while lo < hi:
                mid = (lo + hi + 1) // 2
                if cu_q[mid] == mid:
                    lo = mid
                else:
                    hi = mid - 1
            decode_keys, pairs = cu_k[lo] - cu_k[0], 0
            for r in range(lo, rows):
                lq, lk = cu_q[r + 1] - cu_q[r], cu_k[r + 1] - cu_k[r]
                if lq == 1:
                    decode_keys += lk
                elif lq > 1:  # query j of a prompt row sees lk - lq + j + 1 keys
                    pairs += lq * (lk - lq) + lq * (lq + 1) // 2
            decode_bytes = decode_keys * 2 * self.num_kv_heads * self.head_dim * elem_bytes
            prompt_flops = 4 * self.num_heads * self.head_dim * pairs
            overlap = decode_bytes / DECODE_BYTES_PER_S >= prompt_flops / PROMPT_FLOPS_PER_S
            cache[key] = SCHEDULE_OVERLAP if overlap else SCHEDULE_SERIAL
            decode_s = decode_bytes / DECODE_BYTES_PER_S
            cache[key + ("workgroups",)] = int(prompt_flops / PROMPT_WORKGROUP_FLOPS_PER_S / decode_s) if overlap else 0
            cache[key + ("prompts_only",)] = lo == 0 and all(cu_q[r + 1] - cu_q[r] > 1 for r in range(rows))
        return cache[key]

    def _prompts_only(self, context: Context, elem_bytes: int) -> bool:
        """Whether every row of the step has more than one query, as ``_schedule`` found from the host lengths."""
        cache = context.attn_metadata or {}
        return cache.get(("schedule", self.num_heads, self.num_kv_heads, self.head_dim, elem_bytes, "prompts_only"),
                         False)

    def _prompt_workgroups(self, context: Context, elem_bytes: int) -> int:
        """CUs that hold a prompt workgroup in this step's overlap, as ``_schedule`` sized them (0: the library's
        default, half of them)."""
        cache = context.attn_metadata or {}
        return cache.get(("schedule", self.num_heads, self.num_kv_heads, self.head_dim, elem_bytes, "workgroups"), 0)

    def decode(self, q, k_cache, v_cache, context: Context, out=None):
        """One query per row against its ``context_lens[b]`` cached keys; q ``[B, Hq, D]``."""
        bt, lens = context.block_tables, context.context_lens
        assert bt is not None and lens is not None
        assert lens.numel() == q.size(0) == bt.size(0), (
            f"decode takes one query per row: {q.size(0)} queries, {lens.numel()} context lengths, {bt.size(0)} table "
            "rows (a step whose rows carry drafts is is_prefill and goes to prefill)")
        if checks.ENABLED:
            checks.check_tables(bt, k_cache.size(0))
            checks.check_key_lengths(lens, bt, k_cache.size(1))
        lens = lens if lens.dtype == torch.int32 else lens.to(torch.int32)
        # The table's width bounds every length, so nothing is read back (torch_backend.py:98).
        max_k = bt.size(1) * k_cache.size(1)
        return self._attend(q, k_cache, v_cache, out, context=context, block_tables=bt, cu_seqlens_q=None,
                            seqlens_k=lens, cu_seqlens_k=None, rows=q.size(0), max_seqlen_q=1, max_seqlen_k=max_k)

    def prefill(self, q, k, v, k_cache, v_cache, context: Context, out=None):
        """Varlen causal attention over the step's rows, bottom-right aligned, every key read from the pages;
        rows of one query take the streaming decode path inside the same launch."""
        cu_q, cu_k = context.cu_seqlens_q, context.cu_seqlens_k
        assert cu_q is not None and cu_k is not None
        if context.block_tables is None:  # warmup, or an MLA prompt with no cached context: keys are k, v
            max_q = context.max_seqlen_q or q.size(0)
            o, _ = self._varlen(q, k, v, cu_q, cu_k, max_q, causal=True, want_lse=False, out=out)
            return o
        bt = context.block_tables
        if checks.ENABLED:
            checks.check_query_rows(cu_q, cu_k, q.size(0))
            checks.check_tables(bt, k_cache.size(0))
            checks.check_key_lengths(cu_k[1:] - cu_k[:-1], bt, k_cache.size(1), what="cu_seqlens_k row length")
        max_k = context.max_seqlen_k or bt.size(1) * k_cache.size(1)
        max_q = context.max_seqlen_q or q.size(0)
        return self._attend(q, k_cache, v_cache, out, context=context, block_tables=bt,
                            cu_seqlens_q=cu_q if cu_q.dtype == torch.int32 else cu_q.to(torch.int32), seqlens_k=None,
                            cu_seqlens_k=cu_k if cu_k.dtype == torch.int32 else cu_k.to(torch.int32), rows=cu_q.numel() - 1,
                            max_seqlen_q=max_q, max_seqlen_k=max_k,
                            schedule=self._schedule(context, q.element_size()),
                            prompt_workgroups=self._prompt_workgroups(context, q.element_size()),
                            prompts_only=self._prompts_only(context, q.element_size()))

    def mla_decode(self, q, latent_cache, v_dim, context: Context, out=None):
        """Each row's last ``Lq`` queries against its paged latents, read as one key head shared by every query
        head; values are the latents' first ``v_dim`` entries (``abstract.py:206-219``). q ``[B * Lq, H, 576]``,
        latent_cache ``[N, bs, 576]`` -> ``[B * Lq, H, v_dim]``. Nothing is read back: ``Lq`` comes from the
        shapes and the split-K grid from the block-table width. ``out``, if given, receives the result."""
        bt, lens = context.block_tables, context.context_lens
        assert bt is not None and lens is not None and bt.dtype == torch.int32 and bt.stride(-1) == 1
        lens = lens if lens.dtype == torch.int32 else lens.to(torch.int32)
        if latent_cache.dim() == 4:  # [1, N, bs, latent] as MLA layers allocate it
            latent_cache = latent_cache[0]
        assert q.dtype in _capi.DTYPES and latent_cache.dtype == q.dtype
        assert q.stride(-1) == 1 and latent_cache.stride(-1) == 1
        rows = lens.numel()
        tokens, heads, dim = q.shape
        assert tokens % rows == 0, "every row has the same number of queries"
        if checks.ENABLED:
            checks.check_tables(bt, latent_cache.size(0))
            checks.check_key_lengths(lens, bt, latent_cache.size(1))
        lq = tokens // rows
        max_k = bt.size(1) * latent_cache.size(1)
        if out is None:
            out = torch.empty(tokens, heads, v_dim, dtype=q.dtype, device=q.device)
        assert out.shape == (tokens, heads, v_dim) and out.dtype == q.dtype and out.stride(-1) == 1
        nbytes = _capi.query("lv_mla_decode_workspace_bytes", rows, lq, heads, max_k)
        ws = _WORKSPACE.get(q.device, nbytes)
        _capi.call("lv_mla_decode", q.data_ptr(), q.stride(0), q.stride(1), latent_cache.data_ptr(),
                   latent_cache.stride(0), latent_cache.stride(1), latent_cache.size(1), bt.data_ptr(), bt.stride(0),
                   lens.data_ptr(), rows, lq, heads, dim, v_dim, float(self.scale), max_k, out.data_ptr(),
                   out.stride(0), out.stride(1), _capi.ptr(ws), 0 if ws is None else ws.numel(),
                   _capi.DTYPES[q.dtype], _capi.stream_of(q.device))
        return out

    # -- packed keys (no pages) ----------------------------------------------------------------------------
    def _varlen(self, q, k, v, cu_q, cu_k, max_q, *, causal: bool, want_lse: bool, out=None):
        assert q.dtype in _capi.DTYPES and k.dtype == q.dtype == v.dtype
        assert q.stride(-1) == 1 and k.stride(-1) == 1 and v.stride(-1) == 1
        tokens, heads, dqk = q.shape
        dv = v.size(-1)
        cu_q = cu_q if cu_q.dtype == torch.int32 else cu_q.to(torch.int32)
        cu_k = cu_k if cu_k.dtype == torch.int32 else cu_k.to(torch.int32)
        if out is None:
            out = torch.empty(tokens, heads, dv, dtype=q.dtype, device=q.device)
        assert out.shape == (tokens, heads, dv) and out.stride(-1) == 1 and out.dtype == q.dtype
        lse = torch.empty(tokens, heads, dtype=torch.float32, device=q.device) if want_lse else None
        _capi.call("lv_varlen_attention", q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0),
                   k.stride(1), v.data_ptr(), v.stride(0), v.stride(1), cu_q.data_ptr(), cu_k.data_ptr(),
                   cu_q.numel() - 1, heads, k.size(1), dqk, dv, float(self.scale), int(causal), int(max_q),
                   out.data_ptr(), out.stride(0), out.stride(1), _capi.ptr(lse), heads if want_lse else 0,
                   1 if want_lse else 0, _capi.DTYPES[q.dtype], _capi.stream_of(q.device))
        return out, lse

    def varlen_with_lse(self, q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, causal,
                        host_cu_seqlens=None):
        """Attention over packed keys, bottom-right causal or unmasked, plus the natural log-sum-exp ``[T, H]`` of
        every query row for merging (``abstract.py:187-204``); -inf for a row with no keys. ``host_cu_seqlens``
        is not needed: the grid is sized from ``max_seqlen_q``."""
        return self._varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, causal=causal, want_lse=True)

    def prefill_with_context(self, q, k, v, k_ctx, v_ctx, cu_seqlens_q, cu_seqlens_ctx, max_seqlen_q, out=None,
                             want_lse=False):
        """MLA prefill over cached context in one call: each row's new queries attend all of the row's context
        keys ``k_ctx``/``v_ctx`` (rows by ``cu_seqlens_ctx``) and, causally, its new keys ``k``/``v`` (rows by
        ``cu_seqlens_q``), as one softmax. The same result as ``MLAAttention._prefill``'s causal
        ``varlen_with_lse``, unmasked ``varlen_with_lse`` over the context and ``merge_attention_``
        (``lean_vllm/layers/attention.py:280-316``), without their partial outputs. Returns ``out`` (and the
        natural log-sum-exp ``[T, H]`` with ``want_lse``)."""
        assert q.dtype in _capi.DTYPES and k.dtype == q.dtype == v.dtype == k_ctx.dtype == v_ctx.dtype
        for t in (q, k, v, k_ctx, v_ctx):
            assert t.stride(-1) == 1
        tokens, heads, dqk = q.shape
        dv = v.size(-1)
        assert k.size(0) == tokens and k_ctx.size(1) == k.size(1) and v_ctx.size(-1) == dv
        cu_q = cu_seqlens_q if cu_seqlens_q.dtype == torch.int32 else cu_seqlens_q.to(torch.int32)
        cu_c = cu_seqlens_ctx if cu_seqlens_ctx.dtype == torch.int32 else cu_seqlens_ctx.to(torch.int32)
        assert cu_c.numel() == cu_q.numel()
        if out is None:
            out = torch.empty(tokens, heads, dv, dtype=q.dtype, device=q.device)
        assert out.shape == (tokens, heads, dv) and out.stride(-1) == 1 and out.dtype == q.dtype
        lse = torch.empty(tokens, heads, dtype=torch.float32, device=q.device) if want_lse else None
        _capi.call("lv_varlen_context_attention", q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0),
                   k.stride(1), v.data_ptr(), v.stride(0), v.stride(1), cu_q.data_ptr(), cu_q.data_ptr(),
                   k_ctx.data_ptr(), k_ctx.stride(0), k_ctx.stride(1), v_ctx.data_ptr(), v_ctx.stride(0),
                   v_ctx.stride(1), cu_c.data_ptr(), cu_q.numel() - 1, heads, k.size(1), dqk, dv, float(self.scale),
                   int(max_seqlen_q), out.data_ptr(), out.stride(0), out.stride(1), _capi.ptr(lse),
                   heads if want_lse else 0, 1 if want_lse else 0, _capi.DTYPES[q.dtype], _capi.stream_of(q.device))
        return (out, lse) if want_lse else out
