"""Ragged-batch packing on the GPU: the attention half of ``ModelRunner.prepare_batch``
(``lean_vllm/engine/model_runner.py:349-519``) as one kernel.

The host hands over only per-row integers -- ``num_cached``, ``num_new`` and each row's block list (CSR) -- in one
pinned buffer and one copy. The kernel produces the per-token ``positions`` and ``slot_mapping``, the ``-1``-padded
``block_tables`` and the row prefix sums, in the decode-first row order the reference uses. The host keeps the
row-level ints the ``Context`` carries as host lists (``cu_seqlens_*_host``, ``max_seqlen_*``), which it derives
from the same per-row ints without touching per-token data.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _capi

MIN_CAPACITY = 256


def _host_stage():
    """The host staging extension (built beside liblvattn.so); its absence is an error, as the library's is."""
    try:
        from . import _hoststage
    except ImportError as e:
        raise RuntimeError("lvattn._hoststage is not built; run __graft_entry__.build() (or python -m lvattn._build)"
                           ) from e
    return _hoststage


def decode_query_len(lens: np.ndarray, num_speculative_tokens: int = 0) -> int:
    """The most common query length not above ``1 + num_speculative_tokens``, shorter on ties, else 1
    (``model_runner.py:51-63``)."""
    short = lens[lens <= 1 + num_speculative_tokens]
    if short.size == 0:
        return 1
    return int(np.argmax(np.bincount(short)))


class StagingBuffers:
    """Named device buffers fed from reusable pinned host buffers (``lean_vllm/engine/input_buffers.py:17-56``):
    grow to at least twice their size, copy asynchronously, and fence the host buffers with an event so a step
    never overwrites what the previous step's copy is still reading."""

    def __init__(self, device: torch.device):
        self.device = torch.device(device)
        self._pinned: dict[str, torch.Tensor] = {}
        self._device: dict[str, torch.Tensor] = {}
        self._copied: torch.cuda.Event | None = None

    def begin(self):
        if self._copied is not None:
            self._copied.synchronize()
            self._copied = None

    def end(self):
        self._copied = torch.cuda.Event()
        self._copied.record(torch.cuda.current_stream(self.device))

    def device_buffer(self, name: str, n: int, dtype: torch.dtype) -> torch.Tensor:
        """A device buffer of at least ``n`` elements for a kernel to fill."""
        buf = self._device.get(name)
        if buf is None or buf.numel() < n or buf.dtype != dtype:
            cap = max(n, 2 * (buf.numel() if buf is not None else 0), MIN_CAPACITY)
            buf = torch.empty(cap, dtype=dtype, device=self.device)
            self._device[name] = buf
        return buf[:n]

    def host_view(self, name: str, n: int, dtype: torch.dtype) -> np.ndarray:
        """The first ``n`` elements of this name's pinned host buffer, as a numpy array to fill in place."""
        host = self._pinned.get(name)
        if host is None or host.numel() < n or host.dtype != dtype:
            cap = max(n, 2 * (host.numel() if host is not None else 0), MIN_CAPACITY)
            host = torch.empty(cap, dtype=dtype, pin_memory=True)
            self._pinned[name] = host
        return host[:n].numpy()

    def upload(self, name: str, n: int, dtype: torch.dtype) -> torch.Tensor:
        """Copy the first ``n`` elements of this name's pinned buffer to its device buffer (asynchronously)."""
        dev = self.device_buffer(name, n, dtype)
        dev.copy_(self._pinned[name][:n], non_blocking=True)
        return dev

    def put(self, name: str, values: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
        """Copy host values into this name's device buffer through its pinned buffer."""
        n = values.size
        self.host_view(name, n, dtype)[:] = values.reshape(-1)
        return self.upload(name, n, dtype)


class PackPlan:
    """One step's staged packing inputs (device) and the row-level host ints derived from them."""

    __slots__ = ("rows", "tokens", "width", "slot_count", "query_len", "inputs", "host", "logits")

    def __init__(self, rows, tokens, width, slot_count, query_len, inputs, host, logits=-1):
        self.rows, self.tokens, self.width, self.slot_count = rows, tokens, width, slot_count
        self.query_len, self.inputs, self.host = query_len, inputs, host
        self.logits = logits  # logits rows gathered, or -1 for none (the whole batch samples)


def check_block_lists(num_cached, num_new, lengths, block_size: int) -> None:
    """Every row with a block list must hold a block for each of its ``num_cached + num_new`` tokens (a row without
    one stores nothing, as in warmup); lengths must not be negative. Raises ``ValueError`` naming the first bad row
    (scheduler order). Arrays are numpy."""
    if (num_cached < 0).any() or (num_new < 0).any():
        i = int(np.flatnonzero((num_cached < 0) | (num_new < 0))[0])
        raise ValueError(f"pack: row {i} has num_cached {int(num_cached[i])}, num_new {int(num_new[i])}")
    need = -(-(num_cached.astype(np.int64) + num_new) // block_size)
    short = (lengths > 0) & (lengths < need)
    if short.any():
        i = int(np.flatnonzero(short)[0])
        raise ValueError(f"pack: row {i}'s block list holds {int(lengths[i])} blocks; its "
                         f"{int(num_cached[i])} + {int(num_new[i])} tokens need {int(need[i])}")


class Packer:
    """Builds a step's attention ``Context`` fields on the GPU from per-row scheduler state.

    ``decodes_latents``: the model's attention layers decode cached MLA latents (the runner's ``decodes_latents``,
    ``model_runner.py:380-384``); a step whose rows all carry the same number of drafts is then a decode step."""

    def __init__(self, device, block_size: int, decodes_latents: bool = False):
        self.block_size = block_size
        self.decodes_latents = decodes_latents
        self.buffers = StagingBuffers(device)

    def pack(self, num_cached, num_new, block_lists, num_speculative_tokens: int = 0,
             is_prompt=None, num_logits=None, num_back=None) -> tuple[torch.Tensor, dict]:
        """Per-row ``num_cached``, ``num_new`` (scheduler order) and block lists -> ``(positions, context)``.

        ``context`` has the keys of ``prepare_batch``'s context dict (``model_runner.py:448-462``) that attention
        and the logits gather read, plus ``order`` (batch row -> scheduler row). ``is_prompt`` marks prompt rows
        (default: rows with more than one new token and no drafts allowed, i.e. ``num_new > 1 +
        num_speculative_tokens``); a row that is not a prompt carries ``num_new - 1`` drafts. The step is
        ``is_prefill`` as the reference decides it (``:380-384``): any prompt row, or any drafts unless the model
        decodes latents and every row has the same query length. ``num_logits`` (scheduler order) is the number of
        logits rows each row samples: its drafts + 1, or 0 for a chunk that does not sample (default: drafts + 1
        for every row). As in the reference, ``logits_indices`` is gathered only for an ``is_prefill`` step and is
        None otherwise (every row samples). ``num_back`` (device int32 ``[B]``, scheduler order, optional): drafts
        of the previous step that were rejected, per row; the row's tokens start that many positions earlier
        (``_move_back``, ``:527-551``), and the host lengths stay upper bounds. The returned tensors live in
        buffers the next call reuses.
        """
        self.buffers.begin()
        plan = self.stage(num_cached, num_new, block_lists, num_speculative_tokens, is_prompt, num_logits)
        out = self.run(plan, num_back)
        self.buffers.end()
        return out

    def stage(self, num_cached, num_new, block_lists, num_speculative_tokens: int = 0, is_prompt=None,
              num_logits=None) -> PackPlan:
        """Copy the per-row inputs to the device (one pinned copy) and derive the host-side row ints.

        The rows' Python ints and block lists are laid out straight into the pinned buffer by ``_hoststage``
        (num_cached | num_new | block-list offsets | block ids, then the logits-row counts); the row ints the
        host needs are read back from that buffer as numpy views."""
        rows = len(num_new)
        if rows == 0:
            raise ValueError("pack: a step needs at least one row")
        hs = _host_stage()
        n_ids = hs.count_ids(block_lists)
        base = 3 * rows + 1 + n_ids
        buf = self.buffers.host_view("inputs", base + rows, torch.int32)  # room for the logits-row counts
        _, _, width = hs.stage_rows(num_cached, num_new, block_lists, buf.ctypes.data, base)
        num_cached, num_new = buf[:rows], buf[rows:2 * rows]
        lengths = np.diff(buf[2 * rows:3 * rows + 1])
        check_block_lists(num_cached, num_new, lengths, self.block_size)
        tokens = int(num_new.sum())
        query_len = decode_query_len(num_new, num_speculative_tokens)
        order = np.argsort(num_new != query_len, kind="stable")
        lens_b, ends_b = num_new[order], (num_cached + num_new)[order]
        is_prompt = num_new > 1 + num_speculative_tokens if is_prompt is None else np.asarray(is_prompt, bool)
        drafts = np.where(is_prompt, 0, num_new - 1)
        has_prompt = bool(is_prompt.any())
        uniform = not has_prompt and self.decodes_latents and bool((num_new == query_len).all())
        host = dict(
            is_prefill=has_prompt or (bool(drafts.any()) and not uniform),
            max_seqlen_q=int(lens_b.max()),
            max_seqlen_k=int(ends_b.max()),
            cu_seqlens_q_host=[0, *np.cumsum(lens_b).tolist()],
            cu_seqlens_k_host=[0, *np.cumsum(ends_b).tolist()],
            decode_query_len=query_len,
        )
        logits, size = -1, base
        if host["is_prefill"]:
            n_log = (drafts + 1).astype(np.int32) if num_logits is None else np.asarray(num_logits, dtype=np.int32)
            if n_log.shape != (rows,) or (n_log < 0).any() or (n_log > num_new).any():
                raise ValueError("pack: num_logits must give 0 .. num_new logits rows per row")
            logits = int(n_log.sum())
            buf[base:base + rows] = n_log
            size = base + rows
        inputs = self.buffers.upload("inputs", size, torch.int32)
        slot_count = int(num_new[lengths > 0].sum())
        return PackPlan(rows, tokens, width, slot_count, query_len, inputs, host, logits)

    def run(self, plan: PackPlan, num_back: torch.Tensor | None = None) -> tuple[torch.Tensor, dict]:
        """Launch the pack kernel on staged inputs; returns ``(positions, context)``."""
        buf, rows, width = self.buffers, plan.rows, plan.width
        if num_back is not None:
            assert num_back.dtype == torch.int32 and num_back.shape == (rows,) and num_back.is_contiguous()
        d_cached = plan.inputs[:rows]
        d_new = plan.inputs[rows:2 * rows]
        d_indptr = plan.inputs[2 * rows:3 * rows + 1]
        n_ids = plan.inputs.numel() - (3 * rows + 1) - (rows if plan.logits >= 0 else 0)
        d_ids = plan.inputs[3 * rows + 1:3 * rows + 1 + n_ids]
        d_nlog = plan.inputs[3 * rows + 1 + n_ids:] if plan.logits >= 0 else None
        logits = buf.device_buffer("logits_indices", plan.logits, torch.int64) if plan.logits >= 0 else None
        has_tables = width > 0
        out_order = buf.device_buffer("order", rows, torch.int32)
        cu_q = buf.device_buffer("cu_seqlens_q", rows + 1, torch.int32)
        cu_k = buf.device_buffer("cu_seqlens_k", rows + 1, torch.int32)
        positions = buf.device_buffer("positions", plan.tokens, torch.int64)
        slots = buf.device_buffer("slot_mapping", plan.slot_count, torch.int32)
        context_lens = buf.device_buffer("context_lens", rows, torch.int32)
        tables = buf.device_buffer("block_tables", rows * width, torch.int32) if has_tables else None
        _capi.call("lv_pack", d_cached.data_ptr(), d_new.data_ptr(), d_indptr.data_ptr(),
                   d_ids.data_ptr() if d_ids.numel() else None, rows, plan.query_len, self.block_size, width,
                   plan.tokens, out_order.data_ptr(), cu_q.data_ptr(), cu_k.data_ptr(), positions.data_ptr(),
                   slots.data_ptr() if has_tables else None, context_lens.data_ptr(),
                   tables.data_ptr() if has_tables else None,
                   d_nlog.data_ptr() if plan.logits > 0 else None,
                   logits.data_ptr() if plan.logits > 0 else None, _capi.ptr(num_back), 0,
                   _capi.stream_of(buf.device))
        context = dict(
            plan.host,
            cu_seqlens_q=cu_q,
            cu_seqlens_k=cu_k,
            slot_mapping=slots,
            context_lens=context_lens,
            block_tables=tables.view(rows, width) if has_tables else None,
            logits_indices=logits,
            order=out_order,
        )
        return positions, context
