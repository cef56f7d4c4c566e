"""Full-graph decode steps with the packing on the device: the attention path of ``ModelRunner.capture_cudagraph``
and ``_replay_full`` (``lean_vllm/engine/model_runner.py:585-607,664-701``).

The reference packs a decode step on the host, then copies ``slot_mapping``, ``context_lens`` and
``block_tables`` into the graph's static buffers before every replay; padding rows get slot -1 and context length
0 (``:597-602``). Here the pack kernel runs inside the captured graph, so a replay costs one pinned copy of the
step's per-row ints (``num_cached``, ``num_new``, block lists) and then the graph: pack, store and attention.
A padding row has no block list and ``num_cached = -num_new``: the pack kernel, in dense-slot mode, gives its
tokens slot -1 and its row context length 0, so it stores nothing and attends nothing. Attention plans its work
on the device from the lengths in the graph, so nothing has to be refreshed before a replay.
"""

from __future__ import annotations


import numpy as np
import torch

from . import _capi
from .backend import MI355XAttention
from .context import Context
from .pack import _host_stage

LV_PACK_DENSE_SLOTS = 1


class DecodeGraphs:
    """Captured decode steps of ``query_len`` queries per row, one graph per batch size (smallest that fits is
    replayed). ``max_blocks`` bounds every row's block list (``model_runner.py:661-667``)."""

    def __init__(self, backend: MI355XAttention, k_cache: torch.Tensor, v_cache: torch.Tensor, batch_sizes,
                 max_blocks: int, query_len: int = 1):
        self.backend, self.k_cache, self.v_cache = backend, k_cache, v_cache
        self.device = k_cache.device
        self.block_size = k_cache.size(1)
        self.sizes = sorted(set(int(b) for b in batch_sizes))
        self.max_blocks, self.query_len = int(max_blocks), int(query_len)
        max_bs = self.sizes[-1]
        tokens = max_bs * self.query_len
        heads, kv_heads, dim = backend.num_heads, backend.num_kv_heads, backend.head_dim
        dev, dt = self.device, k_cache.dtype
        self.q = torch.zeros(tokens, heads, dim, dtype=dt, device=dev)
        self.k = torch.zeros(tokens, kv_heads, dim, dtype=dt, device=dev)
        self.v = torch.zeros(tokens, kv_heads, dim, dtype=dt, device=dev)
        self.out = torch.zeros(tokens, heads, dim, dtype=dt, device=dev)
        n_in = 3 * max_bs + 1 + max_bs * self.max_blocks
        self._inputs = torch.zeros(n_in, dtype=torch.int32, device=dev)
        self._host = torch.zeros(n_in, dtype=torch.int32, pin_memory=True)
        self._copied: torch.cuda.Event | None = None
        i32 = dict(dtype=torch.int32, device=dev)
        self.positions = torch.zeros(tokens, dtype=torch.int64, device=dev)
        self.slot_mapping = torch.zeros(tokens, **i32)
        self.context_lens = torch.zeros(max_bs, **i32)
        self.block_tables = torch.zeros(max_bs * self.max_blocks, **i32)
        self.cu_seqlens_q = torch.zeros(max_bs + 1, **i32)
        self.cu_seqlens_k = torch.zeros(max_bs + 1, **i32)
        self.order = torch.zeros(max_bs, **i32)
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self._pool = None

    # -- staging ---------------------------------------------------------------------------------------------
    def _stage(self, bs: int, num_cached, block_lists) -> None:
        """Per-row ints of a ``bs``-row graph into the pinned buffer, real rows first, then padding rows."""
        if self._copied is not None:  # the previous replay's copy may still read the pinned buffer
            self._copied.synchronize()
        rows = len(num_cached)
        q = self.query_len
        host = self._host.numpy()
        # Real rows, then padding rows (num_cached -q: context length 0, no blocks), straight from the Python lists.
        _, at, width = _host_stage().stage_graph_rows(num_cached, block_lists, host.ctypes.data, host.size, bs, q)
        if width > self.max_blocks:
            raise ValueError(f"a block list is longer than the {self.max_blocks} blocks the graphs were sized for")
        lengths = np.diff(host[2 * bs:2 * bs + rows + 1])
        need = -(-(host[:rows] + q) // self.block_size)
        if rows and (lengths < need).any():
            raise ValueError("a row's block list does not cover its context")
        n = 3 * bs + 1 + at
        self._inputs[:n].copy_(self._host[:n], non_blocking=True)
        self._copied = torch.cuda.Event()
        self._copied.record(torch.cuda.current_stream(self.device))

    # -- the captured step -----------------------------------------------------------------------------------
    def _run(self, bs: int) -> None:
        q, w = self.query_len, self.max_blocks
        tokens = bs * q
        d = self._inputs
        _capi.call("lv_pack", d.data_ptr(), d[bs:].data_ptr(), d[2 * bs:].data_ptr(), d[3 * bs + 1:].data_ptr(),
                   bs, q, self.block_size, w, tokens, self.order.data_ptr(), self.cu_seqlens_q.data_ptr(),
                   self.cu_seqlens_k.data_ptr(), self.positions.data_ptr(), self.slot_mapping.data_ptr(),
                   self.context_lens.data_ptr(), self.block_tables.data_ptr(), None, None, None, LV_PACK_DENSE_SLOTS,
                   _capi.stream_of(self.device))
        self.backend.store_kvcache(self.k[:tokens], self.v[:tokens], self.k_cache, self.v_cache,
                                   self.slot_mapping[:tokens])
        ctx = Context(is_prefill=q > 1, cu_seqlens_q=self.cu_seqlens_q[:bs + 1],
                      cu_seqlens_k=self.cu_seqlens_k[:bs + 1], max_seqlen_q=q, max_seqlen_k=w * self.block_size,
                      slot_mapping=self.slot_mapping[:tokens], context_lens=self.context_lens[:bs],
                      block_tables=self.block_tables[:bs * w].view(bs, w))
        if q == 1:
            self.backend.decode(self.q[:tokens], self.k_cache, self.v_cache, ctx, out=self.out[:tokens])
        else:
            self.backend.prefill(self.q[:tokens], None, None, self.k_cache, self.v_cache, ctx, out=self.out[:tokens])

    def capture(self) -> None:
        """Capture every batch size, largest first, each after an eager warmup on padding rows (which grows the
        backend's workspace to what the graph will address)."""
        for bs in reversed(self.sizes):
            self._stage(bs, [], [])
            self._run(bs)
            torch.cuda.synchronize(self.device)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=self._pool):
                self._run(bs)
            self._pool = graph.pool()
            self.graphs[bs] = graph
        torch.cuda.synchronize(self.device)

    def replay(self, num_cached, block_lists, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """One decode step of ``len(num_cached)`` rows (``_replay_full``): stores ``k``, ``v`` at the rows' next
        positions and returns attention ``[rows * query_len, Hq, D]`` (a view of the graphs' output buffer)."""
        rows = len(num_cached)
        bs = next((b for b in self.sizes if b >= rows), None)
        if bs is None or bs not in self.graphs:
            raise ValueError(f"no captured graph holds {rows} rows (sizes {self.sizes})")
        tokens = rows * self.query_len
        self._stage(bs, num_cached, block_lists)
        self.q[:tokens].copy_(q)
        self.k[:tokens].copy_(k)
        self.v[:tokens].copy_(v)
        self.graphs[bs].replay()
        return self.out[:tokens]
