"""Benchmark of the continuous-batching attention path on one MI355X.

A step is one pass of the path over one synthetic batch, all on the GPU with inputs resident in HBM, as a model
runs it per step:
- the pack kernel turns the rows' (num_cached, num_new, block list), staged on the device before timing, into the
  step's metadata (cu_seqlens, positions, slot_mapping, context_lens, padded block_tables) -- once per step;
- then, for each of the model's attention layers (Qwen3-8B 36, Qwen3-0.6B 28, DeepSeek-V2-Lite 27; ``--layers``
  overrides), the store kernel scatters that layer's new K/V (or MLA latents) into its paged cache and the
  attention op attends the whole batch (one varlen launch for decode and prompt rows; MLA latent decode for the
  DeepSeek workload). Every layer reads the one Context the pack produced, so the attention work list is planned
  in the first layer and reused by the rest, as the reference's backends cache per-step plans. The layers rotate
  through enough copies of the cache that each one starts cold (none is still in the 256 MB Infinity Cache).

The JSON line's ``value`` is the primary workload's algorithmic HBM bytes per step / step time (GB/s), and
``tokens_per_s_per_layer`` its tokens / (step time / layers); the timed steps record no events. Default primary:
Qwen3-8B-shaped chunked-prefill mixed batch at token budget 8192 (4 chunks of 1536 new tokens on a cached prefix
U[0, 6144], plus 2048 decode rows with context U[256, 4096]; 32/8 heads, d128, bf16, 256-token pages). The line
also carries per-kernel times from HIP events on the launch stream: the attention op per launch from launches back
to back between one event pair (a step's worth of layers per rep, the first planning), and, from a few further
steps with events around each op, per layer: pack, store and attention (bracketed: these include the events' own
cost, a few microseconds), the attention of the first layer -- which plans -- and of the later ones. Then a
``roofline`` object for the attention op (per launch, back to back), a ``cpu_baseline`` (the
oracle's restatement of the reference PyTorch backend timed over the whole step on the host cores, after every GPU
measurement; batch-256 decode carries one too) and, under
``workloads``, the same figures for the other shapes this path is measured on (Qwen3-8B pure decode at batch 256,
long-context split-K decode, DeepSeek-V2-Lite MLA decode, Qwen3-0.6B mixed, both decode steps again on
lean-vLLM's default 16-token pages, and two steps of prompts -- the Qwen3-8B mixed step's four chunks alone and
DeepSeek-V2-Lite MLA prefill chunks -- which are MFMA work and report TFLOP/s against the bf16 peak).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "lean-vllm_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0
METRIC = "paged-attn HBM GB/s (% of peak) + tokens/s per layer, Qwen3-8B mixed batch"
EXTRA = ("qwen3_8b_decode,qwen3_8b_long,deepseek_v2_lite_mla,qwen3_0_6b_mixed,qwen3_8b_prefill,qwen3_8b_prefix_chunk,"
         "deepseek_v2_lite_mla_prefill,deepseek_v2_lite_mla_prefill_two_pass,qwen3_8b_decode_bs16,"
         "deepseek_v2_lite_mla_bs16,qwen3_8b_mixed_bs16,qwen3_8b_prefill_bs16")
RIDGE_FLOP_PER_BYTE = PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)  # above it a step is MFMA-bound
CPU_ALSO = "qwen3_8b_decode"  # a CPU baseline is also timed for this workload (batch-256 Qwen3-8B decode)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="qwen3_8b_mixed")
    ap.add_argument("--extra", default=EXTRA, help="comma-separated workloads also measured ('none' for none)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--layers", type=int, default=None,
                    help="attention layers per step (default: the model's own count; 1 times a single layer)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB, 5 times (the reference kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes)")
    return ap.parse_args()


def calibrate_copy(mib: int):
    """A plain copy of known size: each launch reads and writes exactly ``mib`` MiB."""
    import torch

    dev = torch.device("cuda:0")
    src = torch.ones(mib << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_per_launch": mib << 20, "launches": 5}), flush=True)


class Arena:
    """Device memory taken once, from the first workload on, and reused by every later one, as a serving engine
    allocates its KV cache once at start (``lean_vllm/engine/model_runner.py:261-277``). Multi-GB caches allocated
    afresh after others were freed land in HBM differently from one allocation to the next: two copies of one cache
    in one process have measured a decode step 2-5% apart. Tensors are views into a few large blocks; ``reset``
    hands the same memory to the next workload."""

    def __init__(self, dev):
        self.dev = dev
        self.blocks: list = []
        self.at = (0, 0)  # (block, byte offset) of the next tensor

    def reset(self):
        self.at = (0, 0)

    def take(self, shape, dtype):
        import math

        import torch

        numel = math.prod(shape)
        n = -(-numel * torch.empty((), dtype=dtype).element_size() // 256) * 256
        b, off = self.at
        while b < len(self.blocks) and off + n > self.blocks[b].numel():
            b, off = b + 1, 0
        if b == len(self.blocks):
            self.blocks.append(torch.empty(max(n, 4 << 30), dtype=torch.uint8, device=self.dev))
        self.at = (b, off + n)
        return self.blocks[b][off:off + n].view(dtype)[:numel].view(shape)


def cache_sets(wl, touched_bytes: int, layers: int) -> int:
    """Copies of the layer state (caches, or MLA prefill's expanded keys) the layers of a step rotate through, so
    that no layer finds the one it attends still in the 256 MB Infinity Cache from an earlier layer."""
    if layers <= 1:
        return 1
    return max(2, min(8, 1 + -(-2 * 256 * 2**20 // max(touched_bytes, 1))))


def measure(name: str, steps: int, warmup: int, seed: int, dev, layers: int | None = None, arena=None):
    """Time ``steps`` steps of one workload; returns (figures, workload, tensors of the first layer).

    A step is what the model runs per step on this path: the pack kernel once, then for each of the model's
    attention layers the store of that layer's new K/V and its attention, every layer reading the one Context the
    pack produced (so the work list is planned in the first layer and reused by the rest, as the reference caches
    per-step plans). The layers rotate through a few copies of the cache so that each starts cold."""
    import torch

    import numpy as np

    from lvattn import Context, MI355XAttention, Packer, merge_attention_
    from lvattn import workloads as W

    wl = W.WORKLOADS[name](seed)
    layers = wl.num_layers if layers is None else layers
    nbytes = W.algorithmic_bytes(wl)
    sets = cache_sets(wl, nbytes["attention"] + nbytes["store"], layers)
    if arena is not None:
        arena.reset()
    ts = [W.materialize(wl, dev, torch.bfloat16, seed=seed + r, alloc=arena.take if arena is not None else None)
          for r in range(sets)]
    t = ts[0]
    heads_kv = wl.num_heads if wl.is_mla else wl.num_kv_heads
    head_dim = wl.expanded[0] if wl.is_mla_prefill else wl.latent_dim if wl.is_mla else wl.head_dim
    backend = MI355XAttention(wl.num_heads, head_dim, wl.scale, heads_kv)
    packer = Packer(dev, wl.block_size)
    # Host time of staging a step's per-row ints (the part of packing left on the host), median of 21; outside the
    # GPU timings, which start from inputs already on the device.
    host_ms = []
    for _ in range(21):
        packer.buffers.begin()
        t0 = time.perf_counter()
        plan = packer.stage(wl.num_cached, wl.num_new, wl.block_lists)
        host_ms.append((time.perf_counter() - t0) * 1e3)
        packer.buffers.end()
    torch.cuda.synchronize()
    host_stage_ms = sorted(host_ms)[len(host_ms) // 2]
    out_dim = wl.expanded[1] if wl.is_mla_prefill else wl.v_dim if wl.is_mla else wl.head_dim
    out = torch.empty(wl.tokens, wl.num_heads, out_dim, dtype=torch.bfloat16, device=dev)
    if wl.is_mla_prefill:  # the cached prefix as one unmasked chunk (layers/attention.py:288-315)
        cu_ctx = torch.tensor([0, *np.cumsum(wl.num_cached).tolist()], dtype=torch.int32, device=dev)
        max_ctx = max(max(wl.num_cached), 1)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)

    def attend(x, ctx, context):
        """One layer's attention op."""
        if wl.is_mla_prefill:
            ex = x.expanded
            cu_q, max_q = ctx["cu_seqlens_q"], ctx["max_seqlen_q"]
            if wl.two_pass:  # the reference layer's calls
                o, lse = backend.varlen_with_lse(ex["q"], ex["k"], ex["v"], cu_q, cu_q, max_q, max_q, True)
                co, clse = backend.varlen_with_lse(ex["q"], ex["k_ctx"], ex["v_ctx"], cu_q, cu_ctx, max_q,
                                                   max_ctx, False)
                merge_attention_(co, clse, o, lse, out)
            else:  # one call over context and new keys
                backend.prefill_with_context(ex["q"], ex["k"], ex["v"], ex["k_ctx"], ex["v_ctx"], cu_q, cu_ctx,
                                             max_q, out=out)
        elif wl.is_mla:
            backend.mla_decode(x.q, x.k_cache, wl.v_dim, context, out=out)
        else:
            backend.forward(x.q, x.k_new, x.v_new, x.k_cache, x.v_cache, context, out=out)

    def step(ev=None):
        """One step; returns the pack's fields. ev: (pack event pair, per layer (start, after the store, after the
        attention)) to record, or None."""
        if ev is not None:
            ev[0][0].record(stream)
        _, ctx = packer.run(plan)
        if ev is not None:
            ev[0][1].record(stream)
        context = Context(**{k: v for k, v in ctx.items() if k in Context.__slots__})
        for layer in range(layers):
            x = ts[layer % sets]
            if ev is not None:
                ev[1][layer][0].record(stream)
            if wl.is_mla:
                backend.store_latents(x.k_new, x.k_cache, ctx["slot_mapping"])
            else:
                backend.store_kvcache(x.k_new, x.v_new, x.k_cache, x.v_cache, ctx["slot_mapping"])
            if ev is not None:
                ev[1][layer][1].record(stream)
            attend(x, ctx, context)
            if ev is not None:
                ev[1][layer][2].record(stream)
        return ctx

    def event():
        return torch.cuda.Event(enable_timing=True)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # The timed steps carry no events: an event costs the GPU a few microseconds, which the layers of a small step
    # would feel (a Qwen3-0.6B layer's attention reads 37.6 us between its own events against 31.9 us per launch back
    # to back).
    t0 = time.perf_counter()
    for _ in range(steps):
        ctx = step()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    # The per-layer breakdown: a few more steps with events around the pack and each layer's store and attention,
    # behind one step without them (so that the GPU is busy when they are queued, as in the timed steps, and no
    # host time between two launches lands between their events).
    n_ev = min(steps, 5)
    ev = [((event(), event()), [(event(), event(), event()) for _ in range(layers)]) for _ in range(n_ev)]
    step()
    for i in range(n_ev):
        step(ev[i])
    torch.cuda.synchronize()
    # The attention op alone, back to back between one event pair: reps steps' worth of layers on the step's pack
    # output, each rep through a fresh Context (its first layer plans, as a step's does), the layers rotating
    # through the cache copies as in a step.
    reps = min(steps, 5)
    e0, e1 = event(), event()
    e0.record(stream)
    for _ in range(reps):
        context = Context(**{k: v for k, v in ctx.items() if k in Context.__slots__})
        for layer in range(layers):
            attend(ts[layer % sets], ctx, context)
    e1.record(stream)
    torch.cuda.synchronize()
    attn_b2b = e0.elapsed_time(e1) / (reps * layers)

    def mean(xs):
        return sum(xs) / len(xs)

    pack_ms = mean([a.elapsed_time(b) for (a, b), _ in ev])
    store_ms = mean([e[0].elapsed_time(e[1]) for _, st in ev for e in st])
    attn_ms = mean([e[1].elapsed_time(e[2]) for _, st in ev for e in st])
    attn_first = mean([st[0][1].elapsed_time(st[0][2]) for _, st in ev])
    attn_later = mean([e[1].elapsed_time(e[2]) for _, st in ev for e in st[1:]]) if layers > 1 else attn_first
    # The attention of the layers on each copy of the cache (later layers): copies are separate allocations, and
    # their placement in HBM moves a decode step's time by a few percent from one allocation to the next.
    by_set = [mean([st[layer][1].elapsed_time(st[layer][2]) for _, st in ev
                    for layer in range(c, layers, sets) if layer > 0 or layers == 1])
              for c in range(min(sets, layers)) if c > 0 or layers == 1 or sets < layers]
    step_ms = wall_ms
    layer_ms = step_ms / layers
    flops = W.algorithmic_flops(wl)
    step_bytes = layers * (nbytes["attention"] + nbytes["store"]) + nbytes["pack"]
    attn_gbs = nbytes["attention"] / (attn_b2b * 1e-3) / 1e9
    figures = {
        "workload": name,
        "rows": wl.rows,
        "tokens": wl.tokens,
        "layers": layers,
        "cache_sets": sets,
        "ms_per_step": round(step_ms, 4),
        "ms_per_layer": round(layer_ms, 4),
        "GBs": round(step_bytes / (step_ms * 1e-3) / 1e9, 1),
        "pct_of_peak_hbm": round(100 * step_bytes / (step_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 2),
        "tokens_per_s_per_layer": round(wl.tokens / (layer_ms * 1e-3), 1),
        # attention: per launch, back to back (a step's mix of planning and reusing layers); the bracketed figures
        # come from an event pair around each layer's op, which adds the events' own cost.
        "kernel_ms": {"pack": round(pack_ms, 4), "store": round(store_ms, 4), "attention": round(attn_b2b, 4),
                      "attention_bracketed": round(attn_ms, 4), "attention_first_layer": round(attn_first, 4),
                      "attention_later_layers": round(attn_later, 4),
                      "attention_by_cache_set": [round(x, 4) for x in by_set]},
        "host_stage_ms": round(host_stage_ms, 4),
        "attention_GBs": round(attn_gbs, 1),
        "attention_frac_of_peak": round(attn_gbs / PEAK_HBM_GBS, 4),
        "attention_TFLOPs": round(flops / (attn_b2b * 1e-3) / 1e12, 2),
        "attention_frac_of_mfma_peak": round(flops / (attn_b2b * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "bound": "mfma" if flops / nbytes["attention"] > RIDGE_FLOP_PER_BYTE else "hbm",
        "bytes": nbytes,
        "flops": flops,
    }
    del ts[1:]
    return figures, wl, t


def cpu_inputs(wl, t, check_rows: int = 64):
    """Host copies of what the CPU baseline reads, taken right after the workload's GPU measurement so that its
    device tensors can be freed: the step's queries, and the pages of every decode row and of every prompt chunk
    (bf16, renumbered). The timing itself runs after every GPU measurement (``cpu_baseline``)."""
    import numpy as np
    import torch

    from lvattn import workloads as W
    from oracle import attention as A

    order = W.batch_order(wl)
    num_new = np.asarray(wl.num_new)[order]
    num_cached = np.asarray(wl.num_cached)[order]
    lists = [wl.block_lists[i] for i in order]
    dec_rows = [r for r in range(wl.rows) if num_new[r] == 1]
    pre_rows = [r for r in range(wl.rows) if num_new[r] > 1]
    q_start = np.concatenate([[0], np.cumsum(num_new)])

    def compact(rows):
        """The rows' pages copied to the host (bf16), renumbered 0..n-1 (the oracle reads only these)."""
        pages = sorted({p for r in rows for p in lists[r]})
        index = {p: i for i, p in enumerate(pages)}
        kc = torch.empty((len(pages),) + tuple(t.k_cache.shape[1:]), dtype=t.k_cache.dtype)
        vc = torch.empty_like(kc)
        for i in range(0, len(pages), 2048):  # bounded device temporaries
            sel = torch.tensor(pages[i:i + 2048], dtype=torch.long, device=t.k_cache.device)
            kc[i:i + 2048] = t.k_cache[sel].cpu()
            vc[i:i + 2048] = t.v_cache[sel].cpu()
        width = max(len(lists[r]) for r in rows)
        bt = torch.full((len(rows), width), -1, dtype=torch.int32)
        for j, r in enumerate(rows):
            bt[j, : len(lists[r])] = torch.tensor([index[p] for p in lists[r]], dtype=torch.int32)
        return kc, vc, bt

    q_all = t.q.float().cpu()
    dec = None
    if dec_rows:
        kc, vc, bt = compact(dec_rows)
        q = q_all[[int(q_start[r]) for r in dec_rows]]
        lens = torch.tensor([int(num_cached[r] + 1) for r in dec_rows], dtype=torch.int32)
        dec = (q, kc, vc, lens, bt)
    pre = []
    if pre_rows:
        kc, vc, bt = compact(pre_rows)
        for j, r in enumerate(pre_rows):
            lq, lk = int(num_new[r]), int(num_cached[r] + num_new[r])
            ctx = A.context(cu_seqlens_q=torch.tensor([0, lq], dtype=torch.int32),
                            cu_seqlens_k=torch.tensor([0, lk], dtype=torch.int32), max_seqlen_q=lq, max_seqlen_k=lk,
                            block_tables=bt[j:j + 1])
            pre.append((q_all[int(q_start[r]): int(q_start[r]) + lq], kc, vc, ctx))
    return {"dec": dec, "pre": pre, "check_rows": min(check_rows, len(dec_rows))}


def cpu_baseline(wl, inputs):
    """The oracle's TorchAttention restatement (page gather, zeroed padding, row padding, bottom-right mask,
    GQA-folded SDPA) in fp32 on all host cores, over the whole step: every decode row and every prompt chunk. One
    warmup pass over the first ``check_rows`` decode rows and the chunks, whose outputs are checked against the
    textbook dense oracle (a few decode rows and prompt queries, max-abs 1e-3), then one timed pass over the whole
    step. Returns the object for the JSON line, in the same algorithmic-byte GB/s as the GPU figures (and tokens/s
    per layer)."""
    import torch

    from lvattn import workloads as W
    from oracle import attention as A

    torch.set_num_threads(len(os.sched_getaffinity(0)))
    cores = torch.get_num_threads()
    dec, pre = inputs["dec"], inputs["pre"]
    math_ = A.TorchMath(wl.num_heads, wl.head_dim, wl.scale, wl.num_kv_heads)

    def one_pass(rows=None):
        times, outs = {}, {}
        if dec is not None:
            q, kc, vc, lens, bt = dec
            n = len(lens) if rows is None else rows
            t0 = time.perf_counter()
            outs["decode"] = A.decode_in_row_chunks(math_, q[:n], kc, vc, lens[:n], bt[:n], rows_per_chunk=16)
            times["decode"] = time.perf_counter() - t0
        if pre:
            t0 = time.perf_counter()
            outs["prefill"] = [math_.prefill(q, None, None, kc, vc, ctx) for q, kc, vc, ctx in pre]
            times["prefill"] = time.perf_counter() - t0
        return times, outs

    _, outs = one_pass(inputs["check_rows"])  # warmup, and the outputs the check reads
    worst = 0.0
    if dec is not None:
        q, kc, vc, lens, bt = dec
        for j in sorted({0, inputs["check_rows"] // 2, inputs["check_rows"] - 1}):
            n = int(lens[j])
            pages = bt[j, : -(-n // wl.block_size)].long()
            k = kc[pages].flatten(0, 1)[:n].float()
            v = vc[pages].flatten(0, 1)[:n].float()
            want = A.dense_attention(q[j:j + 1], k, v, wl.scale, causal=False)
            worst = max(worst, (outs["decode"][j:j + 1] - want).abs().max().item())
    for (q, kc, vc, ctx), o in zip(pre, outs.get("prefill", [])):
        lq, lk = q.size(0), int(ctx.max_seqlen_k)
        pages = ctx.block_tables[0, : -(-lk // wl.block_size)].long()
        k = kc[pages].flatten(0, 1)[:lk].float()
        v = vc[pages].flatten(0, 1)[:lk].float()
        for j in (0, lq - 1):
            want = A.dense_attention(q[j:j + 1], k[:lk - lq + j + 1], v[:lk - lq + j + 1], wl.scale, causal=False)
            worst = max(worst, (o[j:j + 1] - want).abs().max().item())
    if worst > 1e-3:
        raise RuntimeError(f"cpu baseline: the timed restatement differs from the dense oracle by {worst:.2e}")
    timings, _ = one_pass()
    seconds = sum(timings.values())
    nbytes = W.algorithmic_bytes(wl)["attention"]
    n_dec = 0 if dec is None else len(dec[3])
    return {
        "value": round(nbytes / seconds / 1e9, 2),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"{wl.name}, the whole step: oracle TorchAttention restatement (attention only), fp32, {cores} "
                   f"threads, checked against the dense oracle (max abs {worst:.1e}), 1 warmup on {inputs['check_rows']}"
                   f" decode rows, then one timed pass: {len(pre)} prompt chunks ({timings.get('prefill', 0):.2f} s)"
                   f" + all {n_dec} decode rows ({timings.get('decode', 0):.2f} s)"),
        "tokens_per_s_per_layer": round(wl.tokens / seconds, 1),
        "seconds_per_step": round(seconds, 3),
    }


def attention_op(wl) -> str:
    """The kernels of one attention op on this workload (the roofline's subject)."""
    if wl.is_mla_prefill and wl.two_pass:
        return "lv_varlen_attention x2 (causal new tokens, unmasked prefix; varlen_kernel) + lv_merge_attn_states"
    if wl.is_mla_prefill:
        return "lv_varlen_context_attention (varlen_kernel over prefix then causal new keys, one softmax)"
    if wl.is_mla:
        return "lv_mla_decode (mla_run_kernel + mla_run_merge_kernel)"
    if all(n > 1 for n in wl.num_new):  # a step of prompts: the serial schedule, prompt tiles on the whole GPU
        return "lv_paged_attention (plan_kernel + prompt_list_kernel)"
    # The paged steps' kernels as the committed kernel trace of this workload names them.
    f = ROOT / "profiles" / f"traffic_{wl.name}.json"
    if f.exists():
        kernels = [k.removeprefix("lv::") for k in json.loads(f.read_text()).get("kernels", [])]
        if kernels:
            return f"lv_paged_attention ({' + '.join(kernels)})"
    return "lv_paged_attention (plan_kernel + decode kernels)"


def traffic_of(name: str):
    """HBM bytes per attention op (all its kernels, one step) from the committed rocprofv3 counter summary."""
    f = ROOT / "profiles" / f"traffic_{name}.json"
    if f.exists():
        return json.loads(f.read_text()).get("hbm_bytes_per_launch")
    return None


def traffic_source(name: str):
    """Where ``roofline.traffic`` comes from: counters can only be read under the profiler, so it is the committed
    summary of a profiling run (its own machine and session), not this run; its op time is given beside it."""
    f = ROOT / "profiles" / f"traffic_{name}.json"
    if not f.exists():
        return None
    j = json.loads(f.read_text())
    return {"file": f"profiles/traffic_{name}.json", "measured": "rocprofv3 FETCH_SIZE + WRITE_SIZE over the op's "
            "kernels in a profiling run, scaled by the same counters' reading for a 1 GiB copy",
            "op_span_us_in_that_run": j.get("rocprof_op_span_us_median_later_layers"),
            "full_bench_attention_us_in_that_session": j.get("session_full_bench_attention_us")}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported: this path runs on a single GPU and "
              "nothing in it spans GPUs", file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
        return
    import torch

    dev = torch.device("cuda:0")
    # Every GPU measurement first, back to back; the CPU baselines (whose host copies are taken right after their
    # workload's measurement) run last, so no GPU figure follows a long GPU-idle gap.
    cpu_wanted = set() if args.no_cpu_baseline else {args.workload, CPU_ALSO}
    cpu_in = {}
    arena = Arena(dev)
    primary, wl, t = measure(args.workload, args.steps, args.warmup, args.seed, dev, args.layers, arena)
    if args.workload in cpu_wanted and not wl.is_mla:
        cpu_in[args.workload] = (wl, cpu_inputs(wl, t))
    del t
    extras = []
    for name in [n for n in args.extra.split(",") if n and n != "none" and n != args.workload]:
        fig, xwl, t = measure(name, args.steps, args.warmup, args.seed, dev, args.layers, arena)
        extras.append(fig)
        if name in cpu_wanted and not xwl.is_mla:
            cpu_in[name] = (xwl, cpu_inputs(xwl, t))
        del t
    del arena
    torch.cuda.empty_cache()
    cpu = {name: cpu_baseline(*cpu_in.pop(name)) for name in list(cpu_in)}
    for fig in extras:
        if fig["workload"] in cpu:
            fig["cpu_baseline"] = cpu[fig["workload"]]

    result = {
        "metric": METRIC,
        "value": primary["GBs"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": primary["ms_per_step"],
        "ms_per_layer": primary["ms_per_layer"],
        "layers_per_step": primary["layers"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": primary["workload"],
            "rows": primary["rows"],
            "tokens": primary["tokens"],
            "heads": f"{wl.num_heads}/{wl.num_heads if wl.is_mla else wl.num_kv_heads}",
            "head_dim": wl.latent_dim if wl.is_mla else wl.head_dim,
            "block_size": wl.block_size,
            "layers": primary["layers"],
            "parallelism": "single GPU",
        },
        "pct_of_peak_hbm": primary["pct_of_peak_hbm"],
        "tokens_per_s_per_layer": primary["tokens_per_s_per_layer"],
        "kernel_ms": primary["kernel_ms"],
        "host_stage_ms": primary["host_stage_ms"],
        "bytes": primary["bytes"],
        "roofline": {
            "bound": "hbm",
            "achieved": primary["attention_GBs"],
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": primary["attention_frac_of_peak"],
            "traffic": traffic_of(primary["workload"]),
            "traffic_source": traffic_source(primary["workload"]),
            "kernel": attention_op(wl),
            "algorithmic_bytes_per_launch": primary["bytes"]["attention"],
            "tflops": primary["attention_TFLOPs"],
        } if primary["bound"] == "hbm" else {
            "bound": "mfma",
            "achieved": primary["attention_TFLOPs"],
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": primary["attention_frac_of_mfma_peak"],
            "traffic": traffic_of(primary["workload"]),
            "traffic_source": traffic_source(primary["workload"]),
            "kernel": attention_op(wl),
            "algorithmic_flops_per_launch": primary["flops"],
            "GBs": primary["attention_GBs"],
        },
        "flops": primary["flops"],
        "workloads": extras,
    }
    if args.workload in cpu:
        result["cpu_baseline"] = cpu[args.workload]
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
