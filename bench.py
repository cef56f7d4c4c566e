"""Benchmark of the continuous-batching attention path on one MI355X.

A step is one pass of the path over one synthetic batch, all on the GPU with inputs resident in HBM:
- the pack kernel turns the rows' (num_cached, num_new, block list), staged on the device before timing, into the
  step's metadata (cu_seqlens, positions, slot_mapping, context_lens, padded block_tables);
- the store kernel scatters the step's new K/V (or MLA latents) into the paged cache;
- the attention op attends the whole batch (one varlen launch for decode and prompt rows; MLA latent decode for
  the DeepSeek workload).

The JSON line's ``value`` is the primary workload's algorithmic HBM bytes per step / step time (GB/s). Default
primary: Qwen3-8B-shaped chunked-prefill mixed batch at token budget 8192 (4 chunks of 1536 new tokens on a
cached prefix U[0, 6144], plus 2048 decode rows with context U[256, 4096]; 32/8 heads, d128, bf16, 256-token
pages). The line also carries per-kernel times from HIP events on the launch stream, a ``roofline`` object for
the attention op, a ``cpu_baseline`` (the oracle's restatement of the reference PyTorch backend timed on a bounded
sample on the host cores) and, under ``workloads``, the same figures for the other shapes this path is measured on
(Qwen3-8B pure decode at batch 256, long-context split-K decode, DeepSeek-V2-Lite MLA decode, Qwen3-0.6B mixed,
and two steps of prompts -- the Qwen3-8B mixed step's four chunks alone and DeepSeek-V2-Lite MLA prefill chunks --
which are MFMA work and report TFLOP/s against the bf16 peak).
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
EXTRA = ("qwen3_8b_decode,qwen3_8b_long,deepseek_v2_lite_mla,qwen3_0_6b_mixed,qwen3_8b_prefill,"
         "deepseek_v2_lite_mla_prefill,qwen3_8b_decode_bs16,deepseek_v2_lite_mla_bs16")
RIDGE_FLOP_PER_BYTE = PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)  # above it a step is MFMA-bound
# Workloads whose whole working set fits the 256 MB Infinity Cache: each timed step starts from a flushed cache.
FLUSHED = {"qwen3_0_6b_mixed"}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="qwen3_8b_mixed")
    ap.add_argument("--extra", default=EXTRA, help="comma-separated workloads also measured ('none' for none)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seed", type=int, default=0)
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


def measure(name: str, steps: int, warmup: int, seed: int, dev):
    """Time ``steps`` steps of one workload; returns (figures, workload, tensors)."""
    import torch

    import numpy as np

    from lvattn import Context, MI355XAttention, Packer, merge_attention_
    from lvattn import workloads as W

    wl = W.WORKLOADS[name](seed)
    t = W.materialize(wl, dev, torch.bfloat16, seed=seed)
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
        ex = t.expanded
        cu_ctx = torch.tensor([0, *np.cumsum(wl.num_cached).tolist()], dtype=torch.int32, device=dev)
        max_ctx = max(max(wl.num_cached), 1)
    flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev) if name in FLUSHED else None
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    ev = {k: [torch.cuda.Event(enable_timing=True) for _ in range(steps)] for k in ("a", "b", "c", "d")}

    def step(i=None):
        if flush is not None:
            flush.fill_(i or 0)  # evicts the previous step's lines; outside the event brackets
        if i is not None:
            ev["a"][i].record(stream)
        _, ctx = packer.run(plan)
        if i is not None:
            ev["b"][i].record(stream)
        if wl.is_mla:
            backend.store_latents(t.k_new, t.k_cache, ctx["slot_mapping"])
        else:
            backend.store_kvcache(t.k_new, t.v_new, t.k_cache, t.v_cache, ctx["slot_mapping"])
        if i is not None:
            ev["c"][i].record(stream)
        fields = {k: v for k, v in ctx.items() if k in Context.__slots__}
        if wl.is_mla_prefill:
            cu_q, max_q = ctx["cu_seqlens_q"], ctx["max_seqlen_q"]
            o, lse = backend.varlen_with_lse(ex["q"], ex["k"], ex["v"], cu_q, cu_q, max_q, max_q, True)
            co, clse = backend.varlen_with_lse(ex["q"], ex["k_ctx"], ex["v_ctx"], cu_q, cu_ctx, max_q, max_ctx, False)
            merge_attention_(co, clse, o, lse, out)
        elif wl.is_mla:
            backend.mla_decode(t.q, t.k_cache, wl.v_dim, Context(**fields), out=out)
        else:
            backend.forward(t.q, t.k_new, t.v_new, t.k_cache, t.v_cache, Context(**fields), out=out)
        if i is not None:
            ev["d"][i].record(stream)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps

    def avg_ms(x, y):
        return sum(ev[x][i].elapsed_time(ev[y][i]) for i in range(steps)) / steps

    pack_ms, store_ms, attn_ms = avg_ms("a", "b"), avg_ms("b", "c"), avg_ms("c", "d")
    step_ms = avg_ms("a", "d") if flush is not None else wall_ms
    nbytes = W.algorithmic_bytes(wl)
    flops = W.algorithmic_flops(wl)
    attn_gbs = nbytes["attention"] / (attn_ms * 1e-3) / 1e9
    figures = {
        "workload": name,
        "rows": wl.rows,
        "tokens": wl.tokens,
        "ms_per_step": round(step_ms, 4),
        "GBs": round(nbytes["total"] / (step_ms * 1e-3) / 1e9, 1),
        "pct_of_peak_hbm": round(100 * nbytes["total"] / (step_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 2),
        "tokens_per_s_per_layer": round(wl.tokens / (step_ms * 1e-3), 1),
        "kernel_ms": {"pack": round(pack_ms, 4), "store": round(store_ms, 4), "attention": round(attn_ms, 4)},
        "host_stage_ms": round(host_stage_ms, 4),
        "attention_GBs": round(attn_gbs, 1),
        "attention_frac_of_peak": round(attn_gbs / PEAK_HBM_GBS, 4),
        "attention_TFLOPs": round(flops / (attn_ms * 1e-3) / 1e12, 2),
        "attention_frac_of_mfma_peak": round(flops / (attn_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "bound": "mfma" if flops / nbytes["attention"] > RIDGE_FLOP_PER_BYTE else "hbm",
        "bytes": nbytes,
        "flops": flops,
        "cache_flushed_each_step": flush is not None,
    }
    return figures, wl, t


def cpu_baseline(wl, t, dec_sample: int = 256, passes: int = 5):
    """The oracle's TorchAttention restatement (page gather, zeroed padding, row padding, bottom-right mask,
    GQA-folded SDPA) in fp32 on the host cores, on a bounded sample of the step: every prompt chunk in full plus the
    first ``dec_sample`` decode rows, with the rows' pages copied to the host beforehand. One warmup pass, whose
    outputs are first checked against the textbook dense oracle (a few decode rows and prompt queries, max-abs
    1e-3), then the median of ``passes`` timed passes; the decode time is scaled to all decode rows. Returns the
    object for the JSON line, in the same algorithmic-byte GB/s as the GPU figures (and tokens/s per layer)."""
    import numpy as np
    import torch

    from lvattn import workloads as W
    from oracle import attention as A

    torch.set_num_threads(len(os.sched_getaffinity(0)))
    cores = torch.get_num_threads()
    order = W.batch_order(wl)
    num_new = np.asarray(wl.num_new)[order]
    num_cached = np.asarray(wl.num_cached)[order]
    lists = [wl.block_lists[i] for i in order]
    dec_rows = [r for r in range(wl.rows) if num_new[r] == 1]
    pre_rows = [r for r in range(wl.rows) if num_new[r] > 1]
    sample_dec = dec_rows[:dec_sample]
    q_start = np.concatenate([[0], np.cumsum(num_new)])

    def compact(rows):
        """The rows' pages copied to the host (bf16), renumbered 0..n-1 (the oracle reads only these)."""
        pages = sorted({p for r in rows for p in lists[r]})
        index = {p: i for i, p in enumerate(pages)}
        sel = torch.tensor(pages, dtype=torch.long, device=t.k_cache.device)
        kc, vc = t.k_cache[sel].cpu(), t.v_cache[sel].cpu()
        width = max(len(lists[r]) for r in rows)
        bt = torch.full((len(rows), width), -1, dtype=torch.int32)
        for j, r in enumerate(rows):
            bt[j, : len(lists[r])] = torch.tensor([index[p] for p in lists[r]], dtype=torch.int32)
        return kc, vc, bt

    math_ = A.TorchMath(wl.num_heads, wl.head_dim, wl.scale, wl.num_kv_heads)
    q_all = t.q.float().cpu()
    dec = None
    if sample_dec:
        kc, vc, bt = compact(sample_dec)
        q = q_all[[int(q_start[r]) for r in sample_dec]]
        lens = torch.tensor([int(num_cached[r] + 1) for r in sample_dec], dtype=torch.int32)
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

    def one_pass():
        times, outs = {}, {}
        if dec is not None:
            t0 = time.perf_counter()
            outs["decode"] = A.decode_in_row_chunks(math_, *dec, rows_per_chunk=16)
            times["decode"] = time.perf_counter() - t0
        if pre:
            t0 = time.perf_counter()
            outs["prefill"] = [math_.prefill(q, None, None, kc, vc, ctx) for q, kc, vc, ctx in pre]
            times["prefill"] = time.perf_counter() - t0
        return times, outs

    _, outs = one_pass()  # warmup, and the outputs the check reads
    worst = 0.0
    if dec is not None:
        q, kc, vc, lens, bt = dec
        for j in sorted({0, len(sample_dec) // 2, len(sample_dec) - 1}):
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
    runs = [one_pass()[0] for _ in range(passes)]
    timings = {k: sorted(r[k] for r in runs)[passes // 2] for k in runs[0]}
    if "decode" in timings:
        timings["decode"] *= len(dec_rows) / len(sample_dec)
    seconds = sum(timings.values())
    nbytes = W.algorithmic_bytes(wl)["attention"]
    return {
        "value": round(nbytes / seconds / 1e9, 2),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"oracle TorchAttention restatement (attention only), fp32, {cores} threads, checked against the "
                   f"dense oracle (max abs {worst:.1e}), 1 warmup + median of {passes}: all {len(pre_rows)} prompt "
                   f"chunks in full ({timings.get('prefill', 0):.2f} s) + {len(sample_dec)} of {len(dec_rows)} "
                   f"decode rows ({timings.get('decode', 0):.2f} s"
                   f"{'' if len(sample_dec) == len(dec_rows) else ' scaled to all rows'})"),
        "tokens_per_s_per_layer": round(wl.tokens / seconds, 1),
        "seconds_per_step": round(seconds, 3),
    }


def attention_op(wl) -> str:
    """The kernels of one attention op on this workload (the roofline's subject)."""
    if wl.is_mla_prefill:
        return "lv_varlen_attention x2 (causal new tokens, unmasked prefix; varlen_kernel) + lv_merge_attn_states"
    if wl.is_mla:
        return "lv_mla_decode (mla_run_kernel + mla_run_merge_kernel)"
    if all(n > 1 for n in wl.num_new):  # a step of prompts: the serial schedule, prompt tiles on the whole GPU
        return "lv_paged_attention (plan_kernel + prompt_list_kernel)"
    if any(n > 1 for n in wl.num_new):
        return ("lv_paged_attention (plan_kernel + decode_persistent_kernel on a second stream beside "
                "prompt_overlap_kernel + splitk_merge_kernel)")
    return "lv_paged_attention (plan_kernel + decode_persistent_kernel + splitk_merge_kernel)"


def traffic_of(name: str):
    """HBM bytes per attention op (all its kernels, one step) from the committed rocprofv3 counter summary."""
    f = ROOT / "profiles" / f"traffic_{name}.json"
    if f.exists():
        return json.loads(f.read_text()).get("hbm_bytes_per_launch")
    return None


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
    primary, wl, t = measure(args.workload, args.steps, args.warmup, args.seed, dev)
    cpu = None if args.no_cpu_baseline or wl.is_mla else cpu_baseline(wl, t)
    del t
    torch.cuda.empty_cache()
    extras = []
    for name in [n for n in args.extra.split(",") if n and n != "none" and n != args.workload]:
        fig, _, t = measure(name, args.steps, args.warmup, args.seed, dev)
        extras.append(fig)
        del t
        torch.cuda.empty_cache()

    result = {
        "metric": METRIC,
        "value": primary["GBs"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": primary["ms_per_step"],
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
            "kernel": attention_op(wl),
            "algorithmic_flops_per_launch": primary["flops"],
            "GBs": primary["attention_GBs"],
        },
        "flops": primary["flops"],
        "workloads": extras,
    }
    if cpu is not None:
        result["cpu_baseline"] = cpu
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
