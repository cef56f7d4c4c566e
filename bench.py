"""Benchmark of the continuous-batching attention path on one MI355X.

A step is one pass of the path over one synthetic batch, all on the GPU with inputs resident in HBM: the pack
kernel turns the rows' (num_cached, num_new, block list) -- staged on the device before timing -- into the step's
metadata, the store kernel scatters the step's new K/V into the paged cache, and the paged-attention kernel
attends the whole mixed batch. Default workload: Qwen3-8B-shaped chunked-prefill mixed batch at token budget
8192 (4 chunks of 1536 new tokens on a cached prefix U[0, 6144], plus 2048 decode rows with context
U[256, 4096]; 32/8 heads, d128, bf16, 256-token pages).

Prints one JSON line. ``value`` is the step's algorithmic HBM bytes / step time (GB/s); the line also carries
tokens/s per layer, the fraction of the 8 TB/s peak, per-kernel times from HIP events on the launch stream,
a ``roofline`` object for the attention kernel and a ``cpu_baseline`` (the oracle's restatement of the
reference PyTorch backend, timed on a bounded sample on the host cores).
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


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="qwen3_8b_mixed")
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


def cpu_baseline(wl, t, dec_sample: int = 96):
    """The oracle's TorchAttention restatement (page gather, zeroed padding, row padding, bottom-right mask,
    GQA-folded SDPA) in fp32 on the host cores, on a bounded sample of the step: every prompt chunk in full plus
    ``dec_sample`` decode rows, the decode time scaled to all decode rows. Returns the object for the JSON line."""
    import numpy as np
    import torch

    from lvattn.workloads import batch_order
    from oracle import attention as A

    torch.set_num_threads(len(os.sched_getaffinity(0)))
    cores = torch.get_num_threads()
    bs = wl.block_size
    order = batch_order(wl)
    num_new = np.asarray(wl.num_new)[order]
    num_cached = np.asarray(wl.num_cached)[order]
    lists = [wl.block_lists[i] for i in order]
    dec_rows = [r for r in range(wl.rows) if num_new[r] == 1]
    pre_rows = [r for r in range(wl.rows) if num_new[r] > 1]
    sample_dec = dec_rows[:dec_sample]
    q_start = np.concatenate([[0], np.cumsum(num_new)])

    def compact(rows):
        """The rows' pages copied to the host as fp32, renumbered 0..n-1 (the oracle reads only these)."""
        pages = sorted({p for r in rows for p in lists[r]})
        index = {p: i for i, p in enumerate(pages)}
        sel = torch.tensor(pages, dtype=torch.long, device=t.k_cache.device)
        kc = t.k_cache[sel].float().cpu()
        vc = t.v_cache[sel].float().cpu()
        width = max(len(lists[r]) for r in rows)
        bt = torch.full((len(rows), width), -1, dtype=torch.int32)
        for j, r in enumerate(rows):
            bt[j, : len(lists[r])] = torch.tensor([index[p] for p in lists[r]], dtype=torch.int32)
        return kc, vc, bt

    math_ = A.TorchMath(wl.num_heads, wl.head_dim, wl.scale, wl.num_kv_heads)
    q_all = t.q.float().cpu()
    timings = {}
    if sample_dec:
        kc, vc, bt = compact(sample_dec)
        q = q_all[[int(q_start[r]) for r in sample_dec]]
        lens = torch.tensor([int(num_cached[r] + 1) for r in sample_dec], dtype=torch.int32)
        t0 = time.perf_counter()
        A.decode_in_row_chunks(math_, q, kc, vc, lens, bt, rows_per_chunk=16)
        timings["decode"] = (time.perf_counter() - t0) * len(dec_rows) / len(sample_dec)
        del kc, vc
    if pre_rows:
        kc, vc, bt = compact(pre_rows)
        total = 0.0
        for j, r in enumerate(pre_rows):
            lq, lk = int(num_new[r]), int(num_cached[r] + num_new[r])
            q = q_all[int(q_start[r]): int(q_start[r]) + lq]
            ctx = A.context(cu_seqlens_q=torch.tensor([0, lq], dtype=torch.int32),
                            cu_seqlens_k=torch.tensor([0, lk], dtype=torch.int32), max_seqlen_q=lq, max_seqlen_k=lk,
                            block_tables=bt[j:j + 1])
            t0 = time.perf_counter()
            math_.prefill(q, None, None, kc, vc, ctx)
            total += time.perf_counter() - t0
        timings["prefill"] = total
    seconds = sum(timings.values())
    return {
        "value": round(wl.tokens / seconds, 1),
        "unit": "tokens/s per layer",
        "cores": cores,
        "kind": "port",
        "sample": (f"oracle TorchAttention restatement, fp32, {cores} threads: all {len(pre_rows)} prompt chunks "
                   f"in full ({timings.get('prefill', 0):.2f} s) + {len(sample_dec)} of {len(dec_rows)} decode rows "
                   f"scaled to all ({timings.get('decode', 0):.2f} s est.)"),
        "seconds_per_step": round(seconds, 3),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this path runs on a single GPU)",
              file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
        return
    import torch

    from lvattn import Context, MI355XAttention, Packer, _capi
    from lvattn import workloads as W

    dev = torch.device("cuda:0")
    wl = W.WORKLOADS[args.workload](args.seed)
    if wl.is_mla:
        raise SystemExit("the MLA workload is benchmarked by bench_mla (not yet built)")
    t = W.materialize(wl, dev, torch.bfloat16, seed=args.seed)
    backend = MI355XAttention(wl.num_heads, wl.head_dim, wl.scale, wl.num_kv_heads)
    packer = Packer(dev, wl.block_size)
    plan = packer.stage(wl.num_cached, wl.num_new, wl.block_lists)
    torch.cuda.synchronize()
    out = torch.empty_like(t.q)
    stream = torch.cuda.current_stream(dev)

    ev = {k: [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)] for k in ("a", "b", "c", "d")}

    def step(i=None):
        if i is not None:
            ev["a"][i].record(stream)
        _, ctx = packer.run(plan)
        if i is not None:
            ev["b"][i].record(stream)
        backend.store_kvcache(t.k_new, t.v_new, t.k_cache, t.v_cache, ctx["slot_mapping"])
        if i is not None:
            ev["c"][i].record(stream)
        fields = {k: v for k, v in ctx.items() if k in Context.__slots__}
        backend.forward(t.q, t.k_new, t.v_new, t.k_cache, t.v_cache, Context(**fields), out=out)
        if i is not None:
            ev["d"][i].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    def avg_ms(x, y):
        return sum(ev[x][i].elapsed_time(ev[y][i]) for i in range(args.steps)) / args.steps

    pack_ms, store_ms, attn_ms = avg_ms("a", "b"), avg_ms("b", "c"), avg_ms("c", "d")
    ms_per_step = elapsed * 1e3 / args.steps
    nbytes = W.algorithmic_bytes(wl)
    flops = W.algorithmic_flops(wl)
    gbs = nbytes["total"] / (ms_per_step * 1e-3) / 1e9
    attn_gbs = nbytes["attention"] / (attn_ms * 1e-3) / 1e9
    attn_tflops = flops / (attn_ms * 1e-3) / 1e12
    traffic = None
    tfile = ROOT / "profiles" / f"traffic_{wl.name}.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")
    result = {
        "metric": "paged-attn HBM GB/s (% of peak) + tokens/s per layer, Qwen3-8B mixed batch",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": wl.name,
            "rows": wl.rows,
            "tokens": wl.tokens,
            "heads": f"{wl.num_heads}/{wl.num_kv_heads}",
            "head_dim": wl.head_dim,
            "block_size": wl.block_size,
            "parallelism": "single GPU",
        },
        "pct_of_peak_hbm": round(100 * gbs / PEAK_HBM_GBS, 2),
        "tokens_per_s_per_layer": round(wl.tokens / (ms_per_step * 1e-3), 1),
        "kernel_ms": {"pack": round(pack_ms, 4), "store": round(store_ms, 4), "attention": round(attn_ms, 4)},
        "bytes": nbytes,
        "roofline": {
            "bound": "hbm",
            "achieved": round(attn_gbs, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(attn_gbs / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "kernel": "paged_attention_kernel",
            "algorithmic_bytes_per_launch": nbytes["attention"],
            "tflops": round(attn_tflops, 2),
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(wl, t)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
