#!/usr/bin/env python3
"""Benchmark of the branching-decode hot path on one MI355X.

Workload: paged decode attention at Llama-3-8B attention shapes (bf16, 32 q /
8 kv heads, head_dim 128, page size 16, 64 sequences with contexts uniform in
[512, 4096], block tables from a seeded permutation of a 65,536-page pool,
Q/K/V ~ N(0,1), scale 1/sqrt(128)). One step = one decode call over the batch
with every input already resident in HBM.

Prints one JSON line with the whole-job throughput (achieved HBM GB/s of
algorithmic bytes), the roofline fraction against MI355X's 8 TB/s, and the
reference's CPU decode path (gather + per-sequence SDPA, torch on the host
cores) timed beside it on the same inputs.

  python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
METRIC = "branch-decode tokens/sec on 1 GPU; paged-decode achieved HBM GB/s vs peak"
PEAK_HBM_GBS = 8000.0
TRAFFIC_FILE = os.path.join(HERE, "profiles", "paged_decode_llama3_8b_traffic.txt")


def _measured_traffic():
    """HBM bytes per decode launch from the committed rocprofv3 --pmc summary, if any."""
    try:
        text = open(TRAFFIC_FILE).read()
    except OSError:
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", text, flags=re.M)
    return float(m.group(1)) if m else None


def _cpu_baseline(batch, min_seconds: float):
    """The reference's CPU decode path, timed on the host on the same inputs."""
    import torch

    from oracle.attention import reference_cpu_decode

    torch.set_num_threads(max(1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))))
    cores = torch.get_num_threads()
    # Compact host copy of the referenced pages only.
    flat = [p for t in batch.tables for p in t]
    idx = torch.tensor(flat, dtype=torch.long, device=batch.k_pool.device)
    k_host = batch.k_pool[idx].cpu()
    v_host = batch.v_pool[idx].cpu()
    tables, off = [], 0
    for t in batch.tables:
        tables.append(list(range(off, off + len(t))))
        off += len(t)
    q_host = batch.q.cpu()
    reps, t_total = 0, 0.0
    while t_total < min_seconds or reps < 1:
        t0 = time.perf_counter()
        reference_cpu_decode(q_host, k_host, v_host, tables, batch.lens, batch.block_size)
        t_total += time.perf_counter() - t0
        reps += 1
    per = t_total / reps
    return {
        "value": round(batch.algorithmic_bytes() / per / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"the full 64-sequence batch, {reps} repetitions ({t_total:.1f} s): "
                  f"build_packed_kv gather + per-sequence SDPA in bf16, torch CPU",
        "ms_per_step": round(per * 1e3, 3),
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="minimum host time spent on the CPU baseline")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(this build has no multi-GPU path)", file=sys.stderr)
        return 2
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py runs as a single process on one GPU", file=sys.stderr)
        return 2

    import torch

    from mentat_amd import ops
    from mentat_amd._lib import LAYOUT_NATIVE
    from mentat_amd.workloads import paged_decode_batch

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    print("bench: building the workload", file=sys.stderr, flush=True)
    b = paged_decode_batch(device=dev, seed=0, layout=LAYOUT_NATIVE)
    nbytes = b.algorithmic_bytes()
    out = torch.empty_like(b.q)

    def step():
        ops.paged_decode(b.q, b.k_store, b.v_store, layout=b.layout, block_tables=b.block_tables,
                         seq_lens=b.seq_lens, max_seqlen=b.max_seqlen, scale=b.scale, out=out)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    print("bench: warmup done", file=sys.stderr, flush=True)

    stream = torch.cuda.current_stream(dev)  # the stream the kernels are launched on
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    evs[0].record(stream)
    for i in range(args.steps):
        step()
        evs[i + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per_step_ms = [evs[i].elapsed_time(evs[i + 1]) for i in range(args.steps)]
    total_ms = evs[0].elapsed_time(evs[-1])
    ms = total_ms / args.steps
    achieved = nbytes / (ms * 1e-3) / 1e9
    print(f"bench: {args.steps} steps, mean {ms:.4f} ms, median {statistics.median(per_step_ms):.4f} ms, "
          f"wall {wall:.3f} s", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu_baseline:
        print("bench: timing the CPU baseline", file=sys.stderr, flush=True)
        cpu = _cpu_baseline(b, args.cpu_seconds)

    result = {
        "metric": METRIC,
        "value": round(achieved, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) Q/K/V, seeded ragged contexts and page permutation)",
        "config": {
            "workload": "paged decode attention, Llama-3-8B attention shapes",
            "num_seqs": b.q.shape[0],
            "q_heads": b.q.shape[1],
            "kv_heads": b.k_pool.shape[2],
            "head_dim": b.q.shape[2],
            "page_size": b.block_size,
            "context": "uniform [512, 4096], seed 0",
            "sum_context_tokens": sum(b.lens),
            "pool_pages": b.k_pool.shape[0],
            "pool_layout": "native (K [page][kv head][slot][dim], V [page][kv head][dim][slot])",
            "algorithmic_bytes_per_step": nbytes,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": _measured_traffic(),
        },
        "cpu_baseline": cpu,
        "decode_calls_per_s": round(1e3 / ms, 1),
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
