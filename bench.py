#!/usr/bin/env python3
"""Benchmark of the branching-decode hot path on one MI355X.

Default workload (--workload decode): paged decode attention at Llama-3-8B
attention shapes (bf16, 32 q / 8 kv heads, head_dim 128, page size 16, 64
sequences with contexts uniform in [512, 4096], block tables from a seeded
permutation of a 65,536-page pool, Q/K/V ~ N(0,1), scale 1/sqrt(128)). One
step = one decode call over the batch with every input already resident in HBM.

Prints one JSON line with the whole-job throughput (achieved HBM GB/s of
algorithmic bytes), the roofline fraction against MI355X's 8 TB/s, and the
reference's CPU path timed beside it on the same inputs.

With no --workload (or --workload all) the line also carries "workloads": the
tree, rows, prefill and e2e results below, each with its own ms_per_step,
value, roofline and cpu_baseline.

Single workloads (their own JSON line, same fields):
  --workload tree   prefix-tree decode at Qwen3-8B attention shapes: 4 trees
                    of 32 leaves over 2048-token prompts (GB/s of unique bytes)
  --workload rows   fused entropy gate + temperature/top-p sampling over
                    [256, 151936] bf16 logits (GB/s of logits bytes)
  --workload e2e    end-to-end rollout: random-init Llama-3-8B bf16, 16 prompts
                    of 256 ids, 512 new tokens, absolute gate 2.5 nats, up to 8
                    branches per prompt, all prompts continuously batched
                    (branch-decode tokens/s)
  --workload prefill  causal GQA prefill attention, 4 prompts x 2048 positions,
                    Llama-3-8B heads, bf16 (TFLOP/s against the dense bf16 peak)

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload all|decode|tree|rows|e2e|prefill]
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
PEAK_BF16_TFLOPS = 2500.0  # dense bf16 MFMA
TRAFFIC_FILE = os.path.join(HERE, "profiles", "paged_decode_llama3_8b_traffic.txt")
ROWS_TRAFFIC_FILE = os.path.join(HERE, "profiles", "row_stats_sampling.md")
TREE_TRAFFIC_FILE = os.path.join(HERE, "profiles", "tree_decode_qwen3_8b.md")


def _measured_traffic(path: str = TRAFFIC_FILE):
    """HBM bytes per launch from a committed rocprofv3 --pmc summary, if any."""
    try:
        text = open(path).read()
    except OSError:
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", text, flags=re.M)
    return float(m.group(1)) if m else None


def _traffic_source(path: str) -> str | None:
    """Where roofline.traffic comes from: a committed rocprofv3 --pmc summary (not measured in
    this run), with the commit and date it was measured at."""
    try:
        text = open(path).read()
    except OSError:
        return None
    at = re.search(r"^measured_at:\s*(.+)$", text, flags=re.M)
    rel = os.path.relpath(path, HERE)
    return f"committed rocprofv3 --pmc summary {rel}" + (f" ({at.group(1).strip()})" if at else "")


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


def _time_steps(step, steps: int, warmup: int, dev):
    """Untimed warmup, then `steps` calls bracketed by HIP events on the launch stream."""
    import torch

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)  # the stream the kernels are launched on
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    evs[0].record(stream)
    for i in range(steps):
        step()
        evs[i + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = [evs[i].elapsed_time(evs[i + 1]) for i in range(steps)]
    ms = evs[0].elapsed_time(evs[-1]) / steps
    print(f"bench: {steps} steps, mean {ms:.4f} ms, median {statistics.median(per):.4f} ms, wall {wall:.3f} s",
          file=sys.stderr, flush=True)
    return ms


def _line(args, value_gbs: float, ms: float, config: dict, cpu, traffic, extra: dict | None = None) -> dict:
    out = {
        "metric": METRIC,
        "value": round(value_gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded; see config)",
        "config": config,
        "roofline": {
            "bound": "hbm",
            "achieved": round(value_gbs, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(value_gbs / PEAK_HBM_GBS, 4),
            "traffic": traffic,
        },
        "cpu_baseline": cpu,
    }
    if extra:
        out.update(extra)
    return out


def _time_graph(step, steps: int, warmup: int, dev):
    """Untimed warmup on a side stream, then the `steps` calls captured as one
    graph (as the rollout's decode steps run) and replayed once, untimed, and
    once between two HIP events on the replay stream."""
    import torch

    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):  # also creates the side stream's workspace before the capture
        for _ in range(max(warmup, 1)):
            step()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for _ in range(steps):
            step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / steps
    print(f"bench: {steps} steps in one graph replay, mean {ms:.4f} ms, wall {wall:.3f} s", file=sys.stderr,
          flush=True)
    return ms


def run_decode(args, dev) -> dict:
    import torch

    from mentat_amd import ops
    from mentat_amd._lib import LAYOUT_NATIVE
    from mentat_amd.workloads import paged_decode_batch

    print("bench: building the paged decode workload", file=sys.stderr, flush=True)
    b = paged_decode_batch(device=dev, seed=0, layout=LAYOUT_NATIVE)
    nbytes = b.algorithmic_bytes()
    out = torch.empty_like(b.q)
    # Two copies of Q and the K/V stores (same tables), used alternately: each
    # step re-reads data last touched ~1.2 GB of traffic earlier, beyond the
    # 256 MB Infinity Cache.
    g = torch.Generator(device=dev).manual_seed(1)
    sets = [(b.q, b.k_store, b.v_store),
            (torch.randn(b.q.shape, generator=g, device=dev).to(b.q.dtype), b.k_store.clone(), b.v_store.clone())]
    state = {"i": 0}

    def step():
        q, ks, vs = sets[state["i"] & 1]
        state["i"] += 1
        ops.paged_decode(q, ks, vs, layout=b.layout, block_tables=b.block_tables,
                         seq_lens=b.seq_lens, max_seqlen=b.max_seqlen, scale=b.scale, out=out)

    if args.no_graph:
        ms = _time_steps(step, args.steps, args.warmup, dev)
    else:
        ms = _time_graph(step, args.steps, args.warmup, dev)
    cpu = None
    if not args.no_cpu_baseline:
        print("bench: timing the CPU baseline", file=sys.stderr, flush=True)
        cpu = _cpu_baseline(b, args.cpu_seconds)
    config = {
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
        "rotation": "2 copies of Q and the K/V stores used alternately",
        "launch": "eager, one call per step" if args.no_graph else
                  "the timed calls captured as one graph and replayed (the rollout's decode steps are graph replays)",
    }
    line = _line(args, nbytes / (ms * 1e-3) / 1e9, ms, config, cpu, _measured_traffic(),
                 {"decode_calls_per_s": round(1e3 / ms, 1)})
    line["roofline"]["traffic_source"] = _traffic_source(TRAFFIC_FILE)
    line["data"] = "synthetic (seeded N(0,1) Q/K/V, seeded ragged contexts and page permutation)"
    return line


def run_tree(args, dev) -> dict:
    import torch

    from mentat_amd import ops
    from mentat_amd._lib import LAYOUT_NATIVE
    from mentat_amd.tree_plan import build_plan
    from mentat_amd.workloads import prefix_tree_batch

    print("bench: building the prefix-tree workload", file=sys.stderr, flush=True)
    tb = prefix_tree_batch(device=dev, seed=0)
    G = tb.q.shape[1] // tb.k_store.shape[1]
    t0 = time.perf_counter()
    plan = build_plan(tb.tables, tb.lens, tb.rows, block_size=tb.block_size, Hkv=tb.k_store.shape[1], G=G)
    plan_ms = (time.perf_counter() - t0) * 1e3
    out = torch.empty_like(tb.q)
    # Four copies of the stores (same trees and tables), used in turn: each
    # step re-reads data last touched ~240 MB of unique traffic earlier, so the
    # 256 MB Infinity Cache cannot serve the 80 MB working set from one step to
    # the next.
    sets = [(tb.k_store, tb.v_store)] + [(tb.k_store.clone(), tb.v_store.clone()) for _ in range(3)]
    state = {"i": 0}

    def step():
        ks, vs = sets[state["i"] % len(sets)]
        state["i"] += 1
        ops.tree_decode(tb.q, ks, vs, block_tables=tb.block_tables, plan=plan, scale=tb.scale, out=out)

    timer = _time_steps if args.no_graph else _time_graph
    ms = timer(step, args.steps, args.warmup, dev)
    rows_t = torch.tensor(tb.rows, dtype=torch.int32, device=dev)

    def paged():
        ks, vs = sets[state["i"] % len(sets)]
        state["i"] += 1
        ops.paged_decode(tb.q, ks, vs, max_seqlen=max(tb.lens), block_tables=tb.block_tables,
                         seq_lens=tb.seq_lens, seq_rows=rows_t, scale=tb.scale, layout=LAYOUT_NATIVE)

    paged_ms = timer(paged, args.steps, args.warmup, dev)
    ub, lb = tb.unique_bytes(), tb.logical_bytes()
    cpu = None
    if not args.no_cpu_baseline:
        print("bench: timing the CPU baseline", file=sys.stderr, flush=True)
        cpu = _cpu_baseline_tree(tb, args.cpu_seconds)
    config = {
        "workload": "prefix-tree decode attention, Qwen3-8B attention shapes",
        "trees": 4, "leaves_per_tree": 32, "prompt_tokens": 2048, "private_tokens": "0..512 per leaf",
        "q_heads": tb.q.shape[1], "kv_heads": tb.k_store.shape[1], "head_dim": tb.q.shape[2],
        "page_size": tb.block_size, "qk_rmsnorm": True,
        "unique_tokens": tb.unique_tokens(), "logical_tokens": tb.logical_tokens(),
        "unique_bytes_per_step": ub, "logical_bytes_per_step": lb,
        "rotation": "4 copies of the K/V stores used in turn",
        "launch": "eager, one call per step" if args.no_graph else "the timed calls captured as one graph and replayed",
        "plan": {"shared_tasks": plan.n_shared, "solo_items": plan.n_solo, "partial_slots": plan.n_slots,
                 "host_build_ms": round(plan_ms, 2)},
    }
    line = _line(args, ub / (ms * 1e-3) / 1e9, ms, config, cpu, _measured_traffic(TREE_TRAFFIC_FILE), {
        "logical_gbs": round(lb / (ms * 1e-3) / 1e9, 1),
        "paged_decode_same_batch_ms": round(paged_ms, 5),
        "speedup_vs_paged_decode": round(paged_ms / ms, 2),
    })
    line["roofline"]["traffic_source"] = _traffic_source(TREE_TRAFFIC_FILE)
    line["data"] = "synthetic (seeded trees grown through the paged cache manager; RMS-normed N(0,1) q/k, N(0,1) v)"
    return line


def _cpu_baseline_tree(tb, min_seconds: float):
    """The reference's CPU decode path (no prefix sharing) on a sample of the leaves."""
    import torch

    from oracle.attention import reference_cpu_decode

    torch.set_num_threads(max(1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))))
    sample = list(range(0, len(tb.seq_ids), 8))  # 16 of the 128 leaves
    flat = [p for i in sample for p in tb.tables[i]]
    kp = tb.k_store.permute(0, 2, 1, 3)
    vp = tb.v_store.permute(0, 3, 1, 2)
    idx = torch.tensor(flat, dtype=torch.long, device=tb.k_store.device)
    k_host, v_host = kp[idx].contiguous().cpu(), vp[idx].contiguous().cpu()
    tables, off = [], 0
    for i in sample:
        tables.append(list(range(off, off + len(tb.tables[i]))))
        off += len(tb.tables[i])
    q_host = tb.q[sample].cpu()
    lens = [tb.lens[i] for i in sample]
    reps, total = 0, 0.0
    while total < min_seconds or reps < 1:
        t0 = time.perf_counter()
        reference_cpu_decode(q_host, k_host, v_host, tables, lens, tb.block_size)
        total += time.perf_counter() - t0
        reps += 1
    per = total / reps
    Hkv, D = tb.k_store.shape[1], tb.q.shape[2]
    nbytes = sum(lens) * Hkv * D * 2 * 2
    return {"value": round(nbytes / per / 1e9, 3), "unit": "GB/s (logical bytes)", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"16 of the 128 leaves, {reps} repetitions ({total:.1f} s): per-leaf gather + SDPA, bf16, "
                      f"torch CPU (the reference reads every leaf's full context)"}


def run_rows(args, dev) -> dict:
    import torch

    from mentat_amd import ops
    from mentat_amd.workloads import sampling_logits

    print("bench: building the sampling workload", file=sys.stderr, flush=True)
    x, sig = sampling_logits(device=dev, seed=0)
    R, V = x.shape
    nbytes = x.numel() * x.element_size()
    T, TOP_P, THR = 0.7, 0.9, 3.0
    # Four logits sets (seeds 0..3) used in turn, so the 256 MB Infinity Cache
    # cannot hold a step's 78 MB until the next time it is read.
    xs = [x] + [sampling_logits(device=dev, seed=s)[0] for s in (1, 2, 3)]
    state = {"i": 0}
    # One launch of the fused kernel per step through the C ABI, into outputs allocated once
    # (ops.row_stats would add their allocation and a fill of the sample ids).
    from mentat_amd._lib import get_lib, stream_handle

    lib = get_lib()
    ent = torch.empty(R, dtype=torch.float32, device=dev)
    gate = torch.empty(R, dtype=torch.uint8, device=dev)
    smp = torch.empty(R, dtype=torch.int32, device=dev)
    def step():
        xi = xs[state["i"] % len(xs)]
        st = lib.mentat_row_stats(xi.data_ptr(), xi.stride(0), R, V, 2, T, 1.0, None, None, THR, 0, 1, T, TOP_P,
                                  1234, state["i"], ent.data_ptr(), None, None, None, gate.data_ptr(), None,
                                  None, smp.data_ptr(), stream_handle(dev))
        if st != 0:
            raise RuntimeError(f"mentat_row_stats returned {st}")
        state["i"] += 1

    ms = (_time_steps if args.no_graph else _time_graph)(step, args.steps, args.warmup, dev)
    st = ops.row_stats(x, temperature=T, gate_threshold=THR, sample=True, sample_temperature=T, top_p=TOP_P,
                       seed=1234, step=0, pen_stats=False)
    gated = int(st.gate.sum().item())
    cpu = None
    if not args.no_cpu_baseline:
        from oracle.sampling import reference_cpu_rows

        torch.set_num_threads(max(1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))))
        xs = x[:32].cpu()
        reps, total = 0, 0.0
        while total < args.cpu_seconds or reps < 1:
            t0 = time.perf_counter()
            reference_cpu_rows(xs, T, TOP_P, THR)
            total += time.perf_counter() - t0
            reps += 1
        per = total / reps
        cpu = {"value": round(xs.numel() * 2 / per / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
               "kind": "port",
               "sample": f"32 of the 256 rows, {reps} repetitions ({total:.1f} s): compute_entropy + HF top-p "
                         f"(sort, cumsum, multinomial) per row, bf16, torch CPU"}
    config = {
        "workload": "fused entropy gate + temperature/top-p sampling",
        "rows": R, "vocab": V, "sigma": "uniform [0.5, 4] per row", "temperature": T, "top_p": TOP_P,
        "gate_nats": THR, "gated_rows_seed0": gated, "sampler": "Philox4x32-10, seed 1234, step = call index",
        "rotation": "4 logits sets (seeds 0-3) used in turn",
        "logits_bytes_per_step": nbytes,
    }
    line = _line(args, nbytes / (ms * 1e-3) / 1e9, ms, config, cpu, _measured_traffic(ROWS_TRAFFIC_FILE),
                 {"rows_per_s": round(R * 1e3 / ms, 1)})
    line["roofline"]["traffic_source"] = _traffic_source(ROWS_TRAFFIC_FILE)
    line["data"] = "synthetic (seeded N(0, sigma_r) logits)"
    return line


def run_prefill(args, dev) -> dict:
    import torch

    from mentat_amd import ops

    # Llama-3-8B attention shapes; one 2048-token prompt per sequence, batch 4.
    B, S, Hq, Hkv, D = 4, 2048, 32, 8, 128
    print("bench: building the prefill workload", file=sys.stderr, flush=True)
    g = torch.Generator(device=dev).manual_seed(0)
    sets = []
    for _ in range(2):  # two input sets used in turn
        q = torch.randn(B, S, Hq, D, generator=g, device=dev).to(torch.bfloat16)
        k = torch.randn(B, S, Hkv, D, generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn(B, S, Hkv, D, generator=g, device=dev).to(torch.bfloat16)
        sets.append((q, k, v))
    out = torch.empty_like(sets[0][0])
    state = {"i": 0}

    def step():
        q, k, v = sets[state["i"] & 1]
        ops.prefill_attention(q, k, v, out=out)
        state["i"] += 1

    ms = _time_steps(step, args.steps, args.warmup, dev)
    # causal: every query position i multiplies i+1 keys, two products (QK^T, PV) of 2*D flops each
    flops = 4.0 * B * Hq * D * (S * (S + 1) / 2)
    tflops = flops / (ms * 1e-3) / 1e12
    cpu = None
    if not args.no_cpu_baseline:
        from oracle.attention import reference_cpu_prefill

        torch.set_num_threads(max(1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))))
        q, k, v = (t[:1].cpu() for t in sets[0])  # one of the B prompts
        reps, total = 0, 0.0
        while total < args.cpu_seconds or reps < 1:
            t0 = time.perf_counter()
            reference_cpu_prefill(q, k, v)
            total += time.perf_counter() - t0
            reps += 1
        per = total / reps
        cpu = {"value": round(flops / B / per / 1e12, 4), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
               "kind": "port",
               "sample": f"1 of the {B} prompts, {reps} repetitions ({total:.1f} s): GQA expand + causal SDPA, "
                         f"bf16, torch CPU"}
    config = {
        "workload": "causal GQA prefill attention, Llama-3-8B attention shapes",
        "batch": B, "seq_len": S, "q_heads": Hq, "kv_heads": Hkv, "head_dim": D, "window": None,
        "flops_per_step": flops, "rotation": "2 input sets used in turn",
    }
    line = _line(args, 0.0, ms, config, cpu, None)
    line.update({"value": round(tflops, 2), "unit": "TFLOP/s"})
    line["roofline"] = {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(tflops / PEAK_BF16_TFLOPS, 4), "traffic": None}
    line["data"] = "synthetic (seeded N(0,1) Q/K/V)"
    return line


class _IdTokenizer:
    """Prompts are token ids; decoding joins ids (the rollout never needs text)."""

    def __init__(self, eos: int):
        self.eos_token_id = eos

    def decode(self, ids, skip_special_tokens=True):
        return " ".join(str(i) for i in ids)


def _cpu_baseline_e2e(model, prompt, new_tokens: int, knobs: dict, seconds: float) -> dict:
    """The reference's rollout restated on the host cores (oracle.rollout_cpu):
    one prompt (the reference runs prompts one after another), the same weights
    copied to the CPU, decode stopped after `seconds`."""
    import torch

    from oracle.rollout_cpu import reference_cpu_rollout

    torch.set_num_threads(max(1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))))
    print("bench: copying the weights to the host for the CPU baseline", file=sys.stderr, flush=True)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(next(model.parameters()).dtype)
    try:
        with torch.device("meta"):
            cpu_model = type(model)(model.config)
    finally:
        torch.set_default_dtype(prev)
    cpu_model = cpu_model.to_empty(device="cpu")
    with torch.no_grad():
        for (_, pc), (_, pg) in zip(cpu_model.named_parameters(), model.named_parameters()):
            pc.copy_(pg)
        for (_, bc), (_, bg) in zip(cpu_model.named_buffers(), model.named_buffers()):
            bc.copy_(bg)
    cpu_model.eval()
    r = reference_cpu_rollout(cpu_model, prompt, max_new_tokens=new_tokens, time_budget_s=seconds,
                              max_active_branches=knobs["max_active_branches"],
                              branching_factor=knobs["branching_factor"],
                              entropy_threshold=knobs["entropy_threshold"], eos_token_id=128001,
                              block_size=knobs["block_size"])
    del cpu_model
    tps = r["decode_tokens"] / r["decode_s"] if r["decode_s"] > 0 else 0.0
    return {"value": round(tps, 3), "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"1 prompt x {r['steps']} decode steps ({r['decode_tokens']} branch tokens, "
                      f"{r['decode_s']:.1f} s; live leaves {r['trace'][:8]}...): the reference's rollout restated in "
                      f"torch on the host (gather + per-sequence SDPA per layer), bf16; the reference runs "
                      f"prompts one after another, so this rate is also its whole-job rate"}


def run_e2e(args, dev) -> dict:
    import numpy as np
    import torch
    from transformers import LlamaConfig, LlamaForCausalLM

    from mentat_amd.core.batch_generator import MentatBatchGenerator

    print("bench: building random-init Llama-3-8B (bf16)", file=sys.stderr, flush=True)
    cfg = LlamaConfig(hidden_size=4096, num_hidden_layers=32, num_attention_heads=32, num_key_value_heads=8,
                      head_dim=128, intermediate_size=14336, vocab_size=128256, max_position_embeddings=8192,
                      rms_norm_eps=1e-5, initializer_range=0.02, tie_word_embeddings=False)
    cfg.rope_parameters = {"rope_theta": 500000.0, "rope_type": "default"}
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            model = LlamaForCausalLM(cfg)
    finally:
        torch.set_default_dtype(prev)
    model.eval()
    n_prompts, prompt_len, new_tokens = 16, 256, args.e2e_new_tokens
    prompts = [np.random.default_rng(s).integers(0, cfg.vocab_size, prompt_len).tolist() for s in range(n_prompts)]
    knobs = dict(gate="absolute", entropy_threshold=2.5, max_active_branches=8, branching_factor=3,
                 block_size=16, max_blocks=196608)
    with torch.no_grad():
        print("bench: warmup rollout", file=sys.stderr, flush=True)
        warm = MentatBatchGenerator(model, _IdTokenizer(128001), max_new_tokens=8, **knobs)
        warm.generate_batch(prompts[:4])
        del warm
        torch.cuda.empty_cache()
        print("bench: timed rollout", file=sys.stderr, flush=True)
        gen = MentatBatchGenerator(model, _IdTokenizer(128001), max_new_tokens=new_tokens, **knobs)
        results = gen.generate_batch(prompts)
    d = gen.get_batch_diagnostics()
    steps = d["decode_steps"]
    ms = d["decode_time_s"] * 1e3 / max(steps, 1)
    wbytes = sum(p.numel() * p.element_size() for p in model.parameters())
    config = {
        "workload": "end-to-end MENTAT rollout, random-init Llama-3-8B bf16",
        "prompts": n_prompts, "prompt_tokens": prompt_len, "new_tokens": new_tokens,
        "gate": "absolute 2.5 nats", "max_branches_per_prompt": 8, "branching_factor": 3,
        "batching": "all prompts' live leaves in one decode batch per step (continuous batching)",
        "decode_steps": steps, "decode_tokens": d["decode_tokens_total"], "max_live_leaves": d["max_live_leaves"],
        "results": sum(len(r) for r in results), "kv_blocks_peak": d["kv_blocks_peak"],
        "weight_bytes": wbytes,
    }
    graphs = gen.wrapper.graphs
    if graphs is not None:
        config["attention"] = ("prefix-tree decode from layer %d (plans sharing pages: %d steps, without: %d)"
                               % (graphs._tree_from(), graphs.tree_steps, graphs.tree_fallbacks)
                               if graphs.tree else "paged decode")
    cpu = None
    if not args.no_cpu_baseline:
        cpu = _cpu_baseline_e2e(model, prompts[0], new_tokens, knobs, args.cpu_seconds)
    line = _line(args, 0.0, ms, config, cpu, None)
    line.update({"metric": METRIC, "value": round(d["decode_throughput_tps"], 1), "unit": "tokens/s",
                 "steps": steps, "warmup": 1,
                 # graph capture of the decode buckets runs before the decode timer (the reference has
                 # no such phase): its seconds, and the rate with them counted as decode time
                 "capture_s": d["capture_time_s"],
                 "tokens_per_s_incl_capture": d["decode_throughput_tps_incl_capture"]})
    # per-step HBM floor: the weights once per step
    line["roofline"] = {"bound": "hbm", "achieved": round(wbytes / (ms * 1e-3) / 1e9, 1), "peak": PEAK_HBM_GBS,
                        "unit": "GB/s", "frac": round(wbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                        "traffic": None, "note": "achieved = weight bytes per decode step / step time"}
    line["data"] = "synthetic (random-init weights, seed 0; prompts of uniform random ids, seeds 0-15)"
    return line


def _summary(line: dict) -> dict:
    """The fields of a workload's line that its nested entry keeps."""
    keep = ("value", "unit", "ms_per_step", "steps", "warmup", "dtype", "config", "roofline", "cpu_baseline")
    out = {k: line[k] for k in keep if k in line}
    for k, v in line.items():
        if k not in out and k not in ("metric", "n_gpus", "higher_is_better", "scaling", "vs_baseline", "data"):
            out[k] = v
    return out


def run_all(args, dev) -> dict:
    """The headline (paged decode at Llama-3-8B shapes) with the other measured
    workloads nested under "workloads": prefix-tree decode, the fused entropy
    gate + sampling step, prefill attention and the end-to-end rollout
    (branch-decode tokens/s).
    A workload that fails is reported with its error instead of its numbers."""
    import torch

    line = run_decode(args, dev)
    nested = {}
    for name, fn in (("tree", run_tree), ("rows", run_rows), ("prefill", run_prefill), ("e2e", run_e2e)):
        torch.cuda.empty_cache()
        t0 = time.perf_counter()
        try:
            nested[name] = _summary(fn(args, dev))
        except Exception as exc:  # reported, not hidden: the headline still prints
            nested[name] = {"error": f"{type(exc).__name__}: {exc}"}
            print(f"bench: workload {name} failed: {exc!r}", file=sys.stderr, flush=True)
        nested[name]["wall_s"] = round(time.perf_counter() - t0, 1)
        torch.cuda.synchronize()
    line["workloads"] = nested
    return line


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", choices=("all", "decode", "tree", "rows", "e2e", "prefill"), default="all",
                    help="all (default): the paged-decode headline plus tree, rows, prefill and e2e nested "
                         "in one line")
    ap.add_argument("--e2e-new-tokens", type=int, default=512)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="minimum host time spent on the CPU baseline")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true",
                    help="decode workload: launch every timed call eagerly instead of replaying them as one graph")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(mentat_amd has no multi-GPU path)", file=sys.stderr)
        return 2
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py runs as a single process on one GPU", file=sys.stderr)
        return 2

    import torch

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    run = {"all": run_all, "decode": run_decode, "tree": run_tree, "rows": run_rows, "e2e": run_e2e,
           "prefill": run_prefill}[args.workload]
    print(json.dumps(run(args, dev)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
