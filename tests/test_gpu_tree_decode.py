"""Prefix-tree decode (mentat_tree_decode) on the GPU.

Parity: every query's output matches the float64 oracle of the reference's
per-sequence decode (build_packed_kv + SDPA, core/paged_kv_cache.py:289-368,
adapters/attention_backend.py:99-168) within 2e-2 abs + 1e-2 rel, and the
paged decode kernel on the same batch within the same bound. Trees are grown
through PagedKVCacheManager (forks, copy-on-write of shared tails), so the
shared pages are the manager's own.
"""
import numpy as np
import pytest
import torch

from mentat_amd import ops
from mentat_amd._lib import LAYOUT_NATIVE
from mentat_amd.tree_plan import SHARED_MAX_TILES, build_plan
from mentat_amd.workloads import logical_views, prefix_tree_batch
from oracle.attention import paged_decode_f64

pytestmark = pytest.mark.gpu
ATOL, RTOL = 2e-2, 1e-2


def _oracle(tb, idx=None):
    """float64 oracle over a compact copy of the pages the chosen queries use."""
    idx = list(range(len(tb.seq_ids))) if idx is None else idx
    used = sorted({b for i in idx for b in tb.tables[i]})
    remap = {b: j for j, b in enumerate(used)}
    kp, vp = logical_views(tb.k_store, tb.v_store, LAYOUT_NATIVE)
    sel = torch.tensor(used, dtype=torch.long, device=tb.k_store.device)
    kc = kp.index_select(0, sel).float().cpu().numpy()
    vc = vp.index_select(0, sel).float().cpu().numpy()
    tabs = [[remap[b] for b in tb.tables[i]] for i in idx]
    q = tb.q[idx].float().cpu().numpy()
    return paged_decode_f64(q, kc, vc, tabs, [tb.lens[i] for i in idx], tb.block_size, tb.scale)


def _run_tree(tb, chunk_tiles=16, min_groups=3, defaults=False):
    G = tb.q.shape[1] // tb.k_store.shape[1]
    if defaults:  # the plan the bench and the generator use
        plan = build_plan(tb.tables, tb.lens, tb.rows, block_size=tb.block_size, Hkv=tb.k_store.shape[1], G=G)
    else:
        plan = build_plan(tb.tables, tb.lens, tb.rows, block_size=tb.block_size, Hkv=tb.k_store.shape[1], G=G,
                          chunk_tiles=chunk_tiles, shared_chunk_tiles=min(SHARED_MAX_TILES, 2 * chunk_tiles),
                          shared_min_groups=min_groups)
    out = ops.tree_decode(tb.q, tb.k_store, tb.v_store, block_tables=tb.block_tables, plan=plan, scale=tb.scale)
    torch.cuda.synchronize()
    return out, plan


def _close(got, want, what):
    got = np.asarray(got, dtype=np.float64)
    err = np.abs(got - want) - (ATOL + RTOL * np.abs(want))
    assert np.isfinite(got).all(), what
    assert err.max() <= 0, (what, float(np.abs(got - want).max()))


@pytest.mark.parametrize("min_groups,defaults", [(3, False), (1, False), (99, False), (3, True)])
def test_tree_decode_qwen3_8b_trees(gpu, min_groups, defaults):
    """4 trees x 32 leaves over 2048-token prompts, Qwen3-8B attention shapes; shared
    tasks of up to 32 tiles for chunks of >= min_groups member groups (1: all, 99: none),
    and the default plan."""
    print(f"case tree qwen3-8b full min_groups={min_groups} defaults={defaults}", flush=True)
    tb = prefix_tree_batch(device="cuda", seed=0)
    out, plan = _run_tree(tb, min_groups=min_groups, defaults=defaults)
    assert plan.unique_tokens() < 0.1 * tb.logical_tokens()
    rows_t = torch.tensor(tb.rows, dtype=torch.int32, device="cuda")
    ref = ops.paged_decode(tb.q, tb.k_store, tb.v_store, max_seqlen=max(tb.lens), block_tables=tb.block_tables,
                           seq_lens=tb.seq_lens, seq_rows=rows_t, scale=tb.scale, layout=LAYOUT_NATIVE)
    torch.cuda.synchronize()
    idx = list(range(0, len(tb.seq_ids), 4))
    want = _oracle(tb, idx)
    _close(out[idx].float().cpu().numpy(), want, "tree vs oracle")
    _close(out.float().cpu().numpy(), ref.float().cpu().numpy(), "tree vs paged kernel")


@pytest.mark.parametrize("Hq,Hkv,D,B,dtype,chunk", [
    (8, 8, 64, 16, torch.bfloat16, 1),
    (16, 8, 128, 16, torch.float16, 3),
    (32, 8, 128, 32, torch.bfloat16, 2),
    (64, 8, 64, 64, torch.bfloat16, 5),
    (16, 1, 128, 16, torch.bfloat16, 4),
    (32, 2, 64, 16, torch.float16, 64),
])
def test_tree_decode_shapes(gpu, Hq, Hkv, D, B, dtype, chunk):
    tb = prefix_tree_batch(n_trees=2, prefix=150, leaves=9, max_private=70, Hq=Hq, Hkv=Hkv, D=D, block_size=B,
                           max_blocks=512, dtype=dtype, device="cuda", seed=Hq + D + B)
    want = _oracle(tb)
    for min_groups in (1, 2, 99):
        print(f"case tree Hq={Hq} Hkv={Hkv} D={D} B={B} {dtype} chunk={chunk} min_groups={min_groups}", flush=True)
        out, _ = _run_tree(tb, chunk_tiles=chunk, min_groups=min_groups)
        _close(out.float().cpu().numpy(), want, ("tree vs oracle", min_groups))


def test_tree_decode_no_sharing_and_tiny(gpu):
    """Leaves that share nothing but a partial first page, and a 1-token prompt."""
    print("case tree tiny", flush=True)
    for prefix, leaves, priv in ((1, 3, 5), (7, 4, 0), (16, 2, 1)):
        tb = prefix_tree_batch(n_trees=3, prefix=prefix, leaves=leaves, max_private=priv, Hq=8, Hkv=2, D=64,
                               max_blocks=256, device="cuda", seed=prefix)
        want = _oracle(tb)
        for min_groups in (1, 99):
            out, _ = _run_tree(tb, chunk_tiles=1, min_groups=min_groups)
            _close(out.float().cpu().numpy(), want, ("tiny", prefix, leaves, priv, min_groups))


def test_tree_decode_rejects_bad_plans(gpu):
    tb = prefix_tree_batch(n_trees=1, prefix=40, leaves=3, max_private=8, Hq=8, Hkv=2, D=64, max_blocks=128,
                           device="cuda", seed=1)
    plan = build_plan(tb.tables, tb.lens, tb.rows, block_size=16, Hkv=2, G=4)
    plan.members[0] = len(tb.seq_ids)  # member index past the batch
    with pytest.raises(ValueError):
        ops.tree_decode(tb.q, tb.k_store, tb.v_store, block_tables=tb.block_tables, plan=plan)


def test_tree_decode_counted_equals_tree_decode_and_replays_new_plans(gpu):
    """mentat_tree_decode_counted (item counts in device memory, fixed grid of
    workgroups striding over the items) gives tree_decode's output bit for bit
    for the prefix-tree workload and a rollout-shaped batch (16 trees x 9
    leaves under 256-token prompts) written one after the other into the same
    fixed-capacity buffers; captured once in a graph, each replay after a new
    plan is written (and uploaded outside the graph) gives that plan's eager
    result, several times with eager work between the replays."""
    print("case tree decode counted: cfg-3 trees and rollout-shaped trees, eager and captured", flush=True)
    big = prefix_tree_batch(device="cuda", seed=0, max_blocks=8192)
    small = prefix_tree_batch(n_trees=16, prefix=256, leaves=9, max_private=300, device="cuda", seed=4,
                              max_blocks=8192)
    Hkv, G = 8, 4
    Nq = max(len(big.seq_ids), len(small.seq_ids))
    plans, wants = [], []
    for tb in (big, small):
        plan = build_plan(tb.tables, tb.lens, tb.rows, block_size=16, Hkv=Hkv, G=G)
        plan.validate(len(tb.seq_ids), Hkv, G, tb.block_tables.shape[0], tb.block_tables.shape[1], 16)
        plans.append(plan)
        wants.append(ops.tree_decode(tb.q, tb.k_store, tb.v_store, block_tables=tb.block_tables, plan=plan,
                                     scale=tb.scale))
    bufs = ops.TreePlanBuffers(torch.device("cuda"), Nq, Hkv, max_shared=max(p.n_shared for p in plans) + 5,
                               max_solo=max(p.n_solo for p in plans) + 100,
                               max_slots=max(p.n_slots for p in plans) + 64)
    q = torch.zeros(Nq, 32, 128, dtype=torch.bfloat16, device="cuda")
    out = torch.zeros_like(q)

    def load(i):
        tb = (big, small)[i]
        q.zero_()
        q[:len(tb.seq_ids)] = tb.q
        bufs.write(plans[i], len(tb.seq_ids))
        bufs.upload()
        return tb

    # the two batches live in different managers: one call per manager's stores
    for i in (0, 1, 0):
        tb = load(i)
        ops.tree_decode_counted(q, tb.k_store, tb.v_store, block_tables=tb.block_tables, bufs=bufs, scale=tb.scale,
                                out=out)
        torch.cuda.synchronize()
        n = len(tb.seq_ids)
        assert torch.equal(out[:n], wants[i]), i
        assert torch.equal(out[n:], torch.zeros_like(out[n:]))
    # captured: the small batch's stores, plans of that batch with the tables trimmed to fewer queries
    tb = load(1)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ops.tree_decode_counted(q, tb.k_store, tb.v_store, block_tables=tb.block_tables, bufs=bufs, scale=tb.scale,
                                out=out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        ops.tree_decode_counted(q, tb.k_store, tb.v_store, block_tables=tb.block_tables, bufs=bufs, scale=tb.scale,
                                out=out)
    torch.cuda.synchronize()
    for n_keep in (len(tb.seq_ids), 60, 17, len(tb.seq_ids)):
        plan = build_plan([tb.tables[i] for i in range(n_keep)], tb.lens[:n_keep], tb.rows[:n_keep], block_size=16,
                          Hkv=Hkv, G=G)
        plan.validate(n_keep, Hkv, G, tb.block_tables.shape[0], tb.block_tables.shape[1], 16)
        want = ops.tree_decode(tb.q[:n_keep].contiguous(), tb.k_store, tb.v_store, block_tables=tb.block_tables,
                               plan=plan, scale=tb.scale)
        torch.cuda.synchronize()
        q.zero_()
        q[:n_keep] = tb.q[:n_keep]
        bufs.write(plan, n_keep)
        bufs.upload()
        out.fill_(7.0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out[:n_keep], want), n_keep
        assert torch.equal(out[n_keep:Nq], torch.zeros_like(out[n_keep:Nq])), n_keep
