"""Captured decode steps (core/graph_decode.py) against the eager step.

Two managers receive the same prompts, forks, frees and decode steps; one
wrapper runs the eager forward, the other replays captured graphs (batches
padded to buckets, all layers' append plans from plan_append_step). Every
step checks, on the GPU:
  * logits and final hidden of the N real rows against the eager step
    (bf16 model: rows padded into a larger GEMM may take another GEMM
    kernel, so values agree to bf16 rounding, not bit for bit);
  * the device block tables and lengths of every layer: bit-exact (the host
    plans are the same integers);
  * the length-0 padding row stays 0 in every layer.
Replays alternate with eager work (forks, frees, other buckets) and every
replay is checked. A rollout test then compares whole generator runs with
and without capture.
"""
import os
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
sys.path.insert(0, GOLDEN)


def _bf16_model():
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(hidden_size=512, num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=2,
                      head_dim=128, intermediate_size=1024, vocab_size=4096, max_position_embeddings=4096,
                      initializer_range=0.05, tie_word_embeddings=False)
    cfg.rope_parameters = {"rope_theta": 10000.0, "rope_type": "default"}
    torch.manual_seed(3)
    return LlamaForCausalLM(cfg).to(torch.bfloat16).to("cuda").eval()


def _wrapper(model, capture):
    from mentat_amd.adapters.adapter_factory import get_adapter
    from mentat_amd.core.generator_utils import PagedModelWrapper
    from mentat_amd.core.paged_kv_cache import PagedKVCacheManager

    a = get_adapter(model)
    m = PagedKVCacheManager(a.num_hidden_layers, a.num_key_value_heads, a.head_dim, max_blocks=2048, block_size=16,
                            device="cuda", dtype=torch.bfloat16)
    w = PagedModelWrapper(model, m, a)
    if capture:
        w.enable_step_capture()
    return w


@pytest.mark.parametrize("split", [1, 2])
def test_captured_steps_match_eager_steps(gpu, monkeypatch, split):
    """split: layers of the first of the step's two graphs (2 = the whole
    2-layer model, one graph; 1 = two graphs, the second layer's append plans
    made while the first graph runs)."""
    from mentat_amd.core import graph_decode

    monkeypatch.setattr(graph_decode, "SPLIT_LAYERS", split)
    print(f"case graph decode vs eager, bf16 2-layer llama, split={split}", flush=True)
    model = _bf16_model()
    we, wg = _wrapper(model, False), _wrapper(model, True)
    rng = np.random.default_rng(0)
    live = []
    with torch.no_grad():
        for p in range(3):
            ids = torch.tensor([rng.integers(0, 4096, 20 + 13 * p).tolist()], device="cuda")
            se, sg = we.kv_cache_mgr.allocate_sequence(), wg.kv_cache_mgr.allocate_sequence()
            assert se == sg
            we.prefill(ids, se)
            wg.prefill(ids, sg)
            live.append(se)
        last = {s: 1 for s in live}
        sizes = []
        for step in range(24):
            # forks (shared tails: copy-on-write inside the captured append) and frees
            if step % 5 == 1:
                for parent in list(live)[: 2 + step // 5]:
                    for _ in range(3):
                        c = we.kv_cache_mgr.fork_sequence(parent)
                        assert wg.kv_cache_mgr.fork_sequence(parent) == c
                        live.append(c)
                        last[c] = last[parent]
                    live.remove(parent)
                    we.kv_cache_mgr.free_sequence(parent)
                    wg.kv_cache_mgr.free_sequence(parent)
            if step % 7 == 6 and len(live) > 4:
                s = live.pop(3)
                we.kv_cache_mgr.free_sequence(s)
                wg.kv_cache_mgr.free_sequence(s)
            toks = [last[s] for s in live]
            le, he = we.decode_batch_tensor(toks, live)
            lg, hg = wg.decode_batch_tensor(toks, live)
            sizes.append(len(live))
            assert lg.shape == le.shape and hg.shape == he.shape
            scale = float(le.float().abs().max())
            err = float((lg.float() - le.float()).abs().max())
            assert err <= 2e-2 * scale + 2e-2, (step, len(live), err, scale)
            assert float((hg.float() - he.float()).abs().max()) <= 5e-2 * float(he.float().abs().max()) + 2e-2
            me, mg = we.kv_cache_mgr, wg.kv_cache_mgr
            rows_e = [me._sequences[s].row for s in live]
            rows_g = [mg._sequences[s].row for s in live]
            for layer in range(me.num_layers):
                npg = max(len(me._sequences[s].page_table[layer]) for s in live)
                te = me._tables[layer][rows_e, :npg].cpu()
                tg = mg._tables[layer][rows_g, :npg].cpu()
                assert torch.equal(te, tg), (step, layer)
                assert torch.equal(me._lens[layer][rows_e].cpu(), mg._lens[layer][rows_g].cpu())
            assert int(mg._lens[:, mg.empty_row()].abs().sum()) == 0
            for s in live:
                assert me._sequences[s].page_table == mg._sequences[s].page_table
            last = {s: int(t) for s, t in zip(live, le.float().argmax(-1).tolist())}
    g = wg.graphs
    used = {g.bucket(n) for n in sizes}
    assert len(used) >= 3, sizes                     # several buckets were replayed in turn
    assert g.captures == len(used), (g.captures, used)  # each captured once, then replayed
    assert all((b.graph2 is not None) == (split < 2) for b in g._graphs.values())
    # the captured layers after the first graph (all of them with one graph) ran
    # the prefix-tree decode on plans that shared the forked pages
    assert g.tree and g.tree_steps == len(sizes) and g.tree_fallbacks == 0


@pytest.mark.parametrize("split", [1, 2])
def test_steps_queued_without_sync_match_eager(gpu, monkeypatch, split):
    """Captured steps queued back to back with no host synchronisation, behind
    a GPU kept busy, so each step's host-to-device copies of its plans are still
    pending when the host plans the next step: every step's logits and the
    final tables must equal the eager run's (the staging buffer is reused only
    after the previous step's copies have read it)."""
    from mentat_amd.core import graph_decode

    monkeypatch.setattr(graph_decode, "SPLIT_LAYERS", split)
    print(f"case captured steps queued without sync, split={split}", flush=True)
    model = _bf16_model()
    we, wg = _wrapper(model, False), _wrapper(model, True)
    rng = np.random.default_rng(5)
    steps = 8
    with torch.no_grad():
        live = []
        for p in range(4):
            ids = torch.tensor([rng.integers(0, 4096, 9 + 6 * p).tolist()], device="cuda")
            se, sg = we.kv_cache_mgr.allocate_sequence(), wg.kv_cache_mgr.allocate_sequence()
            we.prefill(ids, se)
            wg.prefill(ids, sg)
            live.append(se)
        toks = rng.integers(0, 4096, (steps, len(live))).tolist()
        wg.decode_batch_tensor(toks[0], live)          # capture the bucket first
        ref = [we.decode_batch_tensor(toks[0], live)[0]]
        ref += [we.decode_batch_tensor(toks[t], live)[0] for t in range(1, steps)]
        torch.cuda.synchronize()
        a = torch.randn(4096, 4096, device="cuda")
        for _ in range(40):                            # ~tens of ms of queued GPU work
            a = torch.tanh(a @ a)
        got = [wg.decode_batch_tensor(toks[t], live)[0] for t in range(1, steps)]
        torch.cuda.synchronize()
    for t, (lg, le) in enumerate(zip(got, ref[1:]), start=1):
        scale = float(le.float().abs().max())
        err = float((lg.float() - le.float()).abs().max())
        assert err <= 2e-2 * scale + 2e-2, (t, err, scale)
    me, mg = we.kv_cache_mgr, wg.kv_cache_mgr
    for layer in range(me.num_layers):
        for s in live:
            re_, rg = me._sequences[s].row, mg._sequences[s].row
            n = len(me._sequences[s].page_table[layer])
            assert torch.equal(me._tables[layer][re_, :n].cpu(), mg._tables[layer][rg, :n].cpu())
            assert int(me._lens[layer][re_]) == int(mg._lens[layer][rg])


@pytest.mark.parametrize("gate,thr", [("absolute", 2.0)])
@pytest.mark.parametrize("split", [1, 2])
def test_rollouts_with_and_without_capture(gpu, monkeypatch, gate, thr, split):
    import make_cfg1_trajectory as mk
    from mentat_amd.core import graph_decode
    from mentat_amd.core.batch_generator import MentatBatchGenerator

    monkeypatch.setattr(graph_decode, "SPLIT_LAYERS", split)
    print(f"case rollout capture on/off gate={gate} split={split}", flush=True)
    model = mk.build_model().to("cuda")
    prompts = [np.random.default_rng(s).integers(0, 32000, 40 + 7 * s).tolist() for s in range(3)]
    knobs = dict(max_active_branches=6, branching_factor=3, max_new_tokens=24, block_size=16, max_blocks=4096,
                 gate=gate, entropy_threshold=thr)
    out = {}
    with torch.no_grad():
        for cap in (False, True):
            bg = MentatBatchGenerator(model, mk.StubTokenizer(prompts[0]), capture_steps=cap, **knobs)
            res = bg.generate_batch(prompts, max_trees=2)
            out[cap] = (res, bg.get_batch_diagnostics(), bg)
            assert bg.kv_cache_mgr.allocator.num_used == 0
    (r0, d0, _), (r1, d1, b1) = out[False], out[True]
    assert b1.wrapper.graphs is not None and b1.wrapper.graphs.captures > 0
    assert out[False][2].wrapper.graphs is None
    for a, b in zip(r0, r1):
        assert [x["token_ids"] for x in a] == [x["token_ids"] for x in b]
        for x, y in zip(a, b):
            assert abs(x["log_prob"] - y["log_prob"]) < 1e-4
    assert d0["decode_tokens_total"] == d1["decode_tokens_total"]
    for p in d0["prompts"]:
        assert d0["prompts"][p]["active_branch_trace"] == d1["prompts"][p]["active_branch_trace"]
        assert [x[::2] for x in d0["prompts"][p]["branch_points"]] == \
            [x[::2] for x in d1["prompts"][p]["branch_points"]]


@pytest.mark.parametrize("split", [1, 2])
def test_no_garbage_collection_during_capture(gpu, monkeypatch, split):
    """Captures run with the garbage collector off (collected just before):
    a dropped wrapper's graphs are never torn down inside another capture.
    The forward is spied on; whenever the stream is capturing, gc must be off,
    and gc's state is restored afterwards. split 1 captures each step as two
    graphs (the layout of models deeper than SPLIT_LAYERS), split 2 as one."""
    import gc

    from mentat_amd.core import graph_decode

    print(f"case gc state during capture, split {split}", flush=True)
    monkeypatch.setattr(graph_decode, "SPLIT_LAYERS", split)
    model = _bf16_model()
    seen = []
    orig = graph_decode.DecodeGraphs._forward

    def spy(self, *args, **kwargs):
        seen.append((torch.cuda.is_current_stream_capturing(), gc.isenabled()))
        return orig(self, *args, **kwargs)

    graph_decode.DecodeGraphs._forward = spy
    try:
        with torch.no_grad():
            w0 = _wrapper(model, True)
            s = w0.kv_cache_mgr.allocate_sequence()
            w0.prefill(torch.tensor([[1, 2, 3]], device="cuda"), s)
            w0.decode_batch_tensor([4], [s])
            del w0, s  # its graphs are garbage now
            w1 = _wrapper(model, True)
            s = w1.kv_cache_mgr.allocate_sequence()
            w1.prefill(torch.tensor([[5, 6, 7, 8]], device="cuda"), s)
            for t in range(3):
                w1.decode_batch_tensor([9 + t], [s])
    finally:
        graph_decode.DecodeGraphs._forward = orig
    assert any(c for c, _ in seen) and any(not c for c, _ in seen)
    assert all(not on for capturing, on in seen if capturing)
    # two graphs per bucket capture two forwards per capture
    assert sum(c for c, _ in seen) == (2 if split == 1 else 1) * 2
    assert gc.isenabled()


def test_merged_projections_leave_the_model_alone_and_follow_its_weights(gpu):
    """The captured Llama step runs q/k/v and gate/up as merged GEMMs over its own
    copies of the modules' weights: the modules keep their tensors, and a weight
    rebound (a new tensor) or changed in place is picked up by the next step,
    whose logits follow the new weights (no recapture: the copies are refreshed
    in place). The down projection runs split over its reduction from its own
    sliced copy, refreshed the same way."""
    print("case merged projections after a weight rebind and an in-place change", flush=True)
    model = _bf16_model()
    before = [(b.self_attn.q_proj.weight.data_ptr(), b.mlp.up_proj.weight.data_ptr()) for b in model.model.layers]
    we, wg = _wrapper(model, False), _wrapper(model, True)
    assert [(b.self_attn.q_proj.weight.data_ptr(), b.mlp.up_proj.weight.data_ptr())
            for b in model.model.layers] == before
    with torch.no_grad():
        ids = torch.tensor([[3, 1, 4, 1, 5, 9, 2, 6]], device="cuda")
        se, sg = we.kv_cache_mgr.allocate_sequence(), wg.kv_cache_mgr.allocate_sequence()
        we.prefill(ids, se)
        wg.prefill(ids, sg)
        le, _ = we.decode_batch_tensor([7], [se])
        lg, _ = wg.decode_batch_tensor([7], [sg])
        assert wg.graphs.merged and len(wg.graphs._w_down) == len(model.model.layers)
        assert float((lg.float() - le.float()).abs().max()) <= 2e-2 * float(le.float().abs().max()) + 2e-2
        n0 = wg.graphs.captures
        for b in model.model.layers:  # new tensors, new values
            b.self_attn.q_proj.weight.data = (b.self_attn.q_proj.weight.data * 1.5).clone()
            b.mlp.gate_proj.weight.data = (b.mlp.gate_proj.weight.data * 0.5).clone()
            b.mlp.down_proj.weight.data = (b.mlp.down_proj.weight.data * 1.25).clone()
        le, _ = we.decode_batch_tensor([8], [se])
        lg, _ = wg.decode_batch_tensor([8], [sg])
        assert float((lg.float() - le.float()).abs().max()) <= 2e-2 * float(le.float().abs().max()) + 2e-2
        for b in model.model.layers:  # in place, the same tensors
            b.self_attn.v_proj.weight.mul_(-1.0)
            b.mlp.up_proj.weight.mul_(0.75)
            b.mlp.down_proj.weight.mul_(-0.5)
        le, _ = we.decode_batch_tensor([9], [se])
        lg, _ = wg.decode_batch_tensor([9], [sg])
        assert float((lg.float() - le.float()).abs().max()) <= 2e-2 * float(le.float().abs().max()) + 2e-2
        assert wg.graphs.captures == n0


def test_calibrated_buckets(gpu):
    """buckets="calibrate": the table comes from timings of the step's own
    projection GEMMs on this device at every multiple of 8 rows up to 256. It
    is sorted, ends at 256, and each kept row count is cheaper by more than 1%
    than every larger one. Captured steps on that table match eager steps."""
    print("case calibrated buckets, bf16 2-layer llama", flush=True)
    model = _bf16_model()
    we, wg = _wrapper(model, False), _wrapper(model, False)
    wg.enable_step_capture(buckets="calibrate")
    g = wg.graphs
    b, c = g.buckets, g.bucket_costs
    assert b == tuple(sorted(b)) and b[-1] == 256 and all(r % 8 == 0 for r in b)
    assert sorted(c) == list(range(8, 257, 8)) and all(v > 0 for v in c.values())
    for r in b:
        assert all(c[r2] > 1.01 * c[r] for r2 in c if r2 > r), r
    rng = np.random.default_rng(1)
    live = []
    with torch.no_grad():
        for p in range(2):
            ids = torch.tensor([rng.integers(0, 4096, 30 + 7 * p).tolist()], device="cuda")
            se, sg = we.kv_cache_mgr.allocate_sequence(), wg.kv_cache_mgr.allocate_sequence()
            we.prefill(ids, se)
            wg.prefill(ids, sg)
            live.append(se)
        for parent in list(live):
            c1 = we.kv_cache_mgr.fork_sequence(parent)
            assert wg.kv_cache_mgr.fork_sequence(parent) == c1
            live.append(c1)
        toks = [1] * len(live)
        for _ in range(3):
            le, _ = we.decode_batch_tensor(toks, live)
            lg, _ = wg.decode_batch_tensor(toks, live)
            scale = float(le.float().abs().max())
            assert float((lg.float() - le.float()).abs().max()) <= 2e-2 * scale + 2e-2
            toks = le.float().argmax(-1).tolist()
    assert g.captures >= 1 and g.bucket(len(live)) in b
