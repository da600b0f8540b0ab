"""Cross-prompt continuous batching (MentatBatchGenerator) on the GPU.

Each prompt's rollout inside the batch must be the rollout MentatGenerator
builds for that prompt alone: the same tokens for every result, the same
branch decisions (step, child count) and active-leaf traces, log-probs within
1e-4 (fp32 tiny Llama of the cfg-1 plumbing run, so batched and single GEMMs
differ only in rounding far below the decisions' margins). Two tree slots for
three prompts, so the third prompt is admitted while the others decode.
"""
import os
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
sys.path.insert(0, GOLDEN)

KNOBS = dict(max_active_branches=6, branching_factor=3, max_new_tokens=24, block_size=16, max_blocks=4096)


def _prompts():
    return [np.random.default_rng(s).integers(0, 32000, 40 + 7 * s).tolist() for s in range(3)]


@pytest.mark.parametrize("gate,thr,sim", [("relative", 2.0, None), ("absolute", 2.0, None),
                                          ("absolute", 1.5, 0.2), ("absolute", 1.5, 0.5)])
def test_batched_rollouts_match_single_prompt_rollouts(gpu, gate, thr, sim):
    """sim: a semantic-similarity threshold low enough that leaves are pruned
    (the batch queues its similarity mask before the step's decisions; the
    single-prompt generator computes it after them)."""
    import make_cfg1_trajectory as mk
    from mentat_amd.core.batch_generator import MentatBatchGenerator
    from mentat_amd.core.generator import MentatGenerator

    print(f"case batch generator gate={gate} thr={thr} sim={sim}", flush=True)
    model = mk.build_model().to("cuda")
    prompts = _prompts()
    knobs = dict(KNOBS)
    if sim is not None:
        knobs["semantic_similarity_threshold"] = sim
    singles = []
    with torch.no_grad():
        for ids in prompts:
            g = MentatGenerator(model, mk.StubTokenizer(ids), gate=gate, entropy_threshold=thr, **knobs)
            res = g.generate("stub")
            singles.append((res, g.get_diagnostics()))
            assert g.kv_cache_mgr.allocator.num_used == 0
        bg = MentatBatchGenerator(model, mk.StubTokenizer(prompts[0]), gate=gate, entropy_threshold=thr, **knobs)
        batched = bg.generate_batch(prompts, max_trees=2)
    diag = bg.get_batch_diagnostics()
    assert bg.kv_cache_mgr.allocator.num_used == 0
    for p, ((res, d), got) in enumerate(zip(singles, batched)):
        want_ids = [r["token_ids"] for r in res]
        assert [r["token_ids"] for r in got] == want_ids, p
        for a, b in zip(got, res):
            assert abs(a["log_prob"] - b["log_prob"]) < 1e-4
        pd = diag["prompts"][p]
        assert [tuple(x[::2]) for x in pd["branch_points"]] == [tuple(x[::2]) for x in d["branch_points"]], p
        assert pd["active_branch_trace"] == d["active_branch_trace"], p
        assert pd["diversity_pruning_events"] == d["diversity_pruning_events"], p
        assert len(pd["entropy_trace"]) == len(d["entropy_trace"])
        for (s1, n1, h1), (s2, n2, h2) in zip(pd["entropy_trace"], d["entropy_trace"]):
            assert (s1, n1) == (s2, n2) and abs(h1 - h2) < 1e-4
    # the batch really overlapped prompts: some step carried leaves of two trees
    single_max = max(max(d["active_branch_trace"] or [1]) for _, d in singles)
    assert max(bg.batch_trace) > single_max
    assert diag["decode_tokens_total"] == sum(sum(d["active_branch_trace"]) for _, d in singles)
    if sim is not None:  # the case really pruned
        assert sum(len(diag["prompts"][p]["diversity_pruning_events"]) for p in diag["prompts"]) > 0


def test_cpu_rollout_restatement_follows_the_generator(gpu):
    """The CPU baseline's restatement (oracle.rollout_cpu) against the product
    generator on the fp32 plumbing model, absolute gate: the same live-leaf trace
    and the same sequences."""
    import make_cfg1_trajectory as mk
    from mentat_amd.core.generator import MentatGenerator
    from oracle.rollout_cpu import reference_cpu_rollout

    print("case cpu rollout restatement vs generator", flush=True)
    model = mk.build_model()
    ids = _prompts()[1]
    knobs = dict(max_active_branches=6, branching_factor=3, entropy_threshold=2.0)
    r = reference_cpu_rollout(model, ids, max_new_tokens=20, time_budget_s=1e9, block_size=16, max_blocks=4096,
                              **knobs)
    with torch.no_grad():
        g = MentatGenerator(model.to("cuda"), mk.StubTokenizer(ids), gate="absolute", max_new_tokens=20,
                            block_size=16, max_blocks=4096, **knobs)
        g.generate("stub")
    assert r["trace"] == g.get_diagnostics()["active_branch_trace"]
    assert r["decode_tokens"] == sum(r["trace"])
