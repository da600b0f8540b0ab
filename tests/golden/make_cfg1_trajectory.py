"""Write the golden trajectory of the reference generator on the tiny-Llama
plumbing workload (tests/golden/cfg1_trajectory.json).

Runs the reference's own core/generator.py (imported from /root/reference, in
this container only) on CPU:
  model    LlamaConfig(hidden 256, 2 layers, 4 q / 2 kv heads, head_dim 64,
           vocab 32000, intermediate 1024, rope_theta 10000), fp32, weights from
           HF's initialiser with initializer_range 0.02 after torch.manual_seed(0)
  prompt   128 ids from numpy default_rng(0).integers(0, 32000), stub tokenizer, EOS id 2
  knobs    max_active_branches 8, branching_factor 3, max_new_tokens 64,
           block_size 16, max_blocks 8192, the reference's defaults otherwise
           (relative entropy gate — the reference has no absolute gate)
Recorded per decode step: every live leaf (DFS order) with its generated ids,
cumulative log-prob and sequence id; every live sequence's per-layer page
table; all non-zero refcounts. Per decision: the entropy, tau and the gap
between the top-2 penalised log-probs (to bound how close a decision was).

    python tests/golden/make_cfg1_trajectory.py
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

REF = "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cfg1_trajectory.json")

CONFIG = dict(hidden_size=256, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2, head_dim=64,
              vocab_size=32000, intermediate_size=1024, max_position_embeddings=4096, initializer_range=0.02,
              tie_word_embeddings=False)
KNOBS = dict(max_active_branches=8, branching_factor=3, max_new_tokens=64, block_size=16, max_blocks=8192)
PROMPT_LEN = 128
EOS = 2


class StubTokenizer:
    eos_token_id = EOS

    def __init__(self, ids):
        self.ids = ids

    def __call__(self, prompt, return_tensors="pt"):
        return {"input_ids": torch.tensor([self.ids], dtype=torch.long)}

    def decode(self, ids, skip_special_tokens=True):
        return " ".join(str(i) for i in ids)


def build_model():
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(0)
    cfg = LlamaConfig(**CONFIG)
    cfg.rope_parameters = {"rope_theta": 10000.0, "rope_type": "default"}
    model = LlamaForCausalLM(cfg).float().eval()
    return model


def prompt_ids():
    return np.random.default_rng(0).integers(0, 32000, PROMPT_LEN).tolist()


def main():
    sys.path.insert(0, REF)
    from core.generator import MentatGenerator  # the reference, read-only
    import core.generator_utils as gu

    model = build_model()
    ids = prompt_ids()
    tok = StubTokenizer(ids)

    decisions = []
    steps = []

    class Recording(MentatGenerator):
        def _step_leaf(self, tree, leaf, logits, step, num_active):
            H = gu.compute_entropy(logits, self.temperature)
            ema = H if leaf.entropy_ema is None else (
                self.entropy_ema_alpha * H + (1.0 - self.entropy_ema_alpha) * leaf.entropy_ema)
            tau = ema * gu.adaptive_threshold(self.relative_entropy_multiplier, self.M, num_active) * \
                self._soft_explore_factor(step)
            pen = gu.apply_repetition_penalty(logits, leaf.get_full_sequence(), penalty=self.rep_penalty)
            lp = torch.log_softmax(pen, dim=-1)
            top = torch.topk(lp, 4).values.tolist()
            decisions.append({"step": step, "node": leaf.node_id, "entropy": H, "tau": tau,
                              "top_gap": top[0] - top[1], "kth_gap": top[self.K - 1] - top[self.K]})
            return super()._step_leaf(tree, leaf, logits, step, num_active)

        def _prune_similar(self, tree, step):
            super()._prune_similar(tree, step)
            kv = self.kv_cache_mgr
            steps.append({
                "step": step,
                "leaves": [{"node": l.node_id, "seq": l.seq_id, "tokens": list(l.get_full_sequence()),
                            "lp": l.cumulative_log_prob} for l in tree.get_active_leaves()],
                "tables": {str(s): [list(t) for t in st.page_table] for s, st in kv._sequences.items()},
                "num_tokens": {str(s): list(st.num_tokens) for s, st in kv._sequences.items()},
                "refcounts": {str(b): r for b, r in enumerate(kv.allocator.refcounts) if r},
            })

    gen = Recording(model, tok, **KNOBS)
    with torch.no_grad():
        results = gen.generate("stub")
    diag = gen.get_diagnostics()
    out = {
        "config": CONFIG, "knobs": KNOBS, "eos": EOS, "prompt_ids": ids,
        "results": [{"token_ids": r["token_ids"], "log_prob": r["log_prob"], "norm_prob": r["norm_prob"]}
                    for r in results],
        "branch_points": diag["branch_points"],
        "active_branch_trace": diag["active_branch_trace"],
        "diversity_pruning_events": diag["diversity_pruning_events"],
        "entropy_trace": diag["entropy_trace"],
        "kv_blocks_peak": diag["kv_blocks_peak"],
        "decisions": decisions,
        "steps": steps,
        "versions": {"torch": torch.__version__, "python": sys.version.split()[0]},
    }
    with open(OUT, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print(f"wrote {OUT}: {len(steps)} steps, {len(diag['branch_points'])} branch points, "
          f"{len(results)} results, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
