"""Cross-prompt continuous batching of MENTAT rollouts.

The reference rolls prompts out one after another (mentat_rollout.py:256-259;
the server serialises requests, mentat_server.py:351), so each decode step is
one prompt's handful of branches. Here up to ``max_trees`` prompt trees are
live at once over ONE paged KV cache: every decode step runs all live leaves
of all trees through one batched forward (PagedModelWrapper.decode_batch_tensor)
and one fused row-kernel call, and a finished tree's slot is refilled from the
queue (prefill + its step-0 decision) before the next step.

Each tree keeps the reference's per-prompt rules exactly (core/generator.py:
125-374): its own step counter (soft-explore warm-up, max_new_tokens), its own
num_active frozen at the start of the step (headroom M - num_active, the
relative gate's utilisation), its own EMAs, DFS batch order within the tree and
its own semantic-similarity prune. Given the same logits, a prompt's tree is
the one MentatGenerator.generate would build for it alone; only physical block
ids differ (one allocator serves every tree).

Metric (A12's definition over the whole batch): branch-decode tokens/s =
sum over decode steps of the live leaves / decode wall time (prefill and the
step-0 decisions of the first admitted prompts excluded).
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass, field

import numpy as np
import torch

from .. import ops
from .generator import MentatGenerator
from .generator_utils import PrefixTree, TreeNode

__all__ = ["MentatBatchGenerator"]


@dataclass
class _TreeRun:
    index: int                  # prompt index
    tree: PrefixTree
    step: int = 1               # next decode step of this tree
    prefill_tokens: int = 0
    entropy_trace: list = field(default_factory=list)
    branch_points: list = field(default_factory=list)
    diversity_pruning_events: list = field(default_factory=list)
    active_branch_trace: list = field(default_factory=list)
    decode_tokens: int = 0


class MentatBatchGenerator(MentatGenerator):
    """MentatGenerator over many prompts at once (same constructor)."""

    def generate_batch(self, prompts: list, max_trees: int | None = None) -> list[list[dict]]:
        """Roll out every prompt (strings through the tokenizer, or lists of ids);
        returns each prompt's results, as MentatGenerator.generate does, in prompt order."""
        dev = self.wrapper.device
        on_gpu = dev.type == "cuda"
        if on_gpu:
            torch.cuda.reset_peak_memory_stats(dev)
        max_trees = len(prompts) if max_trees is None else max(1, int(max_trees))
        queue = list(range(len(prompts)))
        live: list[_TreeRun] = []
        done: dict[int, list[dict]] = {}
        self.runs: dict[int, _TreeRun] = {}
        self.batch_trace: list[int] = []
        self._total_tokens_decoded = 0
        self._prefill_tokens = 0
        self._capture_time_s = 0.0
        prefill_s = 0.0

        def admit():
            nonlocal prefill_s
            while queue and len(live) < max_trees:
                idx = queue.pop(0)
                t0 = time.perf_counter()
                run = self._start_tree(idx, prompts[idx])
                if on_gpu:
                    torch.cuda.synchronize(dev)
                prefill_s += time.perf_counter() - t0
                self.runs[idx] = run
                live.append(run)

        admit()
        if self.wrapper.graphs is not None:
            lens = [len(self.tokenizer(p, return_tensors="pt")["input_ids"][0]) if isinstance(p, str) else len(p)
                    for p in prompts]
            self._prepare_capture(max_trees, max(lens))
        t_start = time.perf_counter()
        prefill_before = prefill_s
        while live:
            # retire finished trees, refill their slots
            active = {}
            for run in list(live):
                leaves = run.tree.get_active_leaves() if run.step < self.max_new_tokens else []
                if not leaves:
                    done[run.index] = self._finish_tree(run)
                    live.remove(run)
                else:
                    active[id(run)] = leaves
            admit()
            if not live:
                break
            batch, trees, steps, nacts, logs = [], [], [], [], []
            for run in live:
                leaves = active.get(id(run))
                if leaves is None:  # admitted above
                    leaves = run.tree.get_active_leaves()
                run.active_branch_trace.append(len(leaves))
                run.decode_tokens += len(leaves)
                batch += leaves
                trees += [run.tree] * len(leaves)
                steps += [run.step] * len(leaves)
                nacts += [len(leaves)] * len(leaves)
                logs += [run] * len(leaves)
            self.batch_trace.append(len(batch))
            logits, hidden = self.wrapper.decode_batch_tensor([l.token_ids[-1] for l in batch],
                                                              [l.seq_id for l in batch])
            self._total_tokens_decoded += len(batch)
            self._update_semantic_vectors(batch, hidden)
            launched = self._launch_decisions(batch, logits)
            ahead = self._similarity_ahead(live, batch, logs)   # queued after the decision record
            self._decide_rows(batch, logits, trees, steps, nacts, logs, launched)
            self._prune_runs(live, ahead)
            for run in live:
                if self.step_hook is not None:
                    self.step_hook(run.step, run.tree)
                run.step += 1
        if on_gpu:
            torch.cuda.synchronize(dev)
        # prefill of prompts admitted after the start is not decode time
        self._decode_time_s = time.perf_counter() - t_start - (prefill_s - prefill_before)
        self._prefill_time_s = prefill_s
        if on_gpu:
            self._peak_vram_bytes = torch.cuda.max_memory_allocated(dev)
        return [done[i] for i in range(len(prompts))]

    # ------------------------------------------------------------------
    def _similarity_ahead(self, runs: list, batch: list, logs: list):
        """The prune's similarity mask, queued before the step's decisions.

        Exact when min_steps_before_prune >= 1: after the decisions, a tree's
        eligible leaves are its eligible batch leaves that are still active
        (branched and finished leaves are inactive; new children, created this
        step, are too young), in the same depth-first order, with unchanged
        vectors and parents. So the mask over the batch's eligible leaves,
        restricted to the survivors, is the mask the prune would compute after
        the decisions. Its copy is queued after the decision record's, with an
        event the prune waits for. Returns None when the rule does not apply
        (the prune then computes its own)."""
        if self.min_steps_before_prune < 1 or self.wrapper.device.type != "cuda":
            return None
        gi_of = {id(run): gi for gi, run in enumerate(runs)}
        sv, groups = [], []
        for leaf, run in zip(batch, logs):
            if leaf.semantic_vector is not None and run.step - leaf.creation_step >= self.min_steps_before_prune:
                sv.append(leaf)
                groups.append(gi_of[id(run)])
        if len(sv) <= 1:
            return sv, groups, None, None
        mask = ops.semantic_similar_mask([l.semantic_vector for l in sv], self._similar_keys(sv), groups,
                                         self.semantic_similarity_threshold, wait=False)
        ev = torch.cuda.Event()
        ev.record()
        return sv, groups, mask, ev

    def _prune_runs(self, runs: list, ahead=None) -> None:
        """Every tree's semantic-similarity prune (the rule of _prune_similar, per
        tree) from one similarity matrix over all trees' eligible leaves: pairs
        are kept only within a tree, so each tree sees exactly its own pairs, in
        its own row-major order."""
        if ahead is not None:
            self._prune_runs_ahead(runs, *ahead)
            return
        all_sv, groups, per = [], [], []
        for gi, run in enumerate(runs):
            leaves = run.tree.get_active_leaves()
            sv = []
            if len(leaves) > 1:
                sv = [l for l in leaves if l.semantic_vector is not None
                      and run.step - l.creation_step >= self.min_steps_before_prune]
            if len(sv) <= 1:
                sv = []
            per.append((run, len(all_sv), sv))
            all_sv += sv
            groups += [gi] * len(sv)
        if len(all_sv) <= 1:
            return
        by_group: dict = {}
        for i, j in self._similar_pairs(all_sv, groups):
            by_group.setdefault(groups[i], []).append((i, j))
        for gi, (run, base, sv) in enumerate(per):
            pairs = by_group.get(gi)
            if pairs:
                self._apply_prune(run.tree, sv, [(i - base, j - base) for i, j in pairs], run.step, run)

    def _prune_runs_ahead(self, runs: list, sv: list, groups: list, mask, ev) -> None:
        """_prune_runs from the mask of _similarity_ahead (see there)."""
        # Survivors are active leaves of their tree, so two or more of them also
        # satisfy the rule's "more than one active leaf".
        local = [-1] * len(sv)          # index among the tree's surviving eligible leaves
        members: list = [[] for _ in runs]
        for i, leaf in enumerate(sv):
            if leaf.is_active:
                members[groups[i]].append(i)
        per = [[] for _ in runs]
        for g, idx in enumerate(members):
            if len(idx) <= 1:
                continue
            for k, i in enumerate(idx):
                local[i] = k
            per[g] = [sv[i] for i in idx]
        if mask is None or not any(per):
            return
        ev.synchronize()
        ii, jj = np.nonzero(mask.numpy())
        by_group: dict = {}
        for i, j in zip(ii.tolist(), jj.tolist()):
            if local[i] >= 0 and local[j] >= 0:
                by_group.setdefault(groups[i], []).append((local[i], local[j]))
        for g, pairs in by_group.items():
            run = runs[g]
            self._apply_prune(run.tree, per[g], pairs, run.step, run)

    def _start_tree(self, idx: int, prompt) -> _TreeRun:
        dev = self.wrapper.device
        if isinstance(prompt, str):
            input_ids = self.tokenizer(prompt, return_tensors="pt")["input_ids"].to(dev)
        else:
            input_ids = torch.tensor([list(prompt)], dtype=torch.long, device=dev)
        seq_id = self.kv_cache_mgr.allocate_sequence()
        logits = self.wrapper.prefill(input_ids, seq_id)
        tree = PrefixTree(self.kv_cache_mgr)
        first = TreeNode(node_id=tree.new_id(), token_ids=[], seq_id=seq_id, parent=tree.root,
                         cumulative_log_prob=0.0, depth=0, is_active=True)
        tree.root.children[0] = first
        run = _TreeRun(index=idx, tree=tree, prefill_tokens=int(input_ids.shape[-1]))
        self._prefill_tokens += run.prefill_tokens
        self._decide_rows([first], logits.unsqueeze(0), [tree], [0], [1], [run])
        return run

    def _finish_tree(self, run: _TreeRun) -> list[dict]:
        tree = run.tree
        results = []
        for node in tree.get_complete_sequences() + tree.get_active_leaves():
            tids = node.get_full_sequence()
            length = max(len(tids), 1)
            results.append({
                "token_ids": tids,
                "text": self.tokenizer.decode(tids, skip_special_tokens=True),
                "log_prob": node.cumulative_log_prob,
                "norm_prob": math.exp(node.cumulative_log_prob / length),
            })
        self._free_walk(tree.root)
        results.sort(key=lambda r: r["norm_prob"], reverse=True)
        return results

    def get_batch_diagnostics(self) -> dict:
        """Whole-batch metric plus each prompt's traces (the reference's per-prompt keys)."""
        tps = self._total_tokens_decoded / self._decode_time_s if self._decode_time_s > 0 else 0.0
        with_capture = self._decode_time_s + self._capture_time_s
        tps_cap = self._total_tokens_decoded / with_capture if with_capture > 0 else 0.0
        kv = self.kv_cache_mgr.get_stats()
        return {
            "decode_tokens_total": self._total_tokens_decoded,
            "decode_time_s": round(self._decode_time_s, 4),
            "decode_throughput_tps": round(tps, 2),
            "capture_time_s": round(self._capture_time_s, 4),
            "decode_throughput_tps_incl_capture": round(tps_cap, 2),
            "decode_steps": len(self.batch_trace),
            "max_live_leaves": max(self.batch_trace) if self.batch_trace else 0,
            "prefill_tokens": self._prefill_tokens,
            "prefill_time_s": round(self._prefill_time_s, 4),
            "peak_vram_bytes": self._peak_vram_bytes,
            "kv_blocks_peak": kv["blocks_peak"],
            "peak_kv_cache_bytes_true": kv["peak_kv_cache_bytes_true"],
            "prompts": {
                i: {
                    "num_branch_points": len(r.branch_points),
                    "branch_points": r.branch_points,
                    "entropy_trace": r.entropy_trace,
                    "active_branch_trace": r.active_branch_trace,
                    "diversity_pruning_events": r.diversity_pruning_events,
                    "decode_tokens": r.decode_tokens,
                }
                for i, r in self.runs.items()
            },
        }
