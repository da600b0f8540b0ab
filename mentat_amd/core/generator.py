"""MentatGenerator — entropy-gated prefix-tree decoding over the paged KV cache.

Drop-in for the reference's core/generator.py: same constructor keywords and
defaults (:29-51), generate(prompt) -> results sorted by length-normalised
probability (:125-245), get_diagnostics() keys (:503-555).

Per decode step (reference :174-207, DFS batch order, num_active frozen for
the step):
  1. one batched forward of every live leaf (PagedModelWrapper.decode_batch_tensor);
  2. semantic EMA update (:376-398);
  3. ONE fused row-kernel call over the [N, V] logits (ops.row_stats): gate
     entropy at `temperature` on the raw logits, repetition penalty on each
     leaf's generated ids, top-K log-probs of the penalised row (K =
     branching_factor; top-1 is the greedy extension), entropy of the
     penalised row (branch diagnostics); ONE device-to-host copy of that record;
  4. the host applies _step_leaf's rule to every leaf in batch order (:333-374):
       ema <- H (first) or alpha*H + (1-alpha)*ema
       tau  = ema * base*(1 + 2u^2) * warmup(step),  u = num_active / M
       branch <=> H > tau and (M - num_active) >= K
     with gate="absolute" (new; the reference only has the relative gate)
     replacing `H > tau` by `H > entropy_threshold`;
  5. semantic-similarity prune (:400-497).
"""
from __future__ import annotations

import math
import time
from typing import Optional

import numpy as np
import torch

from .. import ops
from ..adapters.adapter_factory import ModelAdapter, get_adapter
from .generator_utils import PagedModelWrapper, PrefixTree, TreeNode, adaptive_threshold
from .paged_kv_cache import PagedKVCacheManager

__all__ = ["MentatGenerator"]


class MentatGenerator:
    def __init__(
        self,
        model,
        tokenizer,
        *,
        adapter: ModelAdapter | None = None,
        max_active_branches: int = 10,
        branching_factor: int = 3,
        relative_entropy_multiplier: float = 1.25,
        entropy_ema_alpha: float = 0.3,
        max_new_tokens: int = 256,
        temperature: float = 0.7,
        repetition_penalty: float = 1.2,
        block_size: int = 16,
        max_blocks: int = 8192,
        semantic_similarity_threshold: float = 0.85,
        ema_alpha: float = 0.3,
        min_steps_before_prune: int = 5,
        soft_explore_window: int = 10,
        soft_explore_initial: float = 0.3,
        gate: str = "relative",
        entropy_threshold: float = 2.0,
        capture_steps: bool = True,
    ):
        if gate not in ("relative", "absolute"):
            raise ValueError("gate must be 'relative' or 'absolute'")
        if not 1 <= branching_factor <= 8:
            raise ValueError("branching_factor must be in [1, 8]")
        eos = tokenizer.eos_token_id
        if eos is None:
            eos = 2
        self.tokenizer = tokenizer
        self.M = max_active_branches
        self.K = branching_factor
        self.relative_entropy_multiplier = relative_entropy_multiplier
        self.entropy_ema_alpha = entropy_ema_alpha
        self.max_new_tokens = max_new_tokens
        self.temperature = temperature
        self.rep_penalty = repetition_penalty
        self.semantic_similarity_threshold = semantic_similarity_threshold
        self.ema_alpha = ema_alpha
        self.min_steps_before_prune = min_steps_before_prune
        self.soft_explore_window = soft_explore_window
        self.soft_explore_initial = soft_explore_initial
        self.gate = gate
        self.entropy_threshold = entropy_threshold

        if adapter is None:
            adapter = get_adapter(model)
        self.adapter = adapter
        if max_blocks is None:  # reference :84-87
            tokens_budget = max_active_branches * (max_new_tokens + 512)
            max_blocks = max((tokens_budget // block_size + 1) * 2, 256)
        self.kv_cache_mgr = PagedKVCacheManager(
            num_layers=adapter.num_hidden_layers,
            num_key_value_heads=adapter.num_key_value_heads,
            head_dim=adapter.head_dim,
            max_blocks=max_blocks,
            block_size=block_size,
            device=adapter.device,
            dtype=adapter.dtype,
        )
        self.wrapper = PagedModelWrapper(model, self.kv_cache_mgr, adapter, eos_token_id=eos)
        if capture_steps and self.wrapper.device.type == "cuda":
            self.wrapper.enable_step_capture()

        self.branch_points: list[tuple[int, float, int]] = []
        self.pruning_events: list[tuple[int, int]] = []
        self.entropy_trace: list[tuple[int, int, float]] = []
        self.diversity_pruning_events: list[tuple[int, int]] = []
        self.active_branch_trace: list[int] = []
        self._total_tokens_decoded = 0
        self._prefill_tokens = 0
        self._prefill_time_s = 0.0
        self._decode_time_s = 0.0
        self._capture_time_s = 0.0
        self._peak_vram_bytes = 0
        self.step_hook = None  # optional callable(step, tree) after every decode step

    # ------------------------------------------------------------------
    def generate(self, prompt: str) -> list[dict]:
        self.active_branch_trace = []
        self._total_tokens_decoded = 0
        self._prefill_tokens = 0
        self._prefill_time_s = 0.0
        self._decode_time_s = 0.0
        self._capture_time_s = 0.0
        self._peak_vram_bytes = 0
        dev = self.wrapper.device
        on_gpu = dev.type == "cuda"
        if on_gpu:
            torch.cuda.reset_peak_memory_stats(dev)

        enc = self.tokenizer(prompt, return_tensors="pt")
        input_ids = enc["input_ids"].to(dev)
        self._prefill_tokens = input_ids.shape[-1]

        t0 = time.perf_counter()
        seq_id = self.kv_cache_mgr.allocate_sequence()
        logits = self.wrapper.prefill(input_ids, seq_id)
        if on_gpu:
            torch.cuda.synchronize(dev)
        self._prefill_time_s = time.perf_counter() - t0

        tree = PrefixTree(self.kv_cache_mgr)
        first = TreeNode(node_id=tree.new_id(), token_ids=[], seq_id=seq_id, parent=tree.root,
                         cumulative_log_prob=0.0, depth=0, is_active=True)
        tree.root.children[0] = first
        self._decide(tree, [first], logits.unsqueeze(0), step=0, num_active=1)
        self._prepare_capture(1, int(input_ids.shape[-1]))

        t0 = time.perf_counter()
        for step in range(1, self.max_new_tokens):
            active = tree.get_active_leaves()
            if not active:
                break
            num_active = len(active)
            self.active_branch_trace.append(num_active)
            logits, hidden = self.wrapper.decode_batch_tensor([l.token_ids[-1] for l in active],
                                                              [l.seq_id for l in active])
            self._total_tokens_decoded += num_active
            self._update_semantic_vectors(active, hidden)
            self._decide(tree, active, logits, step, num_active)
            self._prune_similar(tree, step)
            if self.step_hook is not None:
                self.step_hook(step, tree)
            if not tree.get_active_leaves():
                break
        if on_gpu:
            torch.cuda.synchronize(dev)
        self._decode_time_s = time.perf_counter() - t0
        if on_gpu:
            self._peak_vram_bytes = torch.cuda.max_memory_allocated(dev)

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
        self.tree = tree
        return results

    def max_leaves_per_tree(self) -> int:
        """Live leaves one tree can reach: every leaf of a step decides against the
        step's frozen num_active, so with a live leaves (a <= M - K) all of them
        may branch into K children each."""
        return max(self.M, (self.M - self.K) * self.K, 1)

    def _prepare_capture(self, trees: int, max_prompt: int) -> None:
        """Capture the decode steps' batch buckets before the decode timer starts;
        the wall time goes to capture_time_s (reported beside the decode time)."""
        graphs = self.wrapper.graphs
        if graphs is None:
            return
        t0 = time.perf_counter()
        leaves = trees * self.max_leaves_per_tree()
        graphs.prepare(leaves, max_prompt + self.max_new_tokens + 1, rows=leaves + trees)
        torch.cuda.synchronize(self.wrapper.device)
        self._capture_time_s += time.perf_counter() - t0

    # ------------------------------------------------------------------
    def _penalty_csr(self, leaves: list[TreeNode]):
        lists = [l.get_full_sequence() for l in leaves]
        off = np.zeros(len(lists) + 1, dtype=np.int32)
        off[1:] = np.cumsum([len(x) for x in lists])
        flat = np.fromiter((t for x in lists for t in x), dtype=np.int32, count=int(off[-1]))
        if flat.size == 0:
            flat = np.zeros(1, dtype=np.int32)
        dev = self.wrapper.device
        if dev.type != "cuda":
            return torch.from_numpy(off).to(dev), torch.from_numpy(flat).to(dev)
        # Pinned staging: the uploads and the row kernel queue behind the step's
        # decode without a host round trip.
        return (torch.from_numpy(off).pin_memory().to(dev, non_blocking=True),
                torch.from_numpy(flat).pin_memory().to(dev, non_blocking=True))

    def _decide(self, tree: PrefixTree, leaves: list[TreeNode], logits: torch.Tensor, step: int,
                num_active: int) -> None:
        """Gate + branch/extend for every leaf of the batch (reference _step_leaf, :333-374)."""
        n = len(leaves)
        self._decide_rows(leaves, logits, [tree] * n, [step] * n, [num_active] * n, [self] * n)

    def _launch_decisions(self, leaves: list[TreeNode], logits: torch.Tensor):
        """Queue the step's row kernel and one device-to-host copy of its
        decision record [H_T, H_pen, K log-probs, K ids (int32 bits carried as
        float32)]; returns (host record, event after its copy). Work queued
        later does not delay the record."""
        off, ids = self._penalty_csr(leaves)
        st = ops.row_stats(
            logits.contiguous(), temperature=self.temperature, penalty=self.rep_penalty,
            pen_offsets=off, pen_ids=ids, topk=self.K, pen_stats=True,
        )
        rec = torch.cat([st.entropy[:, None], st.entropy_pen[:, None], st.topk_lp,
                         st.topk_ids.view(torch.float32)], dim=1)
        if rec.device.type != "cuda":
            return rec, None
        host = torch.empty(rec.shape, dtype=rec.dtype, pin_memory=True)
        host.copy_(rec, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        return host, ev

    def _decide_rows(self, leaves: list[TreeNode], logits: torch.Tensor, trees: list, steps: list,
                     num_actives: list, logs: list, launched=None) -> None:
        """_decide over a batch whose leaves may belong to different trees: leaf i
        follows the rules with its own tree's step, frozen num_active, and appends
        to logs[i].entropy_trace / .branch_points. ``launched``: the result of
        _launch_decisions for these leaves and logits, if already queued."""
        rec, ev = launched if launched is not None else self._launch_decisions(leaves, logits)
        if ev is not None:
            ev.synchronize()
        rec_cpu = rec.numpy()
        ids_cpu = np.ascontiguousarray(rec_cpu[:, 2 + self.K:2 + 2 * self.K]).view(np.int32)
        # Python lists (the float32 values as Python floats) are far cheaper to
        # index per leaf than numpy scalars.
        K = self.K
        rec_rows = rec_cpu.tolist()
        id_rows = ids_cpu.tolist()
        alpha, M = self.entropy_ema_alpha, self.M
        keep = 1.0 - alpha
        relative, thr = self.gate == "relative", self.entropy_threshold
        is_eos = self.wrapper.is_eos
        for i, leaf in enumerate(leaves):
            if not leaf.is_active:
                continue
            tree, step, num_active, log = trees[i], steps[i], num_actives[i], logs[i]
            row = rec_rows[i]
            H = row[0]
            log.entropy_trace.append((step, leaf.node_id, H))
            if leaf.entropy_ema is None:
                leaf.entropy_ema = H
            else:
                leaf.entropy_ema = alpha * H + keep * leaf.entropy_ema
            headroom = M - num_active
            if relative:
                mult = adaptive_threshold(self.relative_entropy_multiplier, M, num_active)
                tau = leaf.entropy_ema * mult * self._soft_explore_factor(step)
                open_gate = H > tau
            else:
                open_gate = H > thr
            top_ids = id_rows[i]
            if open_gate and headroom >= K:
                children = tree.branch_leaf(leaf, top_ids, row[2:2 + K])
                log.branch_points.append((step, row[1], len(children)))
                for child in children:
                    child.creation_step = step
                    self._handle_eos(tree, child)
            else:
                tok = top_ids[0]
                tree.extend_leaf(leaf, tok, row[2])
                if is_eos(tok):
                    self._handle_eos(tree, leaf)

    def _handle_eos(self, tree: PrefixTree, node: TreeNode) -> None:
        if self.wrapper.is_eos(node.token_ids[-1]):
            node.is_eos = True
            node.is_active = False
            if node.seq_id is not None:
                tree.kv_cache_mgr.free_sequence(node.seq_id)
                node.seq_id = None

    def _free_walk(self, node: TreeNode) -> None:
        stack = [node]
        while stack:
            n = stack.pop()
            if n.seq_id is not None:
                self.kv_cache_mgr.free_sequence(n.seq_id)
                n.seq_id = None
            stack.extend(n.children.values())

    def _soft_explore_factor(self, step: int) -> float:
        if step >= self.soft_explore_window:
            return 1.0
        t = step / max(self.soft_explore_window, 1)
        return self.soft_explore_initial + (1.0 - self.soft_explore_initial) * t

    # ---- semantic diversity (reference :376-497) ----------------------------------------
    def _update_semantic_vectors(self, leaves: list[TreeNode], hidden_states: torch.Tensor) -> None:
        """EMA of every leaf's semantic vector (reference :376-398) in one launch
        (ops.semantic_ema): a new leaf takes its hidden state (as h.clone()),
        the others v.mul_(1 - alpha).add_(h, alpha=alpha) with torch's rounding.
        New leaves' vectors are rows of one fresh buffer."""
        if not leaves:
            return
        fresh = [leaf.semantic_vector is None for leaf in leaves]
        n_new = sum(fresh)
        if n_new:
            buf = torch.empty(n_new, hidden_states.shape[1], dtype=hidden_states.dtype, device=hidden_states.device)
            k = 0
            for leaf, f in zip(leaves, fresh):
                if f:
                    leaf.semantic_vector = buf[k]
                    k += 1
        vecs = []
        for leaf in leaves:
            v = leaf.semantic_vector
            if not v.is_contiguous() or v.dtype != hidden_states.dtype:
                v = leaf.semantic_vector = v.to(hidden_states.dtype).contiguous()
            vecs.append(v)
        ops.semantic_ema(vecs, hidden_states.contiguous(), fresh, self.ema_alpha)

    def _prune_similar(self, tree: PrefixTree, step: int, log=None) -> None:
        log = self if log is None else log
        leaves = tree.get_active_leaves()
        if len(leaves) <= 1:
            return
        sv_leaves = [l for l in leaves
                     if l.semantic_vector is not None and step - l.creation_step >= self.min_steps_before_prune]
        M = len(sv_leaves)
        if M <= 1:
            return
        pairs = self._similar_pairs(sv_leaves, [0] * M)
        self._apply_prune(tree, sv_leaves, pairs, step, log)

    def _apply_prune(self, tree: PrefixTree, sv_leaves: list[TreeNode], pairs: list, step: int, log) -> None:
        """Greedy prune over the similar pairs in row-major order (reference :462-497)."""
        if not pairs:
            return
        to_prune: set[int] = set()
        for i, j in pairs:
            li, lj = sv_leaves[i], sv_leaves[j]
            if li.node_id in to_prune or lj.node_id in to_prune:
                continue
            if li.cumulative_log_prob >= lj.cumulative_log_prob:
                to_prune.add(lj.node_id)
            else:
                to_prune.add(li.node_id)
        pruned = 0
        for leaf in sv_leaves:
            if leaf.node_id in to_prune and leaf.is_active:
                tree.prune_branch(leaf)
                pruned += 1
        if pruned:
            log.diversity_pruning_events.append((step, pruned))

    def _similar_keys(self, sv_leaves: list[TreeNode]) -> list:
        """Sibling keys: leaves with one parent share a key; a parentless leaf
        gets a key of its own."""
        keys, parents = [], {}
        for i, leaf in enumerate(sv_leaves):
            if leaf.parent is None:
                keys.append(-1 - i)  # never equal to another leaf's key
            else:
                keys.append(parents.setdefault(id(leaf.parent), len(parents)))
        return keys

    def _similar_pairs(self, sv_leaves: list[TreeNode], groups: list) -> list:
        """(i, j), i < j, row-major: leaves of the same group (tree) whose semantic
        vectors have cosine similarity above the threshold and that are not
        siblings (reference :447-460). The mask is one device call
        (ops.semantic_similar_mask: F.normalize + product in the vectors' dtype,
        triangle, sibling and group masks) read back as M*M bytes."""
        keys = self._similar_keys(sv_leaves)
        mask = ops.semantic_similar_mask([l.semantic_vector for l in sv_leaves], keys, groups,
                                         self.semantic_similarity_threshold)
        ii, jj = np.nonzero(mask)
        return list(zip(ii.tolist(), jj.tolist()))

    # ------------------------------------------------------------------
    def get_diagnostics(self) -> dict:
        decode_tps = self._total_tokens_decoded / self._decode_time_s if self._decode_time_s > 0 else 0.0
        with_capture = self._decode_time_s + self._capture_time_s
        decode_tps_cap = self._total_tokens_decoded / with_capture if with_capture > 0 else 0.0
        prefill_tps = self._prefill_tokens / self._prefill_time_s if self._prefill_time_s > 0 else 0.0
        kv = self.kv_cache_mgr.get_stats()
        return {
            "num_branch_points": len(self.branch_points),
            "total_pruned": sum(n for _, n in self.pruning_events),
            "total_diversity_pruned": sum(n for _, n in self.diversity_pruning_events),
            "branch_points": self.branch_points,
            "pruning_events": self.pruning_events,
            "diversity_pruning_events": self.diversity_pruning_events,
            "entropy_trace": self.entropy_trace,
            "active_branch_trace": self.active_branch_trace,
            "prefill_tokens": self._prefill_tokens,
            "prefill_time_s": round(self._prefill_time_s, 4),
            "prefill_throughput_tps": round(prefill_tps, 2),
            "decode_tokens_total": self._total_tokens_decoded,
            "decode_time_s": round(self._decode_time_s, 4),
            "decode_throughput_tps": round(decode_tps, 2),
            # graph capture of the decode step (before the decode timer starts; the
            # reference has no such phase) and the rate with it counted as decode time
            "capture_time_s": round(self._capture_time_s, 4),
            "decode_throughput_tps_incl_capture": round(decode_tps_cap, 2),
            "peak_vram_bytes": self._peak_vram_bytes,
            "peak_vram_mb": round(self._peak_vram_bytes / 1024 ** 2, 2),
            "peak_kv_cache_bytes": kv["peak_kv_cache_bytes"],
            "peak_kv_cache_mb": round(kv["peak_kv_cache_bytes"] / 1024 ** 2, 2),
            "peak_kv_cache_bytes_true": kv["peak_kv_cache_bytes_true"],
            "kv_blocks_peak": kv["blocks_peak"],
            "kv_blocks_total": kv["blocks_total"],
            "kv_peak_utilization": round(kv["peak_utilization"], 4),
        }
