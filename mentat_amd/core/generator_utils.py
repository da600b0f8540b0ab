"""Prefix tree, reference math helpers and the paged model runner.

Drop-in for the reference's core/generator_utils.py:
  * TreeNode / PrefixTree (:44-189): extend, branch (fork every child, then
    free the parent's sequence), prune with upward cascade, DFS pre-order
    walk over insertion-ordered children (the decode batch order).
  * compute_entropy / apply_repetition_penalty / adaptive_threshold
    (:196-253): the reference's per-leaf torch formulations, kept for
    callers; the generator itself uses the fused row kernel (ops.row_stats).
  * PagedModelWrapper (:259-423): prefill and batched decode through a
    ModelAdapter over the paged KV cache. decode_batch appends each layer's
    new K/V before that layer's attention, as the reference does (:387-404).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch
import torch.nn.functional as F

from .paged_kv_cache import PagedKVCacheManager

__all__ = ["TreeNode", "PrefixTree", "compute_entropy", "apply_repetition_penalty", "adaptive_threshold",
           "PagedModelWrapper"]


@dataclass
class TreeNode:
    node_id: int
    token_ids: list[int] = field(default_factory=list)
    seq_id: Optional[int] = None
    parent: Optional["TreeNode"] = None
    children: dict[int, "TreeNode"] = field(default_factory=dict)
    cumulative_log_prob: float = 0.0
    depth: int = 0
    is_active: bool = True
    is_eos: bool = False
    semantic_vector: Optional[torch.Tensor] = None
    entropy_ema: Optional[float] = None
    creation_step: int = 0
    is_pruned: bool = False

    def get_full_sequence(self) -> list[int]:
        """Generated token ids from the root to this node (the prompt is not part of the tree)."""
        parts = []
        node = self
        while node is not None:
            if node.token_ids:
                parts.append(node.token_ids)
            node = node.parent
        out: list[int] = []
        for seg in reversed(parts):
            out.extend(seg)
        return out


class PrefixTree:
    def __init__(self, kv_cache_mgr: PagedKVCacheManager):
        self.root = TreeNode(node_id=0)
        self._next_id = 1
        self.kv_cache_mgr = kv_cache_mgr

    def new_id(self) -> int:
        nid = self._next_id
        self._next_id += 1
        return nid

    def extend_leaf(self, leaf: TreeNode, token_id: int, log_prob: float) -> TreeNode:
        leaf.token_ids.append(token_id)
        leaf.cumulative_log_prob += log_prob
        leaf.depth += 1
        return leaf

    def branch_leaf(self, leaf: TreeNode, token_ids: list[int], log_probs: list[float]) -> list[TreeNode]:
        """One child per token (a forked cache sequence each); then the parent is
        deactivated and its sequence freed (core/generator_utils.py:102-138)."""
        children = []
        for tid, lp in zip(token_ids, log_probs):
            cid = self.kv_cache_mgr.fork_sequence(leaf.seq_id)
            child = TreeNode(
                node_id=self.new_id(),
                token_ids=[tid],
                seq_id=cid,
                parent=leaf,
                cumulative_log_prob=leaf.cumulative_log_prob + lp,
                depth=leaf.depth + 1,
                is_active=True,
                entropy_ema=leaf.entropy_ema,
                semantic_vector=leaf.semantic_vector.clone() if leaf.semantic_vector is not None else None,
            )
            leaf.children[child.node_id] = child
            children.append(child)
        leaf.is_active = False
        if leaf.seq_id is not None:
            self.kv_cache_mgr.free_sequence(leaf.seq_id)
            leaf.seq_id = None
        return children

    def prune_branch(self, node: TreeNode) -> None:
        """Deactivate and free `node`; cascade to inactive ancestors whose
        children are all pruned (the root is never pruned), :140-169."""
        while True:
            if node.seq_id is not None:
                self.kv_cache_mgr.free_sequence(node.seq_id)
                node.seq_id = None
            node.is_active = False
            node.is_pruned = True
            parent = node.parent
            if parent is None:
                return
            survivors = any(not c.is_pruned for c in parent.children.values())
            if survivors or parent.is_active or parent.parent is None:
                return
            node = parent

    def get_active_leaves(self) -> list[TreeNode]:
        out: list[TreeNode] = []
        self._walk(self.root, out, want_active=True)
        return out

    def get_complete_sequences(self) -> list[TreeNode]:
        out: list[TreeNode] = []
        self._walk(self.root, out, want_active=False)
        return out

    def _walk(self, node: TreeNode, out: list, *, want_active: bool) -> None:
        # Iterative DFS pre-order (children in insertion order), same order as
        # the reference's recursion (:180-189).
        stack = [node]
        while stack:
            n = stack.pop()
            if want_active:
                if n.is_active and not n.children and not n.is_eos:
                    out.append(n)
            elif n.is_eos:
                out.append(n)
            if n.children:
                stack.extend(reversed(list(n.children.values())))


def compute_entropy(logits: torch.Tensor, temperature: float = 1.0) -> float:
    """Shannon entropy (nats) of softmax(logits / T) (core/generator_utils.py:196-202)."""
    probs = F.softmax(logits / temperature, dim=-1)
    log_probs = F.log_softmax(logits / temperature, dim=-1)
    plogp = torch.nan_to_num(probs * log_probs, nan=0.0)
    return -plogp.sum().item()


def apply_repetition_penalty(logits: torch.Tensor, token_ids: list[int], penalty: float = 1.2) -> torch.Tensor:
    """x > 0 ? x / p : x * p on the unique ids (core/generator_utils.py:205-230)."""
    if not token_ids or penalty == 1.0:
        return logits
    logits = logits.clone()
    ids = list(set(token_ids))
    g = logits[ids]
    logits[ids] = torch.where(g > 0, g / penalty, g * penalty)
    return logits


def _find_blocked_tokens(token_ids: list[int], max_n: int) -> set[int]:
    """Tokens that would repeat an n-gram (2 <= n <= max_n): wherever the last
    n-1 tokens occurred earlier, the token that followed them there
    (core/generator_utils.py:233-244; imported by the reference's generator)."""
    blocked: set[int] = set()
    total = len(token_ids)
    for n in range(2, max_n + 1):
        k = n - 1
        if total < n:
            continue
        tail = token_ids[total - k:]
        for start in range(total - k):
            if token_ids[start:start + k] == tail:
                blocked.add(token_ids[start + k])
    return blocked


def adaptive_threshold(base_val: float, max_active: int, current_active: int) -> float:
    util = current_active / max(max_active, 1)
    return base_val * (1.0 + 2.0 * util * util)


class PagedModelWrapper:
    """embed -> per layer (norm, paged attention, residual, norm, MLP, residual) -> norm -> lm_head."""

    def __init__(self, model, kv_cache_mgr: PagedKVCacheManager, adapter, eos_token_id=2):
        self.model = model
        self.kv_cache_mgr = kv_cache_mgr
        self.adapter = adapter
        self.eos_token_id = eos_token_id
        self.device = adapter.device
        self.dtype = adapter.dtype
        self.config = model.config
        self.graphs = None

    def enable_step_capture(self, buckets=None) -> None:
        """Run batched decode steps as captured graph replays (core/graph_decode.py);
        batches above its largest bucket still run eagerly. ``buckets``: the batch
        sizes to capture (default: the tables measured on an MI355X), or
        "calibrate" to measure this device's table first
        (DecodeGraphs.calibrate_buckets; also MENTAT_CALIBRATE_BUCKETS=1)."""
        from .graph_decode import DecodeGraphs

        if self.graphs is None:
            self.graphs = DecodeGraphs(self, buckets=buckets)

    @torch.no_grad()
    def prefill(self, input_ids: torch.LongTensor, seq_id: int) -> torch.Tensor:
        """Run the prompt (1, S) and write its K/V; returns the last position's logits (V,)."""
        a = self.adapter
        hidden = a.embeddings(input_ids)
        for layer_idx, block in enumerate(a.layers):
            attn = a.get_self_attn(block)
            residual = hidden
            x = a.apply_pre_attn_norm(block, hidden)
            attn_out, k_new, v_new = a.forward_paged_prefill(attn, x, layer_idx)
            self.kv_cache_mgr.append_tokens(seq_id, layer_idx, k_new, v_new)
            hidden = a.apply_post_attn_residual(block, residual, attn_out)
            residual = hidden
            x = a.apply_pre_mlp_norm(block, hidden)
            hidden = a.apply_post_mlp_residual(block, residual, a.get_mlp(block)(x))
        hidden = a.final_norm(hidden)
        return a.lm_head(hidden[0, -1, :])

    @torch.no_grad()
    def decode_batch_tensor(self, token_ids_per_seq: list[int], seq_ids: list[int]):
        """One token for each of N sequences: (logits [N, V], final hidden [N, hidden])."""
        a = self.adapter
        N = len(seq_ids)
        assert N == len(token_ids_per_seq)
        if N == 0:
            return (torch.empty(0, self.config.vocab_size, device=self.device, dtype=self.dtype),
                    torch.empty(0, self.config.hidden_size, device=self.device, dtype=self.dtype))
        if self.graphs is not None:
            out = self.graphs.decode(token_ids_per_seq, seq_ids)
            if out is not None:
                return out
        ids = torch.tensor(token_ids_per_seq, dtype=torch.long).to(self.device).unsqueeze(0)
        hidden = a.embeddings(ids)
        offsets = [self.kv_cache_mgr.get_kv_length(s) for s in seq_ids]  # RoPE position of the new token
        for layer_idx, block in enumerate(a.layers):
            attn = a.get_self_attn(block)
            residual = hidden
            x = a.apply_pre_attn_norm(block, hidden)
            k_new, v_new = a.project_kv_for_cache(attn, x, offsets)
            self.kv_cache_mgr.append_tokens_batched(seq_ids=seq_ids, layer_idx=layer_idx, k=k_new, v=v_new)
            attn_out = a.forward_paged_decode(attn, x, self.kv_cache_mgr, seq_ids, offsets, layer_idx)
            hidden = a.apply_post_attn_residual(block, residual, attn_out)
            residual = hidden
            x = a.apply_pre_mlp_norm(block, hidden)
            hidden = a.apply_post_mlp_residual(block, residual, a.get_mlp(block)(x))
        hidden = a.final_norm(hidden).squeeze(0)
        return a.lm_head(hidden), hidden

    @torch.no_grad()
    def decode_batch(self, token_ids_per_seq: list[int], seq_ids: list[int]):
        """Reference signature: (list of N logits rows (V,), hidden [N, hidden])."""
        logits, hidden = self.decode_batch_tensor(token_ids_per_seq, seq_ids)
        return [logits[i] for i in range(logits.shape[0])], hidden

    def is_eos(self, token_id: int) -> bool:
        if isinstance(self.eos_token_id, (list, tuple)):
            return token_id in self.eos_token_id
        return token_id == self.eos_token_id
