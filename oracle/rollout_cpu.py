"""Oracle: the reference's MENTAT rollout on the CPU, for timing (test
infrastructure only: bench.py's end-to-end CPU baseline).

Restates, in torch on the host, one prompt's rollout as the reference runs it
(prompts are serial there, mentat_rollout.py:256-259):
  * prefill (core/generator_utils.py:306-338): the prompt through the model
    with causal SDPA (oracle.attention.reference_cpu_prefill), K/V appended
    into paged pools with the reference's block bookkeeping
    (oracle.paged_cache.OracleCache, copy-on-write copies applied to the pools;
    one store indexed by block id serves every layer);
  * decode steps (core/generator_utils.py:340-418, core/generator.py:174-207):
    every active leaf in DFS order through one batched forward; per layer the
    Q/K/V projections, RoPE at the kv length read before the layer loop, the
    batched append, build_packed_kv's gather and one SDPA per sequence
    (oracle.attention.reference_cpu_decode), o_proj and the MLP;
  * per step, the semantic EMA (core/generator.py:376-398), _step_leaf for
    each leaf in batch order with num_active frozen (:333-374; here the
    absolute gate H_T > threshold with headroom M - num_active >= K, the mode
    the end-to-end workload uses): branch = top-K of log_softmax of the
    repetition-penalised logits, children forked and the parent freed
    (core/generator_utils.py:102-138); extend = argmax; EOS deactivates and
    frees; then the pairwise-similarity prune (:400-497).
Metric as the reference's (core/generator.py:190, :508-511): live leaves
summed over decode steps / decode wall time.

Pinned by tests/test_gpu_batch_generator.py::
test_cpu_rollout_restatement_follows_the_generator: on the fp32 plumbing model
with the absolute gate it produces the product generator's live-leaf trace
(the product generator is in turn pinned by the reference's own cfg-1
trajectory). It is used as a throughput baseline.
"""
from __future__ import annotations

import time

import torch
import torch.nn.functional as F

from .attention import reference_cpu_decode, reference_cpu_prefill
from .paged_cache import OracleCache


class _Leaf:
    __slots__ = ("tokens", "seq", "lp", "parent", "children", "active", "step", "sv")

    def __init__(self, tokens, seq, lp, parent, step):
        self.tokens, self.seq, self.lp, self.parent, self.step = tokens, seq, lp, parent, step
        self.children = []
        self.active = True
        self.sv = None


def _rotate_half(t):
    h = t.shape[-1] // 2
    return torch.cat((-t[..., h:], t[..., :h]), dim=-1)


class _CpuModel:
    """The reference adapter's per-layer decode/prefill on a HF Llama-style model (CPU)."""

    def __init__(self, model, max_blocks: int, block_size: int):
        base = model.model
        self.m, self.base = model, base
        cfg = model.config
        self.L = cfg.num_hidden_layers
        self.Hq, self.Hkv = cfg.num_attention_heads, cfg.num_key_value_heads
        self.D = getattr(cfg, "head_dim", None) or cfg.hidden_size // self.Hq
        self.B = block_size
        dt = next(model.parameters()).dtype
        self.cache = OracleCache(self.L, max_blocks, block_size)
        # One K and one V store indexed by block id for every layer: the single
        # allocator gives each id to one layer at a time, so per-layer pools
        # (core/paged_kv_cache.py:124-138) would hold the same data.
        ks = torch.zeros(max_blocks, block_size, self.Hkv, self.D, dtype=dt)
        vs = torch.zeros(max_blocks, block_size, self.Hkv, self.D, dtype=dt)
        self.kp = [ks] * self.L
        self.vp = [vs] * self.L

    def _apply_copies(self, n0: int) -> None:
        for layer, src, dst in self.cache.copies[n0:]:
            self.kp[layer][dst] = self.kp[layer][src]
            self.vp[layer][dst] = self.vp[layer][src]

    def _qkv(self, attn, hs, pos):
        n, s, _ = hs.shape
        q = attn.q_proj(hs).view(n, s, self.Hq, self.D)
        k = attn.k_proj(hs).view(n, s, self.Hkv, self.D)
        v = attn.v_proj(hs).view(n, s, self.Hkv, self.D)
        cos, sin = self.base.rotary_emb(v, pos)
        cos, sin = cos.unsqueeze(2), sin.unsqueeze(2)
        return q * cos + _rotate_half(q) * sin, k * cos + _rotate_half(k) * sin, v

    def prefill(self, ids: list[int], sid: int):
        x = self.base.embed_tokens(torch.tensor([ids]))
        pos = torch.arange(len(ids)).unsqueeze(0)
        for layer, blk in enumerate(self.base.layers):
            h = blk.input_layernorm(x)
            q, k, v = self._qkv(blk.self_attn, h, pos)
            n0 = len(self.cache.copies)
            self.cache.append(sid, layer, list(range(len(ids))))
            self._apply_copies(n0)
            off = 0
            for b in self.cache.tables[sid][layer]:
                c = min(self.B, len(ids) - off)
                self.kp[layer][b, :c] = k[0, off:off + c]
                self.vp[layer][b, :c] = v[0, off:off + c]
                off += c
            o = reference_cpu_prefill(q, k, v)
            x = x + blk.self_attn.o_proj(o.reshape(1, len(ids), -1))
            x = x + blk.mlp(blk.post_attention_layernorm(x))
        return self.m.lm_head(self.base.norm(x)[0, -1])

    def decode(self, toks: list[int], sids: list[int]):
        n = len(sids)
        x = self.base.embed_tokens(torch.tensor([toks]))
        pos = torch.tensor([self.cache.ntok[s][0] for s in sids]).unsqueeze(1)
        for layer, blk in enumerate(self.base.layers):
            h = blk.input_layernorm(x).squeeze(0).unsqueeze(1)
            q, k, v = self._qkv(blk.self_attn, h, pos)
            n0 = len(self.cache.copies)
            dests = self.cache.append_batched(sids, layer, [0] * n)
            self._apply_copies(n0)
            for i, (b, sl) in enumerate(dests):
                self.kp[layer][b, sl] = k[i, 0]
                self.vp[layer][b, sl] = v[i, 0]
            o = reference_cpu_decode(q.squeeze(1), self.kp[layer], self.vp[layer],
                                     [self.cache.tables[s][layer] for s in sids],
                                     [self.cache.ntok[s][layer] for s in sids], self.B)
            x = x + blk.self_attn.o_proj(o.reshape(1, n, -1))
            x = x + blk.mlp(blk.post_attention_layernorm(x))
        hid = self.base.norm(x).squeeze(0)
        return self.m.lm_head(hid), hid


def reference_cpu_rollout(model, prompt_ids: list[int], *, max_new_tokens: int, time_budget_s: float,
                          max_active_branches: int = 8, branching_factor: int = 3, entropy_threshold: float = 2.5,
                          temperature: float = 0.7, repetition_penalty: float = 1.2, ema_alpha: float = 0.3,
                          semantic_similarity_threshold: float = 0.85, min_steps_before_prune: int = 5,
                          eos_token_id: int = 2, block_size: int = 16, max_blocks: int = 8192) -> dict:
    """One prompt's rollout on the CPU until max_new_tokens or until decode time
    exceeds time_budget_s. Returns decode tokens, decode seconds, steps and the
    live-leaf trace."""
    M, K = max_active_branches, branching_factor
    cm = _CpuModel(model, max_blocks, block_size)
    with torch.no_grad():
        sid = cm.cache.allocate()
        logits = cm.prefill(prompt_ids, sid)
        root = _Leaf([], sid, 0.0, None, 0)
        trace = []

        def leaves(node, out):
            if not node.children:
                if node.active:
                    out.append(node)
                return out
            for c in node.children:
                leaves(c, out)
            return out

        def step_leaf(leaf, row, step, num_active):
            z = row.float() / temperature
            lp = torch.log_softmax(z, -1)
            t = torch.exp(lp) * lp
            H = float(-torch.nan_to_num(t).sum())
            pen = row.clone()
            if leaf.tokens and repetition_penalty != 1.0:
                u = torch.tensor(sorted(set(leaf.tokens)))
                g = pen[u]
                pen[u] = torch.where(g > 0, g / repetition_penalty, g * repetition_penalty)
            keys = torch.log_softmax(pen, -1)
            if H > entropy_threshold and M - num_active >= K:
                vals, ids = torch.topk(keys, K)
                for tok, v in zip(ids.tolist(), vals.tolist()):
                    c = _Leaf(leaf.tokens + [tok], cm.cache.fork(leaf.seq), leaf.lp + v, leaf, step)
                    c.sv = None if leaf.sv is None else leaf.sv.clone()
                    leaf.children.append(c)
                leaf.active = False
                cm.cache.free(leaf.seq)
                for c in leaf.children:
                    if c.tokens[-1] == eos_token_id:
                        c.active = False
                        cm.cache.free(c.seq)
            else:
                tok = int(torch.argmax(keys))
                leaf.tokens.append(tok)
                leaf.lp += float(keys[tok])
                if tok == eos_token_id:
                    leaf.active = False
                    cm.cache.free(leaf.seq)

        step_leaf(root, logits, 0, 1)
        t0 = time.perf_counter()
        decoded, steps = 0, 0
        for step in range(1, max_new_tokens):
            act = leaves(root, [])
            if not act or time.perf_counter() - t0 > time_budget_s:
                break
            trace.append(len(act))
            logits, hid = cm.decode([l.tokens[-1] for l in act], [l.seq for l in act])
            decoded += len(act)
            steps += 1
            for i, leaf in enumerate(act):
                if leaf.sv is None:
                    leaf.sv = hid[i].clone()
                else:
                    leaf.sv.mul_(1.0 - ema_alpha).add_(hid[i], alpha=ema_alpha)
            for i, leaf in enumerate(act):
                step_leaf(leaf, logits[i], step, len(act))
            live = leaves(root, [])
            cand = [l for l in live if l.sv is not None and step - l.step >= min_steps_before_prune]
            if len(live) > 1 and len(cand) > 1:
                sv = F.normalize(torch.stack([l.sv for l in cand]), p=2, dim=1)
                sim = torch.mm(sv, sv.t())
                mask = torch.triu(torch.ones_like(sim, dtype=torch.bool), diagonal=1)
                for i in range(len(cand)):
                    for j in range(i + 1, len(cand)):
                        if cand[i].parent is not None and cand[i].parent is cand[j].parent:
                            mask[i, j] = False
                drop = set()
                for i, j in ((sim * mask) > semantic_similarity_threshold).nonzero().tolist():
                    if id(cand[i]) in drop or id(cand[j]) in drop:
                        continue
                    drop.add(id(cand[j]) if cand[i].lp >= cand[j].lp else id(cand[i]))
                for leaf in cand:
                    if id(leaf) in drop and leaf.active:
                        leaf.active = False
                        cm.cache.free(leaf.seq)
        dt = time.perf_counter() - t0
    return {"decode_tokens": decoded, "decode_s": dt, "steps": steps, "trace": trace}
