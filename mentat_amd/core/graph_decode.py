"""Captured decode steps: two HIP graph launches per batched decode forward.

The eager decode step (PagedModelWrapper.decode_batch_tensor, the reference's
core/generator_utils.py:340-418 loop) launches ~30 kernels per layer from
Python, and at Llama-3-8B size with ~150 live leaves the host, not the GPU,
sets the step time. Here the whole forward for a batch of ``Nb`` sequences —
embedding, every layer's norm, Q/K/V projections, RoPE, KV append (with the
lazy copy-on-write), paged decode attention, output projection, MLP and
residuals, the final norm and the LM head — is captured once per batch-size
bucket ``Nb`` and replayed per step.

Per step the host does what must stay on the host: the allocator and page
tables of every layer (PagedKVCacheManager.plan_append_step_begin / _finish,
the same block ids as the per-layer loop) and pinned host-to-device copies of
the step's int32 inputs (token ids, RoPE positions, table rows and the
[num_layers, 7, Nb] append plans). The forward is captured as two graphs over
one memory pool, the first SPLIT_LAYERS layers and the rest: the first graph
starts once its layers are planned, and the other layers are planned while it
runs and copied in before the second graph in stream order. Batches are padded to
the bucket: padding entries carry the token 0 at position 0, read the
manager's length-0 row (their attention output is zero) and have append plans
whose destination block is -1, which the append kernel skips; their logits are
dropped. A bucket's pinned staging is rewritten only after the event recorded
behind the previous step's copies out of it has completed, so steps queued
back to back without a host sync never overwrite plans not yet read.

A captured graph holds the addresses of the manager's device tables, of the
K/V stores, of its own input buffer and of the paged-decode workspace, so
  * graphs are captured again after the manager reallocates its tables
    (``tables_version``); ``prepare`` reserves table capacity up front;
  * the decode workspace of the capture stream is sized for the largest
    bucket before the first capture, and this object keeps it alive.
Warm-up and capture run with an all-padding input, which writes nothing to
the cache.

For 16-bit HF Llama/Qwen3-style models whose adapter keeps the stock glue, the
captured layer also fuses that glue: each residual add with the RMSNorm that
follows it (across the layer boundary too), RoPE of Q and K in one launch, and
SiLU(gate) * up (ops.rmsnorm, ops.rope_, ops.silu_mul); other models run their
modules as they are. Without QK-norm (Llama) the q/k/v projections also run
as one GEMM and gate/up as another, over per-layer concatenated copies of the
modules' weights (the modules are left as they are); each step refreshes a
copy's rows from any module weight that was rebound or changed in place
since (MERGE_PROJECTIONS selects this, views instead of copies, or no merge).
The RoPE of the merged q/k/v output then also writes k and v straight into
the pages (ops.rope_qkv_append: RoPE and KV append in one launch).

The batch-size buckets are tables measured on an MI355X (BUCKETS,
MERGED_BUCKETS); ``buckets="calibrate"`` measures this device's table instead
(DecodeGraphs.calibrate_buckets).

No object is destroyed while a capture is active: the garbage collector runs
before the captures (once for all the buckets ``prepare`` captures, else just
before the capture) and stays disabled during each capture. (A finished run's
graphs, pools and pinned buffers, if left to the cyclic collector, could
otherwise be torn down in the middle of another capture, where the HIP calls
of that teardown are not allowed and abort the process.) This object also
holds no reference back to its wrapper, so a dropped generator's graphs are
freed by reference counting, outside any capture.
"""
from __future__ import annotations

import gc
import os

import numpy as np
import torch

from .. import ops, tree_plan
from .._lib import LAYOUT_NATIVE, get_lib
from ..adapters.model_adapter import _HFDecoderAdapter

__all__ = ["DecodeGraphs", "BUCKETS"]

# Batch-size buckets (a step of N sequences runs the smallest bucket >= N). The
# step's GEMMs dominate its time, and the library's kernel choice is not
# monotone in the row count: at Llama-3-8B widths on an MI355X the 32-layer
# projections take 5.2 ms for 120 rows but 6.3 ms for 128, 6.0 ms for 152 but
# 7.2 ms for 160, 6.1 ms for 184 but 8.2 ms for 192. The buckets skip those
# row counts and step by 16 where the cost rises with the rows.
BUCKETS = (8, 16, 32, 48, 64, 80, 88, 104, 120, 136, 152, 168, 184, 200, 216, 232, 248, 256)
# With q/k/v and gate/up merged the GEMM costs move again (the merged q/k/v GEMM
# is slow at 128-160 rows: the 32 layers' projections take 5.5-6.1 ms there but
# 5.2 ms at 176): the buckets that no larger one undercuts.
MERGED_BUCKETS = (8, 16, 24, 32, 40, 56, 64, 72, 80, 88, 112, 120, 176, 184, 200, 208, 216, 232, 240, 248, 256)


def _fusable(a, dtype) -> bool:
    """The captured step may fuse the layer glue: stock adapter hooks, HF RMSNorms
    (weight + variance_epsilon), a SiLU-gated MLP, a 16-bit dtype."""
    if dtype not in (torch.bfloat16, torch.float16) or not isinstance(a, _HFDecoderAdapter):
        return False
    for name in ("apply_pre_attn_norm", "apply_pre_mlp_norm", "apply_post_attn_residual", "apply_post_mlp_residual",
                 "apply_rope", "get_mlp", "final_norm"):
        if getattr(type(a), name) is not getattr(_HFDecoderAdapter, name):
            return False

    def norm_ok(n):
        w = getattr(n, "weight", None)
        return (w is not None and hasattr(n, "variance_epsilon") and w.dim() == 1 and w.dtype == dtype
                and w.numel() % 8 == 0 and w.numel() <= 8192)

    for block in a.layers:
        mlp = block.mlp
        act = getattr(mlp, "act_fn", None)
        if not (norm_ok(block.input_layernorm) and norm_ok(block.post_attention_layernorm)
                and all(hasattr(mlp, n) for n in ("gate_proj", "up_proj", "down_proj"))
                and "silu" in type(act).__name__.lower()):
            return False
    return norm_ok(a.final_norm)


def _mergeable(a) -> bool:
    """Q/K/V and gate/up may run as one GEMM each: Llama projections (no
    QK-norm), bias-free linear layers."""
    from ..adapters.llama_adapter import LlamaAdapter

    if type(a).project_qkv is not LlamaAdapter.project_qkv:
        return False
    for block in a.layers:
        attn, mlp = block.self_attn, block.mlp
        for lin in (attn.q_proj, attn.k_proj, attn.v_proj, mlp.gate_proj, mlp.up_proj):
            if not isinstance(lin, torch.nn.Linear) or lin.bias is not None:
                return False
    return True


# How the captured Llama step gets its merged q/k/v and gate/up weights:
# "copy" (default): its own concatenated copies, the modules untouched; every
# step compares each module's weight (the tensor and its in-place version
# counter) with the one copied and refreshes the copy's rows in place when it
# changed (layers of the first graph before it starts, the others while it
# runs). "views": the modules' weights become views of one concatenated tensor
# per layer (no second copy; a rebound weight is merged again and the graphs
# captured again). "off": separate q/k/v and gate/up GEMMs.
MERGE_PROJECTIONS = "copy"

# "copy" mode also runs each layer's down projection split over the reduction:
# its weight is copied as SPLIT_DOWN column slices [S, F/S, H], the activation
# is written as the matching slices [S, nb, F/S], one batched product gives S
# fp32 partials [S, nb, H], and the next RMSNorm sums them and rounds once to
# the dtype (the value the un-split product stores, up to the fp32 summation
# order). At decode row counts the single [nb, F] x [F, H] product has too few
# output tiles to fill the device; S slices give S times as many. 0 or 1: off.
SPLIT_DOWN = 8


def _project(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """The step's product of rows x with a projection weight: linear for an
    [out, in] weight; for split slices w [S, F/S, H], x [rows, F/S] is taken
    as every slice's rows (the shape and cost of the split product)."""
    if w.dim() == 3:
        return torch.bmm(x.unsqueeze(0).expand(w.shape[0], -1, -1).contiguous(), w, out_dtype=torch.float32)
    return torch.nn.functional.linear(x, w)


def _split_copy(w: torch.Tensor, t: torch.Tensor) -> None:
    """w [S, F/S, H] = the linear weight t [H, F] as S slices of its transpose:
    w[s, f, h] = t[h, s * F/S + f]."""
    S, Fs, H = w.shape
    w.copy_(t.view(H, S, Fs).permute(1, 2, 0))


def _merge_linears(lins) -> torch.Tensor:
    """One weight [sum(out), in] for the bias-free linears ``lins``; each
    module's weight becomes a view of its rows ("views" mode)."""
    w = torch.cat([lin.weight.detach() for lin in lins], dim=0)
    off = 0
    for lin in lins:
        n = lin.weight.shape[0]
        lin.weight.data = w[off:off + n]
        off += n
    return w


# Layers in the first of a step's two captured graphs. The host plans those
# layers' appends, starts the first graph, and plans the other layers while it
# runs: their appends are read only by the second graph, whose inputs are
# copied in after the first graph in stream order. At Llama-3-8B size two layers
# of GPU work cover the other 30 layers' planning (one does not: 9.20 ms per
# step at 144 leaves against 9.07 for two and three).
SPLIT_LAYERS = 2

# Attention of the layers after the first graph runs the prefix-tree decode
# (mentat_tree_decode_counted): pages that forked leaves share are read once
# per group of leaves. Its plan is made while the first graph runs, by the
# native planner from the host copy of layer 0's tables (the sharing pattern
# is every layer's), and copied in before the second graph.
TREE_DECODE = True


def _tree_caps(nb: int, Hkv: int, max_len: int, G: int) -> tuple:
    """(max_shared, max_solo, max_slots) of a bucket's plan buffers. A plan
    without sharing (each query one segment, solo items of 4 tiles) needs at
    most nb * ceil(tiles / 4) * Hkv items and slots; a query cut into k
    segments adds at most k - 1 chunks, and k <= 9 is allowed before the
    planner falls back to that plan. Shared tasks (segments of at least
    min_q queries: SHARED_MIN_GROUPS groups of 16 / G) need one item per 32
    tiles per head per 32 queries."""
    tiles = -(-max_len // 16)
    solo = nb * (-(-tiles // tree_plan.CHUNK_TILES) + 8) * Hkv
    min_q = (tree_plan.SHARED_MIN_GROUPS - 1) * (16 // G) + 1
    shared = max(1, -(-nb // min_q)) * (-(-tiles // tree_plan.SHARED_CHUNK_TILES) + 2) * Hkv * 2
    return shared, solo, solo


class _Bucket:
    __slots__ = ("n", "graph", "graph2", "state", "dev", "host", "host_np", "logits", "hidden", "version",
                 "copied", "tree", "tree_read")


class DecodeGraphs:
    """Captured batched decode forwards for one PagedModelWrapper."""

    def __init__(self, wrapper, buckets=None):
        self.a = wrapper.adapter
        self.m = wrapper.kv_cache_mgr
        self.dev = wrapper.device
        self._graphs: dict[int, _Bucket] = {}
        self._stream = torch.cuda.Stream(self.dev)
        self._copy_stream = torch.cuda.Stream(self.dev)  # tree plan copies, overlapping the first graph
        self._ws = None
        self.captures = 0
        self._warm_full = True   # the next capture warms up with the whole forward
        self.fused = _fusable(self.a, self.m.dtype)
        self.merge_mode = MERGE_PROJECTIONS
        self.merged = self.fused and self.merge_mode in ("copy", "views") and _mergeable(self.a)
        self._w_qkv: list = []
        self._w_gu: list = []
        self._w_src: list = []   # "copy": per layer [module params dict, tensor, data_ptr, version, merged, row]
        self._w_down: list = []  # "copy" with SPLIT_DOWN > 1: per layer down weight as [S, F/S, H]
        if self.merged:
            self._merge()
        Hq, Hkv = self.a.num_attention_heads, self.a.num_key_value_heads
        self.G = Hq // Hkv if Hq % Hkv == 0 else 0
        self.tree = bool(TREE_DECODE and self.m.layout == LAYOUT_NATIVE and self.G and 16 % self.G == 0)
        self.tree_steps = 0       # steps whose plan shared pages
        self.tree_fallbacks = 0   # steps planned without sharing (a capacity was exceeded)
        self.bucket_costs: dict = {}
        if buckets is None and os.environ.get("MENTAT_CALIBRATE_BUCKETS", "") == "1":
            buckets = "calibrate"
        if isinstance(buckets, str):
            if buckets != "calibrate":
                raise ValueError(f"buckets must be row counts or 'calibrate', got {buckets!r}")
            buckets = self.calibrate_buckets()
        elif buckets is None:
            buckets = MERGED_BUCKETS if self.merged else BUCKETS
        self.buckets = tuple(sorted(buckets))
        self.max_batch = self.buckets[-1]

    def _projection_weights(self) -> list:
        """The weights of the step's projection GEMMs, in step order: per layer
        q/k/v (merged when the step merges them), o, gate/up (likewise) and
        down (its [S, F/S, H] slices when the step splits it), then the LM head."""
        a = self.a
        mats = []
        for i, b in enumerate(a.layers):
            attn, mlp = a.get_self_attn(b), a.get_mlp(b)
            if self.merged:
                down = self._w_down[i] if self._w_down else mlp.down_proj.weight
                mats += [self._w_qkv[i], attn.o_proj.weight, self._w_gu[i], down]
            else:
                mats += [attn.q_proj.weight, attn.k_proj.weight, attn.v_proj.weight, attn.o_proj.weight,
                         mlp.gate_proj.weight, mlp.up_proj.weight, mlp.down_proj.weight]
        mats.append(a.lm_head.weight)
        return mats

    @torch.no_grad()
    def _warm_gemms(self, nb: int) -> None:
        """One call of each distinct projection GEMM shape at nb rows: the GEMM
        library picks (and loads) its kernels for these shapes outside capture."""
        seen = set()
        for w in self._projection_weights():
            key = (tuple(w.shape), w.dtype)
            if key not in seen:
                seen.add(key)
                _project(torch.zeros(nb, w.shape[-2 if w.dim() == 3 else 1], dtype=w.dtype, device=self.dev), w)

    @torch.no_grad()
    def calibrate_buckets(self, max_batch: int = 256, step: int = 8, reps: int = 3, tol: float = 0.01) -> tuple:
        """A bucket table measured on this device for this model. The step's
        projection GEMMs as the captured step runs them (merged q/k/v and
        gate/up when it merges them, o and down, every layer, and the LM head)
        are timed at each multiple of ``step`` rows up to ``max_batch``; a row
        count is kept unless some larger one costs at most (1 + tol) times as
        much (a batch then runs in that larger bucket at about the same cost).
        BUCKETS / MERGED_BUCKETS were found this way on one MI355X; the GEMM
        library's kernel choice, and with it the cheap row counts, can differ
        with the device and the library version. The timings stay in
        ``bucket_costs`` (ms per step's projections, by row count)."""
        mats = self._projection_weights()
        g = torch.Generator(device=self.dev).manual_seed(0)
        xs = {}
        for w in mats:
            k = w.shape[-2] if w.dim() == 3 else w.shape[1]
            if k not in xs:
                xs[k] = torch.randn(max_batch, k, generator=g, device=self.dev).to(w.dtype)

        def projections(r):
            for w in mats:
                _project(xs[w.shape[-2] if w.dim() == 3 else w.shape[1]][:r], w)

        cost = {}
        for r in range(step, max_batch + 1, step):
            projections(r)   # the library's first call at a shape picks its kernel
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record()
            for _ in range(reps):
                projections(r)
            t1.record()
            t1.synchronize()
            cost[r] = t0.elapsed_time(t1) / reps
        rs = sorted(cost)
        keep = tuple(r for i, r in enumerate(rs) if all(cost[r2] > (1 + tol) * cost[r] for r2 in rs[i + 1:]))
        self.bucket_costs = cost
        return keep

    def _merge(self) -> None:
        groups = lambda b: ((b.self_attn.q_proj, b.self_attn.k_proj, b.self_attn.v_proj),  # noqa: E731
                            (b.mlp.gate_proj, b.mlp.up_proj))
        with torch.no_grad():
            if self.merge_mode == "views":
                self._w_qkv = [_merge_linears(groups(b)[0]) for b in self.a.layers]
                self._w_gu = [_merge_linears(groups(b)[1]) for b in self.a.layers]
                return
            self._w_qkv, self._w_gu, self._w_src, self._w_down = [], [], [], []
            S = SPLIT_DOWN
            split = S > 1 and all(
                isinstance(b.mlp.down_proj, torch.nn.Linear) and b.mlp.down_proj.bias is None
                and b.mlp.down_proj.weight.shape[1] % (8 * S) == 0 for b in self.a.layers)
            for b in self.a.layers:
                recs = []
                if split:
                    t = b.mlp.down_proj._parameters["weight"]
                    w = torch.empty(S, t.shape[1] // S, t.shape[0], dtype=t.dtype, device=t.device)
                    _split_copy(w, t.detach())
                    self._w_down.append(w)
                    recs.append([b.mlp.down_proj._parameters, t, t.data_ptr(), t._version, w, None])
                for lins, dst in zip(groups(b), (self._w_qkv, self._w_gu)):
                    w = torch.cat([lin.weight.detach() for lin in lins], dim=0)
                    dst.append(w)
                    row = 0
                    for lin in lins:
                        t = lin._parameters["weight"]
                        recs.append([lin._parameters, t, t.data_ptr(), t._version, w, row])
                        row += t.shape[0]
                self._w_src.append(recs)

    def _merged_current(self) -> bool:
        """The merged weights can serve this step: "copy" always (they are
        refreshed); "views": the modules' weights still view the merged tensors
        (first and last layer)."""
        if self.merge_mode != "views":
            return True
        layers = self.a.layers
        for i in (0, len(layers) - 1):
            b = layers[i]
            if (b.self_attn.q_proj.weight.data_ptr() != self._w_qkv[i].data_ptr()
                    or b.mlp.gate_proj.weight.data_ptr() != self._w_gu[i].data_ptr()):
                return False
        return True

    def _refresh(self, lo: int, hi: int) -> None:
        """"copy" mode: layers lo .. hi - 1 of the merged copies take the rows of
        any module weight rebound or changed in place since it was copied (in
        stream order, before the graph that reads them). A weight whose shape
        changed cannot be copied in place: ValueError."""
        if not self._w_src:
            return
        for recs in self._w_src[lo:hi]:
            for r in recs:
                t = r[0]["weight"]
                if t is r[1] and t._version == r[3] and t.data_ptr() == r[2]:
                    continue
                w, row = r[4], r[5]
                if row is None:   # a split down projection weight
                    if t.shape != r[1].shape or t.dtype != w.dtype:
                        raise ValueError("DecodeGraphs: a split projection weight changed shape or dtype")
                    with torch.no_grad():
                        _split_copy(w, t.detach())
                    r[1], r[2], r[3] = t, t.data_ptr(), t._version
                    continue
                if t.shape[0] != r[1].shape[0] or t.shape[1:] != w.shape[1:] or t.dtype != w.dtype:
                    raise ValueError("DecodeGraphs: a merged projection weight changed shape or dtype")
                with torch.no_grad():
                    w[row:row + t.shape[0]].copy_(t.detach())
                r[1], r[2], r[3] = t, t.data_ptr(), t._version

    # ------------------------------------------------------------------
    def bucket(self, n: int):
        for b in self.buckets:
            if b >= n:
                return b
        return None

    def prepare(self, max_batch: int, max_len: int, rows: int = 0) -> None:
        """Reserve table capacity for sequences of up to ``max_len`` tokens and
        ``rows`` more live sequences, and capture every bucket up to the one
        that holds ``max_batch``."""
        m = self.m
        m.reserve(rows, -(-max_len // m.block_size))
        top = self.bucket(min(max_batch, self.max_batch))
        gc.collect()   # once for all of them (a full collection costs ~0.1 s at Llama-8B size)
        for b in self.buckets:
            if b <= top:
                self._get(b, collect=False)

    # ------------------------------------------------------------------
    def _inputs_layout(self, nb: int):
        L = self.m.num_layers
        return 3 * nb + L * 7 * nb

    def _fill_padding(self, h: np.ndarray, nb: int, n: int) -> None:
        """Entries n..nb-1 of every field become padding."""
        L = self.m.num_layers
        h[n:nb] = 0                        # token ids
        h[nb + n: 2 * nb] = 0              # positions
        h[2 * nb + n: 3 * nb] = self.m.empty_row()
        plans = h[3 * nb:].reshape(L, 7, nb)
        plans[:, :, n:] = -1               # dst block -1: skipped by the append kernel
        plans[:, 6, n:] = 0

    def _attention(self, q: torch.Tensor, layer_idx: int, rows: torch.Tensor, max_seqlen: int, tree):
        """One layer's decode attention of the step: the prefix-tree decode from
        the layer the tree plan is ready for, the paged decode before it."""
        m = self.m
        if tree is not None and layer_idx >= self._tree_from():
            return ops.tree_decode_counted(q, m._k_store, m._v_store, block_tables=m._tables[layer_idx], bufs=tree)
        return ops.paged_decode(q, m._k_store, m._v_store, layout=m.layout, block_tables=m._tables[layer_idx],
                                seq_lens=m._lens[layer_idx], seq_rows=rows, max_seqlen=max_seqlen)

    def _tree_from(self) -> int:
        """First layer on the tree decode: the second graph's (its plan is made
        while the first runs), or layer 0 with one graph per step."""
        return self._split_layers()

    def _forward(self, buf: torch.Tensor, nb: int, lo: int = 0, hi=None, state=None, tree=None):
        """Layers lo .. hi - 1 of the step (all by default). The first range
        starts from the embeddings; a range that ends before the last layer
        returns the state the next range starts from, the last one returns
        (logits, final hidden)."""
        if self.fused:
            return self._forward_fused(buf, nb, lo, hi, state, tree)
        a, m = self.a, self.m
        L = m.num_layers
        hi = L if hi is None else hi
        ids = buf[0:nb].long().unsqueeze(0)            # [1, nb]
        pos = buf[nb:2 * nb].long().unsqueeze(1)       # [nb, 1]
        rows = buf[2 * nb:3 * nb]                      # [nb] int32
        plans = buf[3 * nb:].view(L, 7, nb)
        max_seqlen = m._pages_cap * m.block_size
        hidden = a.embeddings(ids) if lo == 0 else state
        for layer_idx in range(lo, hi):
            block = a.layers[layer_idx]
            attn = a.get_self_attn(block)
            residual = hidden
            x = a.apply_pre_attn_norm(block, hidden)
            hs = x.squeeze(0).unsqueeze(1)             # [nb, 1, hidden]: one token per sequence
            q, k, v = a.project_qkv(attn, hs)
            q, k = a.apply_rope(attn, q, k, pos, v_for_shape=v)
            ops.kv_append(k.squeeze(1).to(m.dtype).contiguous(), v.squeeze(1).to(m.dtype).contiguous(),
                          m._k_store, m._v_store, plans[layer_idx], block_size=m.block_size, layout=m.layout,
                          block_tables=m._tables[layer_idx], seq_lens=m._lens[layer_idx])
            o = self._attention(q.squeeze(1).contiguous(), layer_idx, rows, max_seqlen, tree)
            attn_out = attn.o_proj(o.reshape(1, nb, -1))
            hidden = a.apply_post_attn_residual(block, residual, attn_out)
            residual = hidden
            x = a.apply_pre_mlp_norm(block, hidden)
            hidden = a.apply_post_mlp_residual(block, residual, a.get_mlp(block)(x))
        if hi < L:
            return hidden
        hidden = a.final_norm(hidden).squeeze(0)
        return a.lm_head(hidden), hidden

    def _forward_fused(self, buf: torch.Tensor, nb: int, lo: int = 0, hi=None, state=None, tree=None):
        """_forward with the layer glue fused (see the module docstring); the
        state between layer ranges is (normalised input, residual stream)."""
        a, m = self.a, self.m
        L = m.num_layers
        hi = L if hi is None else hi
        ids = buf[0:nb].long().unsqueeze(0)
        pos = buf[nb:2 * nb].long().unsqueeze(1)
        rows = buf[2 * nb:3 * nb]
        plans = buf[3 * nb:].view(L, 7, nb)
        max_seqlen = m._pages_cap * m.block_size
        layers = a.layers
        if lo == 0:
            hidden = a.embeddings(ids)                 # [1, nb, H]: the residual stream
            ln = layers[0].input_layernorm
            x, _ = ops.rmsnorm(hidden, ln.weight, ln.variance_epsilon)
        else:
            x, hidden = state
        Hq, Hk = a.num_attention_heads, a.num_key_value_heads
        for layer_idx in range(lo, hi):
            block = layers[layer_idx]
            attn = a.get_self_attn(block)
            if self.merged and m.dtype == x.dtype:
                qkv = torch.nn.functional.linear(x, self._w_qkv[layer_idx])  # [1, nb, (Hq + 2 Hk) * D]
                cos, sin = a._build_cos_sin(pos, qkv)
                # RoPE of q and k with k and v written straight into the pages
                q = ops.rope_qkv_append(qkv, Hq, Hk, cos, sin, m._k_store, m._v_store, plans[layer_idx],
                                        block_size=m.block_size, layout=m.layout,
                                        block_tables=m._tables[layer_idx], seq_lens=m._lens[layer_idx])
            else:
                if self.merged:
                    qkv = torch.nn.functional.linear(x, self._w_qkv[layer_idx])
                    cos, sin = a._build_cos_sin(pos, qkv)
                    q, k, v = ops.rope_qkv(qkv, Hq, Hk, cos, sin)           # dense [nb, H, D]
                else:
                    q, k, v = a.project_qkv(attn, x.squeeze(0).unsqueeze(1))  # one token per sequence
                    cos, sin = a._build_cos_sin(pos, q)
                    q, k = q.contiguous(), k.contiguous()
                    ops.rope_(q, k, cos, sin)
                    q, k, v = q.squeeze(1), k.squeeze(1), v.squeeze(1)
                ops.kv_append(k.to(m.dtype).contiguous(), v.to(m.dtype).contiguous(),
                              m._k_store, m._v_store, plans[layer_idx], block_size=m.block_size, layout=m.layout,
                              block_tables=m._tables[layer_idx], seq_lens=m._lens[layer_idx])
            o = self._attention(q.contiguous(), layer_idx, rows, max_seqlen, tree)
            attn_out = attn.o_proj(o.reshape(1, nb, -1))
            ln = block.post_attention_layernorm
            x, hidden = ops.rmsnorm(attn_out, ln.weight, ln.variance_epsilon, residual=hidden)
            mlp = block.mlp
            if self._w_down:
                gu = torch.nn.functional.linear(x, self._w_gu[layer_idx])
                w_down = self._w_down[layer_idx]
                act = ops.silu_mul_merged_split(gu.view(nb, -1), w_down.shape[0])  # [S, nb, F/S]
                parts = torch.bmm(act, w_down, out_dtype=torch.float32)           # [S, nb, H]
                ln = layers[layer_idx + 1].input_layernorm if layer_idx + 1 < L else a.final_norm
                x, hidden = ops.rmsnorm_partials(parts, ln.weight, ln.variance_epsilon,
                                                 residual=hidden.view(nb, -1))
                x, hidden = x.view(1, nb, -1), hidden.view(1, nb, -1)
                continue
            if self.merged:
                act = ops.silu_mul_merged(torch.nn.functional.linear(x, self._w_gu[layer_idx]))
            else:
                act = ops.silu_mul(mlp.gate_proj(x), mlp.up_proj(x))
            mlp_out = mlp.down_proj(act)
            ln = layers[layer_idx + 1].input_layernorm if layer_idx + 1 < L else a.final_norm
            x, hidden = ops.rmsnorm(mlp_out, ln.weight, ln.variance_epsilon, residual=hidden)
        if hi < L:
            return x, hidden
        x = x.squeeze(0)
        return a.lm_head(x), x

    def _workspace(self) -> None:
        """Size the capture stream's decode workspace for the largest bucket
        (paged decode, and the tree decode's partial slots). It only grows when
        the tables have grown, and then every graph is captured again."""
        a, m = self.a, self.m
        lib = get_lib()
        Hq, Hkv, D = a.num_attention_heads, a.num_key_value_heads, a.head_dim
        nbytes = lib.mentat_paged_decode_workspace_bytes(m.layout, self.max_batch, Hq, Hkv, D, m.block_size,
                                                         m._pages_cap * m.block_size, 0, 0)
        if self.tree:
            slots = _tree_caps(self.max_batch, Hkv, m._pages_cap * m.block_size, self.G)[2]
            nbytes = max(nbytes, lib.mentat_tree_decode_workspace_bytes(slots, Hq, Hkv, D))
        if self._ws is not None and self._ws.numel() >= nbytes:
            return
        with torch.cuda.stream(self._stream):
            self._ws = ops.workspace(self.dev, nbytes)

    def _get(self, nb: int, collect: bool = True) -> _Bucket:
        b = self._graphs.get(nb)
        if b is not None and b.version == self.m.tables_version:
            return b
        self._graphs.pop(nb, None)
        self._workspace()
        m = self.m
        size = self._inputs_layout(nb)
        b = _Bucket()
        b.n = nb
        b.host = torch.empty(size, dtype=torch.int32, pin_memory=True)
        b.host_np = b.host.numpy()
        self._fill_padding(b.host_np, nb, 0)
        b.dev = torch.empty(size, dtype=torch.int32, device=self.dev)
        b.dev.copy_(b.host)
        b.tree = None
        if self.tree:  # zero-filled: no items, every query's output zero, until a plan is written
            caps = _tree_caps(nb, self.a.num_key_value_heads, m._pages_cap * m.block_size, self.G)
            b.tree = ops.TreePlanBuffers(self.dev, nb, self.a.num_key_value_heads, *caps)
            # recorded after each replay of the graph that reads the plan: the
            # next plan's copy waits for it
            b.tree_read = torch.cuda.Event()
            b.tree_read.record(torch.cuda.current_stream(self.dev))
        # Recorded after each step's last copy out of b.host: the next step waits
        # for it before it rewrites the pinned staging.
        b.copied = torch.cuda.Event()
        b.copied.record(torch.cuda.current_stream(self.dev))
        s = self._stream
        s.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(s):
            # Warm-up outside capture on all-padding input. The first capture runs
            # the whole forward (library handles, every kernel's first launch);
            # later ones only meet new GEMM shapes (every other kernel of the
            # step runs the same code at any batch size), so they warm the
            # projection GEMMs at this row count.
            # (The GEMM-only warm-up needs the fused step's HF module layout.)
            if self._warm_full or not self.fused:
                self._forward(b.dev, nb, tree=b.tree)
            else:
                self._warm_gemms(nb)
        torch.cuda.current_stream(self.dev).wait_stream(s)
        g = torch.cuda.CUDAGraph()
        g2 = None
        k = self._split_layers()
        gc_on = gc.isenabled()
        if collect:
            gc.collect()
        gc.disable()
        try:
            if k:
                with torch.cuda.graph(g, stream=s):
                    b.state = self._forward(b.dev, nb, 0, k, tree=b.tree)
                g2 = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g2, pool=g.pool(), stream=s):
                    b.logits, b.hidden = self._forward(b.dev, nb, k, None, b.state, tree=b.tree)
            else:
                b.state = None
                with torch.cuda.graph(g, stream=s):
                    b.logits, b.hidden = self._forward(b.dev, nb, tree=b.tree)
        finally:
            if gc_on:
                gc.enable()
        torch.cuda.current_stream(self.dev).wait_stream(s)
        b.graph, b.graph2 = g, g2
        self._warm_full = False
        b.version = m.tables_version
        self._graphs[nb] = b
        self.captures += 1
        return b

    # ------------------------------------------------------------------
    def decode(self, token_ids: list[int], seq_ids: list[int]):
        """The step of PagedModelWrapper.decode_batch_tensor: (logits [N, V],
        final hidden [N, hidden]); returns None when N exceeds the largest
        bucket (the caller runs the eager step)."""
        n = len(seq_ids)
        nb = self.bucket(n)
        if nb is None:
            return None
        if self.merged and not self._merged_current():
            self._merge()           # ("views") weights were rebound: merge again, capture again
            self._graphs.clear()
        m = self.m
        L = m.num_layers
        k = self._split_layers()
        st = m.plan_append_step_begin(seq_ids, max(k, 1))
        p0 = st["plan"][0]   # layer 0's plan: table rows, and lengths after the append
        rows = p0[3]
        lens = p0[5]
        # Overlap the later layers' planning with the first graph only when every
        # layer's counters agree: then every layer's new token lands on the same
        # page index, so the first layers' plan decides the table capacity.
        overlap = bool(k) and st.get("uniform", False)
        plan = st["plan"] if overlap else m.plan_append_step_finish(st)   # [L, 7, n]
        m._ensure_pages(int(plan[:max(k, 1) if overlap else L, 4].max()) + 1)
        b = self._get(nb)
        # The previous step's non-blocking copies read b.host when the stream
        # reaches them; a caller that queues steps without a host sync could
        # otherwise overwrite its plans before they are read.
        b.copied.synchronize()
        h = b.host_np
        plans_h = h[3 * nb:].reshape(L, 7, nb)
        h[0:n] = token_ids
        h[nb:nb + n] = lens - 1   # RoPE positions: lengths before the append
        h[2 * nb:2 * nb + n] = rows
        self._fill_padding(h, nb, n)
        if overlap:
            cut = 3 * nb + k * 7 * nb
            plans_h[:k, :, :n] = plan[:k]
            b.dev[:cut].copy_(b.host[:cut], non_blocking=True)
            self._refresh(0, k)
            b.graph.replay()
            # while the first graph runs: the tree plan (layer 0's tables are
            # final), the later layers' appends and merged weights
            self._plan_tree(b, rows, lens)
            plan = m.plan_append_step_finish(st)
            self._refresh(k, L)
            if int(plan[k:, 4].max()) >= m._pages_cap:
                raise RuntimeError("DecodeGraphs: a later layer's append needs more table pages than the first")
            plans_h[k:, :, :n] = plan[k:]
            b.dev[cut:].copy_(b.host[cut:], non_blocking=True)
            b.copied.record()
            b.graph2.replay()
            if b.tree is not None:
                b.tree_read.record()
        else:
            plans_h[:, :, :n] = plan
            b.dev.copy_(b.host, non_blocking=True)
            self._plan_tree(b, rows, lens)
            b.copied.record()
            self._refresh(0, L)
            b.graph.replay()
            if b.graph2 is not None:
                b.graph2.replay()
            if b.tree is not None:
                b.tree_read.record()
        return b.logits[:n].clone(), b.hidden[:n].clone()

    def _plan_tree(self, b: _Bucket, rows: np.ndarray, lens: np.ndarray) -> None:
        """The step's prefix-tree plan (after layer 0's appends are planned:
        the tables and lengths attention reads; rows and lens are the batch's
        table rows and lengths after the append) into the bucket's buffers,
        and their copy to the device queued."""
        if b.tree is None:
            return
        m = self.m
        _, _, _, shared = b.tree.plan(m.host_tables0(), rows, lens, m.block_size, self.G)
        if shared:
            self.tree_steps += 1
        else:
            self.tree_fallbacks += 1
        # The copies run on a side stream beside the first graph, once the
        # previous replay has read the device plan; the step's stream waits for
        # them before its next work (the later layers' copy and the second
        # graph), so the staging event recorded after that covers them too.
        main = torch.cuda.current_stream(self.dev)
        cs = self._copy_stream
        cs.wait_event(b.tree_read)
        with torch.cuda.stream(cs):
            b.tree.upload()
        main.wait_stream(cs)

    def _split_layers(self) -> int:
        """Layers of the first graph (0: one graph for the whole step)."""
        L = self.m.num_layers
        return SPLIT_LAYERS if 0 < SPLIT_LAYERS < L else 0
