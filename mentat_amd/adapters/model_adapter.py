"""ModelAdapter: the per-model-family interface of the paged pipeline.

Drop-in for the reference's adapters/model_adapter.py: the same abstract
methods (get_self_attn, get_mlp, apply_pre_attn_norm, apply_pre_mlp_norm,
project_qkv, apply_rope), structural accessors, geometry helpers and the
three high-level ops PagedModelWrapper calls (forward_paged_prefill,
project_kv_for_cache, forward_paged_decode), adapters/model_adapter.py:39-341.

Decode differences from the reference, same results:
  * project_kv_for_cache projects Q, K and V once and keeps the rotated Q
    for the forward_paged_decode call that follows on the same input (the
    reference projects Q, K and V twice per layer);
  * position-id tensors are built once per step, not once per layer;
  * build_packed_kv hands zero-copy paged views to attn_decode.
"""
from __future__ import annotations

import abc
from typing import Optional

import torch

from .attention_backend import BACKEND, attn_decode, attn_prefill  # noqa: F401


class ModelAdapter(abc.ABC):
    def __init__(self, model):
        self.model = model
        self.config = model.config
        p = next(model.parameters())
        self.device = p.device
        self.dtype = p.dtype
        self._embeddings = None
        self._layers = None
        self._final_norm = None
        self._lm_head = None
        self._pos_cache: tuple = (None, None)
        self._pending_q: Optional[tuple] = None

    # ---- structure (reference :66-80) ----
    @property
    def embeddings(self) -> torch.nn.Module:
        return self._embeddings

    @property
    def layers(self) -> torch.nn.ModuleList:
        return self._layers

    @property
    def final_norm(self) -> torch.nn.Module:
        return self._final_norm

    @property
    def lm_head(self) -> torch.nn.Module:
        return self._lm_head

    @abc.abstractmethod
    def get_self_attn(self, layer) -> torch.nn.Module: ...

    @abc.abstractmethod
    def get_mlp(self, layer) -> torch.nn.Module: ...

    @abc.abstractmethod
    def apply_pre_attn_norm(self, layer, hidden: torch.Tensor) -> torch.Tensor: ...

    @abc.abstractmethod
    def apply_pre_mlp_norm(self, layer, hidden: torch.Tensor) -> torch.Tensor: ...

    def apply_post_attn_residual(self, layer, residual, attn_out):
        return residual + attn_out

    def apply_post_mlp_residual(self, layer, residual, mlp_out):
        return residual + mlp_out

    # ---- geometry (reference :115-143) ----
    @property
    def num_layers(self) -> int:
        return self.config.num_hidden_layers

    @property
    def num_attention_heads(self) -> int:
        return self.config.num_attention_heads

    @property
    def num_key_value_heads(self) -> int:
        return getattr(self.config, "num_key_value_heads", None) or self.num_attention_heads

    @property
    def num_hidden_layers(self) -> int:
        return getattr(self.config, "num_hidden_layers", None)

    @property
    def head_dim(self) -> int:
        return getattr(self.config, "head_dim", None) or self.config.hidden_size // self.num_attention_heads

    @property
    def hidden_size(self) -> int:
        return self.config.hidden_size

    # ---- projection + RoPE (reference :150-186) ----
    @abc.abstractmethod
    def project_qkv(self, attn, hidden_states: torch.Tensor):
        """hidden (batch, seq, hidden) -> Q, K, V (batch, seq, heads, head_dim), QK-norms
        included, RoPE not applied."""

    @abc.abstractmethod
    def apply_rope(self, attn, q, k, position_ids, v_for_shape=None):
        """Rotate q and/or k (batch, seq, heads, dim) at position_ids (batch, seq)."""

    # ---- attention wrappers (reference :192-224) ----
    def flash_prefill(self, q, k, v, window_size=None):
        return attn_prefill(q, k, v, window_size)

    def flash_decode(self, q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_k, N, window_size=None):
        return attn_decode(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_k, N, window_size)

    # ---- helpers ----
    def _positions(self, seqlen_offsets, device) -> torch.Tensor:
        """(N, 1) long positions; one host-to-device copy per distinct offset list."""
        key = tuple(int(x) for x in seqlen_offsets)
        if self._pos_cache[0] != key:
            self._pos_cache = (key, torch.tensor(key, dtype=torch.long).to(device).unsqueeze(1))
        return self._pos_cache[1]

    # ---- high-level ops (reference :226-341) ----
    def forward_paged_prefill(self, attn, hidden_states, layer_idx, window_size=None):
        """(1, S, hidden) -> attn_output (1, S, hidden), k_new / v_new (S, Hkv, D) post-RoPE."""
        _, seq_len, _ = hidden_states.size()
        q, k, v = self.project_qkv(attn, hidden_states)
        pp = getattr(self, "_prefill_pos", None)
        if pp is None or pp.shape[1] != seq_len or pp.device != q.device:
            pp = torch.arange(seq_len, device=q.device, dtype=torch.long).unsqueeze(0)
            self._prefill_pos = pp
        pos = pp
        q, k = self.apply_rope(attn, q, k, pos, v_for_shape=v)
        o = self.flash_prefill(q, k, v, window_size)
        o = attn.o_proj(o.reshape(1, seq_len, -1))
        return o, k[0], v[0]

    def project_kv_for_cache(self, attn, hidden_states, seqlen_offsets):
        """(1, N, hidden) -> post-RoPE K and V (N, Hkv, D) for the N new tokens."""
        hs = hidden_states.squeeze(0).unsqueeze(1)  # (N, 1, hidden): one token per sequence
        q, k, v = self.project_qkv(attn, hs)
        pos = self._positions(seqlen_offsets, k.device)
        q, k = self.apply_rope(attn, q, k, pos, v_for_shape=v)
        self._pending_q = (id(attn), hidden_states.data_ptr(), hidden_states._version,
                           tuple(hidden_states.shape), q.squeeze(1))
        return k.squeeze(1), v.squeeze(1)

    def _decode_query(self, attn, hidden_states, seqlen_offsets):
        pend = self._pending_q
        self._pending_q = None
        if pend is not None and pend[:4] == (id(attn), hidden_states.data_ptr(), hidden_states._version,
                                             tuple(hidden_states.shape)):
            return pend[4]
        hs = hidden_states.squeeze(0).unsqueeze(1)
        q, _, _ = self.project_qkv(attn, hs)
        pos = self._positions(seqlen_offsets, q.device)
        q, _ = self.apply_rope(attn, q, None, pos, v_for_shape=q)
        return q.squeeze(1)

    def forward_paged_decode(self, attn, hidden_states, kv_cache_mgr, seq_ids, seqlen_offsets, layer_idx,
                             window_size=None, cached_gather_indices=None):
        """(1, N, hidden) -> attention output (1, N, hidden) over each sequence's cache."""
        N = len(seq_ids)
        _, total_q, _ = hidden_states.size()
        q = self._decode_query(attn, hidden_states, seqlen_offsets)  # (N, Hq, D)
        pk, pv, cu_k, max_k = kv_cache_mgr.build_packed_kv(seq_ids, layer_idx,
                                                           cached_metadata=cached_gather_indices)
        cu_q = torch.arange(0, N + 1, device=q.device, dtype=torch.int32)
        o = self.flash_decode(q, pk, pv, cu_q, cu_k, max_k, N, window_size)
        return attn.o_proj(o.unsqueeze(0).reshape(1, total_q, -1))


def rotate_half(t: torch.Tensor) -> torch.Tensor:
    h = t.shape[-1] // 2
    return torch.cat((-t[..., h:], t[..., :h]), dim=-1)


class _HFDecoderAdapter(ModelAdapter):
    """Shared body of the Llama and Qwen3 adapters (HF layout: model.model.{embed_tokens,
    rotary_emb, layers, norm}, model.lm_head; RoPE from the model-level rotary_emb
    in the model dtype, applied with rotate_half)."""

    def __init__(self, model):
        super().__init__(model)
        base = model.model if hasattr(model, "model") else model
        self._embeddings = base.embed_tokens
        self._layers = base.layers
        self._final_norm = base.norm
        self._lm_head = model.lm_head
        self._rotary_emb = base.rotary_emb

    def get_self_attn(self, layer):
        return layer.self_attn

    def get_mlp(self, layer):
        return layer.mlp

    def apply_pre_attn_norm(self, layer, hidden):
        return layer.input_layernorm(hidden)

    def apply_pre_mlp_norm(self, layer, hidden):
        return layer.post_attention_layernorm(hidden)

    def _build_cos_sin(self, position_ids, ref):
        # Every layer of a decode step rotates at the same positions (the same
        # tensor object from _positions): compute cos/sin once per step. The
        # cache holds the position tensor itself, so identity is reliable.
        c = getattr(self, "_cs_cache", None)
        if (c is not None and c[0] is position_ids and c[1] == position_ids._version
                and c[2] == ref.dtype and c[3] == ref.device):
            return c[4], c[5]
        cos, sin = self._rotary_emb(ref, position_ids)
        cos, sin = cos.unsqueeze(2), sin.unsqueeze(2)
        self._cs_cache = (position_ids, position_ids._version, ref.dtype, ref.device, cos, sin)
        return cos, sin

    @staticmethod
    def _apply_cos_sin(t, cos, sin):
        return t * cos + rotate_half(t) * sin

    def apply_rope(self, attn, q, k, position_ids, v_for_shape=None):
        ref = q if q is not None else (k if k is not None else v_for_shape)
        cos, sin = self._build_cos_sin(position_ids, ref)
        q_rot = self._apply_cos_sin(q, cos, sin) if q is not None else None
        k_rot = self._apply_cos_sin(k, cos, sin) if k is not None else None
        return q_rot, k_rot
