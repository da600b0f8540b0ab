"""Qwen3 adapter (Qwen3ForCausalLM) — drop-in for adapters/qwen3_adapter.py.

As Llama, plus the unconditional per-head RMSNorm q_norm / k_norm applied to Q
and K before RoPE (adapters/qwen3_adapter.py:76-93); K is cached post-norm,
post-RoPE.
"""
from __future__ import annotations

from .model_adapter import _HFDecoderAdapter


class Qwen3Adapter(_HFDecoderAdapter):
    def project_qkv(self, attn, hidden_states):
        b, s, _ = hidden_states.shape
        d = self.head_dim
        q = attn.q_norm(attn.q_proj(hidden_states).view(b, s, -1, d))
        k = attn.k_norm(attn.k_proj(hidden_states).view(b, s, -1, d))
        v = attn.v_proj(hidden_states).view(b, s, -1, d)
        return q, k, v
