"""Llama adapter (LlamaForCausalLM / Llama-3.x) — drop-in for adapters/llama_adapter.py.

Q/K/V projections reshaped to (batch, seq, heads, head_dim), no QK-norm, RoPE
from the model-level rotary_emb in the model dtype (adapters/llama_adapter.py:70-113);
K is cached post-RoPE.
"""
from __future__ import annotations

from .model_adapter import _HFDecoderAdapter


class LlamaAdapter(_HFDecoderAdapter):
    def project_qkv(self, attn, hidden_states):
        b, s, _ = hidden_states.shape
        d = self.head_dim
        q = attn.q_proj(hidden_states).view(b, s, -1, d)
        k = attn.k_proj(hidden_states).view(b, s, -1, d)
        v = attn.v_proj(hidden_states).view(b, s, -1, d)
        return q, k, v
