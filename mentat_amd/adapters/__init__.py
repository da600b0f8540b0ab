"""Model adapters and the attention backend (same module names as the reference's adapters/)."""
from .adapter_factory import LlamaAdapter, ModelAdapter, Qwen3Adapter, get_adapter, register_adapter
from .attention_backend import BACKEND, attn_decode, attn_prefill

__all__ = ["BACKEND", "attn_prefill", "attn_decode", "ModelAdapter", "LlamaAdapter", "Qwen3Adapter",
           "get_adapter", "register_adapter"]
