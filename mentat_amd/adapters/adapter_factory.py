"""Adapter registry — drop-in for adapters/adapter_factory.py (:7-52).

get_adapter(model) matches config.model_type against the registry, then falls
back to the class name ("qwen"/"qwen3" -> Qwen3, "llama" -> Llama), and raises
NotImplementedError otherwise; register_adapter(model_type, cls) adds a family.
"""
from __future__ import annotations

from .llama_adapter import LlamaAdapter
from .model_adapter import ModelAdapter
from .qwen3_adapter import Qwen3Adapter

__all__ = ["ModelAdapter", "LlamaAdapter", "Qwen3Adapter", "get_adapter", "register_adapter"]

_ADAPTER_REGISTRY: dict[str, type] = {
    "qwen3": Qwen3Adapter,
    "llama": LlamaAdapter,
}


def get_adapter(model) -> ModelAdapter:
    model_type = (getattr(model.config, "model_type", "") or "").lower()
    if model_type in _ADAPTER_REGISTRY:
        return _ADAPTER_REGISTRY[model_type](model)
    cls = type(model).__name__.lower()
    if "qwen" in cls:
        return Qwen3Adapter(model)
    if "llama" in cls:
        return LlamaAdapter(model)
    raise NotImplementedError(
        f"No ModelAdapter registered for model_type={model_type!r} (class={type(model).__name__!r}). "
        f"Registered types: {sorted(_ADAPTER_REGISTRY)}. Add a ModelAdapter subclass and register it."
    )


def register_adapter(model_type: str, adapter_cls: type) -> None:
    _ADAPTER_REGISTRY[model_type.lower()] = adapter_cls
