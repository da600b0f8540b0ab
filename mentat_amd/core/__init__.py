"""Paged KV cache, prefix tree and generator (same module names as the reference's core/)."""
