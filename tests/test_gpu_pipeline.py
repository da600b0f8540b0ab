"""Paged pipeline (adapters + PagedKVCacheManager + HIP kernels) against the
model's own dense forward.

Prefill, fork into two children, then decode steps with different tokens per
child, through the drop-in API (PagedModelWrapper / ModelAdapter / attention
backend). After every step each sequence's logits must match HuggingFace's
forward over that sequence's full token history, computed on the CPU in
float32: within 2e-3 for fp32 models, within 5e-2 relative for bf16 models
(bf16 K/V cache and activations).
"""
import numpy as np
import pytest
import torch

from mentat_amd.adapters.adapter_factory import get_adapter
from mentat_amd.core.generator_utils import PagedModelWrapper
from mentat_amd.core.paged_kv_cache import PagedKVCacheManager

pytestmark = pytest.mark.gpu


def _model(kind):
    """A fresh seeded fp32 CPU model (identical weights on every call)."""
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen3Config, Qwen3ForCausalLM

    torch.manual_seed(1)
    common = dict(hidden_size=256, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                  vocab_size=1000, intermediate_size=512, max_position_embeddings=512, tie_word_embeddings=False)
    if kind == "qwen3":
        m = Qwen3ForCausalLM(Qwen3Config(**common))
    else:
        m = LlamaForCausalLM(LlamaConfig(**common))
    return m.float().eval()


@pytest.mark.parametrize("kind", ["qwen3", "llama"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("capture", [False, True])
def test_paged_decode_matches_dense_forward(gpu, kind, dtype, capture):
    """capture: decode steps as captured graphs; in bf16 / f16 these run the fused
    layer glue (Llama: merged q/k/v and gate/up projections too; Qwen3 keeps its
    QK-norm projections and takes the RoPE kernel on the split q/k)."""
    print(f"case pipeline {kind} {dtype} capture={capture}", flush=True)
    cpu_model = _model(kind)
    gpu_model = _model(kind).to(device="cuda", dtype=dtype)
    adapter = get_adapter(gpu_model)
    kv = PagedKVCacheManager(num_layers=2, num_key_value_heads=2, head_dim=64, max_blocks=256, block_size=16,
                             device="cuda", dtype=dtype)
    wrapper = PagedModelWrapper(gpu_model, kv, adapter)
    if capture:
        wrapper.enable_step_capture()
        assert wrapper.graphs.fused == (dtype != torch.float32)
        assert wrapper.graphs.merged == (dtype != torch.float32 and kind == "llama")
    rng = np.random.default_rng(0)
    prompt = rng.integers(0, 1000, 21).tolist()
    s0 = kv.allocate_sequence()
    with torch.no_grad():
        last = wrapper.prefill(torch.tensor([prompt], device="cuda"), s0)
    seqs = {s0: list(prompt)}
    tol = 2e-3 if dtype == torch.float32 else 5e-2

    def check(seq_ids, logits):
        for sid, lg in zip(seq_ids, logits):
            with torch.no_grad():
                want = cpu_model(torch.tensor([seqs[sid]])).logits[0, -1]
            got = lg.float().cpu()
            err = (got - want).abs().max().item() / max(1.0, want.abs().max().item())
            assert err < tol, (kind, dtype, sid, len(seqs[sid]), err)

    check([s0], [last])
    kids = [kv.fork_sequence(s0), kv.fork_sequence(s0)]
    kv.free_sequence(s0)
    for sid in kids:
        seqs[sid] = list(prompt)
    for step in range(5):
        toks = [int(x) for x in rng.integers(0, 1000, len(kids))]
        for sid, t in zip(kids, toks):
            seqs[sid].append(t)
        with torch.no_grad():
            logits, _ = wrapper.decode_batch(toks, kids)
        check(kids, logits)
        if step == 2:  # fork again mid-page, then keep decoding all three
            extra = kv.fork_sequence(kids[0])
            seqs[extra] = list(seqs[kids[0]])
            kids.append(extra)
    if capture:
        assert wrapper.graphs.captures > 0
    for sid in kids:
        kv.free_sequence(sid)
    assert kv.allocator.num_used == 0
