"""Fused layer glue of the captured decode step against the modules it replaces:
HF LlamaRMSNorm (with and without the residual add), the adapters'
t*cos + rotate_half(t)*sin, and LlamaMLP's act_fn(gate) * up.

RoPE is bit-exact (the same three roundings as torch's ops). RMSNorm and
SiLU*up differ from torch only in the fp32 summation order of the mean and in
exp's last bit. A one-ulp change of the fp32 scale can move the rounded
normalised value by one unit, which the weight multiply (|w| up to ~2) can
make two units of the output: RMSNorm is held to two units, SiLU*up to one,
and both to differing from torch in under 1% of elements."""
import pytest
import torch

from mentat_amd import ops
from mentat_amd.adapters.model_adapter import rotate_half

pytestmark = pytest.mark.gpu


def _ulp(ref: torch.Tensor) -> torch.Tensor:
    bits = 8 if ref.dtype == torch.bfloat16 else 11
    mag = ref.float().abs().clamp_min(2.0 ** -14)
    return torch.exp2(torch.floor(torch.log2(mag)) - (bits - 1))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,H", [(1, 4096), (152, 4096), (7, 2048), (33, 5120), (3, 8)])
def test_rmsnorm_matches_hf_module(gpu, dtype, rows, H):
    from transformers.models.llama.modeling_llama import LlamaRMSNorm

    print(f"case rmsnorm {dtype} rows={rows} H={H}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(rows * 7 + H)
    norm = LlamaRMSNorm(H, eps=1e-5).to(gpu, dtype)
    with torch.no_grad():
        norm.weight.copy_((1 + 0.2 * torch.randn(H, generator=g, device=gpu)).to(dtype))
    x = (3 * torch.randn(1, rows, H, generator=g, device=gpu)).to(dtype)
    res = torch.randn(1, rows, H, generator=g, device=gpu).to(dtype)
    with torch.no_grad():
        for residual in (None, res):
            h_ref = x if residual is None else residual + x
            y_ref = norm(h_ref)
            y, h = ops.rmsnorm(x, norm.weight, norm.variance_epsilon, residual=residual)
            if residual is not None:
                assert torch.equal(h, h_ref)  # the residual add rounds as torch's add
            else:
                assert h is None
            diff = (y.float() - y_ref.float()).abs()
            assert bool((diff <= 2 * _ulp(y_ref)).all()), float(diff.max())
            assert (diff > 0).float().mean().item() < 0.01


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,Hq,Hk,D", [(152, 32, 8, 128), (5, 16, 2, 64), (1, 4, 4, 128)])
def test_rope_bit_exact_with_rotate_half(gpu, dtype, n, Hq, Hk, D):
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding

    print(f"case rope {dtype} n={n} Hq={Hq} Hk={Hk} D={D}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(n + Hq + D)
    cfg = LlamaConfig(hidden_size=Hq * D, num_attention_heads=Hq, num_key_value_heads=Hk, head_dim=D,
                      max_position_embeddings=8192)
    rot = LlamaRotaryEmbedding(cfg).to(gpu)
    q = torch.randn(n, 1, Hq, D, generator=g, device=gpu).to(dtype)
    k = torch.randn(n, 1, Hk, D, generator=g, device=gpu).to(dtype)
    pos = torch.randint(0, 8000, (n, 1), generator=g, device=gpu)
    cos, sin = rot(q, pos)
    cos, sin = cos.unsqueeze(2), sin.unsqueeze(2)
    q_ref = q * cos + rotate_half(q) * sin
    k_ref = k * cos + rotate_half(k) * sin
    ops.rope_(q, k, cos, sin)
    assert torch.equal(q, q_ref)
    assert torch.equal(k, k_ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,F", [(152, 14336), (1, 8), (9, 1024)])
def test_silu_mul_matches_mlp_activation(gpu, dtype, rows, F):
    print(f"case silu_mul {dtype} rows={rows} F={F}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(rows + F)
    gate = (4 * torch.randn(1, rows, F, generator=g, device=gpu)).to(dtype)
    up = torch.randn(1, rows, F, generator=g, device=gpu).to(dtype)
    ref = torch.nn.functional.silu(gate) * up
    out = ops.silu_mul(gate, up)
    diff = (out.float() - ref.float()).abs()
    assert bool((diff <= _ulp(ref)).all()), float(diff.max())
    assert (diff > 0).float().mean().item() < 0.01


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rope_qkv_splits_a_merged_projection(gpu, dtype):
    """q/k/v read from one merged projection output: q and k rotated exactly as
    rotate_half does on the split tensors, v copied."""
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding

    n, Hq, Hk, D = 37, 32, 8, 128
    print(f"case rope_qkv {dtype} n={n}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(5)
    cfg = LlamaConfig(hidden_size=Hq * D, num_attention_heads=Hq, num_key_value_heads=Hk, head_dim=D)
    rot = LlamaRotaryEmbedding(cfg).to(gpu)
    qkv = torch.randn(1, n, (Hq + 2 * Hk) * D, generator=g, device=gpu).to(dtype)
    pos = torch.randint(0, 4000, (n, 1), generator=g, device=gpu)
    cos, sin = rot(qkv, pos)
    cos, sin = cos.unsqueeze(2), sin.unsqueeze(2)
    q, k, v = ops.rope_qkv(qkv, Hq, Hk, cos, sin)
    x = qkv.view(n, 1, Hq + 2 * Hk, D)
    q0, k0, v0 = x[:, :, :Hq], x[:, :, Hq:Hq + Hk], x[:, :, Hq + Hk:]
    assert torch.equal(q, (q0 * cos + rotate_half(q0) * sin).squeeze(1))
    assert torch.equal(k, (k0 * cos + rotate_half(k0) * sin).squeeze(1))
    assert torch.equal(v, v0.squeeze(1))


def test_silu_mul_merged_matches_split_halves(gpu):
    g = torch.Generator(device=gpu).manual_seed(6)
    gu = (3 * torch.randn(1, 41, 2 * 14336, generator=g, device=gpu)).to(torch.bfloat16)
    out = ops.silu_mul_merged(gu)
    ref = ops.silu_mul(gu[..., :14336].contiguous(), gu[..., 14336:].contiguous())
    assert torch.equal(out, ref)


def test_captured_step_fuses_the_glue(gpu):
    """A bf16 HF Llama model takes the fused captured path; an fp32 one does not."""
    from transformers import LlamaConfig, LlamaForCausalLM

    from mentat_amd.adapters.adapter_factory import get_adapter
    from mentat_amd.core.graph_decode import _fusable

    cfg = LlamaConfig(hidden_size=256, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                      head_dim=64, intermediate_size=512, vocab_size=1000)
    model = LlamaForCausalLM(cfg).to(gpu)
    assert not _fusable(get_adapter(model), torch.float32)
    model = model.to(torch.bfloat16)
    assert _fusable(get_adapter(model), torch.bfloat16)
    from mentat_amd.core.graph_decode import _mergeable

    assert _mergeable(get_adapter(model))


@pytest.mark.parametrize("split", [2, 4, 8])
@pytest.mark.parametrize("rows,F", [(41, 14336), (1, 64), (176, 1024)])
def test_silu_mul_split_is_the_column_slices(gpu, split, rows, F):
    print(f"case silu_mul_split S={split} rows={rows} F={F}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(rows + F + split)
    gu = (3 * torch.randn(rows, 2 * F, generator=g, device=gpu)).to(torch.bfloat16)
    out = ops.silu_mul_merged_split(gu, split)
    ref = ops.silu_mul_merged(gu).view(rows, split, F // split).permute(1, 0, 2)
    assert out.shape == (split, rows, F // split)
    assert torch.equal(out, ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("S,rows,H", [(4, 152, 4096), (2, 1, 4096), (8, 7, 2048), (4, 33, 5120), (4, 3, 8)])
def test_rmsnorm_partials_is_rmsnorm_of_the_rounded_sum(gpu, dtype, S, rows, H):
    """The partials are summed in slice order in fp32 and rounded once; from
    there the residual add and the norm are rmsnorm's, bit for bit."""
    print(f"case rmsnorm_partials {dtype} S={S} rows={rows} H={H}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(S * 1000 + rows + H)
    parts = torch.randn(S, rows, H, generator=g, device=gpu)
    w = (1 + 0.2 * torch.randn(H, generator=g, device=gpu)).to(dtype)
    res = torch.randn(rows, H, generator=g, device=gpu).to(dtype)
    x = parts[0].clone()
    for s in range(1, S):
        x = x + parts[s]
    x = x.to(dtype)
    for residual in (None, res):
        y_ref, h_ref = ops.rmsnorm(x, w, 1e-5, residual=residual)
        y, h = ops.rmsnorm_partials(parts, w, 1e-5, residual=residual)
        assert torch.equal(y, y_ref)
        assert (h is None) == (residual is None)
        if residual is not None:
            assert torch.equal(h, h_ref)


def test_split_down_projection_refreshes_and_matches(gpu):
    """The split copy of a down weight is its transpose in column slices, and
    an in-place change of the module's weight reaches the copy."""
    from mentat_amd.core.graph_decode import _split_copy

    g = torch.Generator(device=gpu).manual_seed(9)
    W = torch.randn(256, 1024, generator=g, device=gpu).to(torch.bfloat16)
    w = torch.empty(4, 256, 256, dtype=torch.bfloat16, device=gpu)
    _split_copy(w, W)
    act = torch.randn(5, 1024, generator=g, device=gpu).to(torch.bfloat16)
    parts = torch.bmm(act.view(5, 4, 256).permute(1, 0, 2).contiguous(), w, out_dtype=torch.float32)
    ref = act.float() @ W.float().t()
    assert float((parts.sum(0) - ref).abs().max()) < 1e-2 * float(ref.abs().max())
