"""Prefill attention kernel (mentat_prefill_attention) against a float64 CPU
reference of the reference's SDPA prefill (adapters/attention_backend.py:43-96:
causal, GQA by head expansion, sliding window when window_size < seq_len).

Tolerance (bf16/f16 inputs, fp32 accumulation, P rounded to the input dtype
for the P.V product): |got - want| <= 2e-2 + 1e-2 |want|.
Known answers pin the masking independently of the reference formula: with
one position the output is v; with identical keys every position's output
is the mean of V over its window.
"""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _ref(q, k, v, window):
    """float64 CPU attention, explicit masks (q [B,S,Hq,D], k/v [B,S,Hkv,D])."""
    q, k, v = q.double().cpu(), k.double().cpu(), v.double().cpu()
    B, S, Hq, D = q.shape
    G = Hq // k.shape[2]
    k = k.repeat_interleave(G, dim=2)
    v = v.repeat_interleave(G, dim=2)
    s = torch.einsum("bihd,bjhd->bhij", q, k) / math.sqrt(D)
    i = torch.arange(S)[:, None]
    j = torch.arange(S)[None, :]
    mask = j <= i
    if window is not None and window < S:
        mask &= j >= i - window + 1
    s = s.masked_fill(~mask, float("-inf"))
    return torch.einsum("bhij,bjhd->bihd", torch.softmax(s, -1), v)


CASES = [
    # B, S, Hq, Hkv, D, window
    (1, 1, 8, 8, 128, None),
    (2, 17, 32, 8, 128, None),
    (1, 100, 8, 2, 64, None),
    (2, 256, 32, 8, 128, None),
    (1, 333, 16, 1, 64, None),
    (1, 77, 16, 8, 128, None),
    (2, 130, 32, 8, 128, 7),
    (1, 200, 8, 4, 64, 64),
    (1, 90, 32, 8, 128, 1),
    (1, 50, 32, 8, 128, 4096),
    (1, 1000, 32, 8, 128, None),
    # head_dim 128 (the 32-column kernel): 8 and 16 query heads per kv head, and a
    # window spanning several 64-key stages
    (1, 700, 32, 4, 128, 300),
    (1, 129, 16, 1, 128, None),
    (2, 450, 32, 8, 128, 190),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,S,Hq,Hkv,D,window", CASES)
def test_prefill_matches_float64_reference(gpu, dtype, B, S, Hq, Hkv, D, window):
    from mentat_amd import ops

    print(f"case prefill B={B} S={S} Hq={Hq} Hkv={Hkv} D={D} window={window} {dtype}", flush=True)
    g = torch.Generator().manual_seed(S * 131 + Hq)
    q = torch.randn(B, S, Hq, D, generator=g).to(dtype)
    k = torch.randn(B, S, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B, S, Hkv, D, generator=g).to(dtype)
    got = ops.prefill_attention(q.cuda(), k.cuda(), v.cuda(), window_size=window).float().cpu()
    want = _ref(q, k, v, window).float()
    err = (got - want).abs()
    assert bool((err <= 2e-2 + 1e-2 * want.abs()).all()), float(err.max())


F32_CASES = [c for c in CASES if c[2] // c[3] in (1, 2, 4, 8)] + [
    (3, 41, 4, 2, 64, None),   # the fp32 plumbing model's heads
    (2, 300, 4, 2, 64, 33),
]


@pytest.mark.parametrize("B,S,Hq,Hkv,D,window", F32_CASES)
def test_prefill_f32_matches_float64_reference(gpu, B, S, Hq, Hkv, D, window):
    """fp32 prompts run on the VALU decode kernel, one query per position
    (fp32 throughout): |got - want| <= 1e-4 + 1e-4 |want|. attn_prefill
    routes fp32 to it."""
    from mentat_amd import ops
    from mentat_amd.adapters.attention_backend import attn_prefill

    print(f"case prefill f32 B={B} S={S} Hq={Hq} Hkv={Hkv} D={D} window={window}", flush=True)
    g = torch.Generator().manual_seed(S * 17 + Hq)
    q = torch.randn(B, S, Hq, D, generator=g)
    k = torch.randn(B, S, Hkv, D, generator=g)
    v = torch.randn(B, S, Hkv, D, generator=g)
    got = ops.prefill_attention(q.cuda(), k.cuda(), v.cuda(), window_size=window)
    via = attn_prefill(q.cuda(), k.cuda(), v.cuda(), window_size=window)
    torch.cuda.synchronize()
    assert torch.equal(got, via)
    want = _ref(q, k, v, window)
    err = (got.double().cpu() - want).abs()
    assert bool((err <= 1e-4 + 1e-4 * want.abs()).all()), float(err.max())


def test_prefill_known_answers(gpu):
    from mentat_amd import ops

    print("case prefill known answers", flush=True)
    torch.manual_seed(0)
    # one position: o = v of its kv head
    q = torch.randn(3, 1, 8, 128, dtype=torch.bfloat16, device="cuda")
    k = torch.randn(3, 1, 2, 128, dtype=torch.bfloat16, device="cuda")
    v = torch.randn(3, 1, 2, 128, dtype=torch.bfloat16, device="cuda")
    o = ops.prefill_attention(q, k, v)
    assert torch.equal(o, v.repeat_interleave(4, dim=2))
    o = ops.prefill_attention(q.float(), k.float(), v.float())
    assert torch.equal(o, v.float().repeat_interleave(4, dim=2))
    # identical keys: position i outputs the mean of V over keys max(0, i-w+1) .. i
    q = torch.randn(2, 40, 4, 64, device="cuda")
    k = torch.randn(2, 1, 2, 64, device="cuda").expand(2, 40, 2, 64).contiguous()
    v = torch.randn(2, 40, 2, 64, device="cuda")
    for w in (None, 3):
        o = ops.prefill_attention(q, k, v, window_size=w).double().cpu()
        vf = v.double().cpu()
        for i in range(40):
            lo = 0 if w is None else max(0, i - w + 1)
            mean = vf[:, lo:i + 1].mean(1).repeat_interleave(2, dim=1)
            assert (o[:, i] - mean).abs().max() < 1e-5, (w, i)
    S = 70
    for w in (None, 5):
        q = torch.randn(1, S, 4, 64, dtype=torch.float16, device="cuda")
        k = torch.randn(1, 1, 1, 64, dtype=torch.float16, device="cuda").expand(1, S, 1, 64).contiguous()
        v = torch.randn(1, S, 1, 64, dtype=torch.float16, device="cuda")
        o = ops.prefill_attention(q, k, v, window_size=w).float().cpu()
        vf = v.float().cpu()
        for i in range(S):
            lo = 0 if w is None else max(0, i - w + 1)
            mean = vf[0, lo:i + 1, 0].mean(0)
            assert (o[0, i] - mean).abs().max() < 1e-2, (w, i)


def test_prefill_last_row_equals_paged_decode(gpu):
    """The last prompt position's output equals decode over the same cached
    K/V (the paged decode kernel on the prompt's pages)."""
    from mentat_amd import ops
    from mentat_amd._lib import LAYOUT_NATIVE

    print("case prefill last row vs paged decode", flush=True)
    torch.manual_seed(1)
    S, Hq, Hkv, D, B = 181, 32, 8, 128, 16
    q = torch.randn(1, S, Hq, D, dtype=torch.bfloat16, device="cuda")
    k = torch.randn(1, S, Hkv, D, dtype=torch.bfloat16, device="cuda")
    v = torch.randn(1, S, Hkv, D, dtype=torch.bfloat16, device="cuda")
    o = ops.prefill_attention(q, k, v)
    npg = (S + B - 1) // B
    kp = torch.zeros(npg * B, Hkv, D, dtype=torch.bfloat16, device="cuda")
    vp = torch.zeros_like(kp)
    kp[:S], vp[:S] = k[0], v[0]
    k_store = kp.view(npg, B, Hkv, D).permute(0, 2, 1, 3).contiguous()   # native [blk][Hkv][B][D]
    v_store = vp.view(npg, B, Hkv, D).permute(0, 2, 3, 1).contiguous()   # native [blk][Hkv][D][B]
    tables = torch.arange(npg, dtype=torch.int32, device="cuda").view(1, npg)
    lens = torch.tensor([S], dtype=torch.int32, device="cuda")
    d = ops.paged_decode(q[0, S - 1:S].contiguous(), k_store, v_store, layout=LAYOUT_NATIVE, block_tables=tables,
                         seq_lens=lens, max_seqlen=S)
    assert (o[0, S - 1].float() - d[0].float()).abs().max() < 2e-2
