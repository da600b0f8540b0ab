"""Semantic-diversity prune kernels against the reference's torch ops.

EMA (core/generator.py:376-398): one launch must give, bit for bit, what
v.mul_(1 - alpha).add_(h, alpha=alpha) (and h.clone() for a new leaf) give
on the same device, in bf16, f16 and f32.
Similarity mask (core/generator.py:400-460): the pairs above the threshold
must be those of stack + F.normalize + mm + upper-triangle/sibling mask +
compare, in row-major order, on vectors built to put many similarities near
the threshold (a shared direction plus noise of several sizes).
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_semantic_ema_is_bit_exact_with_torch(gpu, dtype):
    from mentat_amd import ops

    print(f"case semantic ema {dtype}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(0)
    n, H, a = 37, 4096, 0.3
    base = torch.randn(n, H, generator=g, device="cuda").to(dtype)
    hid = torch.randn(n, 2 * H, generator=g, device="cuda").to(dtype)[:, :H]  # row stride 2H
    fresh = [i % 5 == 0 for i in range(n)]
    want = []
    for i in range(n):
        if fresh[i]:
            want.append(hid[i].clone())
        else:
            want.append(base[i].clone().mul_(1.0 - a).add_(hid[i], alpha=a))
    got = [base[i].clone() for i in range(n)]
    for step in range(3):  # repeated steps compound the rounding
        ops.semantic_ema(got, hid, fresh if step == 0 else [False] * n, a)
        if step:
            want = [w.mul_(1.0 - a).add_(hid[i], alpha=a) for i, w in enumerate(want)]
        for i in range(n):
            assert torch.equal(got[i], want[i]), (step, i)


def _reference_pairs(vecs, parents, thr):
    sv = torch.stack(vecs, dim=0)
    sim = torch.mm(F.normalize(sv, p=2, dim=1), F.normalize(sv, p=2, dim=1).t().contiguous())
    M = len(vecs)
    mask = torch.triu(torch.ones(M, M, device=sim.device, dtype=torch.bool), diagonal=1)
    for i in range(M):
        for j in range(i + 1, M):
            if parents[i] is not None and parents[i] is parents[j]:
                mask[i, j] = False
    return (sim * mask > thr).nonzero(as_tuple=False).tolist()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_semantic_similar_pairs_match_reference(gpu, dtype):
    from mentat_amd import ops

    print(f"case semantic similar {dtype}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(1)
    M, H, thr = 90, 4096, 0.85
    direction = torch.randn(H, generator=g, device="cuda")
    scales = torch.linspace(0.3, 1.1, M, device="cuda")
    vecs = [(direction + s * torch.randn(H, generator=g, device="cuda")).to(dtype).contiguous() for s in scales]
    objs = [object() for _ in range(12)]
    parents = [objs[i % 12] if i % 7 else None for i in range(M)]
    want = _reference_pairs(vecs, parents, thr)
    keys, pmap = [], {}
    for i, p in enumerate(parents):
        keys.append(-1 - i if p is None else pmap.setdefault(id(p), len(pmap)))
    mask = ops.semantic_similar_mask(vecs, keys, [0] * M, thr)
    ii, jj = np.nonzero(mask)
    got = [[int(a), int(b)] for a, b in zip(ii, jj)]
    assert len(want) > 50 and len(want) < M * (M - 1) // 2  # the threshold splits the pairs
    assert got == want
    # groups: pairs only within a group
    grp = [i % 3 for i in range(M)]
    mask2 = ops.semantic_similar_mask(vecs, keys, grp, thr)
    ii, jj = np.nonzero(mask2)
    got2 = [[int(a), int(b)] for a, b in zip(ii, jj)]
    assert got2 == [p for p in want if grp[p[0]] == grp[p[1]]]
