"""Pins the sampling / entropy / top-K oracle (CPU)."""
import json
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import sampling as S

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_philox_known_answers():
    # Random123's published philox4x32-10 vectors, and rocRAND's engine on more inputs.
    assert S.philox4x32_10([0, 0, 0, 0], [0, 0]) == [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]
    vecs = json.load(open(os.path.join(GOLDEN, "philox_rocrand.json")))
    assert len(vecs) >= 7
    for v in vecs:
        assert S.philox4x32_10(v["counter"], v["key"]) == v["out"], v


def test_det_exp2_exact_on_integers_and_accurate():
    for k in range(0, 64):
        assert S.det_exp2(-float(k)) == 2.0 ** -k
    assert S.det_exp2(-64.5) == 0.0
    ys = np.linspace(-40, 0, 20001, dtype=np.float32)
    got = np.array([S.det_exp2(float(y)) for y in ys])
    rel = np.abs(got / np.exp2(ys.astype(np.float64)) - 1)
    assert rel.max() < 1e-6
    assert np.all(np.diff(got) >= 0)  # monotone on this grid
    assert S.det_q(0.0) == 1 << 40


def test_entropy_closed_forms():
    V = 32000
    assert abs(S.entropy(np.zeros(V)) - math.log(V)) < 1e-12
    x = np.zeros(V)
    x[7] = 1e4
    assert S.entropy(x) < 1e-12
    assert abs(S.entropy(np.zeros(5), temperature=0.3) - math.log(5)) < 1e-12


def _dtype_ulp(v: float, dtype: str) -> float:
    """One unit in the last place of the dtype at |v| (normal range)."""
    bits = {"f32": 23, "bf16": 7, "f16": 10}[dtype]
    return 2.0 ** (math.floor(math.log2(abs(v))) - bits) if v else 0.0


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_entropy_chain_closed_forms(dtype):
    """The dtype chain of compute_entropy on rows whose terms are known in closed
    form: a uniform row (every p = rnd(1/V), lp = rnd(-ln V)) gives exactly
    -rnd(V * rnd(p * lp)); one dominant logit gives 0; a two-value row gives the
    rounded two-term sum."""
    V = 32000
    got = S.entropy_chain(np.zeros(V, dtype=np.float32), 0.7, dtype)
    p = S.round_to(np.array([1.0 / np.float32(V)], dtype=np.float32), dtype)
    lp = S.round_to(np.array([-np.log(np.float32(V))], dtype=np.float32), dtype)
    t = S.round_to(p * lp, dtype)
    want = -float(S.round_to(np.array([np.float32(V * np.float64(t[0]))]), dtype)[0])
    assert got == want
    assert abs(got - math.log(V)) <= 2 * _dtype_ulp(math.log(V), dtype) + 1e-6
    x = np.zeros(V, dtype=np.float32)
    x[7] = 1e4
    assert S.entropy_chain(x, 1.0, dtype) == 0.0
    # two values: n1 tokens at 1.0, the rest at 0.0 (T = 1)
    x = np.zeros(1000, dtype=np.float32)
    x[:10] = 1.0
    e1, e0 = np.exp2(np.float32(0.0) * S.LOG2E_F32), np.exp2(np.float32(-1.0) * S.LOG2E_F32)
    s = np.float32(10 * np.float64(e1) + 990 * np.float64(e0))
    logs = np.log(s)
    terms = []
    for e, d, n in ((e1, np.float32(0.0), 10), (e0, np.float32(-1.0), 990)):
        pr = S.round_to(np.array([e / s], dtype=np.float32), dtype)
        lq = S.round_to(np.array([d - logs], dtype=np.float32), dtype)
        terms.append(n * np.float64(S.round_to(pr * lq, dtype)[0]))
    want = -float(S.round_to(np.array([np.float32(sum(terms))]), dtype)[0])
    assert S.entropy_chain(x, 1.0, dtype) == want


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_entropy_chain_within_a_unit_of_float64(dtype):
    """Rounding every step to the dtype moves H by at most about one unit of the
    dtype from the float64 entropy of the same values (random rows, T = 0.7 and 1)."""
    rng = np.random.default_rng(3)
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[dtype]
    for trial in range(6):
        x = torch.from_numpy(rng.normal(0, 0.5 + trial, 20000).astype(np.float32)).to(tdt).float().numpy()
        for T in (0.7, 1.0):
            H64 = S.entropy(S.round_to(x * (np.float32(1.0) / np.float32(T)), dtype), 1.0)
            Hc = S.entropy_chain(x, T, dtype)
            assert abs(Hc - H64) <= 2 * _dtype_ulp(H64, dtype) + 1e-5, (dtype, trial, T, Hc, H64)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_entropy_and_keys_against_torch(dtype):
    rng = np.random.default_rng(0)
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16}[dtype]
    for trial in range(4):
        x = rng.normal(0, 1 + trial, 5000).astype(np.float32)
        xt = torch.from_numpy(x).to(tdt)
        xr = xt.float().numpy()
        # torch's compute_entropy in float64 on the same (rounded) values
        z = torch.from_numpy(xr.astype(np.float64)) / 0.7
        ref = -(F.softmax(z, -1) * F.log_softmax(z, -1)).sum().item()
        assert abs(S.entropy(xr, 0.7) - ref) < 1e-9
        # keys: torch log_softmax in the dtype (CPU), ours restated
        ids = rng.integers(0, 5000, 40)
        xp = S.penalize(xr, ids, 1.2, dtype)
        pt = torch.from_numpy(xr).to(tdt).clone()
        u = sorted(set(ids.tolist()))
        g = pt[u]
        pt[u] = torch.where(g > 0, g / 1.2, g * 1.2)
        assert np.array_equal(pt.float().numpy(), xp)
        keys = S.log_softmax_keys(xp, dtype)
        tk = F.log_softmax(pt, dim=-1).float().numpy()
        # fp32: the same single-rounding formula. bf16: torch's CPU kernel subtracts
        # an internally rounded log-sum, so the two agree to within 2 bf16 ulps.
        np.testing.assert_allclose(keys, tk, rtol=0 if dtype == "f32" else 2 ** -6,
                                   atol=1e-5 if dtype == "f32" else 0.0)
        ids5, vals5 = S.topk(keys, 5)
        assert int(ids5[0]) == int(torch.argmax(torch.from_numpy(keys)))
        assert list(vals5) == sorted(vals5, reverse=True)


def test_topk_tie_rule():
    keys = np.array([1.0, 3.0, 3.0, 2.0, 3.0], dtype=np.float32)
    ids, vals = S.topk(keys, 4)
    assert ids.tolist() == [1, 2, 4, 3]


def test_gate_formulas():
    assert S.adaptive_threshold(1.25, 10, 0) == 1.25
    assert abs(S.adaptive_threshold(1.25, 10, 5) - 1.25 * 1.5) < 1e-15
    assert S.soft_explore_factor(0, 10, 0.3) == 0.3
    assert abs(S.soft_explore_factor(5, 10, 0.3) - 0.65) < 1e-15
    assert S.soft_explore_factor(10, 10, 0.3) == 1.0


@pytest.mark.parametrize("sigma", [0.5, 2.0, 4.0])
def test_nucleus_matches_hf_top_p_away_from_boundary(sigma):
    rng = np.random.default_rng(int(sigma * 10))
    T, top_p = 0.7, 0.9
    for _ in range(3):
        x = S.round_to((rng.standard_normal(20000) * sigma).astype(np.float32), "bf16")
        idx, kept, Z, need = S.top_p_sample(x, T, top_p, seed=1, step=0, row=0)
        hf = S.hf_top_p_keep(x, T, top_p)
        order = np.lexsort((np.arange(x.size), -x.astype(np.float64)))
        # float64 prefix masses: skip draws whose boundary is within 1e-6 of top_p
        p = np.exp((x.astype(np.float64) - x.max()) / T)
        p /= p.sum()
        cum = np.cumsum(p[order])
        margin = np.min(np.abs(cum[max(kept - 2, 0):kept + 1] - top_p))
        if margin < 1e-6:
            continue
        assert kept == int(hf.sum())
        # Same multiset of kept values; among equal logits at the boundary HF's
        # unstable sort picks arbitrary members, this sampler the lowest indices.
        assert np.array_equal(np.sort(x[order[:kept]]), np.sort(x[hf]))
        assert x[idx] >= x[hf].min()


def test_draws_follow_the_nucleus_distribution():
    # Chi-square of 4000 draws (steps 0..3999) over a 12-token nucleus.
    rng = np.random.default_rng(3)
    x = S.round_to(rng.normal(0, 1.5, 40).astype(np.float32), "bf16")
    T, top_p = 1.0, 0.8
    counts = {}
    kept = None
    for step in range(4000):
        idx, kept, _, _ = S.top_p_sample(x, T, top_p, seed=123, step=step, row=5)
        counts[idx] = counts.get(idx, 0) + 1
    order = np.lexsort((np.arange(x.size), -x.astype(np.float64)))[:kept]
    p = np.exp((x[order].astype(np.float64) - x.max()) / T)
    p /= p.sum()
    assert set(counts) <= set(order.tolist())
    obs = np.array([counts.get(int(i), 0) for i in order], dtype=np.float64)
    exp = 4000 * p
    chi2 = float(((obs - exp) ** 2 / exp).sum())
    # 99.9th percentile of chi-square with kept-1 dof (kept is about 12 here).
    from scipy.stats import chi2 as chi2_dist
    assert chi2 < chi2_dist.ppf(0.999, kept - 1), (chi2, kept)
