"""Pins the attention oracle (CPU): closed forms, GQA mapping, torch SDPA fp64."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.attention import (
    gather_packed_kv,
    paged_decode_f64,
    reference_cpu_decode,
    sdpa_decode_f64,
)


def _random_paged(rng, N, Hq, Hkv, D, B, lens, num_blocks):
    perm = rng.permutation(num_blocks)
    tables, off = [], 0
    for n in lens:
        npg = (n + B - 1) // B
        tables.append(perm[off:off + npg].tolist())
        off += npg
    k_pool = rng.standard_normal((num_blocks, B, Hkv, D))
    v_pool = rng.standard_normal((num_blocks, B, Hkv, D))
    q = rng.standard_normal((N, Hq, D))
    return q, k_pool, v_pool, tables


def test_gather_layout_matches_table_order():
    B, Hkv, D = 4, 1, 2
    pool = np.arange(6 * B * Hkv * D, dtype=np.float64).reshape(6, B, Hkv, D)
    pk, pv, cu, mx = gather_packed_kv(pool, pool, [[5, 2], [1]], [6, 3], B)
    assert cu.tolist() == [0, 6, 9] and mx == 6
    expect_rows = [(5, 0), (5, 1), (5, 2), (5, 3), (2, 0), (2, 1), (1, 0), (1, 1), (1, 2)]
    for r, (b, s) in enumerate(expect_rows):
        np.testing.assert_array_equal(pk[r], pool[b, s])


def test_empty_batch_gather():
    pool = np.zeros((2, 4, 1, 2))
    pk, pv, cu, mx = gather_packed_kv(pool, pool, [], [], 4)
    assert pk.shape[0] == 0 and cu.tolist() == [0] and mx == 0


def test_single_token_returns_v():
    rng = np.random.default_rng(1)
    q = rng.standard_normal((1, 4, 8))
    k = rng.standard_normal((1, 2, 8))
    v = rng.standard_normal((1, 2, 8))
    o = sdpa_decode_f64(q, k, v, np.array([0, 1]))
    for h in range(4):
        np.testing.assert_allclose(o[0, h], v[0, h // 2], rtol=0, atol=1e-15)


def test_identical_keys_give_mean_of_values():
    rng = np.random.default_rng(2)
    L = 37
    k = np.repeat(rng.standard_normal((1, 1, 16)), L, axis=0)
    v = rng.standard_normal((L, 1, 16))
    q = rng.standard_normal((1, 3, 16))
    o = sdpa_decode_f64(q, k, v, np.array([0, L]))
    np.testing.assert_allclose(o[0], np.broadcast_to(v[:, 0].mean(0), (3, 16)), atol=1e-12)


def test_gqa_head_mapping():
    # Each kv head has a distinct constant value vector; q head h must read kv head h // G.
    Hq, Hkv, D, L = 8, 2, 4, 5
    k = np.zeros((L, Hkv, D))
    v = np.zeros((L, Hkv, D))
    v[:, 0] = 1.0
    v[:, 1] = 2.0
    q = np.ones((1, Hq, D))
    o = sdpa_decode_f64(q, k, v, np.array([0, L]))
    np.testing.assert_allclose(o[0, :4], 1.0)
    np.testing.assert_allclose(o[0, 4:], 2.0)


@pytest.mark.parametrize("Hq,Hkv,D", [(4, 2, 64), (32, 8, 128), (8, 8, 32)])
def test_against_torch_sdpa_float64(Hq, Hkv, D):
    rng = np.random.default_rng(Hq * 1000 + D)
    B = 16
    lens = [1, 15, 16, 17, 40, 100]
    q, kp, vp, tables = _random_paged(rng, len(lens), Hq, Hkv, D, B, lens, 64)
    o = paged_decode_f64(q, kp, vp, tables, lens, B)
    G = Hq // Hkv
    for i, n in enumerate(lens):
        pk, pv, _, _ = gather_packed_kv(kp, vp, [tables[i]], [n], B)
        kt = torch.from_numpy(np.repeat(pk, G, axis=1)).permute(1, 0, 2).unsqueeze(0)
        vt = torch.from_numpy(np.repeat(pv, G, axis=1)).permute(1, 0, 2).unsqueeze(0)
        qt = torch.from_numpy(q[i]).unsqueeze(0).unsqueeze(2)
        ref = F.scaled_dot_product_attention(qt, kt, vt).squeeze(0).squeeze(1).numpy()
        np.testing.assert_allclose(o[i], ref, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("w", [1, 5, 16, 33])
def test_decode_window_is_the_last_row_of_the_windowed_prefill_mask(w):
    """The decode window (flash window_size=(w - 1, 0), query at the end of the
    keys) against the reference's sliding-window mask (adapters/
    attention_backend.py:81-86: col <= row and col >= row - w + 1) at the last
    row, through torch's SDPA in float64 with that mask; w >= len gives the
    unwindowed decode, and identical keys give the mean of the last w values."""
    rng = np.random.default_rng(100 + w)
    B, Hq, Hkv, D = 16, 8, 2, 32
    lens = [1, 4, 16, 17, 40, 100]
    q, kp, vp, tables = _random_paged(rng, len(lens), Hq, Hkv, D, B, lens, 64)
    o = paged_decode_f64(q, kp, vp, tables, lens, B, window_size=w)
    G = Hq // Hkv
    for i, n in enumerate(lens):
        pk, pv, _, _ = gather_packed_kv(kp, vp, [tables[i]], [n], B)
        row = torch.arange(n)
        col = torch.arange(n)
        mask = (col <= row.unsqueeze(1)) & (col >= (row - w + 1).unsqueeze(1))
        am = torch.where(mask[-1], 0.0, float("-inf")).to(torch.float64).view(1, 1, 1, n)
        kt = torch.from_numpy(np.repeat(pk, G, axis=1)).permute(1, 0, 2).unsqueeze(0)
        vt = torch.from_numpy(np.repeat(pv, G, axis=1)).permute(1, 0, 2).unsqueeze(0)
        qt = torch.from_numpy(q[i]).unsqueeze(0).unsqueeze(2)
        ref = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=am).squeeze(0).squeeze(1).numpy()
        np.testing.assert_allclose(o[i], ref, rtol=1e-10, atol=1e-12)
    full = paged_decode_f64(q, kp, vp, tables, lens, B)
    np.testing.assert_array_equal(paged_decode_f64(q, kp, vp, tables, lens, B, window_size=100), full)
    for i, n in enumerate(lens):
        if n <= w:
            np.testing.assert_array_equal(o[i], full[i])
    kc = np.broadcast_to(kp[:1, :1], kp.shape).copy()
    oc = paged_decode_f64(q, kc, vp, tables, lens, B, window_size=w)
    for i, n in enumerate(lens):
        pk, pv, _, _ = gather_packed_kv(kc, vp, [tables[i]], [n], B)
        mean = pv[max(0, n - w):].mean(axis=0)  # [Hkv, D]
        np.testing.assert_allclose(oc[i], np.repeat(mean, G, axis=0), rtol=1e-10, atol=1e-12)


def test_reference_cpu_path_matches_f64():
    rng = np.random.default_rng(7)
    B, Hq, Hkv, D = 16, 8, 2, 64
    lens = [3, 33, 70]
    q, kp, vp, tables = _random_paged(rng, len(lens), Hq, Hkv, D, B, lens, 32)
    o64 = paged_decode_f64(q, kp, vp, tables, lens, B)
    o32 = reference_cpu_decode(
        torch.from_numpy(q).float(), torch.from_numpy(kp).float(), torch.from_numpy(vp).float(),
        tables, lens, B,
    ).numpy()
    np.testing.assert_allclose(o32, o64, rtol=1e-4, atol=1e-5)


def test_reference_cpu_prefill_known_answers_and_masks():
    """The CPU prefill baseline (the reference's SDPA path restated): one
    position gives v; identical keys give the mean of V over each position's
    window; and it agrees with explicit float64 masked softmax (GQA expand)."""
    import math

    import torch

    from oracle.attention import reference_cpu_prefill

    g = torch.Generator().manual_seed(0)
    q = torch.randn(2, 1, 4, 16, generator=g, dtype=torch.float64)
    k = torch.randn(2, 1, 2, 16, generator=g, dtype=torch.float64)
    v = torch.randn(2, 1, 2, 16, generator=g, dtype=torch.float64)
    assert torch.allclose(reference_cpu_prefill(q, k, v), v.repeat_interleave(2, dim=2))
    S = 9
    q = torch.randn(1, S, 2, 8, generator=g, dtype=torch.float64)
    k = torch.randn(1, 1, 1, 8, generator=g, dtype=torch.float64).expand(1, S, 1, 8)
    v = torch.randn(1, S, 1, 8, generator=g, dtype=torch.float64)
    for w in (None, 3):
        o = reference_cpu_prefill(q, k, v, window_size=w)
        for i in range(S):
            lo = 0 if w is None else max(0, i - w + 1)
            assert torch.allclose(o[0, i, 0], v[0, lo:i + 1, 0].mean(0))
            assert torch.allclose(o[0, i, 1], v[0, lo:i + 1, 0].mean(0))
    B, S, Hq, Hkv, D = 2, 13, 6, 2, 8
    q = torch.randn(B, S, Hq, D, generator=g, dtype=torch.float64)
    k = torch.randn(B, S, Hkv, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, S, Hkv, D, generator=g, dtype=torch.float64)
    for w in (None, 4, 13):
        o = reference_cpu_prefill(q, k, v, window_size=w)
        for h in range(Hq):
            kh, vh = k[:, :, h // 3], v[:, :, h // 3]
            s = torch.einsum("bid,bjd->bij", q[:, :, h], kh) / math.sqrt(D)
            i = torch.arange(S)[:, None]
            j = torch.arange(S)[None, :]
            m = j <= i
            if w is not None and w < S:
                m &= j >= i - w + 1
            want = torch.einsum("bij,bjd->bid", torch.softmax(s.masked_fill(~m, float("-inf")), -1), vh)
            assert torch.allclose(o[:, :, h], want)
