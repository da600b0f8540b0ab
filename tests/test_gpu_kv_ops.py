"""GPU parity of the KV-cache device ops (append + lazy copy-on-write, page copy,
table row copy) against a host restatement, in both pool layouts. Integer/byte
work: results must be bit-exact."""
import numpy as np
import pytest
import torch

from mentat_amd import ops
from mentat_amd._lib import LAYOUT_NATIVE, LAYOUT_REFERENCE
from mentat_amd.workloads import logical_views

pytestmark = pytest.mark.gpu


def _stores(layout, nb, B, Hkv, D, dtype, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    if layout == LAYOUT_NATIVE:
        ks = torch.randn(nb, Hkv, B, D, generator=g, device=dev).to(dtype)
        vs = torch.randn(nb, Hkv, D, B, generator=g, device=dev).to(dtype)
    else:
        ks = torch.randn(nb, B, Hkv, D, generator=g, device=dev).to(dtype)
        vs = torch.randn(nb, B, Hkv, D, generator=g, device=dev).to(dtype)
    return ks, vs


def _expected_append(kl, vl, k_new, v_new, plan, tables, lens):
    """Host semantics: copy-on-write of the first `slot` tokens, then the token row."""
    kl, vl, tables, lens = kl.copy(), vl.copy(), tables.copy(), lens.copy()
    snap_k, snap_v = kl.copy(), vl.copy()
    dst, slot, cow, row, page, new_len, src = plan
    for i in range(plan.shape[1]):
        if cow[i] >= 0:
            kl[dst[i], :slot[i]] = snap_k[cow[i], :slot[i]]
            vl[dst[i], :slot[i]] = snap_v[cow[i], :slot[i]]
    for i in range(plan.shape[1]):
        kl[dst[i], slot[i]] = k_new[src[i]]
        vl[dst[i], slot[i]] = v_new[src[i]]
        if row[i] >= 0:
            tables[row[i], page[i]] = dst[i]
            if new_len[i] >= 0:
                lens[row[i]] = new_len[i]
    return kl, vl, tables, lens


@pytest.mark.parametrize("layout", [LAYOUT_REFERENCE, LAYOUT_NATIVE])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_kv_append_decode_plan(gpu, layout, dtype):
    if layout == LAYOUT_NATIVE and dtype == torch.float32:
        pytest.skip("the native layout is used for 16-bit pools only")
    print(f"case kv_append decode layout={layout} {dtype}", flush=True)
    nb, B, Hkv, D = 64, 16, 8, 128
    ks, vs = _stores(layout, nb, B, Hkv, D, dtype, gpu, 1)
    k_new = torch.randn(6, Hkv, D, device=gpu).to(dtype)
    v_new = torch.randn(6, Hkv, D, device=gpu).to(dtype)
    # Six sequences, rows 0..5. Seq 0/1 share tail block 10 (seq 0 copies into 20,
    # seq 1, the last sharer, writes in place); seq 2 starts a fresh block 21;
    # seq 3 copies block 11 at slot 0 (nothing to copy); seq 4 plain; seq 5 copies 12 -> 22.
    plan = np.array([
        [20, 10, 21, 23, 30, 22],   # dst block
        [5, 5, 0, 0, 7, 15],        # slot
        [10, -1, -1, 11, -1, 12],   # cow source
        [0, 1, 2, 3, 4, 5],         # row
        [2, 2, 3, 0, 1, 4],         # page
        [38, 38, 49, 1, 24, 80],    # new length
        [0, 1, 2, 3, 4, 5],         # source token
    ], dtype=np.int32)
    tables = torch.randint(0, nb, (8, 6), dtype=torch.int32, device=gpu)
    lens = torch.randint(0, 100, (8,), dtype=torch.int32, device=gpu)
    kl0, vl0 = (t.float().cpu().numpy() for t in logical_views(ks, vs, layout))
    exp = _expected_append(kl0, vl0, k_new.float().cpu().numpy(), v_new.float().cpu().numpy(), plan,
                           tables.cpu().numpy(), lens.cpu().numpy())
    ops.kv_append(k_new, v_new, ks, vs, torch.from_numpy(plan).to(gpu), block_size=B, layout=layout,
                  block_tables=tables, seq_lens=lens)
    torch.cuda.synchronize()
    kl, vl = (t.float().cpu().numpy() for t in logical_views(ks, vs, layout))
    np.testing.assert_array_equal(kl, exp[0])
    np.testing.assert_array_equal(vl, exp[1])
    np.testing.assert_array_equal(tables.cpu().numpy(), exp[2])
    np.testing.assert_array_equal(lens.cpu().numpy(), exp[3])


@pytest.mark.parametrize("layout", [LAYOUT_REFERENCE, LAYOUT_NATIVE])
def test_kv_append_prefill_plan_with_cow(gpu, layout):
    # One sequence appends 21 tokens starting at slot 9 of a shared tail page 3:
    # tokens 0..6 go to a fresh copy (block 40, copy of slots 0..8 of block 3),
    # tokens 7..20 to a new block 41. The copy must not clobber tokens 1..6.
    print(f"case kv_append prefill layout={layout}", flush=True)
    nb, B, Hkv, D = 64, 16, 2, 64
    ks, vs = _stores(layout, nb, B, Hkv, D, torch.bfloat16, gpu, 2)
    n = 21
    k_new = torch.randn(n, Hkv, D, device=gpu).to(torch.bfloat16)
    v_new = torch.randn(n, Hkv, D, device=gpu).to(torch.bfloat16)
    dst = [40] * 7 + [41] * 14
    slot = list(range(9, 16)) + list(range(0, 14))
    cow = [3] + [-1] * 20
    row = [2] * n
    page = [0] * 7 + [1] * 14
    new_len = [-1] * (n - 1) + [30]
    plan = np.array([dst, slot, cow, row, page, new_len, list(range(n))], dtype=np.int32)
    tables = torch.zeros(4, 4, dtype=torch.int32, device=gpu)
    lens = torch.zeros(4, dtype=torch.int32, device=gpu)
    kl0, vl0 = (t.float().cpu().numpy() for t in logical_views(ks, vs, layout))
    exp = _expected_append(kl0, vl0, k_new.float().cpu().numpy(), v_new.float().cpu().numpy(), plan,
                           tables.cpu().numpy(), lens.cpu().numpy())
    ops.kv_append(k_new, v_new, ks, vs, torch.from_numpy(plan).to(gpu), block_size=B, layout=layout,
                  block_tables=tables, seq_lens=lens)
    torch.cuda.synchronize()
    kl, vl = (t.float().cpu().numpy() for t in logical_views(ks, vs, layout))
    np.testing.assert_array_equal(kl, exp[0])
    np.testing.assert_array_equal(vl, exp[1])
    np.testing.assert_array_equal(tables.cpu().numpy(), exp[2])
    assert lens.cpu().tolist() == [0, 0, 30, 0]


def test_page_copy_many_pools(gpu):
    pools = [torch.randn(32, 16, 4, 64, device=gpu).to(torch.bfloat16) for _ in range(6)]
    before = [p.clone() for p in pools]
    src = torch.tensor([1, 5, 7, 9], dtype=torch.int32, device=gpu)
    dst = torch.tensor([2, 6, 30, 99999], dtype=torch.int32, device=gpu)  # last pair out of range: skipped
    ops.page_copy(pools, src, dst)
    torch.cuda.synchronize()
    for p, b in zip(pools, before):
        exp = b.clone()
        exp[2], exp[6], exp[30] = b[1], b[5], b[7]
        assert torch.equal(p, exp)


def test_table_copy_rows(gpu):
    L, R, S = 3, 8, 10
    tables = torch.randint(0, 1000, (L, R, S), dtype=torch.int32, device=gpu)
    lens = torch.randint(0, 100, (L, R), dtype=torch.int32, device=gpu)
    t0, l0 = tables.clone(), lens.clone()
    src = torch.tensor([1, 4], dtype=torch.int32, device=gpu)
    dst = torch.tensor([5, 6], dtype=torch.int32, device=gpu)
    ops.table_copy_rows(tables, lens, src, dst, n_entries=7)
    torch.cuda.synchronize()
    exp_t, exp_l = t0.clone(), l0.clone()
    exp_t[:, 5, :7] = t0[:, 1, :7]
    exp_t[:, 6, :7] = t0[:, 4, :7]
    exp_l[:, 5] = l0[:, 1]
    exp_l[:, 6] = l0[:, 4]
    assert torch.equal(tables, exp_t) and torch.equal(lens, exp_l)


@pytest.mark.parametrize("layout", [LAYOUT_REFERENCE, LAYOUT_NATIVE])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rope_qkv_append_equals_rope_qkv_then_kv_append(gpu, layout, dtype):
    """One launch, the same bits: q, both pools, the tables and the lengths
    equal those of rope_qkv followed by kv_append of its k and v, for a decode
    plan (copy-on-write of shared tails, a padding column with no destination,
    more q rows than plan columns, source rows out of order) and a prefill plan
    (21 tokens over a copied tail page and a fresh page)."""
    decode = np.array([
        [20, 10, 21, 23, 30, 22, -1],   # dst block (-1: padding column)
        [5, 5, 0, 0, 7, 15, 0],         # slot
        [10, -1, -1, 11, -1, 12, -1],   # cow source
        [0, 1, 2, 3, 4, 5, -1],         # row
        [2, 2, 3, 0, 1, 4, 0],          # page
        [38, 38, 49, 1, 24, 80, -1],    # new length
        [3, 0, 8, 1, 5, 2, 7],          # source row
    ], dtype=np.int32)
    n = 21
    prefill = np.array([[40] * 7 + [41] * 14, list(range(9, 16)) + list(range(0, 14)), [3] + [-1] * 20, [2] * n,
                        [0] * 7 + [1] * 14, [-1] * (n - 1) + [30], list(range(n))], dtype=np.int32)
    for name, plan, rows, Hq, Hk, D in (("decode", decode, 9, 32, 8, 128), ("prefill", prefill, n, 8, 2, 64)):
        print(f"case rope_qkv_append {name} layout={layout} {dtype}", flush=True)
        nb, B = 64, 16
        g = torch.Generator(device=gpu).manual_seed(11)
        qkv = torch.randn(1, rows, (Hq + 2 * Hk) * D, generator=g, device=gpu).to(dtype)
        cos = (2 * torch.rand(1, rows, 1, D, generator=g, device=gpu) - 1).to(dtype)
        sin = (2 * torch.rand(1, rows, 1, D, generator=g, device=gpu) - 1).to(dtype)
        ks, vs = _stores(layout, nb, B, Hk, D, dtype, gpu, 3)
        tables = torch.randint(0, nb, (8, 6), dtype=torch.int32, device=gpu)
        lens = torch.randint(0, 100, (8,), dtype=torch.int32, device=gpu)
        ks2, vs2, tables2, lens2 = ks.clone(), vs.clone(), tables.clone(), lens.clone()
        p = torch.from_numpy(plan).to(gpu)
        q, k, v = ops.rope_qkv(qkv, Hq, Hk, cos, sin)
        ops.kv_append(k, v, ks, vs, p, block_size=B, layout=layout, block_tables=tables, seq_lens=lens)
        q2 = ops.rope_qkv_append(qkv, Hq, Hk, cos, sin, ks2, vs2, p, block_size=B, layout=layout,
                                 block_tables=tables2, seq_lens=lens2)
        torch.cuda.synchronize()
        assert torch.equal(q2, q)
        assert torch.equal(ks2, ks) and torch.equal(vs2, vs)
        assert torch.equal(tables2, tables) and torch.equal(lens2, lens)
        assert not torch.equal(ks2, _stores(layout, nb, B, Hk, D, dtype, gpu, 3)[0])  # something was written
