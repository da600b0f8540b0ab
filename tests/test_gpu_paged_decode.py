"""GPU parity of the paged decode kernel (C ABI) against the fp64 oracle.

Tolerance (from the decode contract): 2e-2 abs / 1e-2 rel for bf16/fp16
outputs against the reference computed in fp64 on the same (rounded) inputs;
1e-4 for fp32.
"""
import numpy as np
import pytest
import torch

from mentat_amd import ops
from mentat_amd._lib import LAYOUT_NATIVE, LAYOUT_REFERENCE
from mentat_amd.workloads import paged_decode_batch
from oracle.attention import paged_decode_f64, sdpa_decode_f64

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: (2e-2, 1e-2), torch.float16: (2e-2, 1e-2), torch.float32: (1e-4, 1e-4)}


def _to64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _oracle(batch, rows=None):
    kp = _to64(batch.k_pool)
    vp = _to64(batch.v_pool)
    tables = batch.tables if rows is None else [batch.tables[r] for r in rows]
    lens = batch.lens if rows is None else [batch.lens[r] for r in rows]
    return paged_decode_f64(_to64(batch.q), kp, vp, tables, lens, batch.block_size, batch.scale)


CASES = [
    # (Hq, Hkv, D, dtype, lens)
    (32, 8, 128, torch.bfloat16, [1, 15, 16, 17, 250, 513]),
    (4, 2, 64, torch.float32, [1, 2, 31, 129]),
    (16, 8, 128, torch.bfloat16, [5, 77, 1000]),
    (8, 8, 64, torch.float16, [16, 48, 300]),
    (16, 2, 128, torch.bfloat16, [33, 700]),
    (4, 4, 128, torch.float32, [3, 90]),
]


@pytest.mark.parametrize("Hq,Hkv,D,dtype,lens", CASES)
@pytest.mark.parametrize("chunk", [0, 16, 64])
def test_paged_matches_oracle(gpu, Hq, Hkv, D, dtype, lens, chunk):
    print(f"case reference layout Hq={Hq} Hkv={Hkv} D={D} {dtype} lens={lens} chunk={chunk}", flush=True)
    b = paged_decode_batch(N=len(lens), Hq=Hq, Hkv=Hkv, D=D, dtype=dtype, device=gpu,
                           num_blocks=256, lens=lens, seed=len(lens) + D)
    out = ops.paged_decode(b.q, b.k_store, b.v_store, layout=b.layout, block_tables=b.block_tables,
                           seq_lens=b.seq_lens, max_seqlen=b.max_seqlen, chunk_tokens=chunk,
                           scale=b.scale)
    torch.cuda.synchronize()
    atol, rtol = TOL[dtype]
    np.testing.assert_allclose(_to64(out), _oracle(b), atol=atol, rtol=rtol)


NATIVE_CASES = [
    # (Hq, Hkv, D, dtype, block_size, lens)
    (32, 8, 128, torch.bfloat16, 16, [1, 15, 16, 17, 250, 513]),
    (16, 8, 128, torch.bfloat16, 16, [5, 77, 1000]),
    (8, 8, 64, torch.float16, 16, [16, 48, 300]),
    (16, 2, 128, torch.bfloat16, 32, [33, 700, 0, 64]),
    (32, 2, 128, torch.bfloat16, 16, [2, 40]),
    (4, 4, 64, torch.bfloat16, 64, [3, 90, 129]),
    (64, 8, 128, torch.bfloat16, 16, [100]),
]


@pytest.mark.parametrize("Hq,Hkv,D,dtype,bs,lens", NATIVE_CASES)
def test_native_layout_matches_oracle(gpu, Hq, Hkv, D, dtype, bs, lens):
    print(f"case native layout Hq={Hq} Hkv={Hkv} D={D} {dtype} B={bs} lens={lens}", flush=True)
    b = paged_decode_batch(N=len(lens), Hq=Hq, Hkv=Hkv, D=D, dtype=dtype, device=gpu, block_size=bs,
                           num_blocks=256, lens=lens, seed=len(lens) + D + 7, layout=LAYOUT_NATIVE)
    out = ops.paged_decode(b.q, b.k_store, b.v_store, layout=LAYOUT_NATIVE, block_tables=b.block_tables,
                           seq_lens=b.seq_lens, max_seqlen=max(1, b.max_seqlen), scale=b.scale)
    torch.cuda.synchronize()
    atol, rtol = TOL[dtype]
    np.testing.assert_allclose(_to64(out), _oracle(b), atol=atol, rtol=rtol)


def test_native_many_sequences_stream_k(gpu):
    # Many short and long sequences: units split across persistent wavefronts.
    rng = np.random.default_rng(9)
    lens = rng.integers(1, 700, size=300).tolist()
    b = paged_decode_batch(N=len(lens), Hq=32, Hkv=8, D=128, device=gpu, num_blocks=16384,
                           lens=lens, seed=9, layout=LAYOUT_NATIVE)
    out = ops.paged_decode(b.q, b.k_store, b.v_store, layout=LAYOUT_NATIVE, block_tables=b.block_tables,
                           seq_lens=b.seq_lens, max_seqlen=b.max_seqlen, scale=b.scale)
    torch.cuda.synchronize()
    o = _to64(out)
    q64 = _to64(b.q)
    for i in range(0, len(lens), 7):
        pages = torch.tensor(b.tables[i], dtype=torch.long, device=gpu)
        kp = _to64(b.k_pool[pages]).reshape(-1, 8, 128)[: lens[i]]
        vp = _to64(b.v_pool[pages]).reshape(-1, 8, 128)[: lens[i]]
        ref = sdpa_decode_f64(q64[i:i + 1], kp, vp, np.array([0, lens[i]]), b.scale)
        np.testing.assert_allclose(o[i], ref[0], atol=2e-2, rtol=1e-2, err_msg=f"seq {i}")


def test_native_seq_rows_and_bad_pages(gpu):
    b = paged_decode_batch(N=4, Hq=32, Hkv=8, D=128, device=gpu, num_blocks=64, lens=[40, 3, 200, 16],
                           seed=4, layout=LAYOUT_NATIVE)
    rows = [2, 0, 2, 3, 1]
    rows_t = torch.tensor(rows, dtype=torch.int32, device=gpu)
    g = torch.Generator(device=gpu).manual_seed(1)
    q = torch.randn(5, 32, 128, device=gpu, generator=g).to(torch.bfloat16)
    bad = b.block_tables.clone()
    bad[1, 0] = -5  # row 1 (3 tokens) loses its only page -> zero output
    out = ops.paged_decode(q, b.k_store, b.v_store, layout=LAYOUT_NATIVE, block_tables=bad,
                           seq_lens=b.seq_lens, seq_rows=rows_t, max_seqlen=200, scale=b.scale)
    torch.cuda.synchronize()
    kp, vp = _to64(b.k_pool), _to64(b.v_pool)
    o = _to64(out)
    for i, r in enumerate(rows):
        if r == 1:
            np.testing.assert_array_equal(o[i], 0.0)
            continue
        ref = paged_decode_f64(_to64(q)[i:i + 1], kp, vp, [b.tables[r]], [b.lens[r]], 16, b.scale)
        np.testing.assert_allclose(o[i], ref[0], atol=2e-2, rtol=1e-2)


def test_seq_rows_indirection(gpu):
    b = paged_decode_batch(N=5, Hq=32, Hkv=8, D=128, device=gpu, num_blocks=128,
                           lens=[40, 3, 200, 16, 90], seed=3)
    rows = [4, 0, 2, 2]
    rows_t = torch.tensor(rows, dtype=torch.int32, device=gpu)
    q = b.q[:4].contiguous()
    out = ops.paged_decode(q, b.k_store, b.v_store, layout=b.layout, block_tables=b.block_tables, seq_lens=b.seq_lens,
                           seq_rows=rows_t, max_seqlen=200, chunk_tokens=32, scale=b.scale)
    torch.cuda.synchronize()
    ref = paged_decode_f64(_to64(q), _to64(b.k_pool), _to64(b.v_pool),
                           [b.tables[r] for r in rows], [b.lens[r] for r in rows], 16, b.scale)
    np.testing.assert_allclose(_to64(out), ref, atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_packed_varlen_mode(gpu, dtype):
    g = torch.Generator(device=gpu).manual_seed(11)
    lens = [1, 17, 64, 130]
    total = sum(lens)
    Hq, Hkv, D = 8, 2, 64
    k = torch.randn(total, Hkv, D, device=gpu, generator=g).to(dtype)
    v = torch.randn(total, Hkv, D, device=gpu, generator=g).to(dtype)
    q = torch.randn(len(lens), Hq, D, device=gpu, generator=g).to(dtype)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=gpu)
    for chunk in (0, 16):
        out = ops.paged_decode(q, k, v, cu_seqlens_k=cu, max_seqlen=max(lens), chunk_tokens=chunk)
        torch.cuda.synchronize()
        ref = sdpa_decode_f64(_to64(q), _to64(k), _to64(v), cu.cpu().numpy())
        atol, rtol = TOL[dtype]
        np.testing.assert_allclose(_to64(out), ref, atol=atol, rtol=rtol)


def test_out_of_range_page_ids_are_masked(gpu):
    # A table entry outside [0, num_blocks) is skipped, never dereferenced.
    b = paged_decode_batch(N=2, Hq=8, Hkv=2, D=64, device=gpu, num_blocks=32, lens=[40, 40], seed=5)
    bad = b.block_tables.clone()
    bad[0, 1] = 10_000_000  # tokens 16..31 of sequence 0
    out = ops.paged_decode(b.q, b.k_store, b.v_store, layout=b.layout, block_tables=bad, seq_lens=b.seq_lens,
                           max_seqlen=40, scale=b.scale)
    torch.cuda.synchronize()
    kp, vp = _to64(b.k_pool), _to64(b.v_pool)
    # Oracle with the masked page removed: sequence 0 keeps tokens 0..15 and 32..39.
    t0 = b.tables[0]
    k0 = np.concatenate([kp[t0[0]], kp[t0[2]][:8]])
    v0 = np.concatenate([vp[t0[0]], vp[t0[2]][:8]])
    ref0 = sdpa_decode_f64(_to64(b.q)[:1], k0, v0, np.array([0, 24]), b.scale)
    np.testing.assert_allclose(_to64(out)[0], ref0[0], atol=2e-2, rtol=1e-2)


def test_rejects_bad_shapes_on_host(gpu):
    b = paged_decode_batch(N=2, Hq=8, Hkv=2, D=64, device=gpu, num_blocks=16, lens=[10, 20], seed=1)
    with pytest.raises(ValueError):
        ops.paged_decode(b.q, b.k_store, b.v_store, layout=b.layout, block_tables=b.block_tables, seq_lens=b.seq_lens,
                         max_seqlen=10_000)  # table rows too short for max_seqlen
    with pytest.raises(ValueError):
        ops.paged_decode(b.q.float(), b.k_store, b.v_store, layout=b.layout, block_tables=b.block_tables,
                         seq_lens=b.seq_lens, max_seqlen=20)


@pytest.mark.parametrize("layout", [LAYOUT_NATIVE, LAYOUT_REFERENCE])
def test_llama3_8b_shapes_full_size(gpu, layout):
    """The measured workload at full size (64 seqs, ctx U[512,4096], 64k-page pool)."""
    print(f"case full size layout={layout}", flush=True)
    b = paged_decode_batch(device=gpu, layout=layout)
    out = ops.paged_decode(b.q, b.k_store, b.v_store, layout=b.layout, block_tables=b.block_tables, seq_lens=b.seq_lens,
                           max_seqlen=b.max_seqlen, scale=b.scale)
    torch.cuda.synchronize()
    q64 = _to64(b.q)
    o = _to64(out)
    for i in range(b.q.shape[0]):  # per sequence: copy only its pages to the host
        pages = torch.tensor(b.tables[i], dtype=torch.long, device=gpu)
        kp = _to64(b.k_pool[pages]).reshape(-1, 8, 128)[: b.lens[i]]
        vp = _to64(b.v_pool[pages]).reshape(-1, 8, 128)[: b.lens[i]]
        ref = sdpa_decode_f64(q64[i:i + 1], kp, vp, np.array([0, b.lens[i]]), b.scale)
        np.testing.assert_allclose(o[i], ref[0], atol=2e-2, rtol=1e-2, err_msg=f"seq {i}")


def test_native_split_units_repeat_and_shared_workspace(gpu):
    """The native kernel merges split units through arrival counters kept in the
    workspace's reserved prefix. Repeated calls, interleaved with the other
    entry points on the same workspace, must give identical results and leave
    the counters zero."""
    print("case native repeat + shared workspace", flush=True)
    rng = np.random.default_rng(21)
    lens = rng.integers(1, 3000, size=40).tolist()
    b = paged_decode_batch(N=len(lens), Hq=32, Hkv=8, D=128, device=gpu, num_blocks=16384,
                           lens=lens, seed=21, layout=LAYOUT_NATIVE)
    r = paged_decode_batch(N=6, Hq=32, Hkv=8, D=128, device=gpu, num_blocks=512,
                           lens=[900, 17, 2000, 5, 1200, 333], seed=22)

    def native():
        return ops.paged_decode(b.q, b.k_store, b.v_store, layout=LAYOUT_NATIVE, block_tables=b.block_tables,
                                seq_lens=b.seq_lens, max_seqlen=b.max_seqlen, scale=b.scale)

    first = native()
    for _ in range(3):
        ops.paged_decode(r.q, r.k_store, r.v_store, layout=LAYOUT_REFERENCE, block_tables=r.block_tables,
                         seq_lens=r.seq_lens, max_seqlen=r.max_seqlen, chunk_tokens=16, scale=r.scale)
        again = native()
        torch.cuda.synchronize()
        assert torch.equal(first, again)
    ws = ops.workspace(gpu, 1)
    assert int(ws[:262144].count_nonzero()) == 0
    o = _to64(first)
    q64 = _to64(b.q)
    for i in range(0, len(lens), 3):
        pages = torch.tensor(b.tables[i], dtype=torch.long, device=gpu)
        kp = _to64(b.k_pool[pages]).reshape(-1, 8, 128)[: lens[i]]
        vp = _to64(b.v_pool[pages]).reshape(-1, 8, 128)[: lens[i]]
        ref = sdpa_decode_f64(q64[i:i + 1], kp, vp, np.array([0, lens[i]]), b.scale)
        np.testing.assert_allclose(o[i], ref[0], atol=2e-2, rtol=1e-2, err_msg=f"seq {i}")
