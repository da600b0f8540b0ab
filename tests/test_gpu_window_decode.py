"""Sliding-window decode on the GPU: mentat_paged_decode with window_size w
attends to each sequence's last w tokens (the reference's flash path,
adapters/attention_backend.py:219-228, window_size=(w - 1, 0) with the query
aligned to the end of its keys), against the float64 oracle. Windows start
inside a tile, on a tile or page boundary, and exceed the context; both pool
layouts, packed varlen, split-K chunks of the reference-layout kernel, split
units of the native stream-K kernel, and attn_decode through the zero-copy
views of the cache manager are covered. Tolerances are the unwindowed
decode's: 2e-2 abs / 1e-2 rel for 16-bit, 1e-4 for fp32."""
import numpy as np
import pytest
import torch

from mentat_amd import ops
from mentat_amd._lib import LAYOUT_NATIVE, LAYOUT_REFERENCE
from mentat_amd.workloads import paged_decode_batch
from oracle.attention import paged_decode_f64, sdpa_decode_f64

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: (2e-2, 1e-2), torch.float16: (2e-2, 1e-2), torch.float32: (1e-4, 1e-4)}
LENS = [1, 15, 16, 17, 31, 250, 513, 1000]
WINDOWS = [1, 7, 16, 17, 100, 512, 4096]


def _to64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _oracle(b, w):
    return paged_decode_f64(_to64(b.q), _to64(b.k_pool), _to64(b.v_pool), b.tables, b.lens, b.block_size,
                            b.scale, window_size=w)


@pytest.mark.parametrize("w", WINDOWS)
@pytest.mark.parametrize("layout,dtype,bs", [(LAYOUT_NATIVE, torch.bfloat16, 16), (LAYOUT_NATIVE, torch.float16, 32),
                                             (LAYOUT_REFERENCE, torch.bfloat16, 16),
                                             (LAYOUT_REFERENCE, torch.float32, 16)])
def test_window_matches_oracle(gpu, layout, dtype, bs, w):
    print(f"case window={w} layout={layout} {dtype} B={bs}", flush=True)
    b = paged_decode_batch(N=len(LENS), Hq=32, Hkv=8, D=128, dtype=dtype, device=gpu, block_size=bs,
                           num_blocks=512, lens=LENS, seed=w + bs, layout=layout)
    ref = _oracle(b, w)
    atol, rtol = TOL[dtype]
    chunks = (0, 16, 64) if layout == LAYOUT_REFERENCE else (0,)
    for chunk in chunks:
        out = ops.paged_decode(b.q, b.k_store, b.v_store, layout=layout, block_tables=b.block_tables,
                               seq_lens=b.seq_lens, max_seqlen=b.max_seqlen, scale=b.scale, chunk_tokens=chunk,
                               window_size=w)
        torch.cuda.synchronize()
        np.testing.assert_allclose(_to64(out), ref, atol=atol, rtol=rtol, err_msg=f"chunk {chunk}")
        if w >= max(LENS):  # a window at least every length is the unwindowed decode, bit for bit
            full = ops.paged_decode(b.q, b.k_store, b.v_store, layout=layout, block_tables=b.block_tables,
                                    seq_lens=b.seq_lens, max_seqlen=b.max_seqlen, scale=b.scale,
                                    chunk_tokens=chunk)
            torch.cuda.synchronize()
            assert torch.equal(out, full), f"chunk {chunk}"


def test_window_native_stream_k_split_units(gpu):
    """300 sequences up to 3000 tokens with a 700-token window: units split
    across workgroups and merged in-kernel; also the Llama-3-8B head shapes."""
    print("case window native stream-K 300 seqs w=700", flush=True)
    rng = np.random.default_rng(31)
    lens = rng.integers(1, 3000, size=300).tolist()
    b = paged_decode_batch(N=len(lens), Hq=32, Hkv=8, D=128, device=gpu, num_blocks=65536, lens=lens, seed=31,
                           layout=LAYOUT_NATIVE)
    w = 700
    out = ops.paged_decode(b.q, b.k_store, b.v_store, layout=LAYOUT_NATIVE, block_tables=b.block_tables,
                           seq_lens=b.seq_lens, max_seqlen=b.max_seqlen, scale=b.scale, window_size=w)
    again = ops.paged_decode(b.q, b.k_store, b.v_store, layout=LAYOUT_NATIVE, block_tables=b.block_tables,
                             seq_lens=b.seq_lens, max_seqlen=b.max_seqlen, scale=b.scale, window_size=w)
    torch.cuda.synchronize()
    assert torch.equal(out, again)
    o, q64 = _to64(out), _to64(b.q)
    for i in range(0, len(lens), 5):
        pages = torch.tensor(b.tables[i], dtype=torch.long, device=gpu)
        kp = _to64(b.k_pool[pages]).reshape(-1, 8, 128)[: lens[i]]
        vp = _to64(b.v_pool[pages]).reshape(-1, 8, 128)[: lens[i]]
        ref = sdpa_decode_f64(q64[i:i + 1], kp, vp, np.array([0, lens[i]]), b.scale, window_size=w)
        np.testing.assert_allclose(o[i], ref[0], atol=2e-2, rtol=1e-2, err_msg=f"seq {i} len {lens[i]}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_window_packed_varlen(gpu, dtype):
    g = torch.Generator(device=gpu).manual_seed(12)
    lens = [1, 17, 64, 130, 300]
    total = sum(lens)
    Hq, Hkv, D = 8, 2, 64
    k = torch.randn(total, Hkv, D, device=gpu, generator=g).to(dtype)
    v = torch.randn(total, Hkv, D, device=gpu, generator=g).to(dtype)
    q = torch.randn(len(lens), Hq, D, device=gpu, generator=g).to(dtype)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=gpu)
    for w in (1, 20, 64, 129):
        ref = sdpa_decode_f64(_to64(q), _to64(k), _to64(v), cu.cpu().numpy(), window_size=w)
        for chunk in (0, 16):
            out = ops.paged_decode(q, k, v, cu_seqlens_k=cu, max_seqlen=max(lens), chunk_tokens=chunk,
                                   window_size=w)
            torch.cuda.synchronize()
            atol, rtol = TOL[dtype]
            np.testing.assert_allclose(_to64(out), ref, atol=atol, rtol=rtol, err_msg=f"w {w} chunk {chunk}")


def test_window_rejected_when_not_positive(gpu):
    b = paged_decode_batch(N=2, Hq=8, Hkv=2, D=64, device=gpu, num_blocks=16, lens=[10, 20], seed=1)
    for w in (0, -3):
        with pytest.raises(ValueError):
            ops.paged_decode(b.q, b.k_store, b.v_store, block_tables=b.block_tables, seq_lens=b.seq_lens,
                             max_seqlen=b.max_seqlen, window_size=w)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_attn_decode_window_through_the_manager(gpu, dtype):
    """attn_decode(window_size=w) on the manager's zero-copy views of a forked
    batch equals the oracle over build_packed_kv's gather with the last w
    tokens kept."""
    from mentat_amd.adapters.attention_backend import attn_decode
    from mentat_amd.core.paged_kv_cache import PagedKVCacheManager

    print(f"case attn_decode window via manager {dtype}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(5)
    Hq, Hkv, D, Lyr = 16, 4, 128, 2
    m = PagedKVCacheManager(Lyr, Hkv, D, max_blocks=256, block_size=16, device=gpu, dtype=dtype)
    s0 = m.allocate_sequence()
    for layer in range(Lyr):
        m.append_tokens(s0, layer, torch.randn(70, Hkv, D, device=gpu, generator=g).to(dtype),
                        torch.randn(70, Hkv, D, device=gpu, generator=g).to(dtype))
    kids = [m.fork_sequence(s0) for _ in range(3)]
    seqs = [s0] + kids
    for step in range(21):
        live = seqs if step < 9 else seqs[:3]
        for layer in range(Lyr):
            m.append_tokens_batched(live, layer, torch.randn(len(live), Hkv, D, device=gpu, generator=g).to(dtype),
                                    torch.randn(len(live), Hkv, D, device=gpu, generator=g).to(dtype))
    q = torch.randn(len(seqs), Hq, D, device=gpu, generator=g).to(dtype)
    for layer in range(Lyr):
        kv, vv, cu, mx = m.build_packed_kv(seqs, layer)
        pk, pv, cu2, _ = m.gather_packed_kv(seqs, layer)
        for w in (5, 16, 33, 90, 1000):
            out = attn_decode(q, kv, vv, None, cu, mx, len(seqs), window_size=w)
            torch.cuda.synchronize()
            ref = sdpa_decode_f64(_to64(q), _to64(pk), _to64(pv), cu2.cpu().numpy(), window_size=w)
            atol, rtol = TOL[dtype]
            np.testing.assert_allclose(_to64(out), ref, atol=atol, rtol=rtol, err_msg=f"layer {layer} w {w}")
