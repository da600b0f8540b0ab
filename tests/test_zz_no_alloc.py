"""mentat_paged_decode_noalloc (the allocation-free entry point: its workspace is
a static device array inside the library) against mentat_paged_decode with a
caller-allocated workspace, both called through the C ABI on the same inputs.

Two calls in a row on the static scratch, the second with a smaller input, must
each equal the workspace entry point's output bit for bit (the same kernels
with the same partition; partials are merged in a fixed order). Covered: the
native-layout MFMA path at the Llama-3-8B shapes of the paged-decode workload
(64 sequences, contexts 512-4096, split units in the scratch) and the
reference-layout path with split-K chunks (fp32). Sizes past the scratch are
refused with MENTAT_ESPACE before any launch.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _call(lib, fn, b, out, *, layout, dtype_code, chunk=0, ws=None):
    from mentat_amd._lib import ptr, stream_handle

    N, Hq, D = b.q.shape
    Hkv = b.k_pool.shape[2]
    args = [layout, ptr(b.q), ptr(b.k_store), ptr(b.v_store), ptr(b.block_tables), b.block_tables.shape[1],
            None, ptr(b.seq_lens), None, b.k_store.shape[0], ptr(out), N, Hq, Hkv, D, b.block_size,
            b.max_seqlen, 0, b.scale, dtype_code, chunk]
    if fn == "mentat_paged_decode":
        args += [ptr(ws), ws.numel()]
    args.append(stream_handle(b.q.device))
    return getattr(lib, fn)(*args)


def _both(lib, b, *, layout, dtype_code, chunk=0):
    from mentat_amd._lib import MENTAT_OK

    N, Hq, D = b.q.shape
    Hkv = b.k_pool.shape[2]
    need = lib.mentat_paged_decode_workspace_bytes(layout, N, Hq, Hkv, D, b.block_size, b.max_seqlen, 0, chunk)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=b.q.device)
    ref = torch.empty_like(b.q)
    got = torch.full_like(b.q, float("nan"))
    assert _call(lib, "mentat_paged_decode", b, ref, layout=layout, dtype_code=dtype_code, chunk=chunk,
                 ws=ws) == MENTAT_OK
    assert _call(lib, "mentat_paged_decode_noalloc", b, got, layout=layout, dtype_code=dtype_code,
                 chunk=chunk) == MENTAT_OK
    torch.cuda.synchronize()
    return ref, got


def test_noalloc_native_matches_workspace_entry(gpu):
    from mentat_amd._lib import LAYOUT_NATIVE, get_lib
    from mentat_amd.workloads import paged_decode_batch

    lib = get_lib()
    print("case noalloc native: 64 seqs ctx 512-4096 (Llama-3-8B heads), then 9 seqs", flush=True)
    big = paged_decode_batch(N=64, seed=0, layout=LAYOUT_NATIVE, device=gpu)
    ref, got = _both(lib, big, layout=LAYOUT_NATIVE, dtype_code=2)
    assert torch.equal(ref, got)
    del big
    small = paged_decode_batch(N=9, seed=1, ctx_lo=1, ctx_hi=700, num_blocks=4096, layout=LAYOUT_NATIVE,
                               device=gpu)
    ref, got = _both(lib, small, layout=LAYOUT_NATIVE, dtype_code=2)
    assert torch.equal(ref, got)


def test_noalloc_reference_layout_split_chunks(gpu):
    from mentat_amd._lib import LAYOUT_REFERENCE, get_lib
    from mentat_amd.workloads import paged_decode_batch

    lib = get_lib()
    print("case noalloc reference layout fp32, chunked: 12 seqs then 5 seqs", flush=True)
    a = paged_decode_batch(N=12, Hq=4, Hkv=2, D=64, ctx_lo=100, ctx_hi=1500, num_blocks=2048, seed=2,
                           dtype=torch.float32, device=gpu)
    ref, got = _both(lib, a, layout=LAYOUT_REFERENCE, dtype_code=0, chunk=128)
    assert torch.equal(ref, got)
    b = paged_decode_batch(N=5, Hq=4, Hkv=2, D=64, ctx_lo=1, ctx_hi=300, num_blocks=2048, seed=3,
                           dtype=torch.float32, device=gpu)
    ref, got = _both(lib, b, layout=LAYOUT_REFERENCE, dtype_code=0, chunk=64)
    assert torch.equal(ref, got)


def test_noalloc_refuses_sizes_past_the_scratch(gpu):
    from mentat_amd._lib import LAYOUT_NATIVE, MENTAT_ESPACE, get_lib, stream_handle

    lib = get_lib()
    print("case noalloc size limit", flush=True)
    # 4096 sequences x 8 kv heads of native split units need ~70 MB of partial slots
    assert lib.mentat_paged_decode_workspace_bytes(LAYOUT_NATIVE, 4096, 32, 8, 128, 16, 4096, 0, 0) > 8388608
    # refused on the size alone: the small buffers below are never read
    t = torch.zeros(64, dtype=torch.int32, device=gpu)
    p = t.data_ptr()
    st = lib.mentat_paged_decode_noalloc(LAYOUT_NATIVE, p, p, p, p, 4, None, p, None, 1, p, 4096, 32, 8,
                                         128, 16, 4096, 0, 0.088, 2, 0, stream_handle(gpu))
    assert st == MENTAT_ESPACE
    torch.cuda.synchronize()
