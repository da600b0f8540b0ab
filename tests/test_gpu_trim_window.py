"""trim_to_window on the GPU (core/paged_kv_cache.py:370-417): the product
manager replays the scenarios the reference's own manager recorded
(tests/golden/trim_to_window.json) with K = token tag and V = -tag written
through the HIP append kernel, in the reference pool layout (fp32) and the
native one (bf16, tags < 256 are exact). After every step:
  * host page tables, counters, refcounts and free set equal the vectors;
  * the device table row and lengths of every live sequence and layer equal
    the host lists (the trim re-uploads them);
  * every live sequence's gather (build_packed_kv order) reads the tags the
    reference read, stale slots of a partially trimmed page included; this
    covers the in-place shift of a private page and the copy of a shared one.
At the end, attn_decode over the trimmed cache (zero-copy views, HIP kernel)
matches the float64 oracle over the gathered K/V, with and without a window.

The scenarios copy pages only into blocks no layer has used before. A block
that one layer frees and another reuses would keep the first layer's data in
its unwritten slots here (one store serves every layer), where the reference's
per-layer pool still holds zeros or older data of the second layer.
"""
import json
import os

import numpy as np
import pytest
import torch

from oracle.attention import sdpa_decode_f64

pytestmark = pytest.mark.gpu

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "trim_to_window.json")))
L, NB, OFF = GOLD["num_layers"], GOLD["max_blocks"], GOLD["tag_layer_offset"]
HKV, D = 2, 64

CONFIGS = [(name, dt) for name in sorted(GOLD["cases"]) for dt in (torch.float32, torch.bfloat16)
           if GOLD["cases"][name]["block_size"] == 16 or dt == torch.float32]


def _kv(ts, layer, dtype, dev):
    k = torch.tensor([float(t + OFF * layer) for t in ts], device=dev).view(-1, 1, 1).expand(-1, HKV, D)
    k = k.to(dtype).contiguous()
    return k, (-k).contiguous()


@pytest.mark.parametrize("name,dtype", CONFIGS, ids=[f"{n}-{str(d)[6:]}" for n, d in CONFIGS])
def test_trim_replays_reference_vectors(gpu, name, dtype):
    from mentat_amd._lib import LAYOUT_NATIVE
    from mentat_amd.adapters.attention_backend import attn_decode
    from mentat_amd.core.paged_kv_cache import PagedKVCacheManager

    case = GOLD["cases"][name]
    B = case["block_size"]
    m = PagedKVCacheManager(L, HKV, D, max_blocks=NB, block_size=B, device=gpu, dtype=dtype)
    print(f"case trim {name} {dtype} layout={m.layout}", flush=True)
    assert (m.layout == LAYOUT_NATIVE) == (dtype == torch.bfloat16)
    tag = 0
    for rec in case["steps"]:
        op = rec["step"]
        if op[0] == "alloc":
            m.allocate_sequence()
        elif op[0] == "fork":
            m.fork_sequence(op[1])
        elif op[0] == "free":
            m.free_sequence(op[1])
        elif op[0] == "prefill":
            ts = list(range(tag + 1, tag + 1 + op[2]))
            tag += op[2]
            for layer in range(L):
                m.append_tokens(op[1], layer, *_kv(ts, layer, dtype, gpu))
        elif op[0] == "decode":
            ts = list(range(tag + 1, tag + 1 + len(op[1])))
            tag += len(op[1])
            for layer in range(L):
                m.append_tokens_batched(list(op[1]), layer, *_kv(ts, layer, dtype, gpu))
        elif op[0] == "trim":
            m.trim_to_window(op[1], op[2])
        torch.cuda.synchronize()
        st = rec["state"]
        assert m.allocator.refcounts == st["refcounts"], op
        assert sorted(m.allocator._free) == st["free"], op
        tables, lens = m._tables.cpu(), m._lens.cpu()
        for sid, want in st["seqs"].items():
            seq = m._sequences[int(sid)]
            assert seq.page_table == want["page_table"], (op, sid)
            assert seq.num_tokens == want["num_tokens"], (op, sid)
            assert seq.tokens_in_last_block == want["tokens_in_last_block"], (op, sid)
            for layer in range(L):
                pt = seq.page_table[layer]
                assert tables[layer, seq.row, :len(pt)].tolist() == pt, (op, sid, layer)
                assert int(lens[layer, seq.row]) == seq.num_tokens[layer], (op, sid, layer)
                pk, pv, _, _ = m.gather_packed_kv([int(sid)], layer)
                got = pk[:, 0, 0].float().cpu().numpy()
                assert got.astype(np.int64).tolist() == want["gather"][layer], (op, sid, layer)
                assert torch.equal(pk, pk[:, :1, :1].expand_as(pk)) and torch.equal(pv, -pk), (op, sid, layer)

    # attention over the trimmed cache: the HIP decode through the zero-copy views
    sids = sorted(m._sequences)
    g = torch.Generator(device=gpu).manual_seed(3)
    q = (torch.randn(len(sids), 4 * HKV, D, device=gpu, generator=g) * 0.01).to(dtype)
    for layer in range(L):
        kv, vv, cu, mx = m.build_packed_kv(sids, layer)
        pk, pv, cu2, _ = m.gather_packed_kv(sids, layer)
        for w in (None, 3):
            out = attn_decode(q, kv, vv, None, cu, mx, len(sids), window_size=w)
            torch.cuda.synchronize()
            ref = sdpa_decode_f64(q.double().cpu().numpy(), pk.double().cpu().numpy(), pv.double().cpu().numpy(),
                                  cu2.cpu().numpy(), window_size=w)
            # |V| <= 255: bf16 outputs carry ~1 unit of rounding at that size
            atol, rtol = (1e-3, 1e-4) if dtype == torch.float32 else (1.0, 2e-2)
            np.testing.assert_allclose(out.double().cpu().numpy(), ref, atol=atol, rtol=rtol)
