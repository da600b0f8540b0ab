"""Grouped paged decode (mentat_paged_decode_grouped) on the GPU: decode over
forests of forked sequences (block ids shared as fork_sequence shares them,
core/paged_kv_cache.py:152-170, grown with the oracle cache's bookkeeping),
with each shared page read once per group of queries, against
  * the float64 oracle (build_packed_kv gather + SDPA, oracle/attention.py),
    2e-2 abs / 1e-2 rel, and
  * the plain native paged kernel on the same batch (same tolerance; the two
    differ only in summation order).
Covered: G = 1, 2, 4, 8 (one to eight queries per MFMA tile), kv-head teams
(Hkv % 4 == 0) and single heads, pages of 16 and 32 tokens, bf16 and f16,
depth-first and shuffled batch orders, table rows different from batch
indices, zero-length queries, n_segs below the plan's capacity, long shared
prefixes split across workgroups (stream-K pieces), and repeated calls
(bit-identical, counters left zero)."""
import random

import numpy as np
import pytest
import torch

from mentat_amd import ops
from mentat_amd._lib import LAYOUT_NATIVE
from mentat_amd.group_plan import build_group_plan
from oracle.attention import sdpa_decode_f64
from oracle.paged_cache import OracleCache

pytestmark = pytest.mark.gpu


def _forest(seed, B, roots, prompt, leaves, steps, nb):
    rng = random.Random(seed)
    c = OracleCache(1, nb, B)
    trees = []
    for _ in range(roots):
        r = c.allocate()
        c.append(r, 0, [0] * rng.randint(prompt // 2, prompt))
        trees.append([r])
    for _ in range(steps):
        t = rng.choice(trees)
        leaf = rng.choice(t)
        if rng.random() < 0.25 and len(t) < leaves:
            t.insert(t.index(leaf) + 1, c.fork(leaf))
        else:
            for s in t:
                n = rng.randint(0, 3)
                for _ in range(n):
                    c.append_batched([s], 0, [0])
    return c, [s for t in trees for s in t]


class _Batch:
    def __init__(self, c, order, Hq, Hkv, D, B, nb, dtype, dev, seed, zero_len=()):
        N = len(order)
        g = torch.Generator(device=dev).manual_seed(seed)
        self.k = torch.randn(nb, Hkv, B, D, generator=g, device=dev).to(dtype)
        self.v = torch.randn(nb, Hkv, D, B, generator=g, device=dev).to(dtype)
        self.q = torch.randn(N, Hq, D, generator=g, device=dev).to(dtype)
        self.lens = [0 if i in zero_len else c.ntok[s][0] for i, s in enumerate(order)]
        self.tables = [c.tables[s][0] for s in order]
        P = max(1, max(len(t) for t in self.tables))
        perm = np.random.default_rng(seed).permutation(N) + 2          # table rows != batch indices
        tab = np.zeros((N + 2, P), dtype=np.int32)
        lens_rows = np.zeros(N + 2, dtype=np.int32)
        for i, t in enumerate(self.tables):
            tab[perm[i], :len(t)] = t
            lens_rows[perm[i]] = self.lens[i]
        self.rows = perm
        self.tab_host = tab[perm]
        self.tab = torch.from_numpy(tab).to(dev)
        self.seq_lens = torch.from_numpy(lens_rows).to(dev)
        self.rows_t = torch.from_numpy(perm.astype(np.int32)).to(dev)
        self.B, self.D, self.Hkv, self.scale = B, D, Hkv, D ** -0.5

    def plan(self, per_tile):
        p = build_group_plan(self.tab_host, np.array(self.lens), self.rows, self.B, per_tile)
        p.validate(len(self.lens), self.tab.shape[0], self.tab.shape[1], self.B, per_tile)
        return p

    def grouped(self, plan, max_segs=None):
        segs, n, off, lst = ops.group_plan_device(plan, self.q.device, max_segs)
        return ops.paged_decode_grouped(self.q, self.k, self.v, block_tables=self.tab, seq_lens=self.seq_lens,
                                        segs=segs, n_segs=n, seg_off=off, seg_list=lst, scale=self.scale)

    def plain(self):
        return ops.paged_decode(self.q, self.k, self.v, layout=LAYOUT_NATIVE, block_tables=self.tab,
                                seq_lens=self.seq_lens, seq_rows=self.rows_t,
                                max_seqlen=max(1, max(self.lens)), scale=self.scale)

    def oracle(self, idx):
        q64 = self.q[idx].double().cpu().numpy()
        out = []
        for n, i in enumerate(idx):
            L = self.lens[i]
            if L == 0:
                out.append(np.zeros(q64.shape[1:]))
                continue
            pages = torch.tensor(self.tables[i], dtype=torch.long, device=self.q.device)
            kp = self.k[pages].permute(0, 2, 1, 3).reshape(-1, self.Hkv, self.D)[:L].double().cpu().numpy()
            vp = self.v[pages].permute(0, 3, 1, 2).reshape(-1, self.Hkv, self.D)[:L].double().cpu().numpy()
            out.append(sdpa_decode_f64(q64[n:n + 1], kp, vp, np.array([0, L]), self.scale)[0])
        return np.stack(out)


CASES = [
    # Hq, Hkv, B, dtype
    (32, 8, 16, torch.bfloat16),
    (16, 8, 16, torch.bfloat16),
    (64, 8, 32, torch.float16),
    (8, 8, 16, torch.bfloat16),
    (8, 2, 16, torch.bfloat16),
    (4, 4, 32, torch.bfloat16),
]


@pytest.mark.parametrize("shuffle", [False, True])
@pytest.mark.parametrize("Hq,Hkv,B,dtype", CASES)
def test_grouped_matches_oracle_and_plain_kernel(gpu, Hq, Hkv, B, dtype, shuffle):
    print(f"case grouped Hq={Hq} Hkv={Hkv} B={B} {dtype} shuffle={shuffle}", flush=True)
    nb = 2048
    c, order = _forest(Hq + B, B, roots=3, prompt=300, leaves=9, steps=60, nb=nb)
    if shuffle:
        random.Random(1).shuffle(order)
    b = _Batch(c, order, Hq, Hkv, 128, B, nb, dtype, gpu, seed=Hq * 7 + B, zero_len=(2,))
    per_tile = 16 // (Hq // Hkv)
    plan = b.plan(per_tile)
    got = b.grouped(plan)
    ref = b.plain()
    torch.cuda.synchronize()
    if not shuffle:
        assert plan.tiles_read() < sum((n + 15) // 16 for n in b.lens)   # shared pages read fewer times
    assert torch.equal(got[2], torch.zeros_like(got[2]))
    np.testing.assert_allclose(got.double().cpu().numpy(), ref.double().cpu().numpy(), atol=2e-2, rtol=1e-2)
    idx = list(range(len(order)))
    np.testing.assert_allclose(got.double().cpu().numpy()[idx], b.oracle(idx), atol=2e-2, rtol=1e-2)


def test_grouped_long_shared_prefixes_repeat_and_capacity(gpu):
    """Four trees of up to 32 leaves under ~2k-token prompts (the prefix-tree
    decode workload's shape at Qwen3-8B heads): shared segments split across
    workgroups. Three calls are bit-identical, the arrival counters are left
    zero, and a plan uploaded with spare capacity (n_segs < max_segs) gives
    the same output."""
    print("case grouped long prefixes, 4 trees x 32 leaves", flush=True)
    nb = 16384
    c, order = _forest(5, 16, roots=4, prompt=2048, leaves=32, steps=400, nb=nb)
    b = _Batch(c, order, 32, 8, 128, 16, nb, torch.bfloat16, gpu, seed=9)
    plan = b.plan(4)
    first = b.grouped(plan)
    for _ in range(2):
        again = b.grouped(plan)
        torch.cuda.synchronize()
        assert torch.equal(first, again)
    spare = b.grouped(plan, max_segs=plan.n_segs + 37)
    torch.cuda.synchronize()
    assert torch.equal(first, spare)
    ws = ops.workspace(gpu, 1)
    assert int(ws[:262144].count_nonzero()) == 0
    ref = b.plain()
    torch.cuda.synchronize()
    np.testing.assert_allclose(first.double().cpu().numpy(), ref.double().cpu().numpy(), atol=2e-2, rtol=1e-2)
    idx = list(range(0, len(order), 5))
    np.testing.assert_allclose(first.double().cpu().numpy()[idx], b.oracle(idx), atol=2e-2, rtol=1e-2)
    print(f"  {len(order)} queries, {plan.n_segs} segments, tiles read {plan.tiles_read()} vs "
          f"{sum((n + 15) // 16 for n in b.lens)} unshared", flush=True)
