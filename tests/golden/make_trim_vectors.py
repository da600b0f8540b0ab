"""Writes trim_to_window.json: what the reference's PagedKVCacheManager
(core/paged_kv_cache.py:104-417) holds after scripted allocate / prefill /
fork / decode / free / trim_to_window scenarios, on the CPU with float32 pools
whose K values are token tags (V = -tag), so every slot's contents can be read
back exactly.

Run only where the reference sources are readable (the build container):
    python tests/golden/make_trim_vectors.py /root/reference
The fixture holds inputs (the scenario steps) and outputs (per step: page
tables, token counters, refcounts, free set, and every live sequence's
build_packed_kv gather as tags; at the end, every block's tags per layer); no
reference code is copied into it.

Tags: token j appended by the scenario (counting from 1) is stored as
j + 128 * layer, so tags stay below 256 (exact in bfloat16).
"""
import json
import os
import sys

L = 2
MAX_BLOCKS = 48


def scenarios(B: int) -> dict:
    """Step lists. ("alloc",) / ("fork", parent) name the new sequence by the
    order the manager hands ids out (0, 1, ...)."""
    return {
        # trim inside the second page of a private sequence, then decode and trim again
        "private_partial": [("alloc",), ("prefill", 0, 2 * B + 5), ("trim", 0, B + 3), ("decode", [0]),
                            ("decode", [0]), ("decode", [0]), ("trim", 0, B + 1)],
        # a forked child trims inside a page it shares with its parent (copy-on-write of
        # the kept tail), then both decode; the parent trims across a shared page boundary
        "shared_partial": [("alloc",), ("prefill", 0, 2 * B + 3), ("fork", 0), ("trim", 1, B + 5),
                           ("decode", [0, 1]), ("trim", 0, B), ("decode", [0, 1]), ("free", 1),
                           ("decode", [0])],
        # whole pages evicted; a window at least the length leaves the sequence alone
        "page_aligned": [("alloc",), ("prefill", 0, 3 * B), ("trim", 0, B), ("decode", [0]),
                         ("trim", 0, B + 1), ("trim", 0, 4 * B)],
        # trim to zero tokens keeps the partially evicted last page in the table
        "to_zero": [("alloc",), ("prefill", 0, B + 2), ("trim", 0, 0), ("decode", [0]), ("decode", [0])],
        # a three-leaf tree: tails copied on decode, one leaf freed, another trimmed privately,
        # a new prompt prefilled and trimmed by one token
        "tree": [("alloc",), ("prefill", 0, B + 3), ("fork", 0), ("fork", 0), ("decode", [0, 1, 2]),
                 ("trim", 2, 3), ("free", 1), ("decode", [0, 2]), ("alloc",), ("prefill", 3, B),
                 ("trim", 3, B - 1), ("decode", [0, 2, 3])],
    }


def run(Manager, torch, B: int, steps: list) -> dict:
    m = Manager(L, 1, 1, max_blocks=MAX_BLOCKS, block_size=B, device="cpu", dtype=torch.float32)
    tag = [0]

    def tags(n):
        t = list(range(tag[0] + 1, tag[0] + 1 + n))
        tag[0] += n
        return t

    def kv(ts, layer):
        k = torch.tensor([float(t + 128 * layer) for t in ts], dtype=torch.float32).view(-1, 1, 1)
        return k, -k

    def snapshot():
        seqs = {}
        for sid, st in sorted(m._sequences.items()):
            gathers = []
            for layer in range(L):
                pk, pv, cu, _ = m.build_packed_kv([sid], layer)
                gathers.append([int(x) for x in pk.view(-1).tolist()])
            seqs[str(sid)] = {"page_table": [list(t) for t in st.page_table], "num_tokens": list(st.num_tokens),
                              "tokens_in_last_block": list(st.tokens_in_last_block), "gather": gathers}
        return {"seqs": seqs, "refcounts": list(m.allocator.refcounts), "free": sorted(m.allocator._free)}

    out = []
    for step in steps:
        op = step[0]
        if op == "alloc":
            m.allocate_sequence()
        elif op == "fork":
            m.fork_sequence(step[1])
        elif op == "free":
            m.free_sequence(step[1])
        elif op == "prefill":
            ts = tags(step[2])
            for layer in range(L):
                k, v = kv(ts, layer)
                m.append_tokens(step[1], layer, k, v)
        elif op == "decode":
            ts = tags(len(step[1]))
            for layer in range(L):
                k, v = kv(ts, layer)
                m.append_tokens_batched(list(step[1]), layer, k, v)
        elif op == "trim":
            m.trim_to_window(step[1], step[2])
        else:
            raise ValueError(op)
        out.append({"step": list(step), "state": snapshot()})
    pools = [[[int(x) for x in m.k_pools[layer][b].view(-1).tolist()] for b in range(MAX_BLOCKS)]
             for layer in range(L)]
    vneg = all(torch.equal(m.v_pools[layer], -m.k_pools[layer]) for layer in range(L))
    return {"steps": out, "k_pools": pools, "v_is_minus_k": vneg}


def main() -> None:
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path.insert(0, ref)
    import torch

    from core.paged_kv_cache import PagedKVCacheManager  # the reference's manager

    cases = {}
    for B in (4, 16):
        for name, steps in scenarios(B).items():
            cases[f"{name}_B{B}"] = {"block_size": B, **run(PagedKVCacheManager, torch, B, steps)}
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "trim_to_window.json")
    with open(out, "w") as f:
        json.dump({"source": "core/paged_kv_cache.py:104-417 PagedKVCacheManager (trim_to_window :370-417)",
                   "num_layers": L, "max_blocks": MAX_BLOCKS, "tag_layer_offset": 128, "cases": cases}, f,
                  separators=(",", ":"))
    print(f"wrote {out}: {len(cases)} cases")


if __name__ == "__main__":
    main()
