"""Host-side layout of the captured step's split down projection
(core/graph_decode.py): the weight copy in slices and the batched product
over them, on the CPU in float64 (no kernels involved)."""
import torch

from mentat_amd.core.graph_decode import _project, _split_copy


def test_split_copy_is_the_transpose_in_row_slices():
    H, F, S = 6, 16, 4
    t = torch.arange(H * F, dtype=torch.float64).view(H, F)
    w = torch.empty(S, F // S, H, dtype=torch.float64)
    _split_copy(w, t)
    for s in range(S):
        for f in range(F // S):
            for h in range(H):
                assert w[s, f, h] == t[h, s * (F // S) + f]


def test_slice_products_sum_to_the_linear():
    """act split into column slices, times the matching weight slices, summed
    over the slices: the un-split linear (up to summation order)."""
    g = torch.Generator().manual_seed(0)
    H, F, S, rows = 8, 32, 4, 5
    t = torch.randn(H, F, generator=g, dtype=torch.float64)
    act = torch.randn(rows, F, generator=g, dtype=torch.float64)
    w = torch.empty(S, F // S, H, dtype=torch.float64)
    _split_copy(w, t)
    slices = act.view(rows, S, F // S).permute(1, 0, 2)
    parts = torch.bmm(slices, w)
    assert torch.allclose(parts.sum(0), torch.nn.functional.linear(act, t), rtol=0, atol=1e-12)


def test_project_times_an_unsplit_weight_as_linear():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(3, 8, generator=g)
    t = torch.randn(5, 8, generator=g)
    assert torch.equal(_project(x, t), torch.nn.functional.linear(x, t))
