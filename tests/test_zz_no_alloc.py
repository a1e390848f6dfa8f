"""face_radial_spline_order_noalloc: the table-cell edge order of face_radial_spline_order with its
sort counters in the library's fixed device scratch (no caller workspace, no allocation), for
callers that cannot allocate. Checked against the existing entry point on the same inputs, on
consecutive calls with shrinking and maximal sizes, and its size refusal without a GPU."""
import ctypes

import pytest
import torch

from face_amd import _lib

SCRATCH = 1 << 20            # FACE_SPLINE_ORDER_SCRATCH (int32 entries)
FACE_ERR_SCRATCH = -4


def test_noalloc_order_refuses_oversized_tables_before_launch():
    L = _lib.lib()
    code = L.face_radial_spline_order_noalloc(None, None, 10, 257, 4096, ctypes.c_float(0.01), None, None)
    assert code == FACE_ERR_SCRATCH
    assert "scratch" in L.face_hip_error_string(code).decode()
    assert L.face_radial_spline_order_noalloc(None, None, 10, 2, 4096, ctypes.c_float(0.0), None, None) == -1


def _orders(E, P, G, seed):
    """(order of the workspace entry point, order of the allocation-free one, table cell of each edge).
    Radii sit mid-interval (the cell is exact) and a tenth lie past the grid (clamped to its last
    interval)."""
    gen = torch.Generator(device="cuda").manual_seed(seed)
    dr = 0.01
    icell = torch.randint(0, G - 1, (E,), generator=gen, device="cuda")
    r = (icell.to(torch.float64) + 0.5).mul(dr).float()
    far = E // 10
    r[:far] = (G + 3) * dr
    icell[:far] = G - 2
    pair = torch.randint(0, P, (E,), generator=gen, device="cuda", dtype=torch.int32)
    cell = pair.long() * G + icell
    work = torch.empty(P * G, dtype=torch.int32, device="cuda")
    o1 = torch.full((E,), -1, dtype=torch.int32, device="cuda")
    o2 = torch.full((E,), -1, dtype=torch.int32, device="cuda")
    st = _lib.stream_of(r)
    print(f"spline order E={E} P={P} G={G}", flush=True)
    _lib.call("face_radial_spline_order", r.data_ptr(), pair.data_ptr(), E, P, G, dr, work.data_ptr(),
              o1.data_ptr(), st)
    _lib.call("face_radial_spline_order_noalloc", r.data_ptr(), pair.data_ptr(), E, P, G, dr, o2.data_ptr(), st)
    torch.cuda.synchronize()
    return o1.long(), o2.long(), cell


def _check(o1, o2, cell):
    E = cell.numel()
    ar = torch.arange(E, device="cuda")
    for o in (o1, o2):
        assert torch.equal(torch.sort(o).values, ar)                  # a permutation of the edges
        c = cell[o]
        assert bool((c[1:] >= c[:-1]).all())                          # grouped by cell, cells ascending
    # same cell at every position; within a cell the order is arbitrary (atomic cursors), so each
    # cell's edges are compared as sets
    assert torch.equal(cell[o1], cell[o2])
    k1 = torch.sort(cell[o1] * E + o1).values
    k2 = torch.sort(cell[o2] * E + o2).values
    assert torch.equal(k1, k2)


@pytest.mark.gpu
def test_noalloc_order_matches_workspace_entry_point():
    # a compiled-radial sized table first, then a smaller input (fewer edges and cells) on the same
    # scratch, then the largest table the scratch holds
    for E, P, G, seed in ((300_000, 9, 4096, 0), (40_000, 4, 1024, 1), (120_000, 256, 4096, 2)):
        assert P * G <= SCRATCH
        _check(*_orders(E, P, G, seed))
