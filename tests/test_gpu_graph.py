"""GPU pair-list build vs the fp64 brute-force oracle: bit-exact pair sets, canonical order,
bit-exact shifts, reverse map and padded view (face/neighbors.py:7-37)."""
import sys

import numpy as np
import pytest
import torch

from oracle.neighbors import pair_list, pair_list_cells, padded_graph as oracle_padded

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def oracle_csr(structures, rc, pairs=pair_list):
    I, J, S, off = [], [], [], 0
    for st in structures:
        i, j, s = pairs(st["pos"], st["cell"], st["pbc"], rc)
        I.append(i + off); J.append(j + off); S.append(s)
        off += len(st["pos"])
    return np.concatenate(I), np.concatenate(J), np.concatenate(S)


def check_graph(structures, rc, method="auto", pairs=pair_list):
    from face_amd.neighbors import build_graph
    g = build_graph(structures, rc, method=method)
    i, j, S = oracle_csr(structures, rc, pairs)
    recv, col, Sg = g.recv.cpu().numpy(), g.col.cpu().numpy(), g.S.cpu().numpy()
    assert len(col) == len(j), (len(col), len(j))
    assert np.array_equal(recv, i) and np.array_equal(col, j) and np.array_equal(Sg, S)
    cells = np.concatenate([np.repeat(np.asarray(st["cell"], np.float64)[None], len(st["pos"]), 0)
                            for st in structures])
    sv = np.einsum("ea,eab->eb", S.astype(np.float64), cells[i])
    assert np.array_equal(g.shift.cpu().numpy(), sv.astype(np.float32))
    rev = g.rev.cpu().numpy()
    assert np.array_equal(col[rev], recv) and np.array_equal(recv[rev], col) and np.array_equal(Sg[rev], -Sg)
    assert np.array_equal(rev[rev], np.arange(len(rev)))
    return g


def test_molecule_batch_exact():
    from face_amd import systems
    say("molecule batch")
    check_graph(systems.molecules(64, systems.stream(0)), 4.5)


def test_fcc_864_exact():
    from face_amd import systems
    say("fcc 864")
    st = systems.fcc(4.09, 6, 0.1, systems.stream(2))
    g = check_graph([st], 4.5)
    assert g.max_row == 18


@pytest.mark.parametrize("method", ["cell", "small"])
def test_liquid_3000_exact(method):
    from face_amd import systems
    say("liquid 3000", method)
    st = systems.liquid(3000, np.random.default_rng(5))
    check_graph([st], 5.0, method=method)


@pytest.mark.parametrize("k", [3, 4])
def test_liquid_full_size_exact(k):
    """The 24,000-atom (1.25 M pairs) and 100,000-atom (6.9 M pairs) liquids at full size against
    the bin-candidate fp64 oracle (equal to the brute-force one, pinned on the CPU)."""
    from face_amd import systems
    sts, kw, el, desc = systems.workload(k)
    say("full-size pair list", desc)
    g = check_graph(sts, kw["rc"], pairs=pair_list_cells)
    say(f"  N {g.N} E {g.E} max_row {g.max_row}")
    assert g.N == len(sts[0]["pos"]) and g.E > (1_000_000 if k == 3 else 6_000_000)


@pytest.mark.parametrize("method", ["cell", "small"])
def test_triclinic_and_thin_cells(method):
    say("triclinic", method)
    rng = np.random.default_rng(8)
    cell = np.array([[6.1, 0.0, 0.0], [2.3, 5.7, 0.0], [-1.1, 1.7, 4.2]])   # thinner than 2 rc along c
    pos = rng.random((70, 3)) @ cell + rng.normal(0, 3.0, (70, 3))       # unwrapped positions
    st = {"pos": pos, "Z": np.full(70, 6), "cell": cell, "pbc": np.ones(3, bool)}
    check_graph([st], 4.5, method=method)


def test_mixed_pbc_and_empty_rows():
    say("mixed pbc")
    rng = np.random.default_rng(3)
    cell = np.diag([7.0, 30.0, 7.5])
    st1 = {"pos": rng.random((25, 3)) @ cell, "Z": np.full(25, 8), "cell": cell, "pbc": np.array([1, 0, 1], bool)}
    st2 = {"pos": np.array([[0.0, 0, 0], [20.0, 0, 0]]), "Z": np.array([1, 1]), "cell": np.zeros((3, 3)),
           "pbc": np.zeros(3, bool)}                                      # two isolated atoms
    check_graph([st1, st2], 4.0)


def test_boundary_decisions_match_fp64_oracle():
    """Pairs within a few ulp of rc: the accept test (fp64, fixed order, correctly rounded
    sqrt) must agree with the oracle bit for bit."""
    say("boundary ulps")
    rng = np.random.default_rng(11)
    rc = 4.5
    n = 400
    dirs = rng.normal(size=(n, 3))
    dirs /= np.linalg.norm(dirs, axis=1, keepdims=True)
    scale = rc * (1 + rng.integers(-6, 7, n) * np.finfo(np.float64).eps)
    pos = []
    for k in range(n):
        a = rng.uniform(-50, 50, 3)
        pos += [a, a + dirs[k] * scale[k]]
    pos = np.asarray(pos)
    structures = [{"pos": pos[2 * k:2 * k + 2], "Z": np.array([1, 1]), "cell": np.zeros((3, 3)),
                   "pbc": np.zeros(3, bool)} for k in range(n)]
    g = check_graph(structures, rc)
    say("accepted pairs", g.E, "of", 2 * n)


def test_padded_view_matches_reference_layout():
    from face_amd import systems
    from face_amd.neighbors import padded_graph
    say("padded view")
    mols = systems.molecules(5, np.random.default_rng(4))
    box = [systems.fcc(4.09, 2, 0.1, np.random.default_rng(1))]
    for sts in (mols, box):
        got = padded_graph(sts, 4.5)
        want = oracle_padded(sts, 4.5)
        assert np.array_equal(got["nbr"].cpu().numpy(), want["nbr"].numpy())
        assert np.array_equal(got["mask"].cpu().numpy(), want["mask"].numpy())
        assert np.array_equal(got["shift"].cpu().numpy(), want["shift"].numpy())
        assert np.array_equal(got["batch"].cpu().numpy(), want["batch"].numpy())
        assert np.array_equal(got["pos"].cpu().numpy(), want["pos"].numpy())
