"""Symmetric Cartesian storage used by FACE (oracle restatement of face/cartesian.py:11-81).

Rank-l symmetric tensors over R^3 are stored by their distinct components, one per sorted
index tuple, in the component order of face/cartesian.py:11-17 (1 + 3 + 6 + 10 = 20).

Pinned by: the tables are checked against their defining properties in
tests/test_oracle.py (every sorted tuple appears once, expand() of the monomials equals the
explicit outer products u^{(x)l}, multiplicities sum to 3^l).
"""
import itertools

import torch

SYM_IDX = {
    0: [()],
    1: [(0,), (1,), (2,)],
    2: [(0, 0), (1, 1), (2, 2), (0, 1), (0, 2), (1, 2)],
    3: [(0, 0, 0), (1, 1, 1), (2, 2, 2), (0, 0, 1), (0, 0, 2), (0, 1, 1),
        (1, 1, 2), (0, 2, 2), (1, 2, 2), (0, 1, 2)],
}
RANK_SLICE = {0: slice(0, 1), 1: slice(1, 4), 2: slice(4, 10), 3: slice(10, 20)}
# weights turning sym-storage rank-2 components into u^T M u (off-diagonals appear twice)
Y2_WEIGHT = torch.tensor([1.0, 1.0, 1.0, 2.0, 2.0, 2.0])


def full_to_sym_index(l):
    """Full-tensor flat index (row-major over l axes) -> symmetric component index."""
    pos = {t: k for k, t in enumerate(SYM_IDX[l])}
    return torch.tensor([pos[tuple(sorted(t))] for t in itertools.product(range(3), repeat=l)],
                        dtype=torch.long)


def monomials(u):
    """(...,3) -> (...,20): products u_a u_b ... over each sorted tuple, left to right."""
    cols = []
    for l in range(4):
        for t in SYM_IDX[l]:
            if not t:
                cols.append(torch.ones_like(u[..., 0]))
                continue
            v = u[..., t[0]]
            for a in t[1:]:
                v = v * u[..., a]
            cols.append(v)
    return torch.stack(cols, -1)


def expand(sym, l):
    """(..., k_l) symmetric components -> (..., 3, ..., 3) full rank-l tensor (index gather)."""
    if l == 0:
        return sym
    idx = full_to_sym_index(l).to(sym.device)
    return sym[..., idx].reshape(*sym.shape[:-1], *([3] * l))


def to_sym2(Mfull):
    """(...,3,3) -> (...,6) components xx,yy,zz,xy,xz,yz (upper triangle)."""
    return torch.stack([Mfull[..., a, b] for (a, b) in SYM_IDX[2]], -1)
