"""Hot-path operators as textbook einsums (oracle; CPU, any dtype, autograd for gradients).

Every function here restates a reference computation from its mathematics, not from the
reference's bmm/broadcast tricks, so a transposed operand or dropped term in either
shows up as a mismatch.
"""
import torch

from .cartesian import expand, to_sym2


def factor_density(phi, msg, Y):
    """D[i,x,b*K+k] = sum_m phi[i,m,b] msg[i,m,k] Y[i,m,x]   (face/kernels.py:170-178).

    phi (N,M,B), msg (N,M,K), Y (N,M,X) -> (N,X,B*K). Gradients by autograd.
    Pinned by: brute-force loops on tiny inputs and the reference tolerance spec
    (tests/test_kernels.py:7-20) in tests/test_oracle.py.
    """
    N, M, B = phi.shape
    K = msg.shape[-1]
    return torch.einsum("nmb,nmk,nmx->nxbk", phi, msg, Y).reshape(N, Y.shape[-1], B * K)


def cp_density(R, msg, Y):
    """CP pooling A[i,x,c] = sum_m R[i,m,l(x),c] msg[i,m,c] Y[i,m,x]  (face/model.py:496-502).

    R (N,M,4,C), msg (N,M,C), Y (N,M,20) -> (N,20,C), where l(x) is the rank of monomial x.
    This is the rank-diagonal part of the reference's (N,20,4,C) bmm.
    """
    from .cartesian import RANK_SLICE
    return torch.cat([torch.einsum("nmc,nmx->nxc", R[:, :, l] * msg, Y[..., RANK_SLICE[l]]) for l in range(4)], 1)


def node_algebra_full(P1, Q1, S1, P2, Q2, S2, P3, Q3, a, b):
    """Invariants and gated products on FULL tensors (face/node_kernel.py:212-228,
    face/model.py:252-264,288-291).

    P1,Q1,S1 (...,3); P2,Q2,S2 (...,3,3); P3,Q3 (...,3,3,3); a,b (4,C) broadcast over the
    channel axis (second to last of the leading dims).
    Returns inv (...,8), V (...,3), Mf (...,3,3) (Mf not symmetrised).
    Pinned by: rotation invariance / equivariance and hand-expanded tiny cases in
    tests/test_oracle.py.
    """
    e = torch.einsum
    PQ2 = e("...ab,...bd->...ad", P2, Q2)
    inv = torch.stack([
        e("...a,...a->...", P1, Q1),
        e("...ab,...ab->...", P2, Q2),
        e("...abc,...abc->...", P3, Q3),
        e("...a,...ab,...b->...", P1, Q2, S1),
        e("...ad,...da->...", PQ2, S2),
        e("...abc,...bc,...a->...", P3, Q2, S1),
        e("...abd,...abe,...de->...", P3, Q3, S2),
        e("...abd,...a,...b,...d->...", P3, Q1, S1, Q1),
    ], -1)
    aa = a.t()                                                    # (C,4)
    bb = b.t()
    V = (aa[:, 0, None] * P1 + aa[:, 1, None] * e("...ab,...b->...a", Q2, S1)
         + aa[:, 2, None] * e("...abc,...bc->...a", P3, Q2) + aa[:, 3, None] * e("...ab,...b->...a", P2, Q1))
    Mf = (bb[:, 0, None, None] * P2 + bb[:, 1, None, None] * e("...a,...b->...ab", P1, Q1)
          + bb[:, 2, None, None] * PQ2 + bb[:, 3, None, None] * e("...abc,...c->...ab", P3, S1))
    return inv, V, Mf


def node_algebra_sym(P1, Q1, S1, P2, Q2, S2, P3, Q3, a, b):
    """Same as node_algebra_full but with rank-2/3 inputs in symmetric storage (6 / 10)."""
    return node_algebra_full(P1, Q1, S1, expand(P2, 2), expand(Q2, 2), expand(S2, 2),
                             expand(P3, 3), expand(Q3, 3), a, b)


def transport_sums(phi, u, Vt, Mt, avg_nb):
    """Transport moments of face/model.py:514-533 from explicit per-edge tensors.

    phi (N,M,B), u (N,M,3), Vt (N,M,Kd,3), Mt (N,M,Kd,6) gathered neighbour tensors.
    Returns D1 (N, B*2*Kd, 3) = [sum phi V | sum phi M u] and D2 (N, B*2*Kd, 6) =
    [sum phi M | sum phi sym(u (x) V)], channel index b*2Kd + t*Kd + kd, each / avg_nb.
    Pinned by: the reference's own per-edge check (tests/test_transport_map.py:1-29) restated
    in tests/test_oracle.py.
    """
    N, M, B = phi.shape
    Kd = Vt.shape[2]
    Mfull = expand(Mt, 2)                                         # (N,M,Kd,3,3)
    Mu = torch.einsum("nmkab,nmb->nmka", Mfull, u)
    uV = torch.einsum("nma,nmkb->nmkab", u, Vt)
    suV = to_sym2(0.5 * (uV + uV.transpose(-1, -2)))              # (N,M,Kd,6)
    T1 = torch.stack([Vt, Mu], 2)                                 # (N,M,2,Kd,3)
    T2 = torch.stack([Mt, suV], 2)                                # (N,M,2,Kd,6)
    D1 = torch.einsum("nmb,nmtkq->nbtkq", phi, T1).reshape(N, B * 2 * Kd, 3) / avg_nb
    D2 = torch.einsum("nmb,nmtkq->nbtkq", phi, T2).reshape(N, B * 2 * Kd, 6) / avg_nb
    return D1, D2
