"""GPU parity of the HIP kernels against the CPU oracle (fp64 einsums + autograd).

Tolerances follow the reference's own kernel tests: max-abs error / max-abs reference
< 1e-4 for every output and gradient (tests/test_kernels.py:17-19, tests/test_node_kernel.py:84-89).
"""
import itertools
import sys

import numpy as np
import pytest
import torch

from oracle import cartesian
from oracle import ops as oops

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-4


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


# ----------------------------------------------------------------------------- factor density
@pytest.mark.parametrize("B,K", [(16, 32), (32, 32), (8, 16), (16, 64)])
def test_factor_density_dropin_matches_reference_spec(B, K):
    """tests/test_kernels.py:7-20: N=300, M=37, seed 0, randn inputs and upstream G."""
    from face_amd.kernels import factor_density
    say("factor_density", B, K)
    N, M = 300, 37
    torch.manual_seed(0)
    phi = torch.randn(N, M, B, device=DEV, requires_grad=True)
    msg = torch.randn(N, M, K, device=DEV, requires_grad=True)
    Y = torch.randn(N, M, 20, device=DEV, requires_grad=True)
    G = torch.randn(N, 20, B * K, device=DEV)
    D1 = factor_density(phi, msg, Y)
    g1 = torch.autograd.grad((D1 * G).sum(), (phi, msg, Y))
    ins = [t.detach().double().cpu().requires_grad_(True) for t in (phi, msg, Y)]
    D2 = oops.factor_density(*ins)
    g2 = torch.autograd.grad((D2 * G.double().cpu()).sum(), ins)
    errs = [rel(D1, D2)] + [rel(a, b) for a, b in zip(g1, g2)]
    assert max(errs) < TOL, errs


class _G:
    """Random symmetric CSR graph for operator tests: unique undirected pairs, a hub row,
    isolated atoms; rows sorted by neighbour; reverse map computed on the host."""

    def __init__(self, N, n_pairs, seed, hub=70):
        from face_amd.ops import Graph
        rng = np.random.default_rng(seed)
        pairs = set()
        while len(pairs) < n_pairs:
            i, j = rng.integers(0, N - 3, 2)          # the last 3 atoms stay isolated
            if i != j:
                pairs.add((min(i, j), max(i, j)))
        for j in range(1, min(hub, N - 3)):
            pairs.add((0, j))
        directed = sorted([(i, j) for i, j in pairs] + [(j, i) for i, j in pairs])
        index = {e: k for k, e in enumerate(directed)}
        recv = np.array([e[0] for e in directed], np.int32)
        col = np.array([e[1] for e in directed], np.int32)
        rev = np.array([index[(j, i)] for i, j in directed], np.int32)
        counts = np.bincount(recv, minlength=N)
        row_ptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
        self.counts = counts.tolist()
        t = lambda a: torch.as_tensor(a, device=DEV)
        self.G = Graph(torch.zeros(N, 3, device=DEV), None, None, 1, None, t(row_ptr), t(col), t(recv), None, t(rev),
                       int(counts.max()))


def _pad(x_edge, counts, M):
    """(E, ...) edge tensor -> (N, M, ...) zero padded (for the padded oracle): one gather and a
    mask, so that autograd through it stays linear in the size."""
    N = len(counts)
    if x_edge.shape[0] == 0:
        return x_edge.new_zeros(N, M, *x_edge.shape[1:])
    cnt = torch.as_tensor(counts, dtype=torch.int64, device=x_edge.device)
    start = torch.cumsum(cnt, 0) - cnt
    slot = torch.arange(M, device=x_edge.device)
    valid = slot[None, :] < cnt[:, None]
    idx = (start[:, None] + slot[None, :]).clamp(max=x_edge.shape[0] - 1)
    out = x_edge[idx.reshape(-1)].reshape(N, M, *x_edge.shape[1:])
    return out * valid.reshape(N, M, *([1] * (x_edge.dim() - 1))).to(x_edge.dtype)


@pytest.mark.parametrize("nx,gathered,B,K,lds", [(20, False, 16, 32, None), (20, True, 16, 32, None),
                                                 (4, True, 16, 144, None), (20, False, 8, 16, None),
                                                 (4, True, 8, 36, None), (20, False, 16, 64, "1"),
                                                 (20, True, 16, 32, "1"), (20, False, 16, 48, "1")])
def test_csr_density_ragged_rows(nx, gathered, B, K, lds, monkeypatch):
    """Factor density forward / backward on ragged CSR rows (a 70-edge hub row, isolated atoms)
    against the oracle; lds = "1" forces the backward that stages each atom's G in LDS (the route
    of large systems)."""
    from face_amd import ops
    if lds is not None:
        monkeypatch.setenv("FACE_DENSITY_BWD_LDS", lds)
    say("csr density", nx, gathered, B, K, lds)
    g = _G(57, 500, 2)
    counts = g.counts
    E = sum(counts)
    torch.manual_seed(3)
    phi = torch.randn(E, B + 5, device=DEV)[:, :B].requires_grad_(True)   # strided rows
    tab_rows = 57 if gathered else E
    msg = torch.randn(tab_rows, K, device=DEV, requires_grad=True)
    Y = torch.randn(E, 20, device=DEV, requires_grad=True)
    out = ops.density(phi, msg, Y, g.G, nx, gathered)
    D = torch.cat(out, 0) if nx == 20 else out              # monomial-major (nx, N, B*K)
    assert D.shape == (nx, 57, B * K)
    D = D.permute(1, 0, 2)
    G = torch.randn_like(D)
    gr = torch.autograd.grad((D * G).sum(), (phi, msg, Y))
    # oracle on the padded layout
    M = max(counts)
    col = g.G.col.long().cpu()
    pd = lambda t: _pad(t, counts, M)
    ph = phi.detach().double().cpu().requires_grad_(True)
    ms = msg.detach().double().cpu().requires_grad_(True)
    Yc = Y.detach().double().cpu().requires_grad_(True)
    msg_e = ms[col] if gathered else ms
    D2 = oops.factor_density(pd(ph), pd(msg_e), pd(Yc)[..., :nx])
    gr2 = torch.autograd.grad((D2 * G.double().cpu()).sum(), (ph, ms, Yc))
    errs = [rel(D, D2)] + [rel(a, b) for a, b in zip(gr, gr2)]
    assert max(errs) < TOL, errs
    # bitwise reproducible (no atomics)
    out3 = ops.density(phi, msg, Y, g.G, nx, gathered)
    D3 = (torch.cat(out3, 0) if nx == 20 else out3).permute(1, 0, 2)
    assert torch.equal(D, D3)


@pytest.mark.parametrize("gathered,C", [(False, 160), (True, 160), (False, 96), (True, 40)])
def test_cp_density_ragged_rows(gathered, C):
    from face_amd import ops
    say("cp density", gathered, C)
    g = _G(41, 600, 5)
    counts = g.counts
    E = sum(counts)
    torch.manual_seed(6)
    R = torch.randn(E, 16 + 4 * C, device=DEV)[:, 16:].requires_grad_(True)
    env = torch.rand(E, device=DEV, requires_grad=True)
    msg = torch.randn(41 if gathered else E, C, device=DEV, requires_grad=True)
    Y = torch.randn(E, 20, device=DEV, requires_grad=True)
    A = torch.cat(ops.cp_density(R, env, msg, Y, g.G, gathered), 0).permute(1, 0, 2)   # (N, 20, C)
    G = torch.randn_like(A)
    gr = torch.autograd.grad((A * G).sum(), (R, env, msg, Y))
    M = max(counts)
    col = g.G.col.long().cpu()
    pd = lambda t: _pad(t, counts, M)
    Rc = R.detach().double().cpu().requires_grad_(True)
    ec = env.detach().double().cpu().requires_grad_(True)
    ms = msg.detach().double().cpu().requires_grad_(True)
    Yc = Y.detach().double().cpu().requires_grad_(True)
    A2 = oops.cp_density(pd((Rc * ec[:, None]).view(E, 4, C)), pd(ms[col] if gathered else ms), pd(Yc))
    gr2 = torch.autograd.grad((A2 * G.double().cpu()).sum(), (Rc, ec, ms, Yc))
    errs = [rel(A, A2)] + [rel(a, b) for a, b in zip(gr, gr2)]
    assert max(errs) < TOL, errs


@pytest.mark.parametrize("gathered,C,H,N,pairs", [(False, 160, 64, 41, 600), (True, 160, 64, 41, 600),
                                                  (True, 96, 32, 41, 600), (False, 64, 16, 41, 600),
                                                  (True, 32, 48, 41, 600), (False, 160, 64, 3000, 20000),
                                                  (True, 192, 64, 300, 3000), (False, 320, 64, 41, 600)])
def test_cp_radial_density_fused_backward(gathered, C, H, N, pairs):
    """R = h2 W^T + b feeding the CP pooling, whose backward returns d h2 = dR W from inside the
    pooling kernel: with W^T resident in LDS (H x 4C fp32 up to 160 KB; the 3000-atom graph gives
    every wave of the grid a share of rows), with W^T staged in channel slabs (C = 192, H = 64), or,
    at C = 320 where neither fits, by the pooling backward writing dR and a separate product.
    Outputs and gradients (h2, env, msg, Y) vs the oracle in fp64."""
    from face_amd import ops
    say("cp radial density", gathered, C, H, N, pairs)
    g = _G(N, pairs, 5, hub=70 if N < 100 else 16)
    counts = g.counts
    E = sum(counts)
    torch.manual_seed(C + H)
    h2 = torch.randn(E, H, device=DEV, requires_grad=True)
    W = torch.randn(4 * C, H, device=DEV) / H ** 0.5
    b = torch.randn(4 * C, device=DEV) * 0.1
    env = torch.rand(E, device=DEV, requires_grad=True)
    msg = torch.randn(N if gathered else E, C, device=DEV, requires_grad=True)
    Y = torch.randn(E, 20, device=DEV, requires_grad=True)
    A = torch.cat(ops.cp_radial_density(h2, W, b, env, msg, Y, g.G, gathered), 0).permute(1, 0, 2)   # (N, 20, C)
    G = torch.randn_like(A)
    gr = torch.autograd.grad((A * G).sum(), (h2, env, msg, Y))
    M = max(counts)
    col = g.G.col.long().cpu()
    pd = lambda t: _pad(t, counts, M)
    hc = h2.detach().double().cpu().requires_grad_(True)
    ec = env.detach().double().cpu().requires_grad_(True)
    ms = msg.detach().double().cpu().requires_grad_(True)
    Yc = Y.detach().double().cpu().requires_grad_(True)
    Rc = hc @ W.double().cpu().T + b.double().cpu()
    A2 = oops.cp_density(pd((Rc * ec[:, None]).view(E, 4, C)), pd(ms[col] if gathered else ms), pd(Yc))
    gr2 = torch.autograd.grad((A2 * G.double().cpu()).sum(), (hc, ec, ms, Yc))
    errs = [rel(A, A2)] + [rel(a, b) for a, b in zip(gr, gr2)]
    say("   errs", errs)
    assert max(errs) < TOL, errs


def _ragged_counts(N, seed):
    """Row lengths with runs of empty rows at the start, inside and at the end, a run of one-edge
    rows (16-edge tiles holding up to 16 atom segments) and rows longer than a tile."""
    rng = np.random.default_rng(seed)
    body = rng.integers(0, 60, N - 3 - 40 - 6 - 5)
    body[rng.integers(0, body.size, body.size // 8)] = 0
    return [0, 0, 0] + [1] * 40 + [0] * 6 + body.tolist() + [70, 0, 0, 0, 0]


@pytest.mark.parametrize("C,H,N,gathered,with_b,with_env,with_R", [
    (160, 64, 700, False, True, True, True), (160, 64, 700, True, True, True, True),
    (96, 32, 700, True, False, True, True), (16, 16, 300, False, True, False, True),
    (320, 64, 300, False, True, True, False), (48, 48, 300, True, True, True, True),
    (192, 64, 3000, False, True, True, True), (160, 64, 60, True, True, True, True),
    (160, 64, 24000, False, True, True, True)])
def test_cp_radial_fused_forward_matches_two_launch_route(C, H, N, gathered, with_b, with_env, with_R):
    """The fused CP radial forward (R = h2 W^T + b computed, written and pooled in one launch)
    through the C ABI against the two-launch route on the same inputs (face_edge_linear_fwd then
    face_cp_density_fwd): R bitwise equal, A within fp32 rounding of the edge-serial pooling and
    within TOL of the fp64 oracle; every output row written (outputs start as NaN), empty rows
    exactly zero. Channel widths give 1 to 5 16-channel blocks per part and 1 to 4 parts. The
    24,000-atom case (rows of 30-74 edges, 1.25 M edges: the benchmark liquid's shape, every wave
    of the grid on its own share) is checked against the two-launch route only (the padded fp64
    oracle would need ~10 GB there)."""
    from face_amd import _lib, ops
    say("cp radial fused fwd", C, H, N, gathered, with_b, with_env, with_R)
    full = N >= 10000
    counts = (np.random.default_rng(N).integers(30, 75, N).tolist() if full else _ragged_counts(N, C + H))
    E = int(sum(counts))
    rng = np.random.default_rng(N + C)
    row_ptr = torch.as_tensor(np.concatenate([[0], np.cumsum(counts)]).astype(np.int32), device=DEV)
    col = torch.as_tensor(rng.integers(0, N, E).astype(np.int32), device=DEV)
    torch.manual_seed(C * H + N)
    h2 = torch.randn(E, H, device=DEV)
    W = torch.randn(4 * C, H, device=DEV) / H ** 0.5
    b = torch.randn(4 * C, device=DEV) * 0.1 if with_b else None
    env = torch.rand(E, device=DEV) if with_env else None
    msg = torch.randn(N if gathered else E, C, device=DEV)
    Y = torch.randn(E, 20, device=DEV)
    row = col if gathered else None
    st = _lib.stream_of(h2)
    outs = [torch.full((k, N, C), float("nan"), device=DEV) for k in ops.RANK_K]
    R = torch.full((E, 4 * C), float("nan"), device=DEV) if with_R else None
    P = _lib.ptr
    _lib.call("face_cp_radial_fwd", P(h2), H, H, P(W), P(b), P(env), P(msg), C, P(row), P(Y), 20, P(row_ptr), N, E,
              C, *_lib.ranks_of_blocks(outs), P(R), 4 * C, st)
    R2 = ops.edge_linear(h2, W, b)
    outs2 = [torch.empty(k, N, C, device=DEV) for k in ops.RANK_K]
    _lib.call("face_cp_density_fwd", P(R2), 4 * C, P(env), P(msg), C, P(row), P(Y), 20, P(row_ptr), N, 0, C,
              *_lib.ranks_of_blocks(outs2), st)
    torch.cuda.synchronize()
    if with_R:
        assert torch.equal(R, R2)
    A = torch.cat(outs, 0).permute(1, 0, 2)                               # (N, 20, C)
    A2 = torch.cat(outs2, 0).permute(1, 0, 2)
    assert torch.isfinite(A).all()
    empty = torch.as_tensor(counts, device=DEV) == 0
    assert (A[empty] == 0).all()
    scale = A2.abs().max().item()
    assert (A - A2).abs().max().item() <= 2e-6 * scale
    if full:
        return
    M = max(counts)
    pd = lambda t: _pad(t, counts, M)
    Rc = h2.double().cpu() @ W.double().cpu().T + (b.double().cpu() if with_b else 0)
    ec = env.double().cpu() if with_env else torch.ones(E, dtype=torch.float64)
    ms = msg.double().cpu()
    A3 = oops.cp_density(pd((Rc * ec[:, None]).view(E, 4, C)), pd(ms[col.long().cpu()] if gathered else ms),
                         pd(Y.double().cpu()))
    assert rel(A, A3) < TOL


def test_cp_radial_fused_forward_without_edges():
    """No edges at all: every row of A is zero, and h2 / W may be NULL."""
    from face_amd import _lib, ops
    N, C = 37, 32
    row_ptr = torch.zeros(N + 1, dtype=torch.int32, device=DEV)
    msg = torch.randn(N, C, device=DEV)
    Y = torch.randn(1, 20, device=DEV)
    outs = [torch.full((k, N, C), float("nan"), device=DEV) for k in ops.RANK_K]
    _lib.call("face_cp_radial_fwd", None, 64, 64, None, None, None, _lib.ptr(msg), C, None, _lib.ptr(Y), 20,
              _lib.ptr(row_ptr), N, 0, C, *_lib.ranks_of_blocks(outs), None, 4 * C, _lib.stream_of(msg))
    torch.cuda.synchronize()
    assert all((o == 0).all() for o in outs)


# ----------------------------------------------------------------------------- gated outputs
@pytest.mark.parametrize("N,C", [(1000, 160), (37, 96), (1, 4)])
def test_eq_gate_matches_torch(N, C):
    """V * gv, Ms * gm (face/model.py:286-287): outputs bit-exact against torch fp32, gradients of
    V, Ms and the gate row within fp32 rounding of torch's autograd."""
    from face_amd import ops
    say("eq_gate", N, C)
    torch.manual_seed(N + C)
    V = torch.randn(3, N, C, device=DEV, requires_grad=True)
    Ms = torch.randn(6, N, C, device=DEV, requires_grad=True)
    gvm = torch.randn(N, 2 * C, device=DEV, requires_grad=True)
    Vo, Mo = ops.eq_gate(V, Ms, gvm)
    gv, gm = gvm.chunk(2, dim=-1)
    Vr, Mr = V * gv[None], Ms * gm[None]
    assert torch.equal(Vo, Vr) and torch.equal(Mo, Mr)
    gV, gM = torch.randn_like(Vo), torch.randn_like(Mo)
    g1 = torch.autograd.grad((Vo * gV).sum() + (Mo * gM).sum(), (V, Ms, gvm))
    g2 = torch.autograd.grad((Vr * gV).sum() + (Mr * gM).sum(), (V, Ms, gvm))
    for a, b in zip(g1, g2):
        assert (a - b).abs().max().item() <= 1e-6 * (1 + b.abs().max().item())


@pytest.mark.parametrize("N,F", [(24000, 1440), (37, 864), (5, 4), (300, 2048)])
def test_layer_norm_matches_torch(N, F):
    """Readout LayerNorm (face/model.py:332) and its input gradient against torch's fp32
    LayerNorm on the same device, within fp32 rounding."""
    from face_amd import ops
    say("layer_norm", N, F)
    torch.manual_seed(N + F)
    x = (torch.randn(N, F, device=DEV) * 3 + 1).requires_grad_(True)
    w = torch.randn(F, device=DEV)
    b = torch.randn(F, device=DEV)
    y1 = ops.layer_norm(x, w, b, 1e-5)
    y2 = torch.nn.functional.layer_norm(x, (F,), w, b, 1e-5)
    assert (y1 - y2).abs().max().item() < 1e-5 * (1 + y2.abs().max().item())
    dy = torch.randn_like(y1)
    g1, = torch.autograd.grad((y1 * dy).sum(), x)
    g2, = torch.autograd.grad((y2 * dy).sum(), x)
    assert (g1 - g2).abs().max().item() < 1e-5 * (1 + g2.abs().max().item())


# ----------------------------------------------------------------------------- node algebra
@pytest.mark.parametrize("eq", [True, False])
def test_node_algebra_dropin_matches_reference_spec(eq):
    """tests/test_node_kernel.py:8-28: N=50, C=24, seed 1, outputs and every gradient incl. da, db."""
    from face_amd.node_kernel import node_algebra
    say("node_algebra eq", eq)
    torch.manual_seed(1)
    N, C = 50, 24
    shapes = [(3,), (3,), (3,), (6,), (6,), (6,), (10,), (10,)]
    xs = [torch.randn(N, C, *s, device=DEV, requires_grad=True) for s in shapes]
    a = torch.randn(4, C, device=DEV, requires_grad=True)
    b = torch.randn(4, C, device=DEV, requires_grad=True)
    gI, gV, gM = torch.randn(N, C, 8, device=DEV), torch.randn(N, C, 3, device=DEV), torch.randn(N, C, 3, 3, device=DEV)
    o1 = node_algebra(*xs, a, b, eq)
    L = lambda o, gi, gv, gm: (o[0] * gi).sum() + (((o[1] * gv).sum() + (o[2] * gm).sum()) if eq else 0)
    vars1 = xs + ([a, b] if eq else [])
    g1 = torch.autograd.grad(L(o1, gI, gV, gM), vars1, allow_unused=True)
    xc = [t.detach().double().cpu().requires_grad_(True) for t in xs]
    ac, bc = a.detach().double().cpu().requires_grad_(True), b.detach().double().cpu().requires_grad_(True)
    o2 = oops.node_algebra_sym(*xc, ac, bc)
    vars2 = xc + ([ac, bc] if eq else [])
    g2 = torch.autograd.grad(L(o2, gI.double().cpu(), gV.double().cpu(), gM.double().cpu()), vars2,
                             allow_unused=True)
    outs1 = list(o1[:3] if eq else o1[:1])
    outs2 = list(o2[:3] if eq else o2[:1])
    errs = [rel(u, v) for u, v in zip(outs1 + list(g1), outs2 + list(g2))]
    assert max(errs) < TOL, errs


def test_node_features_product_layout():
    """Strided P/Q/S read from projection outputs, families written into the readout row,
    symmetrised gated products (face/model.py:244-249,274-276)."""
    from face_amd import ops
    say("node features")
    torch.manual_seed(2)
    N, C = 37, 20
    y0 = torch.randn(1, N, C, device=DEV, requires_grad=True)
    y1 = torch.randn(3, N, 3 * C, device=DEV, requires_grad=True)
    y2 = torch.randn(6, N, 3 * C, device=DEV, requires_grad=True)
    y3 = torch.randn(10, N, 2 * C, device=DEV, requires_grad=True)
    a = torch.randn(4, C, device=DEV, requires_grad=True)
    b = torch.randn(4, C, device=DEV, requires_grad=True)
    feats, V, Ms = ops.node_features(y0, y1, y2, y3, a, b, True, C)
    gf, gv, gm = torch.randn_like(feats), torch.randn_like(V), torch.randn_like(Ms)
    vars1 = [y0, y1, y2, y3, a, b]
    g1 = torch.autograd.grad((feats * gf).sum() + (V * gv).sum() + (Ms * gm).sum(), vars1)
    yc = [t.detach().double().cpu().requires_grad_(True) for t in vars1]
    c0, c1, c2, c3, ac, bc = yc
    split = lambda y, k: [y[..., j * C:(j + 1) * C].permute(1, 2, 0) for j in range(k)]
    P1, Q1, S1 = split(c1, 3)
    P2, Q2, S2 = split(c2, 3)
    P3, Q3 = split(c3, 2)
    inv, Vr, Mf = oops.node_algebra_sym(P1, Q1, S1, P2, Q2, S2, P3, Q3, ac, bc)
    feats2 = torch.cat([c0[0]] + list(inv.unbind(-1)), 1)
    Ms2 = cartesian.to_sym2(0.5 * (Mf + Mf.transpose(-1, -2))).permute(2, 0, 1)
    V2 = Vr.permute(2, 0, 1)
    L2 = (feats2 * gf.double().cpu()).sum() + (V2 * gv.double().cpu()).sum() + (Ms2 * gm.double().cpu()).sum()
    g2 = torch.autograd.grad(L2, yc)
    errs = [rel(feats, feats2), rel(V, V2), rel(Ms, Ms2)] + [rel(u, v) for u, v in zip(g1, g2)]
    assert max(errs) < TOL, errs


@pytest.mark.parametrize("N,C,eq,wide", [(37, 20, True, False), (50, 96, True, True), (23, 160, False, False),
                                         (9, 256, True, False), (5, 40, False, True)])
def test_node_layer_norm_fused_matches_oracle(N, C, eq, wide):
    """Node algebra with the readout LayerNorm in one kernel each way (face/model.py:244-264, :332)
    against the oracle's node algebra + torch layer_norm in fp64: the normalised row, V, Ms and
    every input gradient; C not a multiple of the wave width, y0 rows wider than C."""
    from face_amd import ops
    say("node + layer norm", N, C, eq, wide)
    torch.manual_seed(N + C)
    y0 = torch.randn(1, N, 2 * C if wide else C, device=DEV, requires_grad=True)
    y1 = torch.randn(3, N, 3 * C, device=DEV, requires_grad=True)
    y2 = torch.randn(6, N, 3 * C, device=DEV, requires_grad=True)
    y3 = torch.randn(10, N, 2 * C, device=DEV, requires_grad=True)
    a = torch.randn(4, C, device=DEV) if eq else None
    b = torch.randn(4, C, device=DEV) if eq else None
    lw = torch.rand(9 * C, device=DEV) + 0.5
    lb = torch.randn(9 * C, device=DEV) * 0.1
    inv, V, Ms = ops.node_ln(y0, y1, y2, y3, a, b, eq, C, lw, lb, 1e-5)
    gi = torch.randn_like(inv)
    L = (inv * gi).sum()
    if eq:
        gv, gm = torch.randn_like(V), torch.randn_like(Ms)
        L = L + (V * gv).sum() + (Ms * gm).sum()
    vars1 = [y0, y1, y2, y3]
    g1 = torch.autograd.grad(L, vars1)
    yc = [t.detach().double().cpu().requires_grad_(True) for t in vars1]
    c0, c1, c2, c3 = yc
    ac = a.double().cpu() if eq else torch.zeros(4, C, dtype=torch.float64)
    bc = b.double().cpu() if eq else torch.zeros(4, C, dtype=torch.float64)
    split = lambda y, k: [y[..., j * C:(j + 1) * C].permute(1, 2, 0) for j in range(k)]
    P1, Q1, S1 = split(c1, 3)
    P2, Q2, S2 = split(c2, 3)
    P3, Q3 = split(c3, 2)
    invr, Vr, Mf = oops.node_algebra_sym(P1, Q1, S1, P2, Q2, S2, P3, Q3, ac, bc)
    feats = torch.cat([c0[0, :, :C]] + list(invr.unbind(-1)), 1)
    inv2 = torch.nn.functional.layer_norm(feats, (9 * C,), lw.double().cpu(), lb.double().cpu(), 1e-5)
    L2 = (inv2 * gi.double().cpu()).sum()
    outs, refs = [inv], [inv2]
    if eq:
        Ms2 = cartesian.to_sym2(0.5 * (Mf + Mf.transpose(-1, -2))).permute(2, 0, 1)
        V2 = Vr.permute(2, 0, 1)
        L2 = L2 + (V2 * gv.double().cpu()).sum() + (Ms2 * gm.double().cpu()).sum()
        outs += [V, Ms]
        refs += [V2, Ms2]
    g2 = torch.autograd.grad(L2, yc)
    errs = [rel(u, v) for u, v in zip(outs, refs)] + [rel(u, v) for u, v in zip(g1, g2)]
    say("   errs", errs)
    assert max(errs) < TOL, errs
    if wide:
        assert float(g1[0][0, :, C:].abs().max()) == 0.0


# ----------------------------------------------------------------------------- gathers / scatter
def test_gathers_and_force_scatter_match_index_add():
    from face_amd import ops
    from face_amd.neighbors import build_graph
    from face_amd import systems
    say("gathers / scatter")
    (liq,) = [systems.liquid(500, np.random.default_rng(9), rho=0.1, dmin=0.9)]
    g = build_graph([liq], 4.0)
    torch.manual_seed(0)
    X = torch.randn(g.N, 7, device=DEV, requires_grad=True)
    Xj = ops.gather_neighbour(X, g)
    Xi = ops.gather_receiver(X, g)
    col, recv = g.col.long(), g.recv.long()
    assert torch.equal(Xj, X[col]) and torch.equal(Xi, X[recv])
    w1, w2 = torch.randn_like(Xj), torch.randn_like(Xi)
    (gx,) = torch.autograd.grad((Xj * w1).sum() + (Xi * w2).sum(), X)
    ref = torch.zeros_like(X).index_add(0, col, w1).index_add(0, recv, w2)
    assert rel(gx, ref) < 1e-5
    gvec = torch.randn(g.E, 3, device=DEV)
    grad = torch.empty(g.N, 3, device=DEV)
    from face_amd._lib import call, ptr, stream_of
    call("face_force_scatter", ptr(gvec), ptr(g.row_ptr), ptr(g.rev), g.N, 1.0, ptr(grad), stream_of(gvec))
    ref = torch.zeros(g.N, 3, device=DEV).index_add(0, col, gvec).index_add(0, recv, -gvec)
    assert rel(grad, ref) < 1e-5
    # the contiguous row form: reverse slots and per-window own-row sums laid out as the edge backward
    # (face_edge_geom_bwd_seg) writes them, wsum filled only at the last edge of each row in each
    # 64-edge window (NaN elsewhere: never read), then the row pass (both lane widths)
    # (16-byte rows: x, y, z and an unused fourth float, NaN here)
    gvec_rev = torch.full((g.E, 4), float("nan"), device=DEV)
    gvec_rev[:, :3] = gvec[g.rev.long()]
    e_idx = torch.arange(g.E, device=DEV)
    seg = recv * ((g.E + 63) // 64) + e_idx // 64
    _, inv, cnt = torch.unique_consecutive(seg, return_inverse=True, return_counts=True)
    sums = torch.zeros(cnt.numel(), 3, device=DEV).index_add(0, inv, gvec)
    wsum = torch.full((g.E, 4), float("nan"), device=DEV)
    wsum[torch.cumsum(cnt, 0) - 1, :3] = sums
    for mean_row in (16, 40):
        grad2 = torch.full((g.N, 3), float("nan"), device=DEV)
        call("face_force_scatter_rows", ptr(gvec_rev), ptr(wsum), ptr(g.row_ptr), g.N, mean_row, -1.0, ptr(grad2),
             stream_of(gvec))
        assert rel(-grad2, ref) < 1e-5


# ----------------------------------------------------------------------------- edge geometry
@pytest.mark.parametrize("system", ["molecules", "liquid"])
def test_edge_geometry_forward_and_backward(system):
    """Edge geometry, basis and envelope and their backward into dE/dpos (the row-organised edge
    backward and the contiguous force scatter; short molecule rows and ~40-pair periodic rows)."""
    from face_amd import ops
    from face_amd.neighbors import build_graph
    from face_amd import systems
    say("edge geometry", system)
    rc = 4.5
    if system == "molecules":
        st = systems.molecules(6, np.random.default_rng(2))
    else:
        st = [systems.liquid(400, np.random.default_rng(4), rho=0.1, dmin=0.9)]
    g = build_graph(st, rc)
    pos = g.pos.clone().requires_grad_(True)
    freq = (torch.arange(1, 9) * np.pi / rc).float().to(DEV)
    Y, rb, env, rr = ops.edge_geometry(pos, g, freq, rc, with_r=True)
    wY, wr, we, wd = torch.randn_like(Y), torch.randn_like(rb), torch.randn_like(env), torch.randn_like(rr)
    (gp,) = torch.autograd.grad((Y * wY).sum() + (rb * wr).sum() + (env * we).sum() + (rr * wd).sum(), pos)
    # each input handed to several readers as views of one tensor: their gradients, summed in the
    # edge backward, give the same forces as one reader with the summed upstream gradient
    outs = ops.edge_geometry(pos, g, freq, rc, with_r=True, counts=(3, 2, 4, 2))
    assert len(outs) == 11 and all(torch.equal(t, Y) for t in outs[:3]) and torch.equal(outs[3], rb)
    parts = [(outs[0], 0.5 * wY), (outs[1], 0.25 * wY), (outs[2], 0.25 * wY), (outs[3], 0.5 * wr), (outs[4], 0.5 * wr),
             (outs[5], we), (outs[6], 0 * we), (outs[9], 0.5 * wd), (outs[10], 0.5 * wd)]   # one env view unread
    (gp_v,) = torch.autograd.grad(sum((t * w).sum() for t, w in parts), pos)
    assert (gp_v - gp).abs().max() <= 1e-5 * gp.abs().max()
    # without the Bessel rows (compiled radial): rb is empty and the rest unchanged
    Y3, rb3, env3, r3 = ops.edge_geometry(pos.detach(), g, freq, rc, with_rb=False, with_r=True)
    assert rb3.numel() == 0 and torch.equal(Y3, Y.detach()) and torch.equal(r3, rr.detach())
    # oracle: the reference formulas in fp64 on the CPU (face/model.py:670-677, :28-40)
    pc = g.pos.detach().double().cpu().requires_grad_(True)
    col, recv = g.col.long().cpu(), g.recv.long().cpu()
    vec = pc[col] - pc[recv] + g.shift.double().cpu()
    r = torch.sqrt((vec * vec).sum(-1))
    u = vec / r[:, None]
    x = r / rc
    e_ref = (1 - 28 * x ** 6 + 48 * x ** 7 - 21 * x ** 8) * (x < 1)
    bes = torch.sin(torch.arange(1, 9, dtype=torch.float64) * np.pi / rc * r[:, None]) / r[:, None] * np.sqrt(2 / rc)
    Y2, rb2 = cartesian.monomials(u), bes * e_ref[:, None]
    (gp2,) = torch.autograd.grad((Y2 * wY.double().cpu()).sum() + (rb2 * wr.double().cpu()).sum()
                                 + (e_ref * we.double().cpu()).sum() + (r * wd.double().cpu()).sum(), pc)
    errs = [rel(Y, Y2), rel(rb, rb2), rel(env, e_ref), rel(rr, r), rel(gp, gp2)]
    assert max(errs) < TOL, errs


@pytest.mark.parametrize("P,G,F,nb", [(9, 4096, 16, 16), (9, 4096, 16 + 4 * 160, 16), (1, 300, 16, 16),
                                       (4, 64, 37, 5), (2, 33, 6, 0)])
def test_radial_spline_matches_oracle(P, G, F, nb):
    """Compiled radial (face/model.py:407-418, :466-467): phi = S[:, :nb] * env and R = S[:, nb:]
    with their r / env gradients, against the oracle's RadialSpline in fp64 (autograd), for radii
    inside the grid, on grid points, and beyond its end (clamped, zero r-derivative). The tables
    sample smooth functions, as compiled radial functions are: with random, non-smooth tables the
    fp32 rounding of r / dr alone (2e-4 of a cell at 4096 points) moves the value by ~1e-4."""
    from face_amd import ops
    from oracle.model import RadialSpline
    say("spline", P, G, F, nb)
    gen = torch.Generator().manual_seed(G + F)
    rc = 5.0
    dr = rc / (G - 1)
    rg = (torch.arange(G, dtype=torch.float64) * dr)[None, :, None]
    amp, k, ph = (torch.randn(P, 1, F, generator=gen, dtype=torch.float64) for _ in range(3))
    k = 0.3 + 2.5 * k.abs()
    T = (amp * torch.sin(k * rg + ph) + 0.1 * amp * rg ** 2).float()
    dT = (amp * k * torch.cos(k * rg + ph) + 0.2 * amp * rg).float()
    E = 3000
    rng = np.random.default_rng(F)
    r = rng.uniform(1e-4, rc + 0.7, E)
    r[:50] = np.arange(50) % G * dr                              # on grid points
    r = torch.tensor(r, dtype=torch.float32)
    pair = torch.tensor(rng.integers(0, P, E), dtype=torch.int32)
    env = torch.rand(E, generator=gen)
    rd, envd = r.to(DEV).requires_grad_(True), env.to(DEV).requires_grad_(True)
    phi, R = ops.radial_spline(rd, envd, pair.to(DEV), T.to(DEV), dT.to(DEV), dr, nb)
    assert phi.shape == (E, nb) and R.shape == (E, F - nb)
    wp, wq = torch.randn(E, nb, generator=gen), torch.randn(E, F - nb, generator=gen)
    gr, ge = torch.autograd.grad((phi * wp.to(DEV)).sum() + (R * wq.to(DEV)).sum(), (rd, envd))
    sp = RadialSpline(T.double(), dT.double(), dr)
    rc_, ec = r.double().requires_grad_(True), env.double().requires_grad_(True)
    S = sp(rc_, pair.long())
    phi2, R2 = S[:, :nb] * ec[:, None], S[:, nb:]
    gr2, ge2 = torch.autograd.grad((phi2 * wp.double()).sum() + (R2 * wq.double()).sum(), (rc_, ec))
    errs = [rel(phi, phi2) if nb else 0.0, rel(R, R2) if F > nb else 0.0, rel(gr, gr2), rel(ge, ge2) if nb else 0.0]
    assert max(errs) < TOL, errs
    assert float(gr[r.to(DEV) > rc + 1e-3].abs().max()) == 0.0   # clamped: no r-derivative


def test_radial_spline_without_envelope_as_a_reference_binding():
    """The call pattern of a binding inside the reference's RadialSpline.forward (padded (N, M)
    radii and pair indices flattened, no envelope pointer, nb = F): values and r-gradient equal
    the oracle's RadialSpline in fp64."""
    from face_amd._lib import call, ptr, stream_of
    from oracle.model import RadialSpline
    say("spline binding")
    P, G, F, N, M = 9, 4096, 16, 40, 23
    dr = 4.5 / (G - 1)
    gen = torch.Generator().manual_seed(4)
    rg = (torch.arange(G, dtype=torch.float64) * dr)[None, :, None]
    amp, k = torch.randn(P, 1, F, generator=gen, dtype=torch.float64), 0.5 + torch.rand(P, 1, F, generator=gen)
    T, dT = (amp * torch.cos(k * rg)).float(), (-amp * k * torch.sin(k * rg)).float()
    r = torch.rand(N, M, generator=gen) * 4.4 + 0.05
    pair = torch.randint(0, P, (N, M), generator=gen)
    rd, pd = r.reshape(-1).to(DEV), pair.reshape(-1).to(torch.int32).to(DEV)
    E = N * M
    S = torch.empty(E, F, device=DEV)
    Td, dTd = T.to(DEV), dT.to(DEV)
    st = stream_of(rd)
    call("face_radial_spline_fwd", ptr(rd), ptr(pd), E, ptr(Td), ptr(dTd), P, G, F, dr, None, F, None, ptr(S), F,
         None, 0, st)
    w = torch.randn(E, F, generator=gen)
    gr = torch.empty(E, device=DEV)
    call("face_radial_spline_bwd", ptr(rd), ptr(pd), E, ptr(Td), ptr(dTd), P, G, F, dr, None, F, None,
         ptr(w.to(DEV)), F, None, 0, ptr(gr), None, st)
    sp = RadialSpline(T.double(), dT.double(), dr)
    rc = r.double().requires_grad_(True)
    S2 = sp(rc, pair)
    (gr2,) = torch.autograd.grad((S2 * w.double().view(N, M, F)).sum(), rc)
    assert max(rel(S, S2.reshape(E, F)), rel(gr, gr2.reshape(-1))) < TOL


@pytest.mark.parametrize("P,G,F,nb,E", [(5, 700, 24, 8, 20000), (9, 4096, 16 + 4 * 160, 16, 150000),
                                         (4, 4096, 16 + 4 * 256, 16, 40000), (2, 40, 8 + 4 * 32, 8, 3001)])
def test_radial_spline_order_is_a_cell_sorted_permutation(P, G, F, nb, E):
    """face_radial_spline_order: a permutation of the edges with non-decreasing table cell
    (pair * G + grid interval, the same cell the spline kernels use), including radii past the
    grid's end (last interval); the spline outputs in that order (the cell-run kernels, which
    keep each cell's table rows in registers over its run of edges) equal the unordered per-edge
    kernels' bitwise, at the CP widths (16 + 4C columns, C = 160 and 256) too."""
    from face_amd._lib import call, ptr, stream_of
    say("spline order", P, G, F, nb, E)
    rc = 4.0
    dr = rc / (G - 1)
    rng = np.random.default_rng(9)
    r = torch.tensor(rng.uniform(1e-4, rc + 0.5, E), dtype=torch.float32, device=DEV)
    pair = torch.tensor(rng.integers(0, P, E), dtype=torch.int32, device=DEV)
    work = torch.empty(P * G, dtype=torch.int32, device=DEV)
    order = torch.empty(E, dtype=torch.int32, device=DEV)
    st = stream_of(r)
    call("face_radial_spline_order", ptr(r), ptr(pair), E, P, G, dr, ptr(work), ptr(order), st)
    o = order.long().cpu()
    assert torch.equal(torch.sort(o).values, torch.arange(E))
    x = (r.cpu() / dr).clamp(0, G - 1)
    cell = pair.long().cpu() * G + torch.floor(x).long().clamp(max=G - 2)
    assert bool((cell[o][1:] >= cell[o][:-1]).all())
    T = torch.randn(P, G, F, device=DEV)
    dT = torch.randn(P, G, F, device=DEV)
    env = torch.rand(E, device=DEV)
    outs = []
    for od in (None, order):
        phi = torch.empty(E, nb, device=DEV)
        R = torch.empty(E, F - nb, device=DEV)
        call("face_radial_spline_fwd", ptr(r), ptr(pair), E, ptr(T), ptr(dT), P, G, F, dr, ptr(env), nb, ptr(od),
             ptr(phi), nb, ptr(R), F - nb, st)
        gp, gq = torch.ones(E, nb, device=DEV), torch.ones(E, F - nb, device=DEV)
        gr, ge = torch.empty(E, device=DEV), torch.empty(E, device=DEV)
        call("face_radial_spline_bwd", ptr(r), ptr(pair), E, ptr(T), ptr(dT), P, G, F, dr, ptr(env), nb, ptr(od),
             ptr(gp), nb, ptr(gq), F - nb, ptr(gr), ptr(ge), st)
        outs.append((phi, R, gr, ge))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("Kd,B,transport", [(16, 16, True), (4, 8, True), (5, 4, False), (16, 16, False)])
def test_dir_transport_and_gradients(Kd, B, transport, packed, monkeypatch):
    """Directional features d = [u.V_j, u^T M_j u, u.V_i, u^T M_i u] (face/model.py:474-493) and the
    transport sums D1 = [sum phi V, sum phi M u], D2 = [sum phi M, sum phi sym(u V)] (face/model.py:
    514-528) vs gathered einsums and the oracle's explicit per-edge transport tensors, with the
    tables read in place and packed node-major."""
    from face_amd import ops
    monkeypatch.setattr(ops, "DIR_PACK_MIN_BYTES", 0 if packed else 1 << 40)
    say("dir/transport", Kd, B, transport, "packed" if packed else "in place")
    g = _G(37, 300, Kd + 10)
    counts = g.counts
    E = sum(counts)
    nt = 2 if transport else 1
    torch.manual_seed(Kd)
    Vb = torch.randn(3, 37, nt * Kd, device=DEV, requires_grad=True)
    Mb = torch.randn(6, 37, nt * Kd, device=DEV, requires_grad=True)
    phi = torch.randn(E, B, device=DEV, requires_grad=True)
    Y = torch.randn(E, 20, device=DEV, requires_grad=True)
    d, D1, D2 = ops.dir_transport(Vb, Mb, phi, Y, g.G, Kd, transport)
    wd = torch.randn_like(d)
    L = (d * wd).sum()
    if transport:
        w1, w2 = torch.randn_like(D1), torch.randn_like(D2)
        L = L + (D1 * w1).sum() + (D2 * w2).sum()
    ins = [Vb, Mb, Y] + ([phi] if transport else [])
    grads = torch.autograd.grad(L, ins)
    # oracle (fp64, CPU)
    c = [t.detach().double().cpu().requires_grad_(True) for t in ins]
    Vc, Mc, Yc = c[:3]
    col, recv = g.G.col.long().cpu(), g.G.recv.long().cpu()
    u = Yc[:, 1:4]
    Y2 = Yc[:, 4:10] * torch.tensor([1.0, 1, 1, 2, 2, 2], dtype=torch.float64)
    Vj, Mj = Vc[:, col, :Kd], Mc[:, col, :Kd]            # (3|6, E, Kd)
    Vi, Mi = Vc[:, recv, :Kd], Mc[:, recv, :Kd]
    d2 = torch.cat([torch.einsum("ea,aek->ek", u, Vj), torch.einsum("ea,aek->ek", Y2, Mj),
                    torch.einsum("ea,aek->ek", u, Vi), torch.einsum("ea,aek->ek", Y2, Mi)], -1)
    L2 = (d2 * wd.double().cpu()).sum()
    outs, refs = [d], [d2]
    if transport:
        pc = c[3]
        M = max(counts)
        pd = lambda t: _pad(t, counts, M)
        Vt = Vc[:, col, Kd:].permute(1, 2, 0)            # (E, Kd, 3)
        Mt = Mc[:, col, Kd:].permute(1, 2, 0)            # (E, Kd, 6)
        R1, R2 = oops.transport_sums(pd(pc), pd(u), pd(Vt), pd(Mt), 1.0)   # (N, B*2Kd, 3|6)
        R1, R2 = R1.permute(2, 0, 1), R2.permute(2, 0, 1)
        L2 = L2 + (R1 * w1.double().cpu()).sum() + (R2 * w2.double().cpu()).sum()
        outs += [D1, D2]
        refs += [R1, R2]
    grads2 = torch.autograd.grad(L2, c)
    errs = [rel(a, b) for a, b in zip(outs, refs)] + [rel(a, b) for a, b in zip(grads, grads2)]
    assert max(errs) < TOL, errs


# ----------------------------------------------------------------------------- radial MLP
@pytest.mark.parametrize("E,H,F,offset", [(100000, 64, 640, 0), (1001, 16, 128, 0), (37, 48, 640, 0),
                                          (5, 32, 1024, 0), (300, 64, 1280, 0), (4099, 64, 640, 4), (0, 64, 640, 0)])
def test_radial_head_matches_torch(E, H, F, offset):
    """R = h2 w^T + b for the CP columns of the last radial layer vs torch fp64: whole-LDS weight
    images with the rotated (H = 64, F = 640) and padded row layouts, the feature-chunked grid
    (H = 64, F = 1280), ragged edge tiles and a row stride / base offset that is not the width."""
    from face_amd import ops
    say("radial head", E, H, F, offset)
    torch.manual_seed(E + F)
    base = torch.randn(E * (H + offset) + offset, device=DEV)
    h2 = base[offset:offset + E * (H + offset)].view(E, H + offset)[:, :H] if E else torch.empty(0, H, device=DEV)
    w = torch.randn(F, H, device=DEV) / H ** 0.5
    b = torch.randn(F, device=DEV)
    R = ops.radial_head(h2, w, b)
    assert R.shape == (E, F)
    if E == 0:
        return
    ref = h2.double() @ w.double().T + b.double()
    err = rel(R, ref)
    say("   err", err)
    assert err < 1e-5, err


@pytest.mark.parametrize("F,K", [(160, 64), (32, 64), (16, 16), (256, 48), (48, 32)])
def test_edge_message_matches_torch(F, K):
    """gather(msg(h)) + dir_mix(d) (face/model.py:488-493) as one launch, m[e] = T[col e] + d[e] W^T
    + b, and its backward (d T by the reverse-edge reduction, d d = dm W) vs torch fp64 on a
    random symmetric graph with a 70-neighbour hub row (5 edge tiles) and isolated atoms."""
    from face_amd import ops
    say("edge message", F, K)
    gr = _G(700, 9000, F + K)
    g = gr.G
    torch.manual_seed(F * K)
    T = torch.randn(g.N, F, device=DEV, requires_grad=True)
    d = torch.randn(g.E, K, device=DEV, requires_grad=True)
    w = torch.randn(F, K, device=DEV) / K ** 0.5
    b = torch.randn(F, device=DEV)
    m = ops.edge_message(T, d, w, b, g)
    gm = torch.randn_like(m)
    gT, gd = torch.autograd.grad((m * gm).sum(), (T, d))
    Tc = T.detach().double().cpu().requires_grad_(True)
    dc = d.detach().double().cpu().requires_grad_(True)
    mr = Tc[g.col.long().cpu()] + dc @ w.double().cpu().T + b.double().cpu()
    gT2, gd2 = torch.autograd.grad((mr * gm.double().cpu()).sum(), (Tc, dc))
    errs = [rel(m, mr), rel(gT, gT2), rel(gd, gd2)]
    say("   errs", errs)
    assert max(errs) < 1e-5, errs
    assert float(gT[-3:].abs().max()) == 0.0                   # isolated atoms: exact zero rows


@pytest.mark.parametrize("E,nb,H,B,n_pair,want_h2",[(20000, 8, 64, 16, 9, True), (20000, 8, 64, 16, 1, False),
                                                      (1001, 8, 16, 8, 9, False), (37, 8, 32, 20, 4, True),
                                                      (5, 12, 48, 32, 9, True), (0, 8, 64, 16, 9, True)])
def test_radial_mlp_matches_torch(E, nb, H, B, n_pair, want_h2):
    """phi = (silu(silu(rb W_in^T + b_in + pair_tab[pair]) W1^T + b1) W_phi^T + b_phi) * env and h2
    (face/model.py:465-469) vs the same layers in torch fp64, with the gradients of rb and env."""
    from face_amd import ops
    say("radial", E, nb, H, B, n_pair, want_h2)
    torch.manual_seed(E + H)
    rb = torch.randn(E, nb, device=DEV, requires_grad=True)
    env = torch.rand(E, device=DEV, requires_grad=True)
    pair = torch.randint(0, n_pair, (E,), device=DEV, dtype=torch.int32)
    ws = [torch.randn(H, nb) / nb ** 0.5, torch.randn(H) * 0.1, torch.randn(n_pair, H) * 0.3,
          torch.randn(H, H) / H ** 0.5, torch.randn(H) * 0.1, torch.randn(B, H) / H ** 0.5, torch.randn(B) * 0.1]
    ws = [w.to(DEV) for w in ws]
    phi, phi_b, h2 = ops.radial_mlp(rb, env, pair, *ws, want_h2)
    assert phi.shape == (E, B) and h2.shape == ((E, H) if want_h2 else (0, H))
    assert torch.equal(phi, phi_b)
    if E == 0:
        return
    gp = torch.randn_like(phi)
    # the upstream gradient split over the two readers' views (summed in the backward kernel)
    L = (phi * (0.25 * gp)).sum() + (phi_b * (0.75 * gp)).sum()
    gh = torch.randn(E, H, device=DEV)
    if want_h2:
        L = L + (h2 * gh).sum()
    grads = torch.autograd.grad(L, [rb, env])
    # torch fp64 reference
    rc = rb.detach().double().requires_grad_(True)
    ec = env.detach().double().requires_grad_(True)
    w = [t.double() for t in ws]
    hid = torch.nn.functional.silu(rc @ w[0].T + w[1] + w[2][pair.long()])
    h2r = torch.nn.functional.silu(hid @ w[3].T + w[4])
    phir = (h2r @ w[5].T + w[6]) * ec[:, None]
    L2 = (phir * gp.double()).sum() + ((h2r * gh.double()).sum() if want_h2 else 0)
    grads2 = torch.autograd.grad(L2, [rc, ec])
    outs, refs = [phi] + ([h2] if want_h2 else []), [phir] + ([h2r] if want_h2 else [])
    errs = [rel(a, b) for a, b in zip(outs, refs)] + [rel(a, b) for a, b in zip(grads, grads2)]
    say("   errs", errs)
    assert max(errs) < TOL, errs


@pytest.mark.parametrize("E,n_sets,want_h2", [(15552, 2, False), (20000, 2, True), (1001, 3, True), (37, 4, False)])
def test_radial_mlp_sets_equal_single_launches(E, n_sets, want_h2):
    """The radial MLPs of several passes in one launch each way give bitwise the outputs and
    input gradients of one launch per pass (the same instructions per set): rb / envelope read
    through per-pass views, a second phi reader on some passes, no gradient on others."""
    from face_amd import ops
    say("radial sets", E, n_sets, want_h2)
    torch.manual_seed(E + n_sets)
    nb, H, B, n_pair = 8, 64, 16, 9
    base_rb = torch.randn(E, nb, device=DEV, requires_grad=True)
    base_env = torch.rand(E, device=DEV, requires_grad=True)
    pair = torch.randint(0, n_pair, (E,), device=DEV, dtype=torch.int32)
    wsets = []
    for _ in range(n_sets):
        ws = [torch.randn(H, nb) / nb ** 0.5, torch.randn(H) * 0.1, torch.randn(n_pair, H) * 0.3,
              torch.randn(H, H) / H ** 0.5, torch.randn(H) * 0.1, torch.randn(B, H) / H ** 0.5, torch.randn(B) * 0.1]
        wsets.append([w.to(DEV) for w in ws])
    gps = [torch.randn(E, B, device=DEV) for _ in range(n_sets)]
    ghs = [torch.randn(E, H, device=DEV) for _ in range(n_sets)]

    def loss(outs):
        L = 0
        for k, (phi, phi_b, h2) in enumerate(outs):
            L = L + (phi * gps[k]).sum()
            if k % 2 == 1:
                L = L + (phi_b * (0.5 * gps[k])).sum()
            if want_h2 and k != 1:
                L = L + (h2 * ghs[k]).sum()
        return L
    rbs = [base_rb.view(base_rb.shape) for _ in range(n_sets)]
    envs = [base_env.view(base_env.shape) for _ in range(n_sets)]
    outs = ops.radial_mlp_sets(pair, wsets, want_h2, rbs, envs)
    got = torch.autograd.grad(loss(outs), rbs + envs)
    rbs2 = [base_rb.view(base_rb.shape) for _ in range(n_sets)]
    envs2 = [base_env.view(base_env.shape) for _ in range(n_sets)]
    outs2 = [ops.radial_mlp(rbs2[k], envs2[k], pair, *wsets[k], want_h2) for k in range(n_sets)]
    want = torch.autograd.grad(loss(outs2), rbs2 + envs2)
    for a, b in zip(outs, outs2):
        for x, y in zip(a, b):
            assert torch.equal(x, y)
    for a, b in zip(got, want):
        assert torch.equal(a, b)


# ----------------------------------------------------------------------------- row-block linear layers
def _lin_ref(x, w, w_kn, y0, beta, bias, xs, ys, grp, period, s_off):
    x, w = x.double().cpu(), w.double().cpu()
    g = grp.long().cpu()[torch.arange(x.shape[0]) % period] if grp is not None else None
    if xs is not None:
        x = x * xs.double().cpu()[g][:, s_off:s_off + x.shape[1]]
    y = x @ (w if w_kn else w.T)
    if beta:
        y = y + beta * y0.double().cpu()
    if bias is not None:
        y = y + bias.double().cpu()
    if ys is not None:
        y = y * ys.double().cpu()[g][:, s_off:s_off + y.shape[1]]
    return y


@pytest.mark.parametrize("case,kc", [("single", None), ("ranks_proj", None), ("ranks_scaled", None),
                                     ("kn_xscale", None), ("k512", None), ("empty", None), ("k1024", None),
                                     ("ranks_proj", "1"), ("ranks_scaled", "1"), ("kn_xscale", "1"),
                                     ("k512", "1"), ("empty", "1")])
def test_rows_linear_matches_torch(case, kc, monkeypatch):
    """y = (beta y + (x * xs) w^T + bias) * ys over up to four problems per launch (mix / tmix /
    proj with the elem_scale factor and their input gradients) vs torch fp64: ragged row counts,
    weight column slices (ld_w > k), (k, n) weights, K = 512 and 1024, sliced outputs (n = 480), an
    empty problem beside full ones. kc = "1" forces the K-chunked kernel (the route of long K)."""
    from face_amd import ops
    if kc is not None:
        monkeypatch.setenv("FACE_ROWS_GEMM_KC", kc)
    say("rows_linear", case, kc)
    torch.manual_seed(len(case))
    N, C = 1000, 160
    grp = torch.randint(0, 3, (N,), device=DEV, dtype=torch.int32)
    tab = torch.rand(3, 4 * C, device=DEV) + 0.5
    bias = xs = ys = None
    w_kn = False
    probs, refs = [], []
    if case == "single":
        x = torch.randn(10007, C, device=DEV)
        w = torch.randn(C, C, device=DEV) / C ** 0.5
        probs = [(x, w, torch.empty(10007, C, device=DEV), 0, 0.0)]
    elif case == "ranks_proj":
        wide = torch.randn(3 * C, 2 * C, device=DEV) / C ** 0.5           # proj weight over two sets
        for l, (k, n) in enumerate(((1, C), (3, 3 * C), (6, 3 * C), (10, 2 * C))):
            x = torch.randn(k * N, C, device=DEV)
            probs.append((x, wide[:n, C:], torch.randn(k * N, n, device=DEV), 0, 1.0 if l % 2 else 0.0))
    elif case == "ranks_scaled":                                             # mix (+ tmix) * elem_scale
        ys, bias = tab, torch.randn(C, device=DEV)
        for l, k in enumerate((1, 3, 6, 10)):
            x = torch.randn(k * N, C, device=DEV)
            w = torch.randn(C, C, device=DEV) / C ** 0.5
            probs.append((x, w, torch.randn(k * N, C, device=DEV), l * C, 1.0 if l in (1, 2) else 0.0))
    elif case == "kn_xscale":
        w_kn, xs = True, tab
        for l, k in enumerate((1, 3, 6, 10)):
            x = torch.randn(k * N, C, device=DEV)
            w = torch.randn(C, 2 * C + 32, device=DEV)[:, 16:16 + 2 * C] / C ** 0.5   # (k, n), ld_w > n
            probs.append((x, w, torch.empty(k * N, 2 * C, device=DEV), l * C, 0.0))
    elif case == "k512":
        x = torch.randn(6 * N, 512, device=DEV)
        w = torch.randn(C, 512, device=DEV) / 512 ** 0.5
        probs = [(x, w, torch.randn(6 * N, C, device=DEV), 0, 1.0)]
    elif case == "k1024":                                                    # the mix of a K = 64 model
        ys = tab
        x = torch.randn(40 * N, 1024, device=DEV)
        w = torch.randn(C, 1024, device=DEV) / 32
        probs = [(x, w, torch.randn(40 * N, C, device=DEV), C, 1.0)]
    else:
        x = torch.randn(0, C, device=DEV)
        probs = [(x, torch.randn(C, C, device=DEV), torch.empty(0, C, device=DEV), 0, 0.0),
                 (torch.randn(77, C, device=DEV), torch.randn(C, C, device=DEV), torch.empty(77, C, device=DEV), 0, 0.0)]
    for (x, w, y, s, b) in probs:
        refs.append(_lin_ref(x, w, w_kn, y, b, bias, xs, ys, grp if (xs is not None or ys is not None) else None, N, s))
    ops.rows_linear(probs, w_kn=w_kn, bias=bias, xs=xs, ys=ys, group=grp, period=N)
    errs = [rel(p[2], r) if r.numel() else 0.0 for p, r in zip(probs, refs)]
    say("   errs", errs)
    assert max(errs) < 1e-5, errs


def test_rows_linear_launch_shapes_give_bitwise_equal_rows(monkeypatch):
    """face_rows_linear times launch shapes (waves per workgroup, column slices) on the first call of
    a problem signature and keeps the fastest. Every shape must give the same bits: the 864-atom
    factor mix backward (17,280 rows of 96 -> 512 columns, (k, n) weight, input scale; the shape
    the timing changes there) against its first 2,000 rows as a separate call (another signature,
    timed again) and against 17,279 rows with the timing off (the rules' shape), plus torch fp64."""
    from face_amd import ops
    say("rows_linear launch shapes")
    torch.manual_seed(11)
    N, C, BK = 864, 96, 512
    tab = torch.rand(1, 4 * C, device=DEV) + 0.5
    grp = torch.zeros(N, device=DEV, dtype=torch.int32)
    xs = [torch.randn(k * N, C, device=DEV) for k in (1, 3, 6, 10)]
    ws = [torch.randn(C, BK, device=DEV) / C ** 0.5 for _ in range(4)]

    def run(rows):
        ys = [torch.empty(min(rows, x.shape[0]), BK, device=DEV) for x in xs]
        ops.rows_linear([(x[:y.shape[0]], w, y, l * C, 0.0) for l, (x, w, y) in enumerate(zip(xs, ws, ys))],
                        w_kn=True, xs=tab, group=grp, period=N)
        torch.cuda.synchronize()
        return ys

    full = run(10 * N)                                   # timed shapes
    part = run(2000)                                     # another signature, timed separately
    monkeypatch.setenv("FACE_GEMM_TUNE", "0")
    rule = run(10 * N - 1)                               # the rules' shape
    for l, (x, w) in enumerate(zip(xs, ws)):
        ref = (x.double() * tab.double()[0, l * C:(l + 1) * C]) @ w.double()
        assert (full[l].double() - ref).abs().max() <= 1e-5 * ref.abs().max()
        assert torch.equal(part[l], full[l][:part[l].shape[0]])
        assert torch.equal(rule[l], full[l][:rule[l].shape[0]])


def _gemm_shapes(n_widest, ns_max=160):
    """Every (waves per workgroup, column slices) pair face_rows_linear's shape timing tries."""
    out = []
    for nw in (16, 8, 4):
        seen = set()
        for ns in range(16, ns_max + 1, 16):
            k = -(-n_widest // ns)
            if k <= 32 and k not in seen:
                seen.add(k)
                out.append((nw, k))
    return out


@pytest.mark.parametrize("case", ["fcc864_mix_bwd", "liquid24k_mix_fwd"])
def test_rows_linear_every_launch_shape_gives_bitwise_equal_rows(case, monkeypatch):
    """Every launch shape the timing may pick (4, 8, 16 waves per workgroup x every slice count x
    plain / XCD-aware item order, forced through FACE_GEMM_SHAPE) gives the same bits as the rules'
    shape: the 864-atom factor mix backward ((k, n) weight 96 -> 512, input scale: one item per
    workgroup) and the 24,000-atom CP mix forward (480,000 rows of 160 -> 160 over four ranks,
    (n, k) weights, output scale: more tiles than resident workgroups, so the persistent runs)."""
    from face_amd import ops
    say("rows_linear every shape", case)
    torch.manual_seed(13)
    if case == "fcc864_mix_bwd":
        N, C, n = 864, 96, 512
        w_kn, scale = True, "xs"
        ws = [torch.randn(C, n, device=DEV) / C ** 0.5 for _ in range(4)]
    else:
        N, C, n = 24000, 160, 160
        w_kn, scale = False, "ys"
        ws = [torch.randn(n, C, device=DEV) / C ** 0.5 for _ in range(4)]
    tab = torch.rand(3, 4 * max(C, n), device=DEV) + 0.5
    grp = torch.randint(0, 3, (N,), device=DEV, dtype=torch.int32)
    xs = [torch.randn(k * N, C, device=DEV) for k in (1, 3, 6, 10)]

    def run():
        ys = [torch.empty(x.shape[0], n, device=DEV) for x in xs]
        ops.rows_linear([(x, w, y, l * (C if scale == "xs" else n), 0.0)
                         for l, (x, w, y) in enumerate(zip(xs, ws, ys))], w_kn=w_kn,
                        xs=tab if scale == "xs" else None, ys=tab if scale == "ys" else None, group=grp, period=N)
        torch.cuda.synchronize()
        return ys

    monkeypatch.setenv("FACE_GEMM_TUNE", "0")
    rule = run()
    for l, (x, w) in enumerate(zip(xs, ws)):
        g = grp.long().repeat(x.shape[0] // N)
        if scale == "xs":
            ref = (x.double() * tab.double()[g, l * C:(l + 1) * C]) @ w.double()
        else:
            ref = (x.double() @ w.double().T) * tab.double()[g, l * n:(l + 1) * n]
        assert (rule[l].double() - ref).abs().max() <= 1e-5 * ref.abs().max()
    ran = refused = 0
    for nw, n_sl in _gemm_shapes(n):
        for xcd in (0, 1):
            monkeypatch.setenv("FACE_GEMM_SHAPE", f"{nw},{n_sl},{xcd}")
            try:
                out = run()
            except RuntimeError as err:                  # a shape whose slice does not fit LDS
                assert "(code -2)" in str(err), err
                refused += 1
                continue
            for a, b in zip(out, rule):
                assert torch.equal(a, b), (nw, n_sl, xcd)
            ran += 1
    say(f"   {ran} shapes bitwise equal to the rules' shape, {refused} refused")
    assert ran >= 24


@pytest.mark.parametrize("kc", [None, "1"])
@pytest.mark.parametrize("w_kn", [False, True])
def test_rows_linear_split_input_transforms_and_initial_sum(w_kn, kc, monkeypatch):
    """The readout forms of face_rows_linear vs torch fp64: input columns from two tensors
    ([x | x2], the split at k1), silu(x) and x * silu'(xz) applied to the x columns as they load,
    a bias per problem, and the sum started at beta * y0 over the first n_y0 columns of another
    tensor (a residual); four problems of different K in one launch, ragged rows, strided views.
    kc = "1" forces the K-chunked kernel."""
    from face_amd import ops
    if kc is not None:
        monkeypatch.setenv("FACE_ROWS_GEMM_KC", kc)
    say("rows_linear split/ops", w_kn, kc)
    torch.manual_seed(7)
    m = 1203
    silu = lambda t: t * torch.sigmoid(t)
    dsilu = lambda g, z: g * torch.sigmoid(z) * (1 + z * (1 - torch.sigmoid(z)))
    base = torch.randn(m, 400, device=DEV)
    cases = []
    # (x cols k1, x2 cols, n, x_op, bias, y0 cols)
    for k1, k2, n, op, has_b, ny0 in ((144, 16, 64, 0, True, 0), (96, 0, 48, 1, True, 32), (64, 32, 80, 2, False, 80),
                                      (32, 0, 16, 1, True, 16)):
        x = base[:, :k1] if op != 2 else torch.randn(m, k1, device=DEV)          # a strided view
        x2 = torch.randn(m, k2 + 8, device=DEV)[:, :k2] if k2 else None
        xz = torch.randn(m, k1, device=DEV) if op == 2 else None
        k = k1 + k2
        w = torch.randn(k, n, device=DEV) / k ** 0.5 if w_kn else torch.randn(n, k + 4, device=DEV)[:, :k] / k ** 0.5
        bias = torch.randn(n, device=DEV) if has_b else None
        y0 = torch.randn(m, ny0 + 4, device=DEV)[:, :ny0] if ny0 else None
        y = torch.empty(m, n, device=DEV)
        cases.append((ops.lin(x, w, y, x2=x2, x_op=op, xz=xz, bias=bias, y0=y0, beta=1.0 if ny0 else 0.0,
                              n_y0=ny0 if ny0 else None), (x, x2, xz, w, bias, y0, op, ny0)))
    ops.rows_linear([c[0] for c in cases], w_kn=w_kn)
    errs = []
    for pr, (x, x2, xz, w, bias, y0, op, ny0) in cases:
        d = lambda t: None if t is None else t.double().cpu()
        xi = d(x)
        xi = silu(xi) if op == 1 else (dsilu(xi, d(xz)) if op == 2 else xi)
        if x2 is not None:
            xi = torch.cat([xi, d(x2)], 1)
        ref = xi @ (d(w) if w_kn else d(w).T)
        if bias is not None:
            ref = ref + d(bias)
        if ny0:
            ref[:, :ny0] += d(y0)
        errs.append(rel(pr["y"], ref))
    say("   errs", errs)
    assert max(errs) < 1e-5, errs


@pytest.mark.parametrize("C,gate", [(160, True), (160, False), (96, True), (32, False)])
def test_readout_matches_torch(C, gate):
    """The pass readout on the row GEMM (face/model.py:331-339, the gate row of :286-287):
    LayerNorm -> [inv | h] W0^T + b0 -> SiLU -> W1 -> SiLU -> W2 with the energy column and the
    residual h + o[:, 1:], and gvm = inv Wg^T + bg; values and the gradients of feats and h (with
    the gate row's gradient entering the backward) vs torch fp64 autograd."""
    from face_amd import ops
    say("readout", C, gate)
    torch.manual_seed(C + gate)
    N, nf = 777, 9 * C
    feats = torch.randn(N, nf, device=DEV) * 2 + 0.3
    h = torch.randn(N, C + 16, device=DEV)[:, :C]                  # a strided residual, like a previous h_new
    lnw, lnb = torch.rand(nf, device=DEV) + 0.5, torch.randn(nf, device=DEV) * 0.1
    W0 = torch.randn(2 * C, 10 * C + 4, device=DEV) / (10 * C) ** 0.5
    b0 = torch.randn(2 * C, device=DEV) * 0.1
    W1, b1 = torch.randn(2 * C, 2 * C, device=DEV) / (2 * C) ** 0.5, torch.randn(2 * C, device=DEV) * 0.1
    W2, b2 = torch.randn(C + 1, 2 * C, device=DEV) / (2 * C) ** 0.5, torch.randn(C + 1, device=DEV) * 0.1
    Wg, bg = torch.randn(2 * C, nf, device=DEV) / nf ** 0.5, torch.randn(2 * C, device=DEV)
    n_pad = C + 16
    W2p = W2.new_zeros(n_pad, 2 * C)
    W2p[:C], W2p[C] = W2[1:], W2[0]
    b2p = b2.new_zeros(n_pad)
    b2p[:C], b2p[C] = b2[1:], b2[0]
    Wst = torch.cat([W0[:, :nf], Wg], 0).contiguous()
    fd, hd = feats.clone().requires_grad_(True), h.clone().requires_grad_(True)
    e, hn, gvm = ops.readout(fd, hd, lnw, lnb, 1e-5, W0, b0, W1, b1, W2p, b2p, *((Wg, bg, Wst) if gate else (None, None, None)))
    ge, gh = torch.randn(N, 1, device=DEV), torch.randn(N, C, device=DEV)
    gg = torch.randn(N, 2 * C, device=DEV)
    loss = (e * ge).sum() + (hn * gh).sum() + ((gvm * gg).sum() if gate else 0.0)
    gf, ghh = torch.autograd.grad(loss, (fd, hd))
    c = lambda t: t.detach().double().cpu()
    f2, h2 = c(feats).requires_grad_(True), c(h).requires_grad_(True)
    inv = torch.nn.functional.layer_norm(f2, (nf,), c(lnw), c(lnb), 1e-5)
    z = torch.cat([inv, h2, torch.zeros(N, 4, dtype=torch.float64)], 1) @ c(W0).T + c(b0)
    z = torch.nn.functional.silu(z) @ c(W1).T + c(b1)
    o = torch.nn.functional.silu(z) @ c(W2).T + c(b2)
    e2, hn2 = o[:, :1], h2 + o[:, 1:]
    loss2 = (e2 * c(ge)).sum() + (hn2 * c(gh)).sum()
    if gate:
        gvm2 = inv @ c(Wg).T + c(bg)
        loss2 = loss2 + (gvm2 * c(gg)).sum()
    gf2, gh2 = torch.autograd.grad(loss2, (f2, h2))
    errs = [rel(e, e2), rel(hn, hn2), rel(gf, gf2), rel(ghh, gh2)] + ([rel(gvm, gvm2)] if gate else [])
    say("   errs", errs)
    assert max(errs) < 1e-5, errs


@pytest.mark.parametrize("transport,Cin,merge", [(True, 160, True), (True, 160, False), (False, 160, True),
                                                  (False, 512, True), (True, 32, True)])
def test_scaled_mix_forward_backward(transport, Cin, merge, monkeypatch):
    """A_l = (Af_l W_l^T [+ D_l T_l^T]) * s[z] for the four ranks (face/model.py:498-501, :530-533)
    and the gradients of Af_l and D_l vs torch fp64 autograd (the transport-mix backward in the
    mix backward's launch and on its own)."""
    from face_amd import ops
    monkeypatch.setattr(ops, "MIX_MERGE_MAX_ATOMS", 1 << 30 if merge else 0)
    say("scaled mix", transport, Cin, merge)
    torch.manual_seed(Cin + transport)
    N, C, Dw = 517, 96 if Cin != 32 else 32, 64
    grp = torch.randint(0, 3, (N,), device=DEV, dtype=torch.int32)
    s_tab = torch.rand(3, 4 * C, device=DEV) + 0.5
    Af = [torch.randn(k, N, Cin, device=DEV, requires_grad=True) for k in (1, 3, 6, 10)]
    wm = [torch.randn(C, Cin, device=DEV) / Cin ** 0.5 for _ in range(4)]
    D1 = torch.randn(3, N, Dw, device=DEV, requires_grad=True) if transport else None
    D2 = torch.randn(6, N, Dw, device=DEV, requires_grad=True) if transport else None
    wt = [torch.randn(C, Dw, device=DEV) / 8, torch.randn(C, Dw, device=DEV) / 8] if transport else [None, None]
    A = ops.scaled_mix(s_tab, grp, wm, wt, D1, D2, Af)
    G = [torch.randn_like(a) for a in A]
    ins = Af + ([D1, D2] if transport else [])
    gr = torch.autograd.grad(sum((a * g).sum() for a, g in zip(A, G)), ins)
    c = lambda t: t.detach().double().cpu()
    insc = [c(t).requires_grad_(True) for t in ins]
    s = c(s_tab)[grp.long().cpu()].view(N, 4, C)
    A2 = []
    for l in range(4):
        y = insc[l] @ c(wm[l]).T
        if transport and l in (1, 2):
            y = y + insc[3 + l] @ c(wt[l - 1]).T
        A2.append(y * s[None, :, l, :])
    gr2 = torch.autograd.grad(sum((a * c(g)).sum() for a, g in zip(A2, G)), insc)
    errs = [rel(a, b) for a, b in zip(A, A2)] + [rel(a, b) for a, b in zip(gr, gr2)]
    say("   errs", errs)
    assert max(errs) < 1e-5, errs


@pytest.mark.parametrize("n_sets,C,in_row", [(1, 160, False), (2, 160, False), (2, 96, False), (3, 32, False),
                                             (2, 96, True)])
def test_rank_proj_forward_backward(n_sets, C, in_row):
    """proj of the concatenated moment sets for the four ranks (face/model.py:537-544) as one launch
    per set, with the row-sliced weights the node algebra uses (P0 | PQS | PQS | PQ), and the
    sets' gradients, vs torch fp64 autograd; in_row: rank 0 written into the first C columns of a
    wider row buffer (as for the readout row), the other columns left as they were."""
    from face_amd import ops
    say("rank proj", n_sets, C, in_row)
    torch.manual_seed(n_sets * C)
    N = 613
    full = [torch.randn(3 * C, n_sets * C, device=DEV) / C ** 0.5 for _ in range(4)]
    ws = [w[:n] for w, n in zip(full, (C, 3 * C, 3 * C, 2 * C))]
    sets = [[torch.randn(k, N, C, device=DEV, requires_grad=True) for k in (1, 3, 6, 10)] for _ in range(n_sets)]
    buf = torch.full((N, 9 * C), 7.0, device=DEV) if in_row else None
    ys = ops.rank_proj(ws, sets, out0=buf[:, :C] if in_row else None)
    if in_row:
        assert ys[0].data_ptr() == buf.data_ptr() and ys[0].stride(1) == 9 * C
        assert (buf[:, C:] == 7.0).all()
    G = [torch.randn_like(y) for y in ys]
    flat = [t for S in sets for t in S]
    gr = torch.autograd.grad(sum((y * g).sum() for y, g in zip(ys, G)), flat)
    c = lambda t: t.detach().double().cpu()
    flatc = [c(t).requires_grad_(True) for t in flat]
    ys2 = [sum(flatc[4 * s + l] @ c(ws[l][:, s * C:(s + 1) * C]).T for s in range(n_sets)) for l in range(4)]
    gr2 = torch.autograd.grad(sum((y * c(g)).sum() for y, g in zip(ys2, G)), flatc)
    errs = [rel(a, b) for a, b in zip(ys, ys2)] + [rel(a, b) for a, b in zip(gr, gr2)]
    say("   errs", max(errs))
    assert max(errs) < 1e-5, errs


@pytest.mark.parametrize("gathered,K,C,transport", [(False, 32, 96, True), (True, 32, 96, False),
                                                    (False, 64, 256, True), (True, 16, 160, True),
                                                    (False, 48, 32, False)])
def test_density_mix_fused_matches_reference(gathered, K, C, transport):
    """Factor density fused with the per-rank mix and element scale (face/kernels.py:170-178 then
    face/model.py:503-506, :530-533), forward and the gradients of phi, msg, Y and the transport
    sums, against the oracle's factor density + F.linear + scale in fp64 autograd. Ragged rows:
    a hub row, isolated atoms, N not a multiple of the 4-atom tile."""
    from face_amd import ops
    say("density+mix fused", gathered, K, C, transport)
    B, N, Dw = 16, 57, 64
    g = _G(N, 500, 5)
    counts = g.counts
    E = sum(counts)
    torch.manual_seed(K + C)
    phi = torch.randn(E, B, device=DEV, requires_grad=True)
    msg = torch.randn(N if gathered else E, K, device=DEV, requires_grad=True)
    Y = torch.randn(E, 20, device=DEV, requires_grad=True)
    grp = torch.randint(0, 3, (N,), device=DEV, dtype=torch.int32)
    s_tab = torch.rand(3, 4 * C, device=DEV) + 0.5
    wm = [torch.randn(C, B * K, device=DEV) / (B * K) ** 0.5 for _ in range(4)]
    wmt = [w.t().contiguous() for w in wm]
    D1 = torch.randn(3, N, Dw, device=DEV, requires_grad=True) if transport else None
    D2 = torch.randn(6, N, Dw, device=DEV, requires_grad=True) if transport else None
    wt = [torch.randn(C, Dw, device=DEV) / 8, torch.randn(C, Dw, device=DEV) / 8] if transport else [None, None]
    A = ops.density_mix(s_tab, grp, wm, wmt, wt, D1, D2, phi, msg, Y, g.G, gathered)
    assert [tuple(a.shape) for a in A] == [(k, N, C) for k in (1, 3, 6, 10)]
    Gs = [torch.randn_like(a) for a in A]
    ins = [phi, msg, Y] + ([D1, D2] if transport else [])
    gr = torch.autograd.grad(sum((a * gg).sum() for a, gg in zip(A, Gs)), ins)
    # oracle: padded factor density, then the four mixes with the scale
    c = lambda t: t.detach().double().cpu()
    insc = [c(t).requires_grad_(True) for t in ins]
    M = max(counts)
    col = g.G.col.long().cpu()
    pd = lambda t: _pad(t, counts, M)
    msg_e = insc[1][col] if gathered else insc[1]
    Dd = oops.factor_density(pd(insc[0]), pd(msg_e), pd(insc[2]))             # (N, 20, B K)
    s = c(s_tab)[grp.long().cpu()].view(N, 4, C)
    A2 = []
    for l, (x0, x1) in enumerate(((0, 1), (1, 4), (4, 10), (10, 20))):
        y = Dd[:, x0:x1, :].permute(1, 0, 2) @ c(wm[l]).T                      # (k_l, N, C)
        if transport and l in (1, 2):
            y = y + insc[2 + l] @ c(wt[l - 1]).T
        A2.append(y * s[None, :, l, :])
    gr2 = torch.autograd.grad(sum((a * c(gg)).sum() for a, gg in zip(A2, Gs)), insc)
    errs = [rel(a, b) for a, b in zip(A, A2)] + [rel(a, b) for a, b in zip(gr, gr2)]
    say("   errs", [f"{e:.1e}" for e in errs])
    assert max(errs) < TOL, errs
    # bitwise reproducible (fixed summation order)
    A3 = ops.density_mix(s_tab, grp, wm, wmt, wt, D1, D2, phi, msg, Y, g.G, gathered)
    assert all(torch.equal(a, b) for a, b in zip(A, A3))


@pytest.mark.parametrize("with_at,sizes", [(False, [5, 300, 1, 700, 33, 260]), (True, [5, 300, 1, 700, 33, 260]),
                                           (True, [300000]), (False, [140000, 7, 160000])])
def test_atom_energy_matches_index_add(with_at, sizes):
    """Atom energies e0 + scale * e_p added pass by pass and their per-structure sums (face/model.py:
    680-690) against index_add, ragged structures (one of a single atom; structures larger than one
    pass of the per-atom grid) and strided (N, 1) column views; the backward against autograd
    through the torch expression; a second call bitwise equal."""
    from face_amd import ops
    say("atom energy", with_at, len(sizes), sum(sizes))
    torch.manual_seed(3)
    N, nstr = sum(sizes), len(sizes)
    batch = torch.repeat_interleave(torch.arange(nstr), torch.tensor(sizes)).to(DEV)
    sp = torch.tensor([0] + list(np.cumsum(sizes)), dtype=torch.int32, device=DEV)
    e0 = torch.randn(N, device=DEV)
    scale = torch.tensor(0.7, device=DEV)
    rows = [torch.randn(N, w, device=DEV, requires_grad=True) for w in (1, 17, 9)]
    es = [r[:, :1] for r in rows]
    E, e_at = ops.atom_energy(e0, scale, sp, nstr, es)
    ref_at = e0.clone()
    for e in es:
        ref_at = ref_at + scale * e.squeeze(-1)
    ref_E = torch.zeros(nstr, device=DEV).index_add(0, batch, ref_at)
    assert torch.allclose(e_at, ref_at, rtol=1e-6, atol=1e-6)
    assert torch.allclose(E, ref_E, rtol=1e-5, atol=1e-4 * max(1.0, N ** 0.5 / 30))
    E2, e_at2 = ops.atom_energy(e0, scale, sp, nstr, es)
    assert torch.equal(E, E2) and torch.equal(e_at, e_at2)
    gE = torch.randn(nstr, device=DEV)
    g_at = torch.randn(N, device=DEV) if with_at else None
    outs, gouts = ([E, e_at], [gE, g_at]) if with_at else ([E], [gE])
    got = torch.autograd.grad(outs, rows, gouts)
    routs = [ref_E, ref_at] if with_at else [ref_E]
    want = torch.autograd.grad(routs, rows, gouts)
    for a, b in zip(got, want):
        assert torch.allclose(a, b, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("N,C,n", [(864, 96, 32), (37, 160, 48)])
def test_table_linears_match_torch(N, C, n):
    """The pass's directional table linears V pvt^T, Ms pmt^T (face/model.py:474-479) in one
    launch each way, forward and input gradients against torch fp64."""
    from face_amd import ops
    say("table linears", N, C, n)
    torch.manual_seed(N + C)
    V = torch.randn(3, N, C, device=DEV, requires_grad=True)
    Ms = torch.randn(6, N, C, device=DEV, requires_grad=True)
    wv = torch.randn(n, C, device=DEV) / C ** 0.5
    wm = torch.randn(n, C, device=DEV) / C ** 0.5
    Vb, Mb = ops.table_linears(V, Ms, wv, wm)
    gv, gm = torch.randn_like(Vb), torch.randn_like(Mb)
    got = torch.autograd.grad((Vb * gv).sum() + (Mb * gm).sum(), (V, Ms))
    Vc, Mc = V.detach().double().cpu().requires_grad_(True), Ms.detach().double().cpu().requires_grad_(True)
    Vr, Mr = Vc @ wv.double().cpu().T, Mc @ wm.double().cpu().T
    want = torch.autograd.grad((Vr * gv.double().cpu()).sum() + (Mr * gm.double().cpu()).sum(), (Vc, Mc))
    errs = [rel(Vb, Vr), rel(Mb, Mr)] + [rel(a, b) for a, b in zip(got, want)]
    assert max(errs) < 1e-5, errs
