"""Unfused FACE energy + forces in plain torch (oracle; CPU, fp32 or fp64).

Restates the reference's factorised model (face/model.py) for the configurations the hot
path serves: FactorBlock passes (factor=True, cp on/off), optional transport and eqmsg,
LayerNorm readout, no physics terms, every training toggle at its default (off).

Module construction follows the reference's order exactly (face/model.py:99-158 then
:431-458, FACE :559-578), including modules that are created and then replaced or deleted,
because torch.manual_seed(s) followed by construction must reproduce the reference's
random-init weights; the state_dict keys match the reference's.

Pinned by: tests/golden/*.npz, written by tests/golden/make_golden.py from the reference's
own FACE.forward on the CPU (weights, energies and forces at seeded init), and by the
invariance checks of tests/test_symmetry.py restated in tests/test_oracle.py. RadialSpline /
compile_radial: exactness for cubics, the tables against the MLP and its central differences,
and compiled-vs-MLP agreement in fp64 (tests/test_oracle.py).
"""
import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .cartesian import RANK_SLICE, Y2_WEIGHT, monomials, to_sym2
from . import ops


class BesselEnvelope(nn.Module):
    """face/model.py:28-40: bes_n(r) = sin(n pi r / rc) / r * sqrt(2/rc), n = 1..n, and the
    p=6 polynomial envelope 1 - 28 x^6 + 48 x^7 - 21 x^8 (x = r/rc), zero for x >= 1."""

    def __init__(self, n, rc, p=6):
        super().__init__()
        self.rc, self.p = rc, p
        self.register_buffer("freq", torch.arange(1, n + 1) * math.pi / rc)

    def envelope(self, r):
        p, x = self.p, r / self.rc
        c0, c1, c2 = (p + 1) * (p + 2) / 2, p * (p + 2), p * (p + 1) / 2
        return (1 - c0 * x ** p + c1 * x ** (p + 1) - c2 * x ** (p + 2)) * (x < 1)

    def forward(self, r):
        rr = r[..., None]
        return torch.sin(self.freq * rr) / rr * math.sqrt(2 / self.rc), self.envelope(r)


class RadialSpline(nn.Module):
    """face/model.py:383-418: radial functions from a uniform-grid table of values T and exact
    r-derivatives dT (P pairs, G points, columns), cubic Hermite (C1) between grid points."""

    def __init__(self, T, dT, dr):
        super().__init__()
        self.register_buffer("T", T)
        self.register_buffer("dT", dT)
        self.dr = dr

    @staticmethod
    def build(block, basis, rc, n_grid, store_dtype=None):
        """face/model.py:392-405: the radial MLP on r = linspace(0, rc, n_grid).clamp_min(1e-4) per
        element pair; dT column by column by reverse-mode autograd, as the reference does.
        store_dtype: round the tables to that type (and back), as a table stored in it."""
        w = block.rad_in.weight
        r = torch.linspace(0, rc, n_grid, dtype=w.dtype).clamp_min(1e-4)
        P = block.pair.weight.shape[0]
        with torch.enable_grad():
            rr = r[None].expand(P, -1).clone().requires_grad_(True)
            bes, env = basis(rr)
            x = F.silu(block.rad_in(bes * env[..., None]) + block.pair.weight[:, None, :])
            T = block.radial(x)
            dT = torch.stack([torch.autograd.grad(T[..., b].sum(), rr, retain_graph=True)[0]
                              for b in range(T.shape[-1])], -1)
        T, dT = T.detach(), dT.detach()
        if store_dtype is not None:
            T, dT = T.to(store_dtype).to(T.dtype), dT.to(store_dtype).to(dT.dtype)
        return RadialSpline(T, dT, rc / (n_grid - 1))

    def forward(self, r, pair):
        """face/model.py:407-418."""
        P, G, B = self.T.shape
        x = (r / self.dr).clamp(0, G - 1)
        i = torch.floor(x).long().clamp(max=G - 2)
        t = (x - i)[..., None]
        flat = (pair * G + i).reshape(-1)
        T, dT = self.T.reshape(P * G, B), self.dT.reshape(P * G, B)
        sh = (*r.shape, B)
        p0, p1 = T.index_select(0, flat).view(sh), T.index_select(0, flat + 1).view(sh)
        m0, m1 = dT.index_select(0, flat).view(sh) * self.dr, dT.index_select(0, flat + 1).view(sh) * self.dr
        t2, t3 = t * t, t * t * t
        return (2 * t3 - 3 * t2 + 1) * p0 + (t3 - 2 * t2 + t) * m0 + (-2 * t3 + 3 * t2) * p1 + (t3 - t2) * m1


class UnitLinear(nn.Module):
    """face/model.py:43-55: stored weight W/alpha, forward F.linear(x, weight*alpha, bias)."""

    def __init__(self, fan_in, fan_out, bias=True):
        super().__init__()
        self.weight = nn.Parameter(torch.randn(fan_out, fan_in))
        self.bias = nn.Parameter(torch.zeros(fan_out)) if bias else None
        self.alpha = fan_in ** -0.5

    def forward(self, x):
        return F.linear(x, self.weight * self.alpha, self.bias)


def unit_parameterise(module):
    """face/model.py:58-70: every nn.Linear (named_children recursion) -> UnitLinear."""
    for name, child in list(module.named_children()):
        if isinstance(child, nn.Linear):
            u = UnitLinear(child.in_features, child.out_features, child.bias is not None).to(child.weight)
            with torch.no_grad():
                u.weight.copy_(child.weight / u.alpha)
                if child.bias is not None:
                    u.bias.copy_(child.bias)
            setattr(module, name, u)
        else:
            unit_parameterise(child)
    return module


def mlp(sizes):
    """face/model.py:73-77: Linear/SiLU stack without a final activation."""
    layers = []
    for a, b in zip(sizes[:-1], sizes[1:]):
        layers += [nn.Linear(a, b), nn.SiLU()]
    return nn.Sequential(*layers[:-1])


class FactorPass(nn.Module):
    """One interaction pass (reference FactorBlock on top of MomentBlock)."""
    N_INV = 9

    def __init__(self, C, n_basis, n_sets, radial_hidden, n_elem, K_dir, transport, eq_in, eq_out, B, K, cp):
        super().__init__()
        # --- MomentBlock.__init__ (face/model.py:99-158), same module order ---
        self.C, self.n_elem, self.K = C, n_elem, K_dir
        self.eq_in, self.eq_out = eq_in, eq_out
        self.pqs_gate = nn.Embedding(n_elem, 12 * C)
        nn.init.ones_(self.pqs_gate.weight)
        self.register_buffer("mom_scale", torch.ones(4))
        self.register_buffer("eq_scale", torch.ones(2))
        self.register_buffer("inv_scale", torch.ones(self.N_INV))
        self.register_buffer("calibrated", torch.tensor(False))
        self.rad_in = nn.Linear(n_basis, radial_hidden)
        self.pair = nn.Embedding(n_elem * n_elem, radial_hidden)
        nn.init.zeros_(self.pair.weight)
        self.directional = n_sets > 1
        self.transport = transport and self.directional
        self.radial = mlp([radial_hidden, radial_hidden, (8 if self.transport else 4) * C])
        cin = C * n_sets
        self.proj = nn.ModuleList([nn.Linear(cin, 3 * C, bias=False) for _ in range(4)])
        self.elem_scale = nn.Embedding(n_elem, 4 * C)
        nn.init.ones_(self.elem_scale.weight)
        self.out = mlp([self.N_INV * C + C + 4, 2 * C, 2 * C, C + 1])
        self.norm = nn.LayerNorm(self.N_INV * C)
        if self.directional:
            cprev = C if eq_in else C * (n_sets - 1)
            self.pv = nn.Linear(cprev, K_dir, bias=False)
            self.pm = nn.Linear(cprev, K_dir, bias=False)
            self.dir_mix = nn.Linear(4 * K_dir, C)
        if self.transport:
            self.tv = nn.Linear(cprev, C, bias=False)
            self.tm = nn.Linear(cprev, C, bias=False)
        if eq_out:
            self.vpath = nn.Parameter(torch.ones(4, C))
            self.mpath = nn.Parameter(torch.ones(4, C))
            self.gate = nn.Linear(self.N_INV * C, 2 * C)
            nn.init.zeros_(self.gate.weight)
            nn.init.ones_(self.gate.bias)
        # --- FactorBlock.__init__ (face/model.py:431-458) ---
        self.cp = cp
        if cp:
            K = C
        self.B, self.Km = B, K
        self.spline = None              # RadialSpline, set by FACE.compile_radial()
        self._r = None
        self.radial = mlp([radial_hidden, radial_hidden, B + (4 * C if cp else 0)])
        self.msg = nn.Linear(C, K)
        self.mix = nn.ModuleList([nn.Linear(C if cp else B * K, C, bias=False) for _ in range(4)])
        if self.directional:
            self.dir_mix = nn.Linear(4 * K_dir, K)
            nt = 2 if self.transport else 1
            del self.pv, self.pm
            self.pvt = nn.Linear(cprev, nt * K_dir, bias=False)
            self.pmt = nn.Linear(cprev, nt * K_dir, bias=False)
        if self.transport:
            del self.tv, self.tm
            self.tmix1 = nn.Linear(B * 2 * K_dir, C, bias=False)
            self.tmix2 = nn.Linear(B * 2 * K_dir, C, bias=False)
            self.tmix3 = nn.Linear(B * 2 * K_dir, C, bias=False)

    # ---- moments: face/model.py:460-534 ----
    def moments(self, h, rb, Y, nbr, env, zidx, avg_nb, prev_A, eq):
        N, M = nbr.shape
        B, C, Kd = self.B, self.C, self.K
        at_j = lambda x: x[nbr]                                   # (N,M,...) neighbour gather
        zp = zidx[:, None] * self.n_elem + zidx[nbr]
        if self.spline is not None:                               # face/model.py:466-467
            phi = self.spline(self._r, zp) * env[..., None]
        else:
            phi = self.radial(F.silu(self.rad_in(rb) + self.pair(zp))) * env[..., None]
        if self.cp:
            Rcp = phi[..., B:].reshape(N, M, 4, C)
            phi = phi[..., :B]
        mj = at_j(self.msg(h))
        u = Y[..., 1:4]
        if self.directional:
            src1 = eq[0] if self.eq_in else torch.cat([A[1] for A in prev_A], 1)
            src2 = eq[1] if self.eq_in else torch.cat([A[2] for A in prev_A], 1)
            Vb = self.pvt(src1.transpose(1, 2)).transpose(1, 2)           # (N,nt*Kd,3)
            Mb = self.pmt(src2.transpose(1, 2)).transpose(1, 2)           # (N,nt*Kd,6)
            Vi, Mi = Vb[:, :Kd], Mb[:, :Kd]
            Y2 = Y[..., 4:10] * Y2_WEIGHT.to(Y)
            d = torch.cat([
                torch.einsum("nma,nmka->nmk", u, at_j(Vi)),
                torch.einsum("nma,nmka->nmk", Y2, at_j(Mi)),
                torch.einsum("nma,nka->nmk", u, Vi),
                torch.einsum("nma,nka->nmk", Y2, Mi)], -1)
            mj = mj + self.dir_mix(d)
        s = self.elem_scale(zidx).view(N, 4, C) / avg_nb
        if self.cp:
            Af = ops.cp_density(Rcp, mj, Y)                               # (N,20,C)
        else:
            Af = ops.factor_density(phi, mj, Y)                           # (N,20,BK)
        A = [self.mix[l](Af[:, RANK_SLICE[l]]).transpose(1, 2) * s[:, l, :, None] for l in range(4)]
        if self.transport:
            D1, D2 = ops.transport_sums(phi, u, at_j(Vb[:, Kd:]), at_j(Mb[:, Kd:]), avg_nb)
            A[1] = A[1] + self.tmix1(D1.transpose(1, 2)).transpose(1, 2) * (s[:, 1, :, None] * avg_nb)
            A[2] = A[2] + self.tmix2(D2.transpose(1, 2)).transpose(1, 2) * (s[:, 2, :, None] * avg_nb)
        return A

    # ---- invariants + readout: face/model.py:204-249,252-264,272-296,310-339 ----
    def forward(self, h, rb, Y, nbr, env, zidx, avg_nb, prev_A, eq):
        C = self.C
        A = self.moments(h, rb, Y, nbr, env, zidx, avg_nb, prev_A, eq)
        sets = prev_A + [A]
        PQS = []
        for l in range(4):
            x = torch.cat([S[l] for S in sets], 1)                       # (N,cin,k_l)
            y = self.proj[l](x.transpose(1, 2)).transpose(1, 2)           # (N,3C,k_l)
            PQS.append(y.split(C, 1))
        (P0, _, _), (P1, Q1, S1), (P2, Q2, S2), (P3, Q3, _) = PQS
        zero = P1.new_zeros(4, C)
        a = self.vpath if self.eq_out else zero
        b = self.mpath if self.eq_out else zero
        inv8, V, Mf = ops.node_algebra_sym(P1, Q1, S1, P2, Q2, S2, P3, Q3, a, b)
        inv = torch.cat([P0[..., 0]] + list(inv8.unbind(-1)), 1)         # (N,9C) family-major
        inv = self.norm(inv)
        o = self.out(torch.cat([inv, h, inv.new_zeros(inv.shape[0], 4)], 1))
        eq_new = None
        if self.eq_out:
            Ms = to_sym2(0.5 * (Mf + Mf.transpose(-1, -2)))
            gv, gm = self.gate(inv).chunk(2, dim=-1)
            eq_new = (V * gv[..., None], Ms * gm[..., None])
        return o[:, :1], h + o[:, 1:], A, eq_new


class FACE(nn.Module):
    """face/model.py:558-590,665-695 restricted to factor=True and terms=()."""

    def __init__(self, elements, C=64, n_basis=8, rc=5.0, n_passes=2, terms=(), radial_hidden=64, K_dir=16,
                 norm="layer", transport=False, eqmsg=False, factor=True, B=16, K=32, cp=False):
        super().__init__()
        if not factor or terms or norm != "layer":
            raise NotImplementedError("oracle covers factor=True, terms=(), norm='layer'")
        self.rc, self.C = rc, C
        zmap = torch.full((119,), -1, dtype=torch.long)
        for k, z in enumerate(elements):
            zmap[z] = k
        self.register_buffer("zmap", zmap)
        n_el = len(elements)
        self.basis = BesselEnvelope(n_basis, rc)
        self.embed = nn.Embedding(n_el, C)
        self.blocks = nn.ModuleList([
            FactorPass(C, n_basis, t + 1, radial_hidden, n_el, K_dir, transport,
                       eq_in=eqmsg and t > 0, eq_out=eqmsg and t < n_passes - 1, B=B, K=K, cp=cp)
            for t in range(n_passes)])
        self.register_buffer("E0", torch.zeros(n_el))
        self.register_buffer("scale", torch.tensor(1.0))
        self.register_buffer("avg_nb", torch.tensor(10.0))
        self.terms = nn.ModuleDict()

    @torch.no_grad()
    def compile_radial(self, n_grid=4096, on=True, store_dtype=None):
        """face/model.py:644-655 (store_dtype: see RadialSpline.build)."""
        for b in self.blocks:
            b.spline = RadialSpline.build(b, self.basis, self.rc, n_grid, store_dtype) if on else None
        return self

    def forward(self, g, forces=True):
        pos = g["pos"]
        if forces and not pos.requires_grad:
            pos.requires_grad_(True)
        nbr, mask = g["nbr"], g["mask"]
        vec = pos[nbr] - pos[:, None] + g["shift"]
        r2 = (vec * vec).sum(-1)
        r = torch.sqrt(torch.where(mask, r2, torch.ones_like(r2)))
        u = vec / r[..., None]
        bes, env = self.basis(r)
        env = env * mask
        rb = bes * env[..., None]
        Y = monomials(u)
        zidx = self.zmap[g["Z"]]
        h = self.embed(zidx)
        e_at = self.E0[zidx].clone()
        sets, eq = [], None
        for blk in self.blocks:
            blk._r = r
            e, h, A, eq = blk(h, rb, Y, nbr, env, zidx, self.avg_nb, sets, eq)
            sets.append(A)
            e_at = e_at + self.scale * e.squeeze(-1)
        nstr = g["nstr"] if "nstr" in g else int(g["batch"].max()) + 1
        E = torch.zeros(nstr, dtype=e_at.dtype).index_add(0, g["batch"], e_at)
        out = {"energy": E, "atom_energy": e_at}
        if forces:
            (grad,) = torch.autograd.grad(E.sum(), pos)
            out["forces"] = -grad
        return out
