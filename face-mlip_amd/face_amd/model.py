"""FACE energy + forces on the MI355X path (host mirror of face/model.py).

The module tree, parameter names and construction order are those of the reference's
FACE with factorised passes (face/model.py:99-158, :431-458, :559-590), so
torch.manual_seed(s) + FACE(...) gives the reference's random-init weights and
reference state_dicts load unchanged. The forward differs in layout and in where the work
runs:

  * edges are a receiver-grouped CSR list (no padded slots); geometry, basis, envelope and
    monomials come from one HIP kernel whose backward also performs the force scatter
    through the reverse-edge map (no atomics);
  * the factor density (face/kernels.py) and the CP pooling (face/model.py:496-502, with the
    cutoff envelope folded in) run in segmented HIP density kernels; the directional features
    and the transport moments (face/model.py:474-533) run in one fused HIP operator that
    reads the neighbour tables in place and writes the transport sums already mapped;
  * moments are kept monomial-major, one (k_l, N, C) tensor per rank, so `mix`, `proj` and
    the readout are plain row-major GEMMs on contiguous blocks, and the node kernel reads
    P/Q/S straight out of the projection output and writes the invariant families straight
    into the readout row;
  * only the projection columns the algebra uses are computed (P0 of rank 0; P3, Q3 of rank 3).

Supported configuration: factor=True (cp on or off), transport/eqmsg on or off, n_passes >= 1,
norm="layer", terms=(), radial_hidden in {16, 32, 48, 64}, training toggles at their defaults;
evaluation mode and first-order forces (create_graph=False), which is what the reference's fused
kernels support (face/kernels.py:10-11). Parameters enter the forward as constants (frozen()):
energies and forces differentiate through positions only.
"""
import math
import os

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from .neighbors import graph_from_padded
from .ops import Graph

RANKS = [(0, 1), (1, 4), (4, 10), (10, 20)]   # monomial range of each rank (face/cartesian.py:18)
# The readout chain on the row GEMM (ops.readout: 4 launches forward, 5 backward) instead of
# LayerNorm + library GEMMs + elementwise SiLU / residual: measured slower at the benchmark widths
# (24,000-atom C160 step 19.1 -> 21.4 ms, 864-atom C96 0.84 -> 0.96 ms: the whole-K weight
# slices leave the N x 10C -> 2C input layer and its gradient under-occupied, and the small
# 2C-wide layers pay a weight-slice staging per workgroup), so it is opt-in.
READOUT_ROW_GEMM = os.environ.get("FACE_READOUT_ROW_GEMM", "0") == "1"


class BesselEnvelope(nn.Module):
    """Radial basis constants (face/model.py:28-40); evaluated inside the edge kernel."""

    def __init__(self, n, rc, p=6):
        super().__init__()
        if p != 6:
            raise NotImplementedError("the edge kernel implements the p = 6 envelope")
        self.rc, self.p = rc, p
        self.register_buffer("freq", torch.arange(1, n + 1) * math.pi / rc)

    def evaluate(self, r):
        """(bessel (..., n), envelope (...)) in torch (face/model.py:32-40); used to tabulate the
        radial functions, the edge kernel evaluates the same closed forms per edge."""
        p, x = self.p, r / self.rc
        env = 1 - (p + 1) * (p + 2) / 2 * x ** p + p * (p + 2) * x ** (p + 1) - p * (p + 1) / 2 * x ** (p + 2)
        return torch.sin(self.freq * r[..., None]) / r[..., None] * math.sqrt(2 / self.rc), env * (x < 1)


class RadialTables:
    """Compiled radial functions of one pass (face/model.py:383-405): values T and exact
    r-derivatives dT (P element pairs, G grid points, B [+ 4C] columns) on r_g = g * dr."""

    def __init__(self, T, dT, dr):
        self.T, self.dT, self.dr = T, dT, dr

    @staticmethod
    def build(block, basis, rc, n_grid):
        """RadialSpline.build (face/model.py:392-405): the radial MLP on the grid r = linspace(0, rc,
        n_grid) clamped to >= 1e-4, per element pair, and its exact r-derivative. Evaluated in
        float64 and stored in float32 (the reference evaluates in the weights' float32): the
        kernel's r-derivative rests on differences of neighbouring table values, so table entries
        rounded once from exact values keep its round-off at the storage floor. dT by forward-mode
        differentiation: each entry depends on its own grid radius only, so one Jacobian-vector
        product with a unit tangent gives every column (the reference takes one reverse pass per
        column)."""
        f64 = torch.float64
        def lin(m):
            w = m.weight.detach().to(f64)
            return (w * m.alpha) if isinstance(m, UnitLinear) else w, None if m.bias is None else m.bias.detach().to(f64)

        (Wi, bi), (W1, b1), (W2, b2) = lin(block.rad_in), lin(block.radial[0]), lin(block.radial[2])
        pair = block.pair.weight.detach().to(f64)[:, None, :]
        r = torch.linspace(0, rc, n_grid, device=Wi.device, dtype=f64).clamp_min(1e-4)
        rr = r[None].expand(pair.shape[0], -1).contiguous()

        def table(x):
            bes, env = basis.evaluate(x)
            hid = F.silu(F.linear(bes * env[..., None], Wi, bi) + pair)
            return F.linear(F.silu(F.linear(hid, W1, b1)), W2, b2)

        T, dT = torch.func.jvp(table, (rr,), (torch.ones_like(rr),))
        f32 = lambda t: t.detach().to(torch.float32).contiguous()
        return RadialTables(f32(T), f32(dT), rc / (n_grid - 1))


class UnitLinear(nn.Module):
    """Unit-variance stored weight with forward factor fan_in**-0.5 (face/model.py:43-55)."""

    def __init__(self, fan_in, fan_out, bias=True):
        super().__init__()
        self.weight = nn.Parameter(torch.randn(fan_out, fan_in))
        self.bias = nn.Parameter(torch.zeros(fan_out)) if bias else None
        self.alpha = fan_in ** -0.5

    def forward(self, x):
        return F.linear(x, self.weight * self.alpha, self.bias)


def unit_parameterise(module):
    """Swap every nn.Linear for an equal-at-init UnitLinear, in place (face/model.py:58-70)."""
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


def _key(*ts):
    """Cache key of tensors: the tensor objects, an alias of their storage, their in-place version
    counters, data pointers and devices. The entry holds the objects and the storage aliases, so
    neither an object nor a storage the key names can be freed and recycled for another tensor
    while the entry lives; a parameter whose .data is swapped (module.to()) or changed in place
    no longer matches."""
    return tuple((t, t.detach(), t._version, t.data_ptr(), t.device) for t in ts if t is not None)


def _same(a, b):
    return a is not None and len(a) == len(b) and all(
        x[0] is y[0] and x[2:] == y[2:] for x, y in zip(a, b))


def frozen(mod):
    """Effective (weight, bias) of an nn.Linear or UnitLinear as constants of the evaluation
    graph: detached, the UnitLinear factor applied once and cached until a parameter is
    changed in place (version counter) or replaced (storage pointer). Parameters therefore
    take no gradient on this path, and a step reads no per-call weight-scaling kernels."""
    w, b = mod.weight, mod.bias
    key = _key(w, b)
    c = mod.__dict__.get("_frozen")
    if c is None or not _same(c[0], key):
        with torch.no_grad():
            W = (w * mod.alpha) if isinstance(mod, UnitLinear) else w
            c = (key, W.detach(), None if b is None else b.detach())
        mod.__dict__["_frozen"] = c
    return c[1], c[2]


def mlp(sizes):
    layers = []
    for a, b in zip(sizes[:-1], sizes[1:]):
        layers += [nn.Linear(a, b), nn.SiLU()]
    return nn.Sequential(*layers[:-1])


class FactorBlock(nn.Module):
    """One factorised interaction pass; registrations follow MomentBlock then FactorBlock."""
    N_INV = 9

    def __init__(self, C, n_basis, n_sets, radial_hidden=64, n_elem=10, K_dir=16, norm="layer", transport=False,
                 eq_in=False, eq_out=False, B=16, K=32, cp=False):
        super().__init__()
        self.C, self.n_elem, self.K = C, n_elem, K_dir
        self.eq_in, self.eq_out = eq_in, eq_out
        self.pqs_gate = nn.Embedding(n_elem, 4 * 3 * C)
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
        if norm != "layer":
            raise NotImplementedError("norm='layer' only")
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
        # factorised pass
        self.cp = cp
        self.spline = None              # RadialTables, set by FACE.compile_radial()
        if cp:
            K = C
        self.B, self.Km = B, K
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

    # ------------------------------------------------------------------ moments
    def h_products(self, h):
        """(msg(h), b0 + h W0b^T) of a pass whose h is a constant of the evaluation (the first pass's
        embedding rows, a function of the species): cached per h and weights."""
        Wm, bm = frozen(self.msg)
        W0, b0 = frozen(self.out[0])
        nf = self.N_INV * self.C
        key = _key(h, Wm, bm, W0, b0)
        c = self.__dict__.get("_hprod")
        if c is None or not _same(c[0], key):
            with torch.no_grad():
                c = (key, F.linear(h, Wm, bm), torch.addmm(b0, h, W0[:, nf:nf + self.C].t()))
            self.__dict__["_hprod"] = c
        return c[1], c[2]

    def radial_weights(self):
        """(w_in, b_in, pair_tab, w1, b1, w_phi, b_phi) of the fused radial MLP: the phi columns of
        the last radial layer (its CP columns are a GEMM on h2)."""
        Wi, bi = frozen(self.rad_in)
        W1, b1 = frozen(self.radial[0])
        W2, b2 = frozen(self.radial[2])
        return Wi, bi, self.pair.weight.detach(), W1, b1, W2[:self.B], b2[:self.B]

    def moments(self, h, rb, r, Y, env, zp, zidx, zidx32, avg_nb, sets, eq, g, order=None, radial=None):
        """Moments A_l as monomial-major (k_l, N, C) blocks (face/model.py:460-534). Y and env may be
        pairs of views of one tensor, (density reader, directional / radial reader), so that their
        gradients reach the edge backward separately (FACE.forward). radial: this pass's (phi,
        phi again, h2) when the radial MLPs of the passes were evaluated together."""
        N, E = g.N, g.E
        B, C, Kd = self.B, self.C, self.K
        Y, Y_dir = Y if isinstance(Y, tuple) else (Y, Y)
        env, env_rad = env if isinstance(env, tuple) else (env, env)
        W2, b2 = frozen(self.radial[2])
        if self.spline is not None:
            # compiled radial (face/model.py:466-467): phi = spline * env (E, B) and, in CP form,
            # the raw CP radials (E, 4C) whose envelope the pooling kernels apply
            sp = self.spline
            phi, R_sp = ops.radial_spline(r, env_rad, zp, sp.T, sp.dT, sp.dr, B, order)
            phi_dir = phi
        elif radial is not None:
            phi, phi_dir, h2 = radial
        else:
            # hidden layers and phi columns of the radial MLP in one HIP kernel; the CP columns of
            # the last layer are a GEMM on its h2 output; phi once per reader (density, transport)
            phi, phi_dir, h2 = ops.radial_mlp(rb, env_rad, zp, *self.radial_weights(), self.cp)   # (E, B) x2, (E, H)
        # (N, K); the first pass's h is the embedding rows, a constant: its products are cached
        msg_n = self.h_products(h)[0] if not h.requires_grad else F.linear(h, *frozen(self.msg))
        if self.directional:
            if self.eq_in:
                src1, src2 = eq                                                  # (3,N,C), (6,N,C)
            else:
                src1 = torch.cat([S[1] for S in sets], -1)
                src2 = torch.cat([S[2] for S in sets], -1)
            # (3, N, nt*Kd), (6, N, nt*Kd): one launch each way
            Vb, Mb = ops.table_linears(src1, src2, frozen(self.pvt)[0], frozen(self.pmt)[0])
            d, D1, D2 = ops.dir_transport(Vb, Mb, phi_dir, Y_dir, g, Kd, self.transport)   # (E, 4Kd), sums
            # gather(msg(h)) + dir_mix(d) as one per-edge matrix-core launch (and one backward)
            Wd, bd = frozen(self.dir_mix)
            if d.shape[1] % 16 == 0 and d.shape[1] <= 64 and msg_n.shape[1] % 16 == 0 and msg_n.shape[1] <= 256:
                mj = ops.edge_message(msg_n, d, Wd, bd, g)
            else:
                mj = ops.gather_neighbour(msg_n + bd, g).addmm_(d, Wd.t())
            gathered = False
        else:
            mj, gathered = msg_n, True
        s_tab = self._scale_table(avg_nb)                                        # elem_scale / avg_nb (n_el, 4C)
        if self.cp and self.spline is not None:
            Af = ops.cp_density(R_sp, env, mj, Y, g, gathered)                    # 4 x (k_l, N, C)
        elif self.cp:
            # R = h2 W2[B:]^T + b2[B:] (E, 4C) feeds the pooling (envelope applied in-kernel); on the
            # matrix-core shapes the pooling backward also applies W2[B:] and returns d h2 directly
            if C % 32 == 0 and h2.shape[1] % 16 == 0 and h2.shape[1] <= 64:
                Af = ops.cp_radial_density(h2, W2[B:], b2[B:], env, mj, Y, g, gathered)
            else:
                Af = ops.cp_density(F.linear(h2, W2[B:], b2[B:]), env, mj, Y, g, gathered)   # 4 x (k_l, N, C)
        # A_l = (mix_l(Af_l) [+ tmix_l(D_l)]) * s: D1/D2 are the raw transport sums; the reference's
        # 1/avg_nb (face/model.py:522) and its avg_nb factor (:532-533) cancel through the linear tmix,
        # leaving the common factor s = elem_scale / avg_nb, applied in the mix GEMMs' epilogue
        wm = [frozen(self.mix[l])[0] for l in range(4)]
        wt = [frozen(self.tmix1)[0], frozen(self.tmix2)[0]] if self.transport else [None, None]
        D1, D2 = (D1, D2) if self.transport else (None, None)
        if not self.cp:
            if ops.density_mix_fits(B, mj.shape[1], C, N):
                # factor density and mix in one launch each way: D stays on chip
                return list(ops.density_mix(s_tab, zidx32, wm, self._mix_t(wm), wt, D1, D2, phi, mj, Y, g,
                                            gathered))
            Af = ops.density(phi, mj, Y, g, 20, gathered)                         # 4 x (k_l, N, B*K)
        if C % 16 == 0 and Af[0].shape[-1] % 16 == 0:
            return list(ops.scaled_mix(s_tab, zidx32, wm, wt, D1, D2, Af))         # 4 x (k_l, N, C)
        s = s_tab[zidx].view(N, 4, C)
        A = []
        for l in range(4):
            x = Af[l]
            y = x.reshape(-1, x.shape[-1]) @ wm[l].t()
            if l in (1, 2) and self.transport:
                D = D1 if l == 1 else D2
                y.addmm_(D.reshape(-1, D.shape[-1]), wt[l - 1].t())
            A.append(y.view(x.shape[0], N, C) * s[None, :, l, :])                 # (k_l, N, C)
        return A

    def _readout_weights(self):
        """Frozen readout weights in the row GEMM's forms, cached with the parameters:
        (W0 (2C, 10C + 4), b0, W1, b1, W2p (n_pad, 2C), b2p, Wg, bg, Wstack): W2p / b2p hold W2's
        channel rows first, its energy row at C and zero rows up to n_pad = C + 16 (the layer
        writes [h_new | e | 0]); Wstack = [W0[:, :9C]; Wg] (4C, 9C) for the backward of the
        invariant row through both the out MLP and the gate (W0[:, :9C] alone without a gate)."""
        C, nf = self.C, self.N_INV * self.C
        mods = [self.out[0], self.out[2], self.out[4]] + ([self.gate] if self.eq_out else [])
        fr = [frozen(m) for m in mods]
        key = _key(*[t for wb in fr for t in wb])
        c = self.__dict__.get("_rw")
        if c is None or not _same(c[0], key):
            with torch.no_grad():
                (W0, b0), (W1, b1), (W2, b2) = fr[:3]
                n_pad = C + 16
                W2p = W2.new_zeros(n_pad, W2.shape[1])
                W2p[:C] = W2[1:]
                W2p[C] = W2[0]
                b2p = b2.new_zeros(n_pad)
                b2p[:C] = b2[1:]
                b2p[C] = b2[0]
                W0c = W0.contiguous()
                if self.eq_out:
                    Wg, bg = fr[3]
                    Wg, bg = Wg.contiguous(), bg.contiguous()
                    Wst = torch.cat([W0c[:, :nf], Wg], 0).contiguous()
                else:
                    Wg = bg = Wst = None
                vals = (W0c, b0.contiguous(), W1.contiguous(), b1.contiguous(), W2p, b2p, Wg, bg, Wst)
            c = (key, vals)
            self.__dict__["_rw"] = c
        return c[1]

    def _mix_t(self, wm):
        """Contiguous transposes (B K, C) of the four frozen mix weights, cached with them."""
        key = _key(*wm)
        c = self.__dict__.get("_mixT")
        if c is None or not _same(c[0], key):
            with torch.no_grad():
                c = (key, [w.t().contiguous() for w in wm])
            self.__dict__["_mixT"] = c
        return c[1]

    def _scale_table(self, avg_nb):
        """elem_scale / avg_nb per element (n_elem, 4C), cached like the frozen weights."""
        w = self.elem_scale.weight
        key = _key(w, avg_nb)
        c = self.__dict__.get("_stab")
        if c is None or not _same(c[0], key):
            with torch.no_grad():
                c = (key, (w / avg_nb).detach())
            self.__dict__["_stab"] = c
        return c[1]

    # ------------------------------------------------------------------ invariants + readout
    def forward(self, h, rb, r, Y, env, zp, zidx, zidx32, avg_nb, sets, eq, g, order=None, acc=None, last=False,
                radial=None):
        """(e (N, 1), h_new (N, C) | None, A, eq_new) of one pass. acc: the per-forward dict of
        shared moment-set gradients (ops.rank_proj) or None; last: the final pass, whose h_new is
        not computed; radial: precomputed radial MLP outputs (see moments)."""
        C = self.C
        A = self.moments(h, rb, r, Y, env, zp, zidx, zidx32, avg_nb, sets, eq, g, order, radial)
        allsets = sets + [A]
        # only P0 of rank 0 and P3, Q3 of rank 3 are used
        ws = [frozen(self.proj[l])[0][:(C, 3 * C, 3 * C, 2 * C)[l]] for l in range(4)]
        nf = self.N_INV * C
        # node algebra and the readout LayerNorm in one launch each way (the row never written)
        fused_ln = not (READOUT_ROW_GEMM and C % 16 == 0 and nf <= 2048) and C <= 256
        feats_buf = None
        if C % 16 == 0:
            # proj over the concatenated moment sets as a sum of per-set products (no concat copy),
            # all four ranks per launch, later sets accumulating in the epilogue; unless the
            # LayerNorm is fused, P0 (rank 0) is written straight into the first C columns of the
            # readout row
            feats_buf = None if fused_ln else torch.empty(g.N, nf, device=h.device)
            ys = list(ops.rank_proj(ws, allsets, acc,
                                    out0=None if fused_ln else feats_buf[:, :C]))    # (k_l, N, C | 3C | 3C | 2C)
        else:
            ys = []
            for l in range(4):
                y = None
                for si, S in enumerate(allsets):
                    Ws = ws[l][:, si * C:(si + 1) * C]
                    x2 = S[l].reshape(-1, C)
                    y = x2 @ Ws.t() if y is None else y.addmm_(x2, Ws.t())
                ys.append(y.view(S[l].shape[0], S[l].shape[1], -1))
        ab = (self.vpath.detach(), self.mpath.detach()) if self.eq_out else (None, None)
        if fused_ln:
            inv, V, Ms = ops.node_ln(ys[0], ys[1], ys[2], ys[3], *ab, self.eq_out, C, self.norm.weight,
                                     self.norm.bias, self.norm.eps)
        else:
            feats, V, Ms = ops.node_features(ys[0], ys[1], ys[2], ys[3], *ab, self.eq_out, C, feats_buf)
        if not fused_ln and READOUT_ROW_GEMM and C % 16 == 0 and nf <= 2048:
            # LayerNorm, the out MLP and the residual split on the row GEMM (four launches forward;
            # opt-in: slower than the library GEMMs at the benchmark widths)
            rw = self._readout_weights()
            e, h_new, gvm = ops.readout(feats, h, self.norm.weight.detach(), self.norm.bias.detach(), self.norm.eps,
                                        *rw)
            eq_new = None
            if self.eq_out:
                eq_new = ops.eq_gate(V, Ms, gvm)                                  # (3,N,C), (6,N,C)
            return e, h_new, A, eq_new
        if not fused_ln:
            if nf % 4 == 0 and nf <= 2048:
                inv = ops.layer_norm(feats, self.norm.weight.detach(), self.norm.bias.detach(), self.norm.eps)
            else:
                inv = F.layer_norm(feats, (nf,), self.norm.weight.detach(), self.norm.bias.detach(), self.norm.eps)
        W0, b0 = frozen(self.out[0])
        W1, b1 = frozen(self.out[2])
        W2, b2 = frozen(self.out[4])
        Wg, bg = frozen(self.gate) if self.eq_out else (None, None)
        # out MLP on cat([inv, h, 0 (4)]) (two accumulating GEMMs, no concatenated copy), residual
        # and gate row as one autograd node; the last pass computes the energy row only
        hb = self.h_products(h)[1] if not h.requires_grad else None
        e, h_new, gvm = ops.readout_mlp(inv, h, W0[:, :nf], W0[:, nf:nf + C], b0, W1, b1, W2, b2, Wg, bg, last, hb)
        eq_new = None
        if self.eq_out:
            if C % 4 == 0:
                eq_new = ops.eq_gate(V, Ms, gvm)                                  # (3,N,C), (6,N,C)
            else:
                gv, gm = gvm.chunk(2, dim=-1)
                eq_new = (V * gv[None], Ms * gm[None])
        return e, h_new, A, eq_new


class FACE(nn.Module):
    """face/model.py:558-590 (factor=True, terms=()), forward on the HIP path."""

    def __init__(self, elements, C=64, n_basis=8, rc=5.0, n_passes=2, terms=(), radial_hidden=64, K_dir=16,
                 norm="layer", transport=False, eqmsg=False, factor=True, B=16, K=32, cp=False):
        super().__init__()
        if not factor:
            raise NotImplementedError("the MI355X path serves factorised models (factor=True)")
        if terms:
            raise NotImplementedError("physics terms are outside the accelerated path")
        self.rc, self.C = rc, C
        zmap = torch.full((119,), -1, dtype=torch.long)
        for k, z in enumerate(elements):
            zmap[z] = k
        self.register_buffer("zmap", zmap)
        n_el = len(elements)
        self.basis = BesselEnvelope(n_basis, rc)
        self.embed = nn.Embedding(n_el, C)
        self.blocks = nn.ModuleList([FactorBlock(C, n_basis, t + 1, radial_hidden, n_el, K_dir, norm, transport,
                                                 eq_in=eqmsg and t > 0, eq_out=eqmsg and t < n_passes - 1,
                                                 B=B, K=K, cp=cp) for t in range(n_passes)])
        self.register_buffer("E0", torch.zeros(n_el))
        self.register_buffer("scale", torch.tensor(1.0))
        self.register_buffer("avg_nb", torch.tensor(10.0))
        self.terms = nn.ModuleDict()
        self._padded_cache = None          # (topology tensors, their versions, CSR Graph)

    def fuse(self, on=True):
        """Kept for API compatibility (face/model.py:657-663): this path is always fused."""
        return self

    @torch.no_grad()
    def compile_radial(self, n_grid=4096, on=True):
        """face/model.py:644-655: tabulate each pass's radial functions phi_b(r; Z_i, Z_j) (before the
        envelope; B [+ 4C] columns) on n_grid points per element pair; the forward then evaluates
        them by cubic Hermite interpolation (a HIP kernel) instead of the radial MLP. on=False
        returns to the MLP. Build after moving the model to its device."""
        for b in self.blocks:
            b.spline = RadialTables.build(b, self.basis, self.rc, n_grid) if on else None
        return self

    def _graph(self, g):
        if isinstance(g, Graph):
            return g
        if "csr" in g:
            gr = g["csr"]
            return gr if gr.pos is g["pos"] else gr.with_pos(g["pos"])
        # The CSR graph of a padded dict is reused only for the very same topology tensors, unchanged
        # since (identity and in-place version counter). The entry holds strong references to them,
        # so a freed dict's storage cannot be handed to a new dict of the same shape while its graph
        # is cached: a fresh dict on every call (the reference calculator's pattern,
        # face/calculator.py:52) always rebuilds.
        src = tuple(g[k] for k in ("nbr", "mask", "shift", "Z", "batch"))
        ver = tuple(t._version for t in src) + (g.get("nstr"),)
        c = self._padded_cache
        if c is None or c[1] != ver or any(a is not b for a, b in zip(c[0], src)):
            self._padded_cache = None                  # drop the old entry before building the new one
            c = (src, ver, graph_from_padded(g))
            self._padded_cache = c
        return c[2].with_pos(g["pos"])

    def forward(self, g, forces=True, create_graph=False):
        if create_graph:
            raise NotImplementedError("first-order forces only (inference / MD)")
        if self.training and torch.is_grad_enabled():
            raise NotImplementedError("this path evaluates energies and forces of a trained model: call .eval() "
                                      "(the fused radial kernel gives no weight gradients)")
        graph = self._graph(g)
        pos = graph.pos
        if forces and not pos.requires_grad:
            pos.requires_grad_(True)
        splines = [b.spline is not None for b in self.blocks]
        # each reader of Y, rb, the envelope and r gets its own view, so that the edge backward sums
        # their gradients (no addition launches): per pass, Y is read by the density and the
        # directional features, the envelope by the radial functions and the CP pooling
        readers = [(1 + b.directional, int(b.spline is None), 1 + int(b.cp), int(b.spline is not None))
                   for b in self.blocks]
        counts = [sum(x[i] for x in readers) for i in range(4)]
        geo = ops.edge_geometry(pos, graph, self.basis.freq, self.rc, with_rb=not all(splines), with_r=any(splines),
                                counts=counts)
        views, k = [], 0
        for c in counts:
            c = max(1, min(ops.EDGE_GRAD_SLOTS, c))
            views.append(list(geo[k:k + c]))
            k += c

        def take(i):
            """The next view of input i (the last one is shared once the slots run out)."""
            v = views[i]
            return v.pop(0) if len(v) > 1 else v[0]
        r = views[3][0]                  # the spline order (no gradient) reads the first r view
        # per-atom element index, element-pair row of every edge, the embedding rows and the energy
        # offsets: functions of the graph's species and of constants only, cached on the graph per
        # model (keyed like every weight cache: the tensors it depends on, their in-place versions,
        # data pointers and devices, so it can be neither recycled by another model nor outlive a
        # change of the weights, in place or by a swapped .data)
        w, E0 = self.embed.weight, self.E0
        dep = _key(self.zmap, w, E0)
        akey = ("atoms", id(self))
        ent = graph.cache.get(akey)
        if ent is None or not _same(ent[0], dep):
            zidx = self.zmap[graph.Z]
            zp = (zidx[graph.recv.long()] * len(E0) + zidx[graph.col.long()]).to(torch.int32)
            ent = (dep, (zidx, zidx.to(torch.int32), zp, F.embedding(zidx, w.detach()), E0[zidx]))
            graph.cache[akey] = ent
        zidx, zidx32, zp, h, e0 = ent[1]
        # table-cell edge order for large compiled tables: one sort per step, shared by the passes
        order = None
        big = [b.spline for b in self.blocks if b.spline is not None and ops.spline_wants_order(b.spline.T)]
        if big:
            P, G = big[0].T.shape[:2]
            if all(s.T.shape[:2] == (P, G) and s.dr == big[0].dr for s in big):
                order = ops.spline_order(r, zp, P, G, big[0].dr)
        # moment sets read only by the projections (every directional pass takes its tables from
        # the previous pass's gated outputs): their gradients accumulate in place across passes
        acc = {} if all(b.eq_in or not b.directional for b in self.blocks) else None
        sets, eq, es = [], None, []
        nb = len(self.blocks)
        rb0, r0 = views[1][0], views[3][0]
        # the radial MLPs of all MLP passes in one launch each way (they read only the edge basis)
        mlp = [t for t, b in enumerate(self.blocks) if b.spline is None]
        radial, pre = {}, {}
        if len(mlp) > 1 and len({self.blocks[t].cp for t in mlp}) == 1 and \
                len({tuple(w.shape for w in self.blocks[t].radial_weights()) for t in mlp}) == 1:
            for t in mlp:
                pre[t] = (take(1), take(2))
            outs = ops.radial_mlp_sets(zp, [self.blocks[t].radial_weights() for t in mlp], self.blocks[mlp[0]].cp,
                                       [pre[t][0] for t in mlp], [pre[t][1] for t in mlp])
            radial = dict(zip(mlp, outs))
        for t, blk in enumerate(self.blocks):
            y_d = take(0)
            y_t = take(0) if blk.directional else y_d
            if t in pre:
                rb_b, env_r = pre[t]
            else:
                rb_b = take(1) if blk.spline is None else rb0
                env_r = take(2)
            env_d = take(2) if blk.cp else env_r
            r_b = take(3) if blk.spline is not None else r0
            e, h, A, eq = blk(h, rb_b, r_b, (y_d, y_t), (env_d, env_r), zp, zidx, zidx32, self.avg_nb, sets, eq, graph,
                              order, acc, last=t == nb - 1, radial=radial.get(t))
            sets.append(A)
            es.append(e)
        E, e_at = ops.atom_energy(e0, self.scale, graph.struct_ptr, graph.nstr, es)
        out = {"energy": E, "atom_energy": e_at}
        if forces:
            # forces = -dE/dpos directly: the backward is seeded with -1 per structure
            key = ("neg_ones", graph.nstr)
            seed = graph.cache.get(key)
            if seed is None or seed.device != E.device:
                seed = torch.full((graph.nstr,), -1.0, device=E.device)
                graph.cache[key] = seed
            # the backward runs on this thread: handing it to autograd's device thread cost ~1.4 ms
            # per eager 864-atom step (4.1 -> 2.7 ms) in cross-thread scheduling of ~90 small launches
            with torch.autograd.set_multithreading_enabled(False):
                (out["forces"],) = torch.autograd.grad(E, pos, grad_outputs=seed)
        return out
