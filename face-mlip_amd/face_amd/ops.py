"""Autograd operators over the HIP kernels (CSR edge layout).

Every operator here launches the kernels of libface_hip.so on torch's current stream; none
has a torch or CPU fallback. Edge tensors are grouped by receiver atom (CSR `row_ptr`), and
the backward of every neighbour gather is a row reduction through the reverse-edge map
(`rev`) instead of an atomic scatter, so forces are bitwise reproducible.
"""
import math
import os

import torch

from . import _lib
from ._lib import call, ptr


def _rows(t, width):
    """(rows, >= width) fp32 view with unit column stride -> (tensor, row stride)."""
    if t.dtype != torch.float32:
        t = t.float()
    if t.dim() != 2 or t.stride(1) != 1 or t.stride(0) < width:
        t = t.contiguous()
    return t, t.stride(0)


class Graph:
    """Receiver-grouped (CSR) edge list of a batch of structures on the device.

    pos (N,3) fp32, Z (N,) int64, batch (N,) int64, nstr, struct_ptr (nstr+1) int32,
    row_ptr (N+1) int32, col (E) int32 neighbour, recv (E) int32 receiver, shift (E,3) fp32,
    rev (E) int32 reverse edge, max_row (host int), optional S (E,3) int32 image offsets.
    """

    def __init__(self, pos, Z, batch, nstr, struct_ptr, row_ptr, col, recv, shift, rev, max_row, S=None):
        self.pos, self.Z, self.batch, self.nstr = pos, Z, batch, nstr
        self.struct_ptr, self.row_ptr, self.col, self.recv = struct_ptr, row_ptr, col, recv
        self.shift, self.rev, self.max_row, self.S = shift, rev, max_row, S
        self.cache = {}

    @property
    def N(self):
        return self.pos.shape[0]

    @property
    def E(self):
        return self.col.shape[0]

    def with_pos(self, pos):
        g = Graph(pos, self.Z, self.batch, self.nstr, self.struct_ptr, self.row_ptr, self.col, self.recv,
                  self.shift, self.rev, self.max_row, self.S)
        g.cache = self.cache
        return g


# ----------------------------------------------------------------------------- edge geometry
EDGE_GRAD_SLOTS = 4                 # gradient buffers per edge input the edge backward sums


class EdgeGeometry(torch.autograd.Function):
    """pos -> (Y (E,20), rb (E,nb), env (E), r (E)) for the edges of `graph` (face/model.py:670-677).
    With_r False: r is an empty tensor; with_rb False (compiled radial, which reads r instead of
    the Bessel rows): rb is an empty tensor and is not computed. counts = (n_y, n_rb, n_env, n_r):
    each input is returned that many times, as views of one tensor, one per reader, so that the
    readers' gradients arrive separately and the edge backward sums them (no addition launches)."""

    @staticmethod
    def forward(ctx, pos, graph, freq, rc, bes_scale, with_rb, with_r, counts):
        _lib.require_gpu(pos)
        pos = pos.contiguous().float()
        E, nb = graph.E, freq.numel()
        Y = torch.empty(E, 20, device=pos.device)
        rb = torch.empty(E if with_rb else 0, nb, device=pos.device)
        env = torch.empty(E, device=pos.device)
        r = torch.empty(E if with_r else 0, device=pos.device)
        call("face_edge_geom_fwd", ptr(pos), ptr(graph.recv), ptr(graph.col), ptr(graph.shift), None, E, ptr(freq),
             nb, float(rc), float(bes_scale), ptr(Y), ptr(rb) if with_rb else None, ptr(env),
             ptr(r) if with_r else None, _lib.stream_of(pos), label="edge_fwd")
        ctx.save_for_backward(pos, freq)
        ctx.graph, ctx.rc, ctx.bes_scale, ctx.counts = graph, rc, bes_scale, counts
        ctx.set_materialize_grads(False)
        out = []
        for t, n in zip((Y, rb, env, r), counts):
            out += [t] + [t.view(t.shape) for _ in range(n - 1)]
        return tuple(out)

    @staticmethod
    def backward(ctx, *grads):
        pos, freq = ctx.saved_tensors
        g = ctx.graph
        gvec = torch.empty(g.E, 4, device=pos.device)          # 16-byte rows (x, y, z, unused)
        keep = []

        def slots(gs):
            ts = [t.contiguous().float() for t in gs if t is not None and t.numel() > 0]
            if not ts:
                return None
            keep.extend(ts)
            return _lib.ptr_array(ts + [None] * (EDGE_GRAD_SLOTS - len(ts)))

        groups, i = [], 0
        for n in ctx.counts:
            groups.append(slots(grads[i:i + n]))
            i += n
        st = _lib.stream_of(pos)
        # edge backward: each edge's dL/dvec lands in its reverse edge's slot and the own-row sums are
        # reduced per 64-edge window in the same pass (wsum), so the scatter reads one contiguous row
        # per atom, no reverse-edge gathers: grad_k = sum_{e in row k} gvec[rev e] - gvec[e]
        wsum = torch.empty(g.E, 4, device=pos.device)
        call("face_edge_geom_bwd_seg", ptr(pos), ptr(g.recv), ptr(g.col), ptr(g.shift), ptr(g.rev), g.E, ptr(freq),
             freq.numel(), float(ctx.rc), float(ctx.bes_scale), *groups, ptr(gvec), ptr(wsum), st, label="edge_bwd")
        gpos = torch.empty_like(pos)
        mean_row = (g.E + max(g.N, 1) - 1) // max(g.N, 1)
        call("face_force_scatter_rows", ptr(gvec), ptr(wsum), ptr(g.row_ptr), g.N, mean_row, 1.0, ptr(gpos), st,
             label="force_scatter")
        return gpos, None, None, None, None, None, None, None


def edge_geometry(pos, graph, freq, rc, with_rb=True, with_r=False, counts=(1, 1, 1, 1)):
    """(Y..., rb..., env..., r...): each input counts[i] times (views, one per reader; at most
    EDGE_GRAD_SLOTS each); rb / r are empty tensors when not asked for."""
    counts = tuple(max(1, min(EDGE_GRAD_SLOTS, int(c))) for c in counts)
    return EdgeGeometry.apply(pos, graph, freq, rc, math.sqrt(2.0 / rc), with_rb, with_r, counts)


# ----------------------------------------------------------------------------- gathers
class GatherNeighbour(torch.autograd.Function):
    """X (N,F) -> X[col] (E,F); backward dX[k] = sum_{e in row k} g[rev e] (no atomics)."""

    @staticmethod
    def forward(ctx, X, graph):
        X, ld = _rows(X, X.shape[1])
        F = X.shape[1]
        out = torch.empty(graph.E, F, device=X.device)
        call("face_gather_rows", ptr(X), ld, ptr(graph.col), graph.E, F, ptr(out), F, _lib.stream_of(X))
        ctx.graph, ctx.N = graph, X.shape[0]
        return out

    @staticmethod
    def backward(ctx, g):
        gr = ctx.graph
        g, ld = _rows(g, g.shape[1])
        F = g.shape[1]
        dX = torch.empty(ctx.N, F, device=g.device)
        call("face_gather_rows_bwd", ptr(g), ld, ptr(gr.row_ptr), ptr(gr.rev), gr.N, F, ptr(dX), F,
             _lib.stream_of(g))
        return dX, None


class GatherReceiver(torch.autograd.Function):
    """X (N,F) -> X[recv] (E,F); backward is the row sum dX[k] = sum_{e in row k} g[e]."""

    @staticmethod
    def forward(ctx, X, graph):
        X, ld = _rows(X, X.shape[1])
        F = X.shape[1]
        out = torch.empty(graph.E, F, device=X.device)
        call("face_gather_rows", ptr(X), ld, ptr(graph.recv), graph.E, F, ptr(out), F, _lib.stream_of(X))
        ctx.graph, ctx.N = graph, X.shape[0]
        return out

    @staticmethod
    def backward(ctx, g):
        gr = ctx.graph
        g, ld = _rows(g, g.shape[1])
        F = g.shape[1]
        dX = torch.empty(ctx.N, F, device=g.device)
        call("face_segment_sum", ptr(g), ld, ptr(gr.row_ptr), gr.N, F, ptr(dX), F, _lib.stream_of(g))
        return dX, None


def gather_neighbour(X, graph):
    # 2-d tables come back as the operator's own output (not a view of it), so callers may
    # accumulate into it in place without autograd copying the gradient
    shp = X.shape
    out = GatherNeighbour.apply(X.reshape(shp[0], -1), graph)
    return out if X.dim() == 2 else out.view(graph.E, *shp[1:])


def gather_receiver(X, graph):
    shp = X.shape
    out = GatherReceiver.apply(X.reshape(shp[0], -1), graph)
    return out if X.dim() == 2 else out.view(graph.E, *shp[1:])


# directional tables of at most this many bytes are read in place by the edge kernels
DIR_PACK_MIN_BYTES = 4 << 20


class DirTransport(torch.autograd.Function):
    """Directional edge features and transport moments from the node tables Vb (3, N, nt*Kd),
    Mb (6, N, nt*Kd) (component-major; channels [0, Kd) directional, [Kd, 2Kd) transport).

    d (E, 4Kd) = [u.V_j | u^T M_j u | u.V_i | u^T M_i u]          (face/model.py:474-493)
    D1 (3, N, B*2Kd), D2 (6, N, B*2Kd): sum_e phi[e, b] F(u, V_j, M_j)  (face/model.py:514-528)
    One autograd node for both, so the tables' gradient is assembled in place (no slices). Tables
    larger than an L2 (DIR_PACK_MIN_BYTES) are read node-major, packed as P (N, nt, 9, Kd)
    ([node][directional | transport][V0..V2, M0..M5][channel]): a neighbour's 9 component rows of
    one part are 36 Kd contiguous bytes instead of 9 rows each in its own cache line; smaller ones
    (held in L2 whatever the layout) are read where the linears wrote them, with no packing
    copies either way.
    """

    @staticmethod
    def _tables(V, M, N, nt, Kd, packed, t):
        """(V, v_sn, v_sq, M, m_sn, m_sq) pointers and strides of part t (0 directional, 1
        transport): in the packed P (V is P, M unused) or in place in the (3|6, N, nt*Kd) tables."""
        if packed:
            base = ptr(V) + 4 * t * 9 * Kd
            sn = nt * 9 * Kd
            return base, sn, Kd, base + 4 * 3 * Kd, sn, Kd
        return ptr(V) + 4 * t * Kd, nt * Kd, N * nt * Kd, ptr(M) + 4 * t * Kd, nt * Kd, N * nt * Kd

    @staticmethod
    def forward(ctx, Vb, Mb, phi, Y, graph, Kd, transport):
        _lib.require_gpu(Vb, Mb, phi, Y)
        Y = Y.contiguous().float()
        N, E = graph.N, graph.E
        dev = Vb.device
        st = _lib.stream_of(Vb)
        nt = Vb.shape[2] // Kd
        # tables that fit in an L2 are read in place (no packing copies); larger ones are packed
        packed = 9 * N * nt * Kd * 4 > DIR_PACK_MIN_BYTES
        if packed:
            P = torch.empty(N, nt, 9, Kd, device=dev)
            P[:, :, :3].copy_(Vb.float().view(3, N, nt, Kd).permute(1, 2, 0, 3))
            P[:, :, 3:].copy_(Mb.float().view(6, N, nt, Kd).permute(1, 2, 0, 3))
            tabs = (P, P)
        else:
            tabs = (Vb.contiguous().float(), Mb.contiguous().float())
        tab = lambda t: DirTransport._tables(tabs[0], tabs[1], N, nt, Kd, packed, t)
        d = torch.empty(E, 4 * Kd, device=dev)
        call("face_dir_feats_fwd", *tab(0), Kd, ptr(graph.recv), ptr(graph.col), ptr(Y), E, ptr(d), st,
             label="dir_fwd")
        D1 = D2 = None
        phi_ = phi
        if transport:
            phi_, ld_phi = _rows(phi, phi.shape[1])
            B = phi.shape[1]
            D1 = torch.empty(3, N, B * 2 * Kd, device=dev)
            D2 = torch.empty(6, N, B * 2 * Kd, device=dev)
            call("face_transport_fwd", ptr(phi_), ld_phi, B, *tab(1), Kd, ptr(Y), 20,
                 ptr(graph.col), ptr(graph.row_ptr), N, 1.0, ptr(D1), ptr(D2), st, label="transport_fwd")
        ctx.save_for_backward(tabs[0], tabs[1] if not packed else torch.empty(0),
                              phi_ if transport else torch.empty(0), Y)
        ctx.graph, ctx.Kd, ctx.transport, ctx.nt, ctx.packed = graph, Kd, transport, nt, packed
        return d, D1, D2

    @staticmethod
    def backward(ctx, gd, gD1, gD2):
        T0, T1, phi, Y = ctx.saved_tensors
        g, Kd, nt, packed = ctx.graph, ctx.Kd, ctx.nt, ctx.packed
        N, E = g.N, g.E
        dev = T0.device
        st = _lib.stream_of(T0)
        tabs = (T0, T0) if packed else (T0, T1)
        gtabs = (torch.empty_like(T0),) * 2 if packed else (torch.empty_like(T0), torch.empty_like(T1))
        tab = lambda t: DirTransport._tables(tabs[0], tabs[1], N, nt, Kd, packed, t)
        gtab = lambda t: DirTransport._tables(gtabs[0], gtabs[1], N, nt, Kd, packed, t)
        gd = torch.zeros(E, 4 * Kd, device=dev) if gd is None else gd.contiguous().float()
        gY = torch.empty_like(Y)
        g0 = gtab(0)
        call("face_dir_feats_bwd", *tab(0), Kd, ptr(g.row_ptr), ptr(g.recv), ptr(g.col), ptr(g.rev), ptr(Y),
             ptr(gd), N, E, g0[0], g0[3], ptr(gY), st, label="dir_bwd")
        dphi = None
        if ctx.transport:
            B = phi.shape[1]
            W = B * 2 * Kd
            gD1 = torch.zeros(3, N, W, device=dev) if gD1 is None else gD1.contiguous().float()
            gD2 = torch.zeros(6, N, W, device=dev) if gD2 is None else gD2.contiguous().float()
            dphi = torch.empty(E, B, device=dev)
            dT = torch.empty(E, 9, Kd, device=dev)
            g1 = gtab(1)
            call("face_transport_bwd", ptr(phi), phi.stride(0), B, *tab(1), Kd, ptr(Y), 20,
                 ptr(g.col), ptr(g.row_ptr), ptr(g.rev), N, g.max_row, 1.0, ptr(gD1), ptr(gD2), ptr(dphi), B, ptr(dT),
                 g1[0], g1[3], ptr(gY), st, label="transport_bwd")
        if not packed:
            return gtabs[0], gtabs[1], dphi, gY, None, None, None
        gP = gtabs[0]
        gVb = gP[:, :, :3].permute(2, 0, 1, 3).reshape(3, N, nt * Kd)
        gMb = gP[:, :, 3:].permute(2, 0, 1, 3).reshape(6, N, nt * Kd)
        return gVb, gMb, dphi, gY, None, None, None


class EqGate(torch.autograd.Function):
    """Gated equivariant outputs of a pass, V * gv and Ms * gm per (atom, channel), with the gate
    row gvm = [gv | gm] (N, 2C) (face/model.py:286-287, :295-296): one launch each way (the
    backward also gives the gate row's gradient)."""

    @staticmethod
    def forward(ctx, V, Ms, gvm):
        _lib.require_gpu(V, Ms, gvm)
        V, Ms, gvm = V.contiguous().float(), Ms.contiguous().float(), gvm.contiguous().float()
        N, C = gvm.shape[0], gvm.shape[1] // 2
        Vo, Mo = torch.empty_like(V), torch.empty_like(Ms)
        call("face_eq_gate_fwd", ptr(V), ptr(Ms), ptr(gvm), N, C, ptr(Vo), ptr(Mo), _lib.stream_of(V),
             label="eq_gate_fwd")
        ctx.save_for_backward(V, Ms, gvm)
        return Vo, Mo

    @staticmethod
    def backward(ctx, gVo, gMo):
        V, Ms, gvm = ctx.saved_tensors
        N, C = gvm.shape[0], gvm.shape[1] // 2
        gVo = torch.zeros_like(V) if gVo is None else gVo.contiguous().float()
        gMo = torch.zeros_like(Ms) if gMo is None else gMo.contiguous().float()
        dV, dMs, dgvm = torch.empty_like(V), torch.empty_like(Ms), torch.empty_like(gvm)
        call("face_eq_gate_bwd", ptr(V), ptr(Ms), ptr(gvm), ptr(gVo), ptr(gMo), N, C, ptr(dV), ptr(dMs), ptr(dgvm),
             _lib.stream_of(V), label="eq_gate_bwd")
        return dV, dMs, dgvm


def eq_gate(V, Ms, gvm):
    """V (3, N, C), Ms (6, N, C), gvm (N, 2C) -> (V * gv, Ms * gm)."""
    return EqGate.apply(V, Ms, gvm)


class LayerNorm(torch.autograd.Function):
    """nn.LayerNorm of the readout's invariant row with frozen weight and bias (face/model.py:140,
    :332): one wave per row each way; the input gradient only."""

    @staticmethod
    def forward(ctx, x, w, b, eps):
        _lib.require_gpu(x, w, b)
        x = x.contiguous().float()
        N, F_ = x.shape
        y = torch.empty_like(x)
        mean = torch.empty(N, device=x.device)
        rstd = torch.empty(N, device=x.device)
        call("face_layer_norm_fwd", ptr(x), N, F_, ptr(w), ptr(b), float(eps), ptr(y), ptr(mean), ptr(rstd),
             _lib.stream_of(x), label="ln_fwd")
        ctx.save_for_backward(x, w, mean, rstd)
        return y

    @staticmethod
    def backward(ctx, dy):
        if ctx.needs_input_grad[1] or ctx.needs_input_grad[2]:
            raise NotImplementedError("the readout LayerNorm gives no weight gradients (forces only)")
        x, w, mean, rstd = ctx.saved_tensors
        dy = dy.contiguous().float()
        dx = torch.empty_like(x)
        call("face_layer_norm_bwd", ptr(x), ptr(dy), x.shape[0], x.shape[1], ptr(w), ptr(mean), ptr(rstd), ptr(dx),
             _lib.stream_of(x), label="ln_bwd")
        return dx, None, None, None


def layer_norm(x, w, b, eps):
    """x (N, F) -> LayerNorm over F with frozen w, b (F % 4 == 0, F <= 2048)."""
    return LayerNorm.apply(x, w.contiguous(), b.contiguous(), eps)


class TableLinears(torch.autograd.Function):
    """The directional table linears of a pass, Vb = V pvt^T (3, N, n) and Mb = Ms pmt^T (6, N, n)
    (face/model.py:474-479), as one row-GEMM launch of two problems each way (input gradients
    only; the weights are constants of the evaluation)."""

    @staticmethod
    def forward(ctx, V, Ms, wv, wm):
        _lib.require_gpu(V, Ms, wv, wm)
        C = V.shape[-1]
        V_, Ms_ = V.contiguous().float(), Ms.contiguous().float()
        Vb = torch.empty(V.shape[0], V.shape[1], wv.shape[0], device=V.device)
        Mb = torch.empty(Ms.shape[0], Ms.shape[1], wm.shape[0], device=V.device)
        rows_linear([(V_.view(-1, C), wv, Vb.view(-1, wv.shape[0]), 0, 0.0),
                     (Ms_.view(-1, C), wm, Mb.view(-1, wm.shape[0]), 0, 0.0)], label="table_linear_fwd")
        ctx.wv, ctx.wm, ctx.shapes = wv, wm, (V.shape, Ms.shape)
        ctx.set_materialize_grads(False)
        return Vb, Mb

    @staticmethod
    def backward(ctx, gVb, gMb):
        wv, wm = ctx.wv, ctx.wm
        (sv, sm), dev = ctx.shapes, wv.device
        probs, dV, dMs = [], None, None
        if gVb is not None and ctx.needs_input_grad[0]:
            dV = torch.empty(sv, device=dev)
            probs.append((gVb.contiguous().float().view(-1, wv.shape[0]), wv, dV.view(-1, sv[-1]), 0, 0.0))
        if gMb is not None and ctx.needs_input_grad[1]:
            dMs = torch.empty(sm, device=dev)
            probs.append((gMb.contiguous().float().view(-1, wm.shape[0]), wm, dMs.view(-1, sm[-1]), 0, 0.0))
        if probs:
            rows_linear(probs, w_kn=True, label="table_linear_bwd")
        return dV, dMs, None, None


def table_linears(V, Ms, wv, wm):
    """(V wv^T, Ms wm^T) for (3|6, N, C) tables: one launch each way (C and the output width
    multiples of 16), else torch's linears."""
    if V.shape[-1] % 16 == 0 and wv.shape[0] % 16 == 0 and wm.shape[0] % 16 == 0:
        return TableLinears.apply(V, Ms, wv.contiguous(), wm.contiguous())
    return torch.nn.functional.linear(V, wv), torch.nn.functional.linear(Ms, wm)


def dir_transport(Vb, Mb, phi, Y, graph, Kd, transport):
    return DirTransport.apply(Vb, Mb, phi, Y, graph, Kd, transport)


class ReadoutMLP(torch.autograd.Function):
    """The readout after the LayerNorm on the library GEMMs (face/model.py:331-339, the gate of
    :286-287): z0 = [inv | h] W0^T + b0 (two accumulating GEMMs, no concatenated copy),
    o = W2 silu(W1 silu(z0) + b1) + b2, e = o[:, :1], h_new = h + o[:, 1:], gvm = inv Wg^T + bg.
    As one autograd node its backward accumulates where autograd would add: d inv takes the gate
    term in the second GEMM's epilogue, d h = gh + dz0 W0[:, 9C:10C] in one GEMM. last (the final
    pass, whose h_new nobody reads): only the energy row of the last layer is computed and its
    input gradient is the outer product ge W2[0]. W0a / W0b are the inv / h column blocks of W0.
    Weights receive no gradient; h's only when h takes one (the first pass's rows are constants)."""

    @staticmethod
    def forward(ctx, inv, h, W0a, W0b, b0, W1, b1, W2, b2, Wg, bg, last, hb):
        if hb is not None:                                # b0 + h W0b^T precomputed (h a constant)
            z0 = torch.addmm(hb, inv, W0a.t())
        else:
            z0 = torch.addmm(b0, inv, W0a.t())
            z0.addmm_(h, W0b.t())
        z1 = torch.addmm(b1, torch.nn.functional.silu(z0), W1.t())
        a1 = torch.nn.functional.silu(z1)
        if last:
            e = torch.addmm(b2[:1], a1, W2[:1].t())                               # (N, 1)
            h_new = None
        else:
            o = torch.addmm(b2, a1, W2.t())                                       # (N, 1 + C)
            e = o[:, :1]
            h_new = torch.add(h, o[:, 1:])
        gvm = torch.addmm(bg, inv, Wg.t()) if Wg is not None else None
        ctx.save_for_backward(z0, z1)
        ctx.w = (W0a, W0b, W1, W2, Wg)
        ctx.last = last
        return e, h_new, gvm

    @staticmethod
    def backward(ctx, ge, gh, ggvm):
        z0, z1 = ctx.saved_tensors
        W0a, W0b, W1, W2, Wg = ctx.w
        N = z0.shape[0]
        C = W0b.shape[1]
        if ge is None:
            ge = z0.new_zeros(N, 1)
        if ctx.last:
            da1 = ge * W2[:1]                                                     # (N, 2C)
        else:
            if gh is None:
                gh = z0.new_zeros(N, C)
            da1 = torch.cat([ge, gh], 1) @ W2
        da0 = torch.ops.aten.silu_backward(da1, z1) @ W1
        dz0 = torch.ops.aten.silu_backward(da0, z0)
        dinv = dz0 @ W0a
        if ggvm is not None and Wg is not None:
            dinv.addmm_(ggvm, Wg)
        dh = None
        if ctx.needs_input_grad[1]:                       # not for the first pass's constant rows
            dh = torch.addmm(gh, dz0, W0b) if (not ctx.last) else dz0 @ W0b
        return dinv, dh, None, None, None, None, None, None, None, None, None, None, None


def readout_mlp(inv, h, W0a, W0b, b0, W1, b1, W2, b2, Wg=None, bg=None, last=False, hb=None):
    """(e (N, 1), h_new (N, C) | None when last, gvm (N, 2C) | None); see ReadoutMLP. hb: b0 + h W0b^T
    when h is a constant of the evaluation (no gradient), computed once."""
    return ReadoutMLP.apply(inv, h, W0a, W0b, b0, W1, b1, W2, b2, Wg, bg, last, hb)


class AtomEnergy(torch.autograd.Function):
    """Atom energies e_at = e0 + scale * e_1 + scale * e_2 + ... (N,) and their per-structure sums
    E (nstr,) (face/model.py:680-690) in two launches (the atoms over the whole device, then one
    fixed-order sum per structure; atoms of a structure contiguous, ranges struct_ptr); the
    backward gives every pass the same gradient scale * (gE[structure] + g_at) in one launch.
    e_p may be strided (N, 1) column views."""

    @staticmethod
    def forward(ctx, e0, scale, struct_ptr, nstr, *es):
        _lib.require_gpu(e0, scale, *es)
        N = e0.shape[0]
        dev = e0.device
        e0_ = e0.contiguous().float()
        sc = scale.detach().float().contiguous().view(1)
        cols = [e if (e.dtype == torch.float32 and e.dim() == 2 and e.stride(1) == 1) else e.float().view(N, 1)
                for e in es]
        e_at = torch.empty(N, device=dev)
        E = torch.empty(nstr, device=dev)
        call("face_atom_energy_fwd", ptr(e0_), ptr(sc), _lib.ptr_array(cols), _lib.i64_array([c.stride(0) for c in cols]),
             len(cols), ptr(struct_ptr), nstr, ptr(e_at), ptr(E), _lib.stream_of(e0_), label="atom_energy")
        ctx.save_for_backward(struct_ptr, sc)
        ctx.n, ctx.N, ctx.nstr = len(es), N, nstr
        ctx.set_materialize_grads(False)                 # e_at is usually not differentiated
        return E, e_at

    @staticmethod
    def backward(ctx, gE, g_at):
        if gE is None and g_at is None:
            return (None,) * (4 + ctx.n)
        struct_ptr, sc = ctx.saved_tensors
        gE_ = gE.contiguous().float() if gE is not None else None
        ga_ = g_at.contiguous().float() if g_at is not None else None
        ge = torch.empty(ctx.N, 1, device=sc.device)
        call("face_atom_energy_bwd", ptr(gE_), ptr(ga_), ptr(sc), ptr(struct_ptr), ctx.nstr, ptr(ge),
             _lib.stream_of(sc), label="atom_energy_bwd")
        return (None, None, None, None) + (ge,) * ctx.n


def atom_energy(e0, scale, struct_ptr, nstr, es):
    """(E (nstr,), e_at (N,)); see AtomEnergy."""
    return AtomEnergy.apply(e0, scale, struct_ptr, nstr, *es)


class Readout(torch.autograd.Function):
    """The readout of a pass (face/model.py:331-339, with the gate row of an eq_out pass,
    face/model.py:286-287), forward and input gradients on the row GEMM:
        inv = LayerNorm(feats);  z1 = [inv | h] W0^T + b0;  z2 = silu(z1) W1^T + b1;
        o = silu(z2) W2^T + b2;  e = o[:, 0];  h_new = h + o[:, 1:];  gvm = inv Wg^T + bg.
    The SiLUs are applied to the GEMM inputs as they load and their derivatives likewise in the
    backward chain, [inv | h] and [dz1 | dgvm] are read as two column ranges without copies, and
    the residual h enters the last layer as its initial sum: W2p = W2 with the energy row moved
    last and zero rows to a multiple of 16 (n_pad), so one launch writes [h_new | e | 0] (N, n_pad).
    Four launches forward (LayerNorm and three GEMMs), five backward. Weights receive no
    gradient. Returns (e (N, 1), h_new (N, C), gvm (N, 2C) or an empty tensor)."""

    @staticmethod
    def forward(ctx, feats, h, ln_w, ln_b, eps, w0, b0, w1, b1, w2p, b2p, wg, bg, wstack):
        _lib.require_gpu(feats, h)
        dev = feats.device
        N, nf = feats.shape
        C = h.shape[1]
        H1, H2, n_pad = w0.shape[0], w1.shape[0], w2p.shape[0]
        feats = feats.contiguous().float()
        inv = torch.empty_like(feats)
        mean = torch.empty(N, device=dev)
        rstd = torch.empty(N, device=dev)
        st = _lib.stream_of(feats)
        call("face_layer_norm_fwd", ptr(feats), N, nf, ptr(ln_w), ptr(ln_b), float(eps), ptr(inv), ptr(mean),
             ptr(rstd), st, label="ln_fwd")
        z1 = torch.empty(N, H1, device=dev)
        probs = [lin(inv, w0, z1, x2=h, bias=b0)]
        gvm = torch.empty(0, device=dev)
        if wg is not None:
            gvm = torch.empty(N, wg.shape[0], device=dev)
            probs.append(lin(inv, wg, gvm, bias=bg))
        rows_linear(probs, label="readout_in")
        z2 = torch.empty(N, H2, device=dev)
        rows_linear([lin(z1, w1, z2, x_op=1, bias=b1)], label="readout_hid")
        out = torch.empty(N, n_pad, device=dev)
        rows_linear([lin(z2, w2p, out, x_op=1, bias=b2p, beta=1.0, y0=h, n_y0=C)], label="readout_out")
        ctx.save_for_backward(feats, ln_w, mean, rstd, z1, z2)
        ctx.w = (w0, w1, w2p, wstack)
        ctx.dims = (N, nf, C, n_pad, wg is not None)
        return out[:, C:C + 1], out[:, :C], gvm

    @staticmethod
    def backward(ctx, ge, gh, dgvm):
        feats, ln_w, mean, rstd, z1, z2 = ctx.saved_tensors
        w0, w1, w2p, wstack = ctx.w
        N, nf, C, n_pad, gate = ctx.dims
        dev = feats.device
        gh = gh if gh is not None else feats.new_zeros(N, C)
        ge = ge if ge is not None else feats.new_zeros(N, 1)
        do = torch.cat([gh, ge, feats.new_zeros(N, n_pad - C - 1)], 1)          # (N, n_pad): [gh | ge | 0]
        gh = do[:, :C]
        da2 = torch.empty(N, w1.shape[0], device=dev)
        rows_linear([lin(do, w2p, da2)], w_kn=True, label="readout_out_bwd")
        da1 = torch.empty(N, w0.shape[0], device=dev)
        rows_linear([lin(da2, w1, da1, x_op=2, xz=z2)], w_kn=True, label="readout_hid_bwd")
        dinv = torch.empty(N, nf, device=dev)
        dh = torch.empty(N, C, device=dev)
        use_gate = gate and dgvm is not None and dgvm.numel() > 0
        pa = lin(da1, wstack if use_gate else w0[:, :nf], dinv, x_op=2, xz=z1,
                 x2=dgvm.contiguous() if use_gate else None)
        pb = lin(da1, w0[:, nf:nf + C], dh, x_op=2, xz=z1, beta=1.0, y0=gh)
        rows_linear([pa, pb], w_kn=True, label="readout_in_bwd")
        dfeats = torch.empty_like(feats)
        call("face_layer_norm_bwd", ptr(feats), ptr(dinv), N, nf, ptr(ln_w), ptr(mean), ptr(rstd), ptr(dfeats),
             _lib.stream_of(feats), label="ln_bwd")
        return dfeats, dh, None, None, None, None, None, None, None, None, None, None, None, None


def readout(feats, h, ln_w, ln_b, eps, w0, b0, w1, b1, w2p, b2p, wg=None, bg=None, wstack=None):
    """(e (N, 1), h_new (N, C), gvm (N, 2C) | empty); see Readout."""
    return Readout.apply(feats, h, ln_w, ln_b, eps, w0, b0, w1, b1, w2p, b2p, wg, bg, wstack)


# ----------------------------------------------------------------------------- densities
RANK_K = (1, 3, 6, 10)


def _ranks_xmajor(t):
    """Rank descriptor of one (NX, N, W) monomial-major tensor."""
    NX, N, W = t.shape
    base = t.data_ptr()
    nr = 4 if NX == 20 else 2
    ptrs = [base + 4 * _lib.RANK_X0[l] * N * W if l < nr else None for l in range(4)]
    return (_lib.P * 4)(*ptrs), W, N * W


class Density(torch.autograd.Function):
    """Factor density sum over row i of phi (x) msg (x) Y[:, :nx]  (face/kernels.py:170-178).

    nx = 20: returns the four rank blocks D_l (k_l, N, B*K) (monomial-major), each a separate
    tensor so the channel-mixing GEMMs read them in place and their gradients arrive without
    slice/concat copies. nx = 4: returns one (4, N, B*K) tensor.
    msg is per edge (E, K) when gathered is False, else a node table (N, K) read through col
    (its gradient is then reduced back to the table through the reverse-edge map).
    """

    @staticmethod
    def forward(ctx, phi, msg, Y, graph, nx, gathered):
        _lib.require_gpu(phi, msg, Y)
        B, K = phi.shape[1], msg.shape[1]
        phi_, ld_phi = _rows(phi, B)
        msg_, ld_msg = _rows(msg, K)
        Y_, ld_Y = _rows(Y, nx)
        N = graph.N
        if nx == 20:
            outs = [torch.empty(k, N, B * K, device=phi.device) for k in RANK_K]
            desc = _lib.ranks_of_blocks(outs)
        else:
            outs = [torch.empty(nx, N, B * K, device=phi.device)]
            desc = _ranks_xmajor(outs[0])
        row = graph.col if gathered else None
        call("face_density_fwd", ptr(phi_), ld_phi, ptr(msg_), ld_msg, ptr(row), ptr(Y_), ld_Y, nx, ptr(graph.row_ptr),
             N, 0, B, K, *desc, _lib.stream_of(phi), label=f"density_fwd{nx}")
        ctx.save_for_backward(phi_, msg_, Y_)
        ctx.graph, ctx.nx, ctx.gathered, ctx.BK = graph, nx, gathered, (B, K)
        ctx.ywidth = Y.shape[1]
        return tuple(outs) if nx == 20 else outs[0]

    @staticmethod
    def backward(ctx, *grads):
        phi, msg, Y = ctx.saved_tensors
        g, nx, (B, K) = ctx.graph, ctx.nx, ctx.BK
        dev = phi.device
        if nx == 20:
            Gs = [(t.contiguous().float() if t is not None else torch.zeros(k, g.N, B * K, device=dev))
                  for t, k in zip(grads, RANK_K)]
            desc = _lib.ranks_of_blocks(Gs)
        else:
            Gs = [grads[0].contiguous().float()]
            desc = _ranks_xmajor(Gs[0])
        need_phi, need_msg, need_Y = ctx.needs_input_grad[:3]
        dphi = torch.empty(g.E, B, device=dev) if need_phi else None
        dmsg = torch.empty(g.E, K, device=dev) if need_msg else None
        dY = torch.empty(g.E, nx, device=dev) if need_Y else None
        row = g.col if ctx.gathered else None
        st = _lib.stream_of(phi)
        call("face_density_bwd", ptr(phi), phi.stride(0), ptr(msg), msg.stride(0), ptr(row), ptr(Y), Y.stride(0), nx,
             ptr(g.row_ptr), g.N, 0, g.max_row, B, K, *desc, ptr(dphi), B, ptr(dmsg), K, ptr(dY), nx, st,
             label=f"density_bwd{nx}")
        if dmsg is not None and ctx.gathered:
            dtab = torch.empty(g.N, K, device=dev)
            call("face_gather_rows_bwd", ptr(dmsg), K, ptr(g.row_ptr), ptr(g.rev), g.N, K, ptr(dtab), K, st,
                 label="gather_bwd")
            dmsg = dtab
        if dY is not None and ctx.ywidth != nx:
            dY = torch.nn.functional.pad(dY, (0, ctx.ywidth - nx))
        return dphi, dmsg, dY, None, None, None


def density(phi, msg, Y, graph, nx=20, gathered=False):
    return Density.apply(phi, msg, Y, graph, nx, gathered)


class DensityMix(torch.autograd.Function):
    """Factor density fused with the per-rank mix and the element scale (face/kernels.py:170-178,
    face/model.py:503-506, the scale of :530-533): A_l = (Af_l W_l^T [+ D_l T_l^T]) * s[z] with
    Af = the factor density of phi, msg, Y, in one launch each way (the density D never leaves the
    chip). The transport mix (D1, D2 with weights wt) is a separate GEMM written first and
    accumulated in the fused epilogue. wm: 4 mix weights (C, B K); wmt: their transposes (B K, C),
    contiguous. Weights receive no gradient."""

    @staticmethod
    def forward(ctx, s_tab, group, wm, wmt, wt, D1, D2, phi, msg, Y, graph, gathered):
        _lib.require_gpu(phi, msg, Y)
        B, K = phi.shape[1], msg.shape[1]
        C = wm[0].shape[0]
        N = graph.N
        # dense rows (16-byte aligned row strides for the backward's vector loads; a no-op in the model)
        phi_, msg_, Y_ = phi.float().contiguous(), msg.float().contiguous(), Y.float().contiguous()
        ld_phi, ld_msg, ld_Y = B, K, Y_.shape[1]
        dev = phi.device
        outs = [torch.empty(k, N, C, device=dev) for k in RANK_K]
        beta = 0
        for l, D in ((1, D1), (2, D2)):
            if D is not None:
                torch.mm(D.reshape(-1, D.shape[-1]), wt[l - 1].t(), out=outs[l].view(-1, C))
                beta |= 1 << l
        row = graph.col if gathered else None
        call("face_density_mix_fwd", ptr(phi_), ld_phi, ptr(msg_), ld_msg, ptr(row), ptr(Y_), ld_Y,
             ptr(graph.row_ptr), N, B, K, C, _lib.ptr_array(wm), wm[0].stride(0), _lib.ptr_array(outs), C, N * C,
             ptr(s_tab), s_tab.stride(0), ptr(group), beta, _lib.stream_of(phi), label="density_mix_fwd")
        ctx.save_for_backward(s_tab, group, phi_, msg_, Y_)
        ctx.graph, ctx.gathered, ctx.wmt, ctx.wt = graph, gathered, wmt, wt
        ctx.has_D = (D1 is not None, D2 is not None)
        ctx.ywidth = Y.shape[1]
        return tuple(outs)

    @staticmethod
    def backward(ctx, *gA):
        s_tab, group, phi, msg, Y = ctx.saved_tensors
        g = ctx.graph
        N, B, K = g.N, phi.shape[1], msg.shape[1]
        C = ctx.wmt[0].shape[1]
        dev = phi.device
        gA = [(t.contiguous() if t is not None else torch.zeros(k, N, C, device=dev)) for t, k in zip(gA, RANK_K)]
        need_D1, need_D2, need_phi, need_msg, need_Y = ctx.needs_input_grad[5:10]
        dphi = torch.empty(g.E, B, device=dev) if need_phi else None
        dmsg = torch.empty(g.E, K, device=dev) if need_msg else None
        dY = torch.empty(g.E, 20, device=dev) if need_Y else None
        st = _lib.stream_of(phi)
        row = g.col if ctx.gathered else None
        call("face_density_mix_bwd", ptr(phi), phi.stride(0), ptr(msg), msg.stride(0), ptr(row), ptr(Y), Y.stride(0),
             ptr(g.row_ptr), N, B, K, C, _lib.ptr_array(ctx.wmt), ctx.wmt[0].stride(0), _lib.ptr_array(gA), C, N * C,
             ptr(s_tab), s_tab.stride(0), ptr(group), ptr(dphi), B, ptr(dmsg), K, ptr(dY), 20, st,
             label="density_mix_bwd")
        if dmsg is not None and ctx.gathered:
            dtab = torch.empty(N, K, device=dev)
            call("face_gather_rows_bwd", ptr(dmsg), K, ptr(g.row_ptr), ptr(g.rev), N, K, ptr(dtab), K, st,
                 label="gather_bwd")
            dmsg = dtab
        if dY is not None and ctx.ywidth != 20:
            dY = torch.nn.functional.pad(dY, (0, ctx.ywidth - 20))
        # transport mix: dD_l = (gA_l * s_l) wt, the scale applied to the rows as they load
        dD = [None, None]
        tp = []
        for i, (l, need) in enumerate(((1, need_D1), (2, need_D2))):
            if ctx.has_D[i] and need:
                w = ctx.wt[i]
                dD[i] = torch.empty(gA[l].shape[0], N, w.shape[1], device=dev)
                tp.append((gA[l].view(-1, C), w, dD[i].view(-1, w.shape[1]), l * C, 0.0))
        if tp:
            rows_linear(tp, w_kn=True, xs=s_tab, group=group, period=N, label="tmix_bwd")
        return (None, None, None, None, None, dD[0], dD[1], dphi, dmsg, dY, None, None)


def density_mix(s_tab, group, wm, wmt, wt, D1, D2, phi, msg, Y, graph, gathered=False):
    """4 x (k_l, N, C) moments of a factorised pass from the fused density + mix kernels."""
    return DensityMix.apply(s_tab, group, wm, wmt, wt, D1, D2, phi, msg, Y, graph, gathered)


def density_mix_fits(B, K, C, N, nx=20):
    """Whether the model takes the fused density + mix route for this shape: the kernels serve
    B = 16, K <= 64 and C <= 256 (multiples of 16), and the route is taken for systems of at most
    DENSITY_MIX_MAX_ATOMS atoms. Measured on the flagship workloads (864-atom FCC, 1,344-atom
    molecule batch) the fused kernels are slower than the density kernel + row GEMM pair they
    replace (fwd 65 / 114 us against 54 / 74 us, bwd 121 / 227 us against 80 / 95 us): every
    4-atom workgroup streams all four mix weights from L2 and pads its rank blocks to 16 rows
    (71 % useful), and these launches are latency-bound single rounds. The default therefore
    keeps D in memory (DENSITY_MIX_MAX_ATOMS = 0); set it to use the fused route."""
    return (nx == 20 and B == 16 and K % 16 == 0 and K <= 64 and C % 16 == 0 and C <= 256
            and N <= DENSITY_MIX_MAX_ATOMS)


DENSITY_MIX_MAX_ATOMS = int(os.environ.get("FACE_DENSITY_MIX_MAX_ATOMS", "0"))


def _cp_label(base, gathered):
    """Timing label of a CP pooling launch: "_tab" when the messages are node-table rows gathered
    through col (N x C read) rather than per-edge rows (E x C)."""
    return base + ("_tab" if gathered else "")


class CPDensity(torch.autograd.Function):
    """CP pooling A_l (k_l, N, C) = sum over row i of env R[:, l, c] msg[:, c] Y[:, x in l]
    (face/model.py:496-502, envelope of face/model.py:469 folded in); four rank blocks."""

    @staticmethod
    def forward(ctx, R, env, msg, Y, graph, gathered):
        _lib.require_gpu(R, env, msg, Y)
        C = msg.shape[1]
        R_, ld_R = _rows(R, 4 * C)
        env_ = env.contiguous().float()
        msg_, ld_msg = _rows(msg, C)
        Y_, ld_Y = _rows(Y, 20)
        outs = [torch.empty(k, graph.N, C, device=R.device) for k in RANK_K]
        row = graph.col if gathered else None
        call("face_cp_density_fwd", ptr(R_), ld_R, ptr(env_), ptr(msg_), ld_msg, ptr(row), ptr(Y_), ld_Y,
             ptr(graph.row_ptr), graph.N, 0, C, *_lib.ranks_of_blocks(outs), _lib.stream_of(R),
             label=_cp_label("cp_fwd", gathered))
        ctx.save_for_backward(R_, env_, msg_, Y_)
        ctx.graph, ctx.gathered, ctx.C = graph, gathered, C
        return tuple(outs)

    @staticmethod
    def backward(ctx, *grads):
        R, env, msg, Y = ctx.saved_tensors
        g, C = ctx.graph, ctx.C
        dev = R.device
        Gs = [(t.contiguous().float() if t is not None else torch.zeros(k, g.N, C, device=dev))
              for t, k in zip(grads, RANK_K)]
        need_R, need_env, need_msg, need_Y = ctx.needs_input_grad[:4]
        dR = torch.empty(g.E, 4 * C, device=dev) if need_R else None
        denv = torch.empty(g.E, device=dev) if need_env else None
        dmsg = torch.empty(g.E, C, device=dev) if need_msg else None
        dY = torch.empty(g.E, 20, device=dev) if need_Y else None
        row = g.col if ctx.gathered else None
        st = _lib.stream_of(R)
        call("face_cp_density_bwd", ptr(R), R.stride(0), ptr(env), ptr(msg), msg.stride(0), ptr(row), ptr(Y),
             Y.stride(0), ptr(g.row_ptr), g.N, 0, g.max_row, C, *_lib.ranks_of_blocks(Gs), ptr(dR), 4 * C, ptr(dmsg),
             C, ptr(dY), 20, ptr(denv), st, label=_cp_label("cp_bwd", ctx.gathered))
        if dmsg is not None and ctx.gathered:
            dtab = torch.empty(g.N, C, device=dev)
            call("face_gather_rows_bwd", ptr(dmsg), C, ptr(g.row_ptr), ptr(g.rev), g.N, C, ptr(dtab), C, st,
                 label="gather_bwd")
            dmsg = dtab
        return dR, denv, dmsg, dY, None, None


def cp_density(R, env, msg, Y, graph, gathered=False):
    return CPDensity.apply(R, env, msg, Y, graph, gathered)


class CPRadialDensity(torch.autograd.Function):
    """CP pooling fed by the CP columns of the last radial layer: R = h2 W_cp^T + b_cp (E, 4C), then
    A_l as in CPDensity (face/model.py:469-472, 496-502). With per-edge messages the forward computes
    R on the matrix cores and pools it in the same launch (R is written once, for the backward, and
    not read back: 1.85 ms against 2.03 ms for the two launches at 24,000 atoms, C = 160; 0.345
    against 0.385 ms at 512 molecules); with node-table messages gathered through col, and for
    shapes that launch cannot serve, R comes from the radial head and is pooled in a second launch
    (1.89 ms against 2.03 ms fused there). The
    backward multiplies the pooling's dR by W_cp on the matrix cores inside the pooling kernel and
    returns d h2 (E, H) without writing dR. W_cp / b_cp receive no gradient (forces only)."""

    @staticmethod
    def forward(ctx, h2, w_cp, b_cp, env, msg, Y, graph, gathered):
        _lib.require_gpu(h2, env, msg, Y)
        C = msg.shape[1]
        env_ = env.contiguous().float()
        msg_, ld_msg = _rows(msg, C)
        Y_, ld_Y = _rows(Y, 20)
        outs = [torch.empty(k, graph.N, C, device=h2.device) for k in RANK_K]
        row = graph.col if gathered else None
        h2_, w_, b_ = _aligned_rows(h2.detach()), _aligned16(w_cp.detach()), _aligned16(b_cp.detach())
        H = h2_.shape[1]
        code = _lib.FACE_ERR_UNSUPPORTED
        if not gathered:
            R = torch.empty(graph.E, 4 * C, device=h2.device)
            code = _lib.call_status("face_cp_radial_fwd", ptr(h2_), h2_.stride(0), H, ptr(w_), ptr(b_), ptr(env_),
                                    ptr(msg_), ld_msg, None, ptr(Y_), ld_Y, ptr(graph.row_ptr), graph.N, graph.E, C,
                                    *_lib.ranks_of_blocks(outs), ptr(R), 4 * C, _lib.stream_of(R),
                                    label="cp_radial_fwd")
        if code == _lib.FACE_ERR_UNSUPPORTED:
            R = radial_head(h2_, w_, b_)                                                          # (E, 4C)
            call("face_cp_density_fwd", ptr(R), R.stride(0), ptr(env_), ptr(msg_), ld_msg, ptr(row), ptr(Y_), ld_Y,
                 ptr(graph.row_ptr), graph.N, 0, C, *_lib.ranks_of_blocks(outs), _lib.stream_of(R),
                 label=_cp_label("cp_fwd", gathered))
        ctx.save_for_backward(R, w_cp.detach(), env_, msg_, Y_)
        ctx.graph, ctx.gathered, ctx.C = graph, gathered, C
        return tuple(outs)

    @staticmethod
    def backward(ctx, *grads):
        if ctx.needs_input_grad[1] or ctx.needs_input_grad[2]:
            raise NotImplementedError("the fused CP radial backward gives no weight gradients (forces only)")
        R, w_cp, env, msg, Y = ctx.saved_tensors
        g, C = ctx.graph, ctx.C
        dev = R.device
        H = w_cp.shape[1]
        Gs = [(t.contiguous().float() if t is not None else torch.zeros(k, g.N, C, device=dev))
              for t, k in zip(grads, RANK_K)]
        need_h2, need_env, need_msg, need_Y = (ctx.needs_input_grad[0], ctx.needs_input_grad[3],
                                               ctx.needs_input_grad[4], ctx.needs_input_grad[5])
        w_t = w_cp.t().contiguous()                                                          # (H, 4C)
        dh2 = torch.empty(g.E, H, device=dev)
        denv = torch.empty(g.E, device=dev) if need_env else None
        dmsg = torch.empty(g.E, C, device=dev) if need_msg else None
        dY = torch.empty(g.E, 20, device=dev) if need_Y else None
        row = g.col if ctx.gathered else None
        st = _lib.stream_of(R)
        code = _lib.call_status("face_cp_radial_bwd", ptr(R), R.stride(0), ptr(env), ptr(msg), msg.stride(0), ptr(row),
                                ptr(Y), Y.stride(0), ptr(g.row_ptr), g.N, 0, C, *_lib.ranks_of_blocks(Gs), ptr(w_t), H,
                                ptr(dh2), H, ptr(dmsg), C, ptr(dY), 20, ptr(denv), st,
                                label=_cp_label("cp_radial_bwd", ctx.gathered))
        if code == _lib.FACE_ERR_UNSUPPORTED:
            # widths whose staging exceeds the fused kernel's LDS: the pooling backward writes dR
            # and d h2 = dR W_cp is a separate GEMM
            dR = torch.empty(g.E, 4 * C, device=dev)
            call("face_cp_density_bwd", ptr(R), R.stride(0), ptr(env), ptr(msg), msg.stride(0), ptr(row), ptr(Y),
                 Y.stride(0), ptr(g.row_ptr), g.N, 0, g.max_row, C, *_lib.ranks_of_blocks(Gs), ptr(dR), 4 * C,
                 ptr(dmsg), C, ptr(dY), 20, ptr(denv), st, label=_cp_label("cp_bwd", ctx.gathered))
            torch.mm(dR, w_cp, out=dh2)
        if dmsg is not None and ctx.gathered:
            dtab = torch.empty(g.N, C, device=dev)
            call("face_gather_rows_bwd", ptr(dmsg), C, ptr(g.row_ptr), ptr(g.rev), g.N, C, ptr(dtab), C, st,
                 label="gather_bwd")
            dmsg = dtab
        return (dh2 if need_h2 else None), None, None, denv, dmsg, dY, None, None


def cp_radial_density(h2, w_cp, b_cp, env, msg, Y, graph, gathered=False):
    return CPRadialDensity.apply(h2, w_cp, b_cp, env, msg, Y, graph, gathered)


def _aligned16(t):
    t = t.contiguous().float()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _aligned_rows(x):
    """x itself when its rows are unit-stride, 16-byte aligned float rows; else an aligned copy."""
    ok = x.dtype == torch.float32 and x.stride(1) == 1 and x.stride(0) % 4 == 0 and x.data_ptr() % 16 == 0
    return x if ok else _aligned16(x)


def edge_linear(x, w, b=None, tab=None, idx=None, label="edge_linear"):
    """y (E, F) = x w^T + b + tab[idx] on the matrix cores, no gradient (x (E, K), w (F, K),
    K in {16, 32, 48, 64}, F a multiple of 16)."""
    _lib.require_gpu(x, w)
    E, K = x.shape
    F_ = w.shape[0]
    x_ = x if (x.stride(1) == 1 and x.stride(0) % 4 == 0 and x.data_ptr() % 16 == 0) else _aligned16(x)
    w_ = _aligned16(w)
    b_ = None if b is None else _aligned16(b)
    tab_ = None if tab is None else _aligned16(tab)
    y = torch.empty(E, F_, device=x.device)
    call("face_edge_linear_fwd", ptr(x_), x_.stride(0), E, K, ptr(w_), ptr(b_), F_, ptr(tab_),
         0 if tab_ is None else tab_.stride(0), ptr(idx), ptr(y), F_, _lib.stream_of(y), label=label)
    return y


def radial_head(h2, w, b):
    """R (E, F) = h2 w^T + b for the CP columns of the last radial layer (no gradient)."""
    return edge_linear(h2, w, b, label="radial_head")


class EdgeMessage(torch.autograd.Function):
    """Per-edge message of a directional pass, m[e] = msg_n[col e] + d[e] W_d^T + b_d
    (face/model.py:488-493: gather(msg(h)) + dir_mix(d)), in one launch; the backward gives
    d msg_n (reduction over each atom's reverse edges, no atomics) and d d = dm W_d in one launch.
    W_d / b_d receive no gradient (forces only)."""

    @staticmethod
    def forward(ctx, msg_n, d, w, b, graph):
        _lib.require_gpu(msg_n, d)
        y = edge_linear(d.detach(), w.detach(), b.detach(), msg_n.detach(), graph.col, label="edge_msg_fwd")
        ctx.save_for_backward(_aligned16(w.detach()))
        ctx.graph, ctx.K = graph, d.shape[1]
        return y

    @staticmethod
    def backward(ctx, gy):
        if ctx.needs_input_grad[2] or ctx.needs_input_grad[3]:
            raise NotImplementedError("the fused edge message gives no weight gradients (forces only)")
        (w,) = ctx.saved_tensors
        g = ctx.graph
        gy = _aligned16(gy)
        F_ = gy.shape[1]
        dtab = torch.empty(g.N, F_, device=gy.device) if ctx.needs_input_grad[0] else None
        dd = torch.empty(g.E, ctx.K, device=gy.device) if ctx.needs_input_grad[1] else None
        call("face_edge_linear_bwd", ptr(gy), gy.stride(0), F_, ptr(w), ctx.K, ptr(g.row_ptr), ptr(g.rev), g.N,
             ptr(dd), ctx.K, ptr(dtab), F_, _lib.stream_of(gy), label="edge_msg_bwd")
        return dtab, dd, None, None, None


def edge_message(msg_n, d, w, b, graph):
    return EdgeMessage.apply(msg_n, d, w, b, graph)


# ----------------------------------------------------------------------------- radial MLP
class RadialMLP(torch.autograd.Function):
    """phi (E, B) = (silu(silu(rb W_in^T + b_in + pair_tab[pair]) W1^T + b1) W_phi^T + b_phi) * env and,
    when want_h2, the last hidden activation h2 (E, H) (face/model.py:465-469). Gradients flow to rb and
    env only: the fused radial kernel serves forces, not training."""

    @staticmethod
    def forward(ctx, rb, env, pair, w_in, b_in, pair_tab, w1, b1, w_phi, b_phi, want_h2):
        _lib.require_gpu(rb, env)
        E, nb = rb.shape
        H, B = w1.shape[0], w_phi.shape[0]
        rb_, ld_rb = _rows(rb, nb)
        env_ = env.contiguous().float()
        ws = [t.detach().contiguous().float() for t in (w_in, b_in, pair_tab, w1, b1, w_phi, b_phi)]
        h2 = torch.empty(E, H, device=rb.device) if want_h2 else torch.empty(0, H, device=rb.device)
        phi = torch.empty(E, B, device=rb.device)
        call("face_radial_fwd", ptr(rb_), ld_rb, nb, ptr(pair), ptr(env_), E, ptr(ws[0]), ptr(ws[1]), ptr(ws[2]),
             ws[2].shape[0], H, ptr(ws[3]), ptr(ws[4]), ptr(ws[5]), ptr(ws[6]), B, ptr(h2) if want_h2 else None, H,
             ptr(phi), B, _lib.stream_of(rb), label="radial_fwd")
        ctx.save_for_backward(rb_, env_, pair, *ws)
        ctx.dims = (E, nb, H, B)
        ctx.set_materialize_grads(False)
        return phi, phi.view(phi.shape), h2

    @staticmethod
    def backward(ctx, gphi, gphi2, gh2):
        if any(ctx.needs_input_grad[2:]):
            raise NotImplementedError("the fused radial MLP gives no weight gradients (forces only)")
        rb, env, pair, *ws = ctx.saved_tensors
        E, nb, H, B = ctx.dims
        dev = rb.device
        gp = [t.contiguous().float() for t in (gphi, gphi2) if t is not None]
        if not gp:
            gp = [torch.zeros(E, B, device=dev)]
        gh2 = gh2.contiguous().float() if (gh2 is not None and gh2.numel()) else None
        grb = torch.empty(E, nb, device=dev) if ctx.needs_input_grad[0] else None
        genv = torch.empty(E, device=dev) if ctx.needs_input_grad[1] else None
        call("face_radial_bwd", ptr(rb), rb.stride(0), nb, ptr(pair), ptr(env), E, ptr(ws[0]), ptr(ws[1]), ptr(ws[2]),
             ws[2].shape[0], H, ptr(ws[3]), ptr(ws[4]), ptr(ws[5]), ptr(ws[6]), B, ptr(gh2), H, ptr(gp[0]),
             ptr(gp[1]) if len(gp) > 1 else None, B, ptr(grb), nb, ptr(genv), _lib.stream_of(rb), label="radial_bwd")
        return grb, genv, None, None, None, None, None, None, None, None, None


class RadialMLPSets(torch.autograd.Function):
    """The radial MLPs of several passes over the same edges (face/model.py:465-469 per pass) in one
    launch each way: the passes' radial functions depend only on the edge basis, so they are
    evaluated together (twice the waves of one pass per launch) and differentiated together once
    every pass's gradients have arrived. rb_env: one rb view and one envelope view per pass (views
    of the same tensors, so that each reader's gradient comes back on its own)."""

    @staticmethod
    def forward(ctx, pair, wsets, want_h2, *rb_env):
        n = len(wsets)
        rbs, envs = rb_env[:n], rb_env[n:]
        _lib.require_gpu(*rb_env)
        rb, env = rbs[0], envs[0]
        if any(t.data_ptr() != rb.data_ptr() or t.stride() != rb.stride() for t in rbs) or \
                any(t.data_ptr() != env.data_ptr() for t in envs):
            raise ValueError("radial_mlp_sets: the rb (and envelope) views must be views of one tensor")
        E, nb = rb.shape
        rb_, ld_rb = _rows(rb, nb)
        env_ = env.contiguous().float()
        ws = [t.detach().contiguous().float() for w in wsets for t in w]
        H, B, n_pair = ws[3].shape[0], ws[5].shape[0], ws[2].shape[0]
        dev = rb.device
        h2 = [torch.empty(E, H, device=dev) if want_h2 else torch.empty(0, H, device=dev) for _ in range(n)]
        phi = [torch.empty(E, B, device=dev) for _ in range(n)]
        call("face_radial_fwd_sets", ptr(rb_), ld_rb, nb, ptr(pair), ptr(env_), E, n, _lib.ptr_array(ws), n_pair, H, B,
             _lib.ptr_array(h2) if want_h2 else None, H, _lib.ptr_array(phi), B, _lib.stream_of(rb_),
             label=f"radial_fwd*{n}")
        ctx.save_for_backward(rb_, env_, pair, *ws)
        ctx.dims = (E, nb, H, B, n_pair, n)
        ctx.set_materialize_grads(False)
        out = []
        for k in range(n):
            out += [phi[k], phi[k].view(phi[k].shape), h2[k]]
        return tuple(out)

    @staticmethod
    def backward(ctx, *grads):
        rb, env, pair, *ws = ctx.saved_tensors
        E, nb, H, B, n_pair, n = ctx.dims
        dev = rb.device
        gphi, gphi2, gh2 = [], [], []
        for k in range(n):
            g1, g2, gh = grads[3 * k:3 * k + 3]
            g1 = g1.contiguous().float() if g1 is not None else None
            g2 = g2.contiguous().float() if g2 is not None else None
            if g1 is None:
                g1, g2 = (g2, None) if g2 is not None else (torch.zeros(E, B, device=dev), None)
            gphi.append(g1)
            gphi2.append(g2)
            gh2.append(gh.contiguous().float() if (gh is not None and gh.numel()) else None)
        need_rb = ctx.needs_input_grad[3:3 + n]
        need_env = ctx.needs_input_grad[3 + n:3 + 2 * n]
        grb = [torch.empty(E, nb, device=dev) if need_rb[k] else None for k in range(n)]
        genv = [torch.empty(E, device=dev) if need_env[k] else None for k in range(n)]
        call("face_radial_bwd_sets", ptr(rb), rb.stride(0), nb, ptr(pair), ptr(env), E, n, _lib.ptr_array(ws), n_pair,
             H, B, _lib.ptr_array(gh2), H, _lib.ptr_array(gphi), _lib.ptr_array(gphi2), B, _lib.ptr_array(grb), nb,
             _lib.ptr_array(genv), _lib.stream_of(rb), label=f"radial_bwd*{n}")
        return (None, None, None, *grb, *genv)


def radial_mlp_sets(pair, wsets, want_h2, rbs, envs):
    """Per pass (phi, phi again as a view for a second reader, h2) of the radial MLPs of several
    passes in one launch each way; wsets: per pass (w_in, b_in, pair_tab, w1, b1, w_phi, b_phi)."""
    out = RadialMLPSets.apply(pair, wsets, want_h2, *rbs, *envs)
    return [tuple(out[3 * k:3 * k + 3]) for k in range(len(wsets))]


def radial_mlp(rb, env, pair, w_in, b_in, pair_tab, w1, b1, w_phi, b_phi, want_h2):
    """(phi, phi again as a view for a second reader (its gradient is summed in the backward
    kernel), h2)."""
    return RadialMLP.apply(rb, env, pair, w_in, b_in, pair_tab, w1, b1, w_phi, b_phi, want_h2)


class RadialSpline(torch.autograd.Function):
    """Compiled radial functions (face/model.py:407-418, :466-467): cubic Hermite interpolation of
    the tables T, dT (P, G, F) at r (E) for element pair `pair` (E); returns phi (E, nb) = the
    first nb columns times env, and R (E, F - nb) = the other columns as they are (the CP radials,
    enveloped inside the pooling kernels). Gradients flow to r and env (the tables are constants
    of the compiled model). Tables far larger than L2 (the CP columns) are read in table-cell
    order (spline_order)."""

    @staticmethod
    def forward(ctx, r, env, pair, T, dT, dr, nb, order):
        _lib.require_gpu(r, env, pair, T, dT)
        if pair.dtype != torch.int32 or T.dtype != torch.float32 or dT.dtype != torch.float32:
            raise TypeError("radial_spline: pair must be int32 and the tables float32")
        P, G, F = T.shape
        E = r.shape[0]
        r_, env_ = r.contiguous().float(), env.contiguous().float()
        phi = torch.empty(E, nb, device=r.device)
        R = torch.empty(E, F - nb, device=r.device)
        st = _lib.stream_of(r)
        if order is None and spline_wants_order(T):
            order = spline_order(r_, pair, P, G, dr)
        call("face_radial_spline_fwd", ptr(r_), ptr(pair), E, ptr(T), ptr(dT), P, G, F, float(dr), ptr(env_), nb,
             ptr(order), ptr(phi), nb, ptr(R), F - nb, st, label="spline_fwd")
        ctx.save_for_backward(r_, env_, pair, T, dT, order)
        ctx.dr, ctx.nb = dr, nb
        return phi, R

    @staticmethod
    def backward(ctx, gphi, gR):
        r, env, pair, T, dT, order = ctx.saved_tensors
        P, G, F = T.shape
        E, nb = r.shape[0], ctx.nb
        gp, ldp = _rows(gphi, nb) if (gphi is not None and nb > 0) else (None, nb)
        gq, ldq = _rows(gR, F - nb) if (gR is not None and F > nb) else (None, F - nb)
        gr = torch.empty(E, device=r.device)
        genv = torch.empty(E, device=r.device) if ctx.needs_input_grad[1] else None
        call("face_radial_spline_bwd", ptr(r), ptr(pair), E, ptr(T), ptr(dT), P, G, F, float(ctx.dr), ptr(env), nb,
             ptr(order), ptr(gp), ldp, ptr(gq), ldq, ptr(gr), ptr(genv), _lib.stream_of(r), label="spline_bwd")
        return gr, genv, None, None, None, None, None, None


SPLINE_SORT_BYTES = 16 << 20                 # both tables above this: visit the edges cell by cell


def spline_wants_order(T):
    """Whether the spline kernels should visit the edges in table-cell order (tables of (P, G, F)
    far larger than L2, e.g. with the CP columns)."""
    return 8 * T.numel() > SPLINE_SORT_BYTES


def spline_order(r, pair, P, G, dr):
    """int32 (E,) permutation of the edges sorted by table cell (pair, grid interval of r); the
    same for every pass of a step (they share r, the pair index and the grid)."""
    _lib.require_gpu(r, pair)
    if pair.dtype != torch.int32:
        raise TypeError("spline_order: pair must be int32")
    E = r.shape[0]
    order = torch.empty(E, dtype=torch.int32, device=r.device)
    if E:
        work = torch.empty(P * G, dtype=torch.int32, device=r.device)
        call("face_radial_spline_order", ptr(r.detach().contiguous().float()), ptr(pair), E, P, G, float(dr),
             ptr(work), ptr(order), _lib.stream_of(r), label="spline_order")
    return order


def radial_spline(r, env, pair, T, dT, dr, nb, order=None):
    """(phi (E, nb), R (E, F - nb)) from the compiled tables; see RadialSpline. order: a
    spline_order() permutation to reuse (computed here when the tables want one and it is None)."""
    return RadialSpline.apply(r, env, pair, T, dT, dr, nb, order)


# ----------------------------------------------------------------------------- node algebra
def _s3(t):
    """(atom, channel, component) element strides of a 3-d view."""
    return [t.stride(0), t.stride(1), t.stride(2)]


def _pqs_views(y1, y2, y3, C):
    """(atom, channel, component) views of P1..Q3 inside monomial-major projection outputs
    y1 (3, N, 3C), y2 (6, N, 3C), y3 (10, N, >=2C)."""
    v = lambda y, j: y[:, :, j * C:(j + 1) * C].permute(1, 2, 0)
    return [v(y1, 0), v(y1, 1), v(y1, 2), v(y2, 0), v(y2, 1), v(y2, 2), v(y3, 0), v(y3, 1)]


class NodeFeatures(torch.autograd.Function):
    """Invariant families and gated products from the monomial-major projection outputs.

    y0 (1, N, >=C), y1 (3, N, 3C), y2 (6, N, 3C), y3 (10, N, >=2C): P|Q|S blocks of C channels.
    Returns feats (N, 9C) = [P0 | inv1..inv8] (family-major, face/model.py:244-249,254-264) and,
    when eq: V (3, N, C), Ms (6, N, C) = symmetrised Mf in sym storage (face/model.py:288-294).
    """

    @staticmethod
    def forward(ctx, y0, y1, y2, y3, a, b, eq, C, out):
        _lib.require_gpu(y0, y1, y2, y3)
        N = y1.shape[1]
        dev = y1.device
        y1, y2, y3 = [y.contiguous().float() for y in (y1, y2, y3)]
        ins = _pqs_views(y1, y2, y3, C)
        feats = out[0] if out else torch.empty(N, 9 * C, device=dev)
        if not (y0.data_ptr() == feats.data_ptr() and y0.stride(1) == feats.stride(0) and y0.shape[2] == C):
            feats[:, :C] = y0[0, :, :C]                 # P0 not already written in place
        inv_view = feats[:, C:].view(N, 8, C).transpose(1, 2)                   # (N,C,8)
        st = sum((_s3(t) for t in ins), [])
        V = Ms = None
        z3 = [0, 0, 0]
        if eq:
            V = torch.empty(3, N, C, device=dev)
            Ms = torch.empty(6, N, C, device=dev)
            a_, b_ = a.contiguous().float(), b.contiguous().float()
        else:
            a_ = b_ = None
        call("face_node_fwd", _lib.ptr_array(ins), _lib.i64_array(st), ptr(a_), ptr(b_), ptr(inv_view),
             _lib.i64_array(_s3(inv_view)), ptr(V), _lib.i64_array(_s3(V.permute(1, 2, 0)) if eq else z3),
             ptr(Ms), _lib.i64_array(_s3(Ms.permute(1, 2, 0)) if eq else z3), 1, N, C, int(bool(eq)),
             _lib.stream_of(y1), label="node_fwd")
        ctx.save_for_backward(y1, y2, y3, a_ if eq else torch.empty(0), b_ if eq else torch.empty(0))
        ctx.eq, ctx.C, ctx.y0_shape = eq, C, y0.shape
        if eq:
            return feats, V, Ms
        return feats, None, None

    @staticmethod
    def backward(ctx, gfeats, gV, gMs):
        y1, y2, y3, a, b = ctx.saved_tensors
        C, eq, y0_shape = ctx.C, ctx.eq, ctx.y0_shape
        N = y1.shape[1]
        dev = y1.device
        ins = _pqs_views(y1, y2, y3, C)
        st = sum((_s3(t) for t in ins), [])
        dy1 = torch.empty_like(y1)
        dy2 = torch.empty_like(y2)
        dy3 = torch.empty_like(y3)
        if dy3.shape[2] > 2 * C:
            dy3[:, :, 2 * C:] = 0
        outs = _pqs_views(dy1, dy2, dy3, C)
        gI = None
        z3 = [0, 0, 0]
        if gfeats is not None:
            gfeats = gfeats.contiguous().float()
            gI = gfeats[:, C:].view(N, 8, C).transpose(1, 2)
        # P0 was copied into the readout row: its gradient is that row's first C columns, handed
        # on as a strided view when y0 has exactly C channels (the projection backward reads rows
        # at any stride)
        if gfeats is not None and y0_shape[2] == C:
            dy0 = gfeats[:, :C].unsqueeze(0)
        else:
            dy0 = torch.zeros(y0_shape, device=dev)
            if gfeats is not None:
                dy0[0, :, :C] = gfeats[:, :C]
        need_ab = eq and (ctx.needs_input_grad[4] or ctx.needs_input_grad[5])
        da = torch.empty(N, C, 4, device=dev) if need_ab else None
        db = torch.empty(N, C, 4, device=dev) if need_ab else None
        if gV is not None:
            gV = gV.contiguous().float()
        if gMs is not None:
            gMs = gMs.contiguous().float()
        call("face_node_bwd", _lib.ptr_array(ins), _lib.i64_array(st), ptr(a) if eq else None,
             ptr(b) if eq else None, ptr(gI), _lib.i64_array(_s3(gI) if gI is not None else z3),
             ptr(gV), _lib.i64_array(_s3(gV.permute(1, 2, 0)) if gV is not None else z3),
             ptr(gMs), _lib.i64_array(_s3(gMs.permute(1, 2, 0)) if gMs is not None else z3), 1,
             _lib.ptr_array(outs), _lib.i64_array(sum((_s3(t) for t in outs), [])), ptr(da), ptr(db), N, C,
             int(bool(eq)), _lib.stream_of(y1), label="node_bwd")
        ga = da.sum(0).t() if need_ab else None
        gb = db.sum(0).t() if need_ab else None
        return dy0, dy1, dy2, dy3, ga, gb, None, None, None


def node_features(y0, y1, y2, y3, a, b, eq, C, out=None):
    """(feats, V | None, Ms | None); out: an (N, 9C) buffer for feats, whose first C columns may
    already hold P0 (y0 a view of them, as rank_proj writes it with out0)."""
    return NodeFeatures.apply(y0, y1, y2, y3, a, b, eq, C, (out,) if out is not None else ())


class NodeLN(torch.autograd.Function):
    """NodeFeatures followed by the readout LayerNorm (face/model.py:244-264, :140, :332) in one
    launch each way: returns inv = LayerNorm([P0 | inv_1..inv_8]) (N, 9C) and, when eq, V, Ms.
    The un-normalised row is never written (the backward recomputes it); the LayerNorm weight and
    bias and the coefficients a, b are frozen."""

    @staticmethod
    def forward(ctx, y0, y1, y2, y3, a, b, eq, C, lw, lb, eps):
        _lib.require_gpu(y0, y1, y2, y3)
        N = y1.shape[1]
        dev = y1.device
        y1, y2, y3 = [y.contiguous().float() for y in (y1, y2, y3)]
        p0 = y0[0, :, :C]
        if p0.stride(1) != 1:
            p0 = p0.contiguous()
        ins = _pqs_views(y1, y2, y3, C)
        st = sum((_s3(t) for t in ins), [])
        lw_, lb_ = lw.detach().contiguous().float(), lb.detach().contiguous().float()
        inv = torch.empty(N, 9 * C, device=dev)
        stats = torch.empty(N, 2, device=dev)
        V = Ms = None
        z3 = [0, 0, 0]
        if eq:
            V = torch.empty(3, N, C, device=dev)
            Ms = torch.empty(6, N, C, device=dev)
            a_, b_ = a.contiguous().float(), b.contiguous().float()
        else:
            a_ = b_ = None
        call("face_node_ln_fwd", _lib.ptr_array(ins), _lib.i64_array(st), ptr(p0), p0.stride(0), ptr(a_), ptr(b_),
             ptr(lw_), ptr(lb_), float(eps), ptr(inv), 9 * C, ptr(stats), ptr(V),
             _lib.i64_array(_s3(V.permute(1, 2, 0)) if eq else z3), ptr(Ms),
             _lib.i64_array(_s3(Ms.permute(1, 2, 0)) if eq else z3), 1, N, C, int(bool(eq)), _lib.stream_of(y1),
             label="node_ln_fwd")
        ctx.save_for_backward(p0, y1, y2, y3, a_ if eq else torch.empty(0), b_ if eq else torch.empty(0), lw_, stats)
        ctx.eq, ctx.C, ctx.y0_shape = eq, C, y0.shape
        ctx.set_materialize_grads(False)
        return inv, V, Ms

    @staticmethod
    def backward(ctx, ginv, gV, gMs):
        p0, y1, y2, y3, a, b, lw, stats = ctx.saved_tensors
        C, eq = ctx.C, ctx.eq
        N = y1.shape[1]
        dev = y1.device
        ins = _pqs_views(y1, y2, y3, C)
        st = sum((_s3(t) for t in ins), [])
        dy1 = torch.empty_like(y1)
        dy2 = torch.empty_like(y2)
        dy3 = torch.empty_like(y3)
        if dy3.shape[2] > 2 * C:
            dy3[:, :, 2 * C:] = 0
        outs = _pqs_views(dy1, dy2, dy3, C)
        ginv = torch.zeros(N, 9 * C, device=dev) if ginv is None else ginv.contiguous().float()
        # the kernel writes P0's gradient; wider y0 rows (other channels unused) start at zero
        dy0 = torch.empty(ctx.y0_shape, device=dev) if ctx.y0_shape[2] == C else torch.zeros(ctx.y0_shape, device=dev)
        need_ab = eq and (ctx.needs_input_grad[4] or ctx.needs_input_grad[5])
        da = torch.empty(N, C, 4, device=dev) if need_ab else None
        db = torch.empty(N, C, 4, device=dev) if need_ab else None
        z3 = [0, 0, 0]
        if gV is not None:
            gV = gV.contiguous().float()
        if gMs is not None:
            gMs = gMs.contiguous().float()
        dp0 = dy0[0, :, :C]
        call("face_node_ln_bwd", _lib.ptr_array(ins), _lib.i64_array(st), ptr(p0), p0.stride(0),
             ptr(a) if eq else None, ptr(b) if eq else None, ptr(lw), ptr(ginv), 9 * C, ptr(stats),
             ptr(gV), _lib.i64_array(_s3(gV.permute(1, 2, 0)) if gV is not None else z3),
             ptr(gMs), _lib.i64_array(_s3(gMs.permute(1, 2, 0)) if gMs is not None else z3), 1,
             _lib.ptr_array(outs), _lib.i64_array(sum((_s3(t) for t in outs), [])), ptr(dp0), dp0.stride(0),
             ptr(da), ptr(db), N, C, int(bool(eq)), _lib.stream_of(y1), label="node_ln_bwd")
        ga = da.sum(0).t() if need_ab else None
        gb = db.sum(0).t() if need_ab else None
        return dy0, dy1, dy2, dy3, ga, gb, None, None, None, None, None


def node_ln(y0, y1, y2, y3, a, b, eq, C, lw, lb, eps):
    """(LayerNorm(feats) (N, 9C), V | None, Ms | None): node_features and the readout LayerNorm in
    one launch each way (C <= 256)."""
    return NodeLN.apply(y0, y1, y2, y3, a, b, eq, C, lw, lb, eps)


# ----------------------------------------------------------------------------- row-block linear layers
def lin(x, w, y, s_off=0, beta=0.0, x2=None, x_op=0, xz=None, bias=None, y0=None, n_y0=None):
    """One problem of rows_linear: y = (beta y0 + op(x | x2) w^T + bias) [* scales]; x (m, k1),
    x2 (m, k - k1) the rest of the input columns (no concatenated copy), x_op on the x columns:
    0 none, 1 silu, 2 x * silu'(xz); y0 the initial sum (default y) over its first n_y0 columns.
    2-d fp32 views with unit column stride."""
    return dict(x=x, w=w, y=y, s_off=s_off, beta=beta, x2=x2, x_op=x_op, xz=xz, bias=bias, y0=y0, n_y0=n_y0)


def rows_linear(probs, w_kn=False, bias=None, xs=None, ys=None, group=None, period=1, label="rows_linear"):
    """One launch of up to eight row-block linear problems (no autograd). probs: lin() dicts or
    (x (m, k), w, y (m, n), s_off, beta) tuples; w is (n, k) or, with w_kn, (k, n).
    y[r] = (beta y0[r] + (op(x)[r] * xs[g(r), s_off:]) w^T + bias) * ys[g(r), s_off:],
    g(r) = group[r % period]; xs / ys are (n_groups, ld) tables or None; `bias` applies to the
    problems without their own."""
    arr = (_lib.LinProblem * len(probs))()
    ref = None
    for i, pr in enumerate(probs):
        if not isinstance(pr, dict):
            pr = lin(*pr)
        x, w, y, x2, xz, y0 = pr["x"], pr["w"], pr["y"], pr["x2"], pr["xz"], pr["y0"]
        b = pr["bias"] if pr["bias"] is not None else bias
        assert x.dim() == 2 and y.dim() == 2 and w.dim() == 2 and x.stride(1) == 1 and y.stride(1) == 1
        assert w.stride(1) == 1 and x.shape[0] == y.shape[0]
        k1 = x.shape[1]
        k = k1 + (x2.shape[1] if x2 is not None else 0)
        for t in (x2, xz, y0):
            assert t is None or (t.dim() == 2 and t.stride(1) == 1 and t.shape[0] == x.shape[0])
        n_y0 = pr["n_y0"] if pr["n_y0"] is not None else (y0.shape[1] if y0 is not None else y.shape[1])
        arr[i] = _lib.LinProblem(x.data_ptr(), x.stride(0), x.shape[0], w.data_ptr(), w.stride(0), y.data_ptr(),
                                 y.stride(0), y.shape[1], k, int(pr["s_off"]), float(pr["beta"]),
                                 ptr(x2), 0 if x2 is None else x2.stride(0), k1, int(pr["x_op"]),
                                 ptr(xz), 0 if xz is None else xz.stride(0), ptr(b),
                                 ptr(y0), 0 if y0 is None else y0.stride(0), int(n_y0), 0)
        ref = y
    tab = xs if xs is not None else ys
    if xs is not None and ys is not None and xs.shape[0] != ys.shape[0]:
        raise ValueError("rows_linear: xs and ys must have the same number of groups")
    call("face_rows_linear", arr, len(probs), 1 if w_kn else 0, ptr(xs), ptr(ys),
         0 if tab is None else tab.stride(0), 0 if tab is None else tab.shape[0], ptr(group), int(period),
         _lib.stream_of(ref), label=label)


# mix and transport-mix backward in one launch up to this many atoms (launch-bound sizes; at
# 24,000 atoms the six-problem launch measured 646 us against 238 + 354 us for the two)
MIX_MERGE_MAX_ATOMS = 4096


class ScaledMix(torch.autograd.Function):
    """A_l = (Af_l W_l^T [+ D_l T_l^T]) * s[z] for the four ranks l (face/model.py:498-501, the
    transport terms of :530-533 for l = 1, 2): s = elem_scale / avg_nb per atom (s_tab (n_el, 4C),
    group = element index per atom, int32). The four mix GEMMs run in one launch with the scale
    (and the accumulation onto the tmix products) in their epilogue; the backward applies the
    scale to the upstream rows as it loads them. Weights receive no gradient."""

    @staticmethod
    def forward(ctx, s_tab, group, wm, wt, D1, D2, *Af):
        N = group.shape[0]
        C = wm[0].shape[0]
        dev = Af[0].device
        outs = [torch.empty(a.shape[0], N, C, device=dev) for a in Af]
        Ds = {1: D1, 2: D2}
        for l, D in Ds.items():
            if D is not None:
                torch.mm(D.reshape(-1, D.shape[-1]), wt[l - 1].t(), out=outs[l].view(-1, C))
        probs = [(a.reshape(-1, a.shape[-1]), wm[l], outs[l].view(-1, C), l * C,
                  1.0 if Ds.get(l) is not None else 0.0) for l, a in enumerate(Af)]
        rows_linear(probs, ys=s_tab, group=group, period=N, label="mix_fwd")
        ctx.save_for_backward(s_tab, group)
        ctx.wm, ctx.wt, ctx.has_D = wm, wt, (D1 is not None, D2 is not None)
        ctx.shapes = [a.shape for a in Af]
        return tuple(outs)

    @staticmethod
    def backward(ctx, *gA):
        s_tab, group = ctx.saved_tensors
        N = group.shape[0]
        C = ctx.wm[0].shape[0]
        dev = s_tab.device
        gA = [(g.contiguous() if g is not None else torch.zeros(sh[0], N, C, device=dev))
              for g, sh in zip(gA, ctx.shapes)]
        dAf = [torch.empty(sh, device=dev) for sh in ctx.shapes]
        probs = [(g.view(-1, C), ctx.wm[l], dAf[l].view(-1, dAf[l].shape[-1]), l * C, 0.0) for l, g in enumerate(gA)]
        # transport mix: dD_l = (gA_l * s_l) wt, the scale applied to the rows as they load; for
        # small systems in the same launch as the mix backward (same scale table, 6 problems)
        dD = [None, None]
        tp = []
        for i, l in enumerate((1, 2)):
            if ctx.has_D[i] and ctx.needs_input_grad[4 + i]:
                wt = ctx.wt[i]
                dD[i] = torch.empty(gA[l].shape[0], N, wt.shape[1], device=dev)
                tp.append((gA[l].view(-1, C), wt, dD[i].view(-1, wt.shape[1]), l * C, 0.0))
        if tp and N <= MIX_MERGE_MAX_ATOMS:
            rows_linear(probs + tp, w_kn=True, xs=s_tab, group=group, period=N, label="mix_tmix_bwd")
        else:
            rows_linear(probs, w_kn=True, xs=s_tab, group=group, period=N, label="mix_bwd")
            if tp:
                rows_linear(tp, w_kn=True, xs=s_tab, group=group, period=N, label="tmix_bwd")
        return (None, None, None, None, dD[0], dD[1], *dAf)


def scaled_mix(s_tab, group, wm, wt, D1, D2, Af):
    return ScaledMix.apply(s_tab, group, wm, wt, D1, D2, *Af)


def _row_view(t, n):
    """(k, N, n) -> (k N, n) rows with unit column stride: a view where the strides allow one
    (e.g. a column block of a wider row-major tensor), else a contiguous copy."""
    if t.stride(-1) == 1 and t.stride(1) >= n and (t.shape[0] == 1 or t.stride(0) == t.shape[1] * t.stride(1)):
        return t.as_strided((t.shape[0] * t.shape[1], n), (t.stride(1), 1))
    return t.contiguous().view(-1, n)


class SetGrad:
    """The input gradient of one moment set read by several RankProj nodes (the set of pass p is
    projected again by every later pass): the first backward to run writes it, the later ones
    accumulate onto it in the GEMM epilogue (beta = 1) and hand autograd None, so no separate
    accumulation add runs. Valid only when RankProj nodes are the set's only readers; reset once
    all of them have run (a second backward through the same graph starts again)."""
    __slots__ = ("readers", "arrived", "g")

    def __init__(self):
        self.readers, self.arrived, self.g = 0, 0, None


class RankProj(torch.autograd.Function):
    """y_l = sum_s S_s,l W_l[:, s C:(s + 1) C]^T for the four ranks l over the moment sets s
    (face/model.py:537-544, the proj of the concatenated sets as a sum of per-set products):
    one launch per set, the sets after the first accumulating in the epilogue. The backward
    gives each set's input gradient, again one launch per set (accumulated across the nodes
    that share a set through its SetGrad, when given). Weights receive no gradient."""

    @staticmethod
    def forward(ctx, ws, n_sets, acc, out0, *S):
        C = S[0].shape[-1]
        N = S[0].shape[1]
        dev = S[0].device
        sets = [S[4 * s:4 * s + 4] for s in range(n_sets)]
        ys = [torch.empty(sets[0][l].shape[0], N, w.shape[0], device=dev) for l, w in enumerate(ws)]
        if out0:
            ys[0] = out0[0].unsqueeze(0)                 # rank 0 (one monomial) into the caller's rows
        # two sets per launch as one product of K = 2C (the second set's rows as the split input
        # columns), a third accumulating in the epilogue of the next launch
        for s in range(0, n_sets, 2):
            pair = s + 1 < n_sets
            rows_linear([lin(sets[s][l].reshape(-1, C), ws[l][:, s * C:(s + 1 + pair) * C],
                             ys[l].reshape(-1, ws[l].shape[0]), 0, 1.0 if s else 0.0,
                             x2=sets[s + 1][l].reshape(-1, C) if pair else None) for l in range(4)],
                        label="proj_fwd*2" if pair else "proj_fwd")
        slots = None
        if acc is not None:
            # one SetGrad per set, keyed by its rank-0 tensor (the entry holds the tensor itself, so
            # the key cannot be recycled while the dict lives)
            slots = []
            for S_s in sets:
                ent = acc.get(id(S_s[0]))
                if ent is None or ent[0] is not S_s[0]:
                    ent = (S_s[0], SetGrad())
                    acc[id(S_s[0])] = ent
                ent[1].readers += 1
                slots.append(ent[1])
        ctx.ws, ctx.n_sets, ctx.C, ctx.slots = ws, n_sets, C, slots
        ctx.shapes = [t.shape for t in S]
        return tuple(ys)

    @staticmethod
    def backward(ctx, *gy):
        C, ws = ctx.C, ctx.ws
        dev = ws[0].device
        gy = [(_row_view(g, w.shape[0]) if g is not None else torch.zeros(sh[0] * sh[1], w.shape[0], device=dev))
              for g, w, sh in zip(gy, ws, ctx.shapes[:4])]
        grads, probs, n_in = [], [], 0
        for s in range(ctx.n_sets):
            need = [ctx.needs_input_grad[4 + 4 * s + l] for l in range(4)]
            slot = ctx.slots[s] if ctx.slots is not None else None
            if slot is not None and slot.g is not None:
                d, beta, out = slot.g, 1.0, [None] * 4
            else:
                d = [torch.empty(ctx.shapes[4 * s + l], device=dev) if need[l] else None for l in range(4)]
                beta, out = 0.0, d
                if slot is not None:
                    slot.g = d
            # the four ranks of two sets per launch
            probs += [(gy[l], ws[l][:, s * C:(s + 1) * C], d[l].view(-1, C), 0, beta) for l in range(4) if need[l]]
            n_in += 1
            if len(probs) > 4 or s == ctx.n_sets - 1:
                if probs:
                    rows_linear(probs, w_kn=True, label="proj_bwd*2" if n_in == 2 else "proj_bwd")
                probs, n_in = [], 0
            if slot is not None:
                slot.arrived += 1
                if slot.arrived == slot.readers:
                    slot.g, slot.arrived = None, 0
            grads += out
        return (None, None, None, None, *grads)


def rank_proj(ws, sets, acc=None, out0=None):
    """ws: 4 frozen proj weights (n_l, n_sets C); sets: list of 4-tuples of (k_l, N, C) moments;
    acc: a dict shared by the rank_proj calls of one forward whose sets nothing else reads (their
    gradients then accumulate in place, see SetGrad), or None; out0: (N, n_0) rows (unit column
    stride, any row stride) that receive the rank-0 output, returned as a (1, N, n_0) view."""
    return RankProj.apply(ws, len(sets), acc, (out0,) if out0 is not None else (), *[t for S in sets for t in S])
