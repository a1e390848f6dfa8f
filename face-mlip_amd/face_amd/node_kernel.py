"""Drop-in replacement of face/node_kernel.py: the fused node algebra on gfx950.

node_algebra(P1,Q1,S1,P2,Q2,S2,P3,Q3,a,b,eq) keeps the reference signature and shapes
(face/node_kernel.py:207-209): symmetric storage in, inv (N,C,8), V (N,C,3), Mf (N,C,3,3)
out, a/b gradients returned summed over atoms as (4,C). Operands are read through their own
strides, so the split/transposed projection views of face/model.py:227-232 need no copy.
"""
import torch

from . import _lib
from ._lib import call, ptr


def _s3(t):
    return [t.stride(0), t.stride(1), t.stride(2)]


class NodeAlgebra(torch.autograd.Function):
    """face/node_kernel.py:164-204."""

    @staticmethod
    def forward(ctx, P1, Q1, S1, P2, Q2, S2, P3, Q3, a, b, eq):
        ins = [t if t.dtype == torch.float32 else t.float() for t in (P1, Q1, S1, P2, Q2, S2, P3, Q3)]
        _lib.require_gpu(*ins)
        N, C = P1.shape[:2]
        widths = [3, 3, 3, 6, 6, 6, 10, 10]
        for t, w in zip(ins, widths):
            if t.shape != (N, C, w):
                raise ValueError(f"node_algebra: expected (N,C,{w}), got {tuple(t.shape)}")
        dev = P1.device
        inv = torch.empty(N, C, 8, device=dev)
        V = torch.empty(N, C, 3, device=dev)
        Mf = torch.empty(N, C, 3, 3, device=dev)
        a_, b_ = a.contiguous().float(), b.contiguous().float()
        Mv = Mf.view(N, C, 9)
        call("face_node_fwd", _lib.ptr_array(ins), _lib.i64_array(sum((_s3(t) for t in ins), [])), ptr(a_), ptr(b_),
             ptr(inv), _lib.i64_array(_s3(inv)), ptr(V), _lib.i64_array(_s3(V)), ptr(Mv), _lib.i64_array(_s3(Mv)),
             0, N, C, int(bool(eq)), _lib.stream_of(P1))
        ctx.save_for_backward(*ins, a_, b_)
        ctx.eq = eq
        return inv, V, Mf

    @staticmethod
    def backward(ctx, gI, gV, gM):
        *ins, a, b = ctx.saved_tensors
        N, C = ins[0].shape[:2]
        dev = ins[0].device
        eq = bool(ctx.eq)
        outs = [torch.empty(t.shape, device=dev) for t in ins]
        cont = lambda t: None if t is None else t.contiguous().float()
        gI, gV = cont(gI), cont(gV)
        gM = None if gM is None else cont(gM).view(N, C, 9)
        if not eq:
            gV = gM = None
        need_ab = ctx.needs_input_grad[8] or ctx.needs_input_grad[9]
        da = torch.zeros(N, C, 4, device=dev) if need_ab else None
        db = torch.zeros(N, C, 4, device=dev) if need_ab else None
        z3 = [0, 0, 0]
        call("face_node_bwd", _lib.ptr_array(ins), _lib.i64_array(sum((_s3(t) for t in ins), [])), ptr(a), ptr(b),
             ptr(gI), _lib.i64_array(_s3(gI) if gI is not None else z3), ptr(gV),
             _lib.i64_array(_s3(gV) if gV is not None else z3), ptr(gM),
             _lib.i64_array(_s3(gM) if gM is not None else z3), 0, _lib.ptr_array(outs),
             _lib.i64_array(sum((_s3(t) for t in outs), [])), ptr(da) if eq else None, ptr(db) if eq else None,
             N, C, int(eq), _lib.stream_of(ins[0]))
        ga = da.sum(0).t() if need_ab else None
        gb = db.sum(0).t() if need_ab else None
        return (*outs, ga, gb, None)


def node_algebra(P1, Q1, S1, P2, Q2, S2, P3, Q3, a, b, eq=True):
    """P2,Q2,S2: (N,C,6) and P3,Q3: (N,C,10) symmetric components (no expansion to full tensors)."""
    return NodeAlgebra.apply(P1, Q1, S1, P2, Q2, S2, P3, Q3, a, b, eq)
