"""Drop-in replacement of face/kernels.py: the fused factor density on gfx950.

factor_density(phi, msg, Y) keeps the reference signature and shapes
(face/kernels.py:170-172): (N,M,B), (N,M,K), (N,M,20) -> (N,20,B*K), first-order
differentiable, launched on torch's current stream, outputs allocated by torch. The padded
layout is handed to the kernels as-is (row i = edges i*M .. i*M+M-1); masked slots carry
phi = 0 and so contribute nothing.
"""
import torch

from . import _lib
from ._lib import call, ptr


class FactorDensity(torch.autograd.Function):
    """face/kernels.py:135-167 (forward :137-149, backward :151-167)."""

    @staticmethod
    def forward(ctx, phi, msg, Y):
        _lib.require_gpu(phi, msg, Y)
        N, M, B = phi.shape
        K = msg.shape[-1]
        if msg.shape[:2] != (N, M) or Y.shape != (N, M, 20):
            raise ValueError(f"factor_density: shapes {tuple(phi.shape)}, {tuple(msg.shape)}, {tuple(Y.shape)}")
        phi, msg, Y = phi.contiguous().float(), msg.contiguous().float(), Y.contiguous().float()
        D = torch.empty(N, 20, B * K, device=phi.device, dtype=torch.float32)
        call("face_density_fwd", ptr(phi), B, ptr(msg), K, None, ptr(Y), 20, 20, None, N, M, B, K,
             *_lib.ranks_of_dense(D), _lib.stream_of(phi))
        ctx.save_for_backward(phi, msg, Y)
        return D

    @staticmethod
    def backward(ctx, G):
        phi, msg, Y = ctx.saved_tensors
        N, M, B = phi.shape
        K = msg.shape[-1]
        G = G.contiguous().float()
        dphi, dmsg, dY = torch.empty_like(phi), torch.empty_like(msg), torch.empty_like(Y)
        call("face_density_bwd", ptr(phi), B, ptr(msg), K, None, ptr(Y), 20, 20, None, N, M, M, B, K,
             *_lib.ranks_of_dense(G), ptr(dphi), B, ptr(dmsg), K, ptr(dY), 20, _lib.stream_of(G))
        return dphi, dmsg, dY


def factor_density(phi, msg, Y):
    """(N,M,B), (N,M,K), (N,M,20) -> (N,20,B*K); first-order differentiable."""
    return FactorDensity.apply(phi, msg, Y)
