"""CPU checks of host-side autograd nodes built from torch ops only (no kernel calls): the readout
MLP node against plain autograd of the reference's readout (face/model.py:331-339, the gate of
:286-287) in fp64, values and input gradients, for every combination of gate / last pass."""
import pytest
import torch
import torch.nn.functional as F


@pytest.mark.parametrize("gate", [True, False])
@pytest.mark.parametrize("last", [True, False])
def test_readout_mlp_matches_autograd_of_the_reference_readout(gate, last):
    from face_amd import ops
    torch.manual_seed(0)
    N, C = 7, 4
    nf = 9 * C
    dt = torch.float64
    inv = torch.randn(N, nf, dtype=dt, requires_grad=True)
    h = torch.randn(N, C, dtype=dt, requires_grad=True)
    W0, b0 = torch.randn(2 * C, nf + C + 4, dtype=dt), torch.randn(2 * C, dtype=dt)
    W1, b1 = torch.randn(2 * C, 2 * C, dtype=dt), torch.randn(2 * C, dtype=dt)
    W2, b2 = torch.randn(C + 1, 2 * C, dtype=dt), torch.randn(C + 1, dtype=dt)
    Wg, bg = torch.randn(2 * C, nf, dtype=dt), torch.randn(2 * C, dtype=dt)

    # the reference's formulation: out MLP on cat([inv, h, 0 (4)]), e = o[:, :1], h + o[:, 1:]
    z = F.linear(torch.cat([inv, h, torch.zeros(N, 4, dtype=dt)], 1), W0, b0)
    o = F.linear(F.silu(F.linear(F.silu(z), W1, b1)), W2, b2)
    ref = (o[:, :1], None if last else h + o[:, 1:], F.linear(inv, Wg, bg) if gate else None)

    got = ops.readout_mlp(inv, h, W0[:, :nf], W0[:, nf:nf + C], b0, W1, b1, W2, b2,
                          Wg if gate else None, bg if gate else None, last)
    for a, b in zip(got, ref):
        assert (a is None) == (b is None)
        if a is not None:
            torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)
    # input gradients under random upstream gradients of every output, then of the energy alone
    up = [torch.randn_like(t) if t is not None else None for t in ref]
    for ws in (up, [up[0], None, None]):
        L = lambda outs: sum((t * w).sum() for t, w in zip(outs, ws) if t is not None and w is not None)
        g_got = torch.autograd.grad(L(got), (inv, h), retain_graph=True)
        g_ref = torch.autograd.grad(L(ref), (inv, h), retain_graph=True)
        for a, b in zip(g_got, g_ref):
            torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)
