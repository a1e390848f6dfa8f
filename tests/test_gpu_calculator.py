"""The calculator / MD loop around the hot path (face/calculator.py:35-56): pair lists built on
the device with a skin and reused, HIP-graph replay, velocity-Verlet NVE."""
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
SMALL = dict(C=16, n_basis=8, n_passes=2, radial_hidden=16, K_dir=4, transport=True, eqmsg=True, factor=True, B=8,
             K=16, rc=3.5)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _model(**over):
    from face_amd import model as fm
    torch.manual_seed(0)
    return fm.unit_parameterise(fm.FACE([1, 6, 8], **dict(SMALL, **over))).to(DEV).eval()


def _liquid(n=300):
    from face_amd import systems
    (liq,), _, _, _ = systems.workload(3, n_atoms=n)
    return liq


def _exact(m, pos, Z, cell, pbc):
    from face_amd.neighbors import build_graph
    g = build_graph([{"pos": pos.double().cpu().numpy(), "Z": Z, "cell": cell, "pbc": pbc}], m.rc, DEV)
    o = m(g.with_pos(pos.clone()))
    return o["energy"][0].detach(), o["forces"].detach()


def _close(e, f, e2, f2, tol_e=1e-6, tol_f=1e-5):
    de = abs(float(e) - float(e2)) / max(abs(float(e2)), 1e-12)
    rms = f2.pow(2).mean().sqrt().item()
    df = (f - f2).abs().max().item() / max(rms, 1e-12)
    return de < tol_e and df < tol_f, (de, df)


@pytest.mark.parametrize("periodic", [True, False])
def test_skin_list_equals_exact_list(periodic):
    from face_amd.calculator import FACECalculator
    say("skin list", periodic)
    m = _model()
    if periodic:
        s = _liquid()
        pos, Z, cell, pbc = torch.as_tensor(s["pos"], dtype=torch.float32, device=DEV), s["Z"], s["cell"], True
    else:
        from face_amd import systems
        mols, _, _, _ = systems.workload(0)
        s = mols[0]
        pos, Z, cell, pbc = torch.as_tensor(s["pos"], dtype=torch.float32, device=DEV), s["Z"], None, False
    calc = FACECalculator(m, skin=0.8)
    e, f = calc.compute(pos, Z, cell, pbc)
    e2, f2 = _exact(m, pos, Z, cell, pbc)
    ok, errs = _close(e, f, e2, f2)
    assert ok, errs


def test_reuse_rebuild_and_unwrapped_positions():
    from face_amd.calculator import FACECalculator
    say("reuse / rebuild")
    m = _model()
    s = _liquid()
    cell = s["cell"]
    pos0 = torch.as_tensor(s["pos"], dtype=torch.float32, device=DEV)
    calc = FACECalculator(m, skin=0.8)
    calc.compute(pos0, s["Z"], cell, True)
    g = torch.Generator(device="cpu").manual_seed(5)
    step = (torch.rand(pos0.shape, generator=g) - 0.5).to(DEV) * 0.2          # |d| < 0.18 < skin / 2
    pos1 = pos0 + step
    e, f = calc.compute(pos1, s["Z"], cell, True)
    assert calc.n_builds == 1
    ok, errs = _close(e, f, *_exact(m, pos1, s["Z"], cell, True))
    assert ok, errs
    # lattice-shifted copies of some atoms: same energy and forces, and a rebuild
    shift = torch.zeros_like(pos1)
    shift[::7] = torch.as_tensor(cell[0] - 2 * cell[2], dtype=torch.float32, device=DEV)
    e2, f2 = calc.compute(pos1 + shift, s["Z"], cell, True)
    assert calc.n_builds == 2
    ok, errs = _close(e2, f2, e, f, 1e-6, 1e-4)           # fp32 rounding of ~30 A coordinates
    assert ok, errs


def test_graph_replay_equals_eager():
    from face_amd.calculator import FACECalculator
    say("calculator graph vs eager")
    m = _model()
    s = _liquid()
    pos = torch.as_tensor(s["pos"], dtype=torch.float32, device=DEV)
    a = FACECalculator(m, skin=0.5, use_graph=True)
    b = FACECalculator(m, skin=0.5, use_graph=False)
    for k in range(3):
        p = pos + 0.01 * k
        ea, fa = a.compute(p, s["Z"], s["cell"], True)
        eb, fb = b.compute(p, s["Z"], s["cell"], True)
        ok, errs = _close(ea, fa, eb, fb, 1e-6, 1e-5)
        assert ok, (k, errs)


def test_nve_energy_error_is_second_order():
    """Velocity Verlet conserves the total energy up to O(dt^2) only if the forces are the
    exact negative gradient of the energy: halving dt must cut the energy error about 4x."""
    from face_amd.calculator import FACECalculator, run_nve
    say("nve")
    m = _model()
    s = _liquid(200)
    masses = np.array([{1: 1.008, 6: 12.011, 8: 15.999}[int(z)] for z in s["Z"]])
    rng = np.random.default_rng(3)
    kT = 0.025                                                    # eV
    vel = rng.normal(size=(len(masses), 3)) * np.sqrt(kT / masses)[:, None]
    errs = []
    for dt, n in ((2.0, 20), (1.0, 40)):
        calc = FACECalculator(m, skin=0.8)
        _, _, hist = run_nve(calc, s["pos"], vel, masses, s["Z"], s["cell"], True, dt_fs=dt, steps=n)
        errs.append(np.abs(hist - hist[0]).max())
        say("   dt", dt, "max |dE_tot|", errs[-1], "builds", calc.n_builds)
    ratio = errs[0] / max(errs[1], 1e-30)
    assert 2.5 < ratio < 6.5, (errs, ratio)
