"""Write the golden vectors of tests/golden/ from the reference's own torch path (CPU).

Runs in the build container only (it reads /root/reference, which does not exist on the GPU
host). For each case it builds the reference FACE (face/model.py) with a fixed seed,
unit-parameterises it, evaluates energy and forces with the UNFUSED reference path on a
padded graph, and stores: the graph, the full state_dict (small models) or per-tensor
checksums (benchmark widths), energies, per-atom energies and forces.

The padded graphs come from the oracle's brute-force pair list (ASE is not installed); the
reference forward is independent of the within-row order up to fp rounding.

Usage: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
REF = "/root/reference"
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.join(REPO, "face-mlip_amd"))
sys.path.insert(0, REF)
sys.path.insert(0, HERE)

from face.model import FACE, unit_parameterise  # noqa: E402  (the reference, CPU, torch only)

from oracle.neighbors import padded_graph  # noqa: E402
from face_amd import systems  # noqa: E402
from cases import SMALL_CASES, BIG_CASES  # noqa: E402


def small_structures(seed):
    """Two aspirin-order molecules (non-periodic) + one small periodic box, as oracle dicts."""
    rng = np.random.default_rng(seed)
    mols = systems.molecules(2, rng)
    box = systems.liquid(40, rng, rho=0.08, dmin=1.0)   # 40 atoms, L ~ 7.9 A (> 2 rc for rc 3.5)
    return mols, [box]


def run_case(name, structures, kw, elements, dtype, seed=0, store_state=True):
    torch.set_default_dtype(dtype)
    torch.manual_seed(seed)
    m = FACE(elements, **kw)
    unit_parameterise(m)
    m.eval()
    g = padded_graph(structures, kw["rc"], dtype=dtype)
    gg = {k: g[k] for k in ("pos", "Z", "nbr", "shift", "mask", "batch")}
    gg["pos"] = gg["pos"].clone()
    o = m(gg)
    out = {
        "pos": g["pos"].numpy(), "Z": g["Z"].numpy(), "nbr": g["nbr"].numpy(), "shift": g["shift"].numpy(),
        "mask": g["mask"].numpy(), "batch": g["batch"].numpy(),
        "energy": o["energy"].detach().numpy(), "atom_energy": o["atom_energy"].detach().numpy(),
        "forces": o["forces"].detach().numpy(),
    }
    sd = m.state_dict()
    keys = list(sd.keys())
    out["state_keys"] = np.array(keys)
    for k in keys:
        v = sd[k].detach().double().numpy()
        if store_state:
            out["state/" + k] = sd[k].detach().numpy()
        out["sum/" + k] = np.array([v.sum(), np.abs(v).sum(), (v * v).sum()])
        out["head/" + k] = v.reshape(-1)[:4].copy()
    torch.set_default_dtype(torch.float32)
    return out


def main():
    mols, box = small_structures(7)
    sets = {"mols": mols, "box": box}
    for dt, tag in ((torch.float64, "f64"), (torch.float32, "f32")):
        for name, (kw, el, which) in SMALL_CASES.items():
            out = run_case(name, sets[which], kw, el, dt)
            np.savez_compressed(os.path.join(HERE, f"{name}_{tag}.npz"), **out)
            print(name, tag, "E =", out["energy"], flush=True)
    # benchmark widths: checksums of the seeded weights + E/F on two molecules / small cells
    rng = np.random.default_rng(11)
    sets = {"two": systems.molecules(2, rng),
            "fcc": [systems.fcc(4.09, 2, 0.1, rng)],                # 32 atoms, L = 8.18 A
            "liq": [systems.liquid(60, rng, rho=0.10, dmin=0.9)]}   # 60 atoms, L = 8.43 A
    for name, (kw, el, which) in BIG_CASES.items():
        out = run_case(name, sets[which], kw, el, torch.float32, store_state=False)
        np.savez_compressed(os.path.join(HERE, f"{name}_f32.npz"), **out)
        print(name, "E =", out["energy"], flush=True)


if __name__ == "__main__":
    main()
