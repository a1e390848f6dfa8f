"""ASE-style calculator and an on-device molecular-dynamics loop over the MI355X path.

FACECalculator follows face/calculator.py:35-56 (energy + forces of one structure from a
FACE model in evaluation mode; like the reference on CUDA, face/calculator.py:41-43, it
tabulates the radial functions with model.compile_radial() unless the model already has
tables or compile_radial=False) with three differences that keep every step on the device:

  * the pair list is built on the GPU with cutoff rc + skin and reused until some atom has
    moved more than skin / 2 since the build (the reference rebuilds the padded list on the
    CPU on every call, face/calculator.py:52; its padded_graph already takes the skin,
    face/neighbors.py:7). Pairs in the skin shell contribute exactly zero: the cutoff envelope
    and its derivative vanish for r >= rc (face/model.py:28-40), so the energy is the
    exact-list energy up to summation order;
  * positions stay unwrapped between rebuilds (the list carries integer image offsets);
  * the E+F step of a list is captured once as a HIP graph and replayed (runner.StepGraph).

Units follow ASE: positions in Angstrom, energies in eV, forces in eV/Angstrom, masses in amu,
time in ASE units (1 fs = FS ASE time units).
"""
import numpy as np
import torch

from .neighbors import build_graph
from .runner import StepGraph

FS = 0.09822694788464063            # 1 fs in ASE time units (Angstrom sqrt(amu / eV))


class FACECalculator:
    """Energy and forces of one structure (positions, Z, cell, pbc) with pair-list reuse."""

    implemented_properties = ("energy", "forces")

    def __init__(self, model, skin=0.5, use_graph=True, e_shift=0.0, device="cuda", tune_gemms=False,
                 compile_radial=True):
        if tune_gemms:                     # library GEMM solutions timed on the first step
            from .runner import tune_library_gemms
            tune_library_gemms()
        if model.training:
            raise ValueError("FACECalculator needs the model in evaluation mode (model.eval())")
        if skin < 0:
            raise ValueError("skin must be >= 0")
        if compile_radial and getattr(model.blocks[0], "spline", 1) is None:
            model.compile_radial()
        self.model, self.skin, self.use_graph = model, float(skin), bool(use_graph)
        self.rc = float(model.rc)
        self.e_shift = float(e_shift)
        self.device = torch.device(device)
        self.n_builds = 0
        self._graph = self._runner = self._pos0 = self._key = None

    # ------------------------------------------------------------------ pair list
    def _structure_key(self, Z, cell, pbc):
        cell = np.zeros((3, 3)) if cell is None else np.asarray(cell, dtype=np.float64).reshape(3, 3)
        pbc = np.broadcast_to(np.asarray(pbc, dtype=bool), (3,))
        return (np.asarray(Z, dtype=np.int64).tobytes(), cell.tobytes(), pbc.tobytes()), cell, pbc

    def _rebuild(self, pos, Z, cell, pbc, key):
        st = {"pos": pos.detach().double().cpu().numpy(), "Z": np.asarray(Z, dtype=np.int64), "cell": cell,
              "pbc": pbc}
        self._graph = build_graph([st], self.rc + self.skin, self.device)
        self._pos0 = pos.detach().clone()
        self._key = key
        self._runner = StepGraph(self.model, self._graph) if self.use_graph else None
        self.n_builds += 1

    def needs_rebuild(self, pos, key):
        if self._graph is None or key != self._key:
            return True
        if self.skin == 0.0:
            return True
        disp = (pos.detach() - self._pos0).norm(dim=1).max()
        return bool(disp > 0.5 * self.skin)          # one device-to-host read

    # ------------------------------------------------------------------ evaluation
    def compute(self, pos, Z, cell=None, pbc=False):
        """Energy (0-d tensor) and forces (N, 3) on the device for device positions (N, 3)."""
        pos = torch.as_tensor(pos, dtype=torch.float32, device=self.device)
        key, cell_a, pbc_a = self._structure_key(Z, cell, pbc)
        if self.needs_rebuild(pos, key):
            self._rebuild(pos, Z, cell_a, pbc_a, key)
        if self._runner is not None:
            energy, forces = self._runner(pos)
            return energy[0] + self.e_shift, forces
        out = self.model(self._graph.with_pos(pos.clone()))
        return out["energy"][0].detach() + self.e_shift, out["forces"].detach()

    def calculate(self, structure):
        """face/calculator.py:46-56: {'pos','Z','cell','pbc'} -> {'energy': float, 'forces': (N,3) array}."""
        e, f = self.compute(structure["pos"], structure["Z"], structure.get("cell"), structure.get("pbc", False))
        return {"energy": float(e), "forces": f.double().cpu().numpy()}


def run_nve(calc, pos, vel, masses, Z, cell=None, pbc=False, dt_fs=0.5, steps=100, record=True):
    """Velocity-Verlet NVE trajectory on the device. pos, vel (N, 3) in Angstrom and
    Angstrom / ASE-time, masses (N,) amu. Returns the final positions and velocities and, if
    record, the per-step total energy (potential + kinetic, eV) as a host array."""
    dev = calc.device
    pos = torch.as_tensor(pos, dtype=torch.float32, device=dev).clone()
    vel = torch.as_tensor(vel, dtype=torch.float32, device=dev).clone()
    inv_m = 1.0 / torch.as_tensor(masses, dtype=torch.float32, device=dev)[:, None]
    m = torch.as_tensor(masses, dtype=torch.float32, device=dev)[:, None]
    dt = dt_fs * FS
    e, f = calc.compute(pos, Z, cell, pbc)
    f = f.clone()
    totals = []
    for _ in range(steps):
        vel += (0.5 * dt) * f * inv_m
        pos += dt * vel
        e, f = calc.compute(pos, Z, cell, pbc)
        f = f.clone()
        vel += (0.5 * dt) * f * inv_m
        if record:
            totals.append(e + 0.5 * (m * vel * vel).sum())
    hist = torch.stack(totals).double().cpu().numpy() if record and totals else None
    return pos, vel, hist
