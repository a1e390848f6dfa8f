"""ASE-style calculator and an on-device molecular-dynamics loop over the MI355X path.

load_face(path, device) and FACECalculator(path, device, fused, e_shift) follow
face/calculator.py:10-56: the calculator is built from a training checkpoint (or from a live
model), evaluates energy + forces of one structure in evaluation mode and, as the reference
does on CUDA (face/calculator.py:41-43), tabulates the radial functions with
model.compile_radial() -- for models without CP passes: for FACE-CP the compiled CP radials
are evaluated by a separate spline kernel that writes the (E, 4C) radial rows, which the MLP
route fuses away, so the MLP route is the faster one there (compile_radial=True forces the
tables). Three differences keep every step on the device:

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
import os

import numpy as np
import torch

from .neighbors import build_graph
from .runner import StepGraph

FS = 0.09822694788464063            # 1 fs in ASE time units (Angstrom sqrt(amu / eV))


# Checkpoint switches of face/calculator.py:21-28 and the value this path implements for each
# (the model's defaults); a checkpoint trained with another value raises NotImplementedError.
_TOGGLES = {"standardise": 0, "momnorm": 0, "calib": 0, "calib_ln": 0, "eq_linear": 0, "max_body": 5,
            "elem_proj": 0, "poly": 0, "t3": 0}
# state_dict keys a checkpoint may lack (face/calculator.py:30): buffers and parameters added
# after some checkpoints were written, left at their construction values
_OPTIONAL_KEYS = ("inv_scale", "calibrated", "mom_scale", "eq_scale", "pqs_gate.weight", "tmix3.weight")


def _load_checkpoint(path, device):
    """torch.load with weights_only=True: tensors, containers and primitives only, plus numpy
    scalars and dtypes (the reference stores Eref as a numpy float64, face/train.py:83,161);
    nothing in the file is executed."""
    safe = [np.dtype, type(np.dtype(np.float64))]
    core = getattr(np, "_core", None) or getattr(np, "core")
    safe.append(core.multiarray.scalar)
    with torch.serialization.safe_globals(safe):
        return torch.load(path, map_location=device, weights_only=True)


def load_face(path, device="cuda"):
    """face/calculator.py:10-32: (model in evaluation mode, checkpoint dict) from a training
    checkpoint {"state", "args", "elements" | "E0", "Eref", ...}. The checkpoint is read with
    torch.load(weights_only=True). Raises NotImplementedError for a configuration outside this
    path (factor=False, physics terms, non-default switches)."""
    from .model import FACE, unit_parameterise
    c = _load_checkpoint(path, device)
    a = c["args"]
    terms = [t for t in a.get("terms", "").split(",") if t]
    for k, v in _TOGGLES.items():
        if k in a and a[k] is not None and a[k] != v:
            raise NotImplementedError(f"checkpoint switch {k}={a[k]!r}: this path implements {k}={v!r}")
    m = FACE(c.get("elements", sorted(c.get("E0", {}))), C=a["C"], n_basis=a.get("nbasis", 8), rc=a["rc"],
             n_passes=a["passes"], terms=terms, radial_hidden=a.get("radial_hidden", 64), K_dir=a.get("kdir", 16),
             norm=a.get("norm", "layer"), transport=bool(a.get("transport", 0)), eqmsg=bool(a.get("eqmsg", 0)),
             factor=bool(a.get("factor", 0)), B=a.get("B", 16), K=a.get("K", 32), cp=bool(a.get("cp", 0)))
    m = m.to(device)
    if a.get("unit", 0):
        unit_parameterise(m)
    missing, unexpected = m.load_state_dict(c["state"], strict=False)
    if unexpected or not all(k.endswith(_OPTIONAL_KEYS) for k in missing):
        raise RuntimeError(f"checkpoint does not match the model: missing {missing}, unexpected {unexpected}")
    m.eval()
    return m, c


class FACECalculator:
    """Energy and forces of one structure (positions, Z, cell, pbc) with pair-list reuse.

    path: a checkpoint file (loaded by load_face; its Eref is added to e_shift, as
    face/calculator.py:45) or a FACE model of this package in evaluation mode. fused: kept for
    the reference's signature (this path is always fused); like the reference on CUDA it enables
    the compiled radial tables (compile_radial=None: for models without CP passes)."""

    implemented_properties = ("energy", "forces")

    def __init__(self, path, device="cuda", fused=True, e_shift=0.0, skin=0.5, use_graph=True, tune_gemms=False,
                 compile_radial=None):
        if tune_gemms:                     # library GEMM solutions timed on the first step
            from .runner import tune_library_gemms
            tune_library_gemms()
        e_shift = float(e_shift)
        if isinstance(path, (str, os.PathLike)):
            model, ck = load_face(path, device)
            e_shift += float(ck.get("Eref", 0.0))
        else:
            model = path
        if model.training:
            raise ValueError("FACECalculator needs the model in evaluation mode (model.eval())")
        if skin < 0:
            raise ValueError("skin must be >= 0")
        if compile_radial is None:
            compile_radial = bool(fused) and not any(b.cp for b in model.blocks)
        if compile_radial and getattr(model.blocks[0], "spline", 1) is None:
            model.compile_radial()
        self.model, self.skin, self.use_graph = model, float(skin), bool(use_graph)
        self.rc = float(model.rc)
        self.e_shift = e_shift
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
