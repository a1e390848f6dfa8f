"""Checkpoint loading (face/calculator.py:10-44): load_face / FACECalculator(path) read a training
checkpoint with torch.load(weights_only=True) into this package's FACE. CPU: the weights land
bit for bit (reference-written state of a golden case), Eref reaches the energy shift, unsafe or
unsupported checkpoints are refused. GPU: the loaded model reproduces the golden E/F."""
import os
import pickle

import numpy as np
import pytest
import torch

from golden.cases import SMALL_CASES

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASE = "small_flag_mol"


def _args(kw):
    """Training-script arguments (face/train.py) of a golden case's model settings."""
    return {"C": kw["C"], "nbasis": kw["n_basis"], "rc": kw["rc"], "passes": kw["n_passes"], "terms": "",
            "radial_hidden": kw["radial_hidden"], "kdir": kw["K_dir"], "norm": kw["norm"],
            "transport": int(kw["transport"]), "eqmsg": int(kw["eqmsg"]), "factor": int(kw["factor"]),
            "B": kw["B"], "K": kw["K"], "cp": int(kw.get("cp", False)), "unit": 1, "standardise": 0,
            "momnorm": 0, "calib": 0, "eq_linear": 0, "max_body": 5, "elem_proj": 0, "poly": 0, "t3": 0,
            "seed": 0, "dtype": "float32"}


def _write(path, case=CASE, dtype="f32", **extra_args):
    kw, el, _ = SMALL_CASES[case]
    d = np.load(os.path.join(GOLD, f"{case}_{dtype}.npz"))
    state = {str(k): torch.as_tensor(d["state/" + str(k)]) for k in d["state_keys"]}
    ck = {"state": state, "args": dict(_args(kw), **extra_args), "elements": el, "Eref": np.float64(-123.25),
          "epoch": 7}
    torch.save(ck, path)
    return d, state


def test_load_face_restores_reference_state(tmp_path):
    from face_amd.calculator import load_face
    path = tmp_path / "ck.pt"
    d, state = _write(path)
    m, ck = load_face(str(path), device="cpu")
    assert not m.training
    sd = m.state_dict()
    assert list(sd) == [str(k) for k in d["state_keys"]]              # registration order as the reference
    for k, v in state.items():
        assert torch.equal(sd[k], v), k
    assert float(ck["Eref"]) == -123.25


def test_calculator_from_path_adds_eref(tmp_path):
    from face_amd.calculator import FACECalculator
    path = tmp_path / "ck.pt"
    _write(path)
    calc = FACECalculator(str(path), device="cpu", e_shift=0.5, compile_radial=False)
    assert calc.e_shift == pytest.approx(0.5 - 123.25)
    assert calc.model.blocks[0].spline is None
    # default: compiled radial tables for models without CP passes (the reference's CUDA setting)
    calc2 = FACECalculator(str(path), device="cpu")
    assert calc2.model.blocks[0].spline is not None


def test_cp_checkpoint_keeps_the_mlp_radial_by_default(tmp_path):
    from face_amd.calculator import FACECalculator
    path = tmp_path / "ck.pt"
    _write(path, case="small_cp_mol")
    calc = FACECalculator(str(path), device="cpu")
    assert calc.model.blocks[0].cp and calc.model.blocks[0].spline is None


class _Payload:
    def __reduce__(self):
        return (os.getcwd, ())


def test_unsafe_checkpoint_is_refused(tmp_path):
    from face_amd.calculator import load_face
    path = tmp_path / "bad.pt"
    torch.save({"args": {"C": 8}, "state": {}, "x": _Payload()}, path)
    with pytest.raises(pickle.UnpicklingError):
        load_face(str(path), device="cpu")


@pytest.mark.parametrize("switch,value", [("momnorm", 1), ("max_body", 3), ("poly", 1), ("t3", 1)])
def test_unsupported_switch_is_refused(tmp_path, switch, value):
    from face_amd.calculator import load_face
    path = tmp_path / "ck.pt"
    _write(path, **{switch: value})
    with pytest.raises(NotImplementedError):
        load_face(str(path), device="cpu")


@pytest.mark.gpu
def test_loaded_checkpoint_matches_golden(tmp_path):
    from face_amd.calculator import load_face
    path = tmp_path / "ck.pt"
    d, _ = _write(path)
    m, _ = load_face(str(path), device="cuda")
    t = lambda k, dt=None: torch.as_tensor(d[k], device="cuda", dtype=dt)
    o = m({"pos": t("pos", torch.float32), "Z": t("Z"), "nbr": t("nbr"), "shift": t("shift", torch.float32),
           "mask": t("mask"), "batch": t("batch")})
    E, F = o["energy"].detach().cpu().double().numpy(), o["forces"].detach().cpu().double().numpy()
    assert np.abs(E - d["energy"]).max() <= 1e-5 * np.abs(d["energy"]).max()
    assert np.abs(F - d["forces"]).max() <= 1e-4 * np.sqrt((d["forces"].astype(np.float64) ** 2).mean())
