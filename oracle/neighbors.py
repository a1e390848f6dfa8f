"""ctypes front of the brute-force pair list (oracle/neighbors.c) and the padded-dense graph
layout of face/neighbors.py:7-37 / face/datasets.py:62-97 (oracle; test infrastructure only).
"""
import ctypes
import os
import subprocess

import numpy as np
import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def build():
    """Compile oracle/neighbors.c (gcc, -ffp-contract=off) into oracle/build/."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "build", "liboracle_nbr.so")
        if not os.path.exists(path):
            build()
        lib = ctypes.CDLL(path)
        lib.oracle_pair_list.restype = ctypes.c_int64
        lib.oracle_pair_list.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p,
                                         ctypes.c_double, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                         ctypes.c_int64]
        lib.oracle_pair_list_cells.restype = ctypes.c_int64
        lib.oracle_pair_list_cells.argtypes = lib.oracle_pair_list.argtypes
        _LIB = lib
    return _LIB


def pair_list(pos, cell, pbc, rc):
    """All (i, j, S) with |pos_j - pos_i + S.cell| < rc (fp64), canonical order (i, j, S-lex).

    pos (n,3) float64, cell (3,3) float64 (rows = lattice vectors), pbc (3,) bool.
    Returns i (E,), j (E,), S (E,3) as int64 numpy arrays.
    """
    return _pairs("oracle_pair_list", pos, cell, pbc, rc)


def pair_list_cells(pos, cell, pbc, rc):
    """pair_list for cells periodic on all three axes in about O(n) time: the same per-pair image
    loop and arithmetic, the j loop narrowed to the atoms of adjacent bins of the fractional
    coordinates (bins no narrower than rc / face distance, so no pair within rc is skipped).
    Raises ValueError unless all three axes are periodic."""
    if not all(bool(b) for b in np.asarray(pbc).reshape(3)):
        raise ValueError("pair_list_cells needs a cell periodic on all three axes")
    return _pairs("oracle_pair_list_cells", pos, cell, pbc, rc)


def _pairs(fn, pos, cell, pbc, rc):
    pos = np.ascontiguousarray(pos, dtype=np.float64)
    cell = np.ascontiguousarray(cell, dtype=np.float64)
    pbc_a = np.ascontiguousarray(np.asarray(pbc, dtype=np.int32).reshape(3))
    n = len(pos)
    f = getattr(_lib(), fn)
    args = (pos.ctypes.data, n, cell.ctypes.data, pbc_a.ctypes.data, float(rc))
    # one pass into a buffer of 96 pairs per atom, a second one sized to the count if that is short
    cap = 0 if fn == "oracle_pair_list" else 96 * n + 1024
    while True:
        oi = np.zeros(cap, np.int32)
        oj = np.zeros(cap, np.int32)
        oS = np.zeros((cap, 3), np.int32)
        E = f(*args, oi.ctypes.data if cap else None, oj.ctypes.data if cap else None,
              oS.ctypes.data if cap else None, cap)
        if E < 0:
            raise RuntimeError(f"{fn} failed ({E})")
        if E <= cap:
            break
        cap = E
    return oi[:E].astype(np.int64), oj[:E].astype(np.int64), oS[:E].astype(np.int64)


def padded_graph(structures, rc, device="cpu", dtype=torch.float32):
    """Padded-dense batch of face/neighbors.py:7-37 from oracle pair lists.

    structures: list of dicts with 'pos' (n,3), 'Z' (n,), 'cell' (3,3), 'pbc' (3,).
    Layout: per structure the pairs sorted by i (canonical within-row order: j, then S),
    slot = rank within the row, M = max row length over the batch, padding slots point at
    the structure's first atom with mask False and zero shift; shift = S @ cell in fp64
    then cast to `dtype`, as the reference does (face/neighbors.py:13,34).
    Also returns the flat pair list ('pairs': i, j (global indices), S).
    """
    rows, off = [], 0
    for st in structures:
        n = len(st["pos"])
        i, j, S = pair_list(st["pos"], st["cell"], st["pbc"], rc)
        sv = S @ np.asarray(st["cell"], dtype=np.float64)
        cnt = np.bincount(i, minlength=n)
        rows.append((n, i, j, S, sv, cnt, off))
        off += n
    M = max(int(r[5].max()) if len(r[5]) else 1 for r in rows)
    N = off
    NB = np.zeros((N, M), np.int64)
    SH = np.zeros((N, M, 3))
    MK = np.zeros((N, M), bool)
    pos, Z, bt, PI, PJ, PS = [], [], [], [], [], []
    for k, (n, i, j, S, sv, cnt, o) in enumerate(rows):
        start = np.concatenate([[0], np.cumsum(cnt)[:-1]])
        slot = np.arange(len(i)) - start[i]
        NB[o + i, slot] = o + j
        SH[o + i, slot] = sv
        MK[o + i, slot] = True
        NB[o:o + n][~MK[o:o + n]] = o
        st = structures[k]
        pos.append(np.asarray(st["pos"], np.float64))
        Z.append(np.asarray(st["Z"]))
        bt.append(np.full(n, k))
        PI.append(i + o); PJ.append(j + o); PS.append(S)
    t = lambda x, dt=dtype: torch.as_tensor(np.asarray(x), device=device, dtype=dt)
    return {"pos": t(np.concatenate(pos)), "Z": t(np.concatenate(Z), torch.long),
            "nbr": t(NB, torch.long), "shift": t(SH), "mask": t(MK, torch.bool),
            "batch": t(np.concatenate(bt), torch.long), "nstr": len(structures),
            "pairs": (np.concatenate(PI), np.concatenate(PJ), np.concatenate(PS))}
