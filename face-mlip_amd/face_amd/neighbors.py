"""GPU pair-list build: replaces face/neighbors.py (ASE neighbor_list on the CPU).

build_graph(...) returns the receiver-grouped CSR `Graph` the model consumes;
padded_graph(atoms_list, rc, ...) keeps the reference's signature and dict layout
(face/neighbors.py:7-37) and adds the CSR graph under the key "csr".

Pair set: ASE neighbor_list("ijS") semantics (face/neighbors.py:12): |pos_j - pos_i + S.cell| < rc
in fp64, integer S (0 on non-periodic axes), (i,i,0) excluded. Rows are ordered by (j, S);
ASE's own within-row order comes from an unstable sort and is not reproduced.
Shift vectors are fp32(S.cell) with S.cell formed in fp64 (face/neighbors.py:13,34).
"""
import math

import numpy as np
import torch

from . import _lib
from ._lib import call, ptr
from .ops import Graph

# Structures with more atoms than this that are periodic on all three axes use the cell list;
# all others use the all-pairs generator of their own structure.
CELL_LIST_MIN_ATOMS = 128


def _as_struct(s):
    """dict {'pos','Z','cell','pbc'} or an ASE-like object -> (pos f64 (n,3), Z, cell (3,3), pbc (3,))."""
    if isinstance(s, dict):
        pos, Z, cell, pbc = s["pos"], s["Z"], s.get("cell"), s.get("pbc", False)
    else:
        pos, Z, cell, pbc = s.positions, s.numbers, s.cell, s.pbc
    cell = getattr(cell, "array", cell)
    cell = np.zeros((3, 3)) if cell is None else np.asarray(cell, dtype=np.float64).reshape(3, 3)
    pbc = np.broadcast_to(np.asarray(pbc, dtype=bool), (3,)).copy()
    return np.asarray(pos, dtype=np.float64).reshape(-1, 3), np.asarray(Z, dtype=np.int64), cell, pbc


def _inv_cell(cell, pbc):
    return np.linalg.inv(cell) if pbc.any() else np.zeros((3, 3))


def _grid(cell, rc):
    """Bins per axis (each >= rc wide along its reciprocal axis) and bins searched per side."""
    inv = np.linalg.inv(cell)
    fd = 1.0 / np.linalg.norm(inv, axis=0)            # face distances (reciprocal axes = columns)
    nb = np.maximum(1, np.floor(fd / rc).astype(np.int64))
    while nb.prod() > (1 << 22):
        nb = np.maximum(1, nb // 2)
    s = np.ceil(rc * nb / fd - 1e-12).astype(np.int64)
    s = np.maximum(s, 1)
    return [int(x) for x in nb] + [int(x) for x in s]


def _build_one_cell_list(pos64, cell, rc, dev, st):
    """CSR rows for one fully periodic structure with the cell-list generator."""
    N = pos64.shape[0]
    nbh = _grid(cell, rc)
    nb_arr = (_lib.I32 * 6)(*nbh)
    nbins = nbh[0] * nbh[1] * nbh[2]
    cell_d = torch.as_tensor(cell.reshape(9), dtype=torch.float64, device=dev)
    inv_d = torch.as_tensor(np.linalg.inv(cell).reshape(9), dtype=torch.float64, device=dev)
    i32 = dict(dtype=torch.int32, device=dev)
    bin_of = torch.empty(N, **i32)
    wrap = torch.empty(N, 3, **i32)
    bin_count = torch.empty(nbins, **i32)
    bin_start = torch.empty(nbins + 1, **i32)
    bin_fill = torch.empty(nbins, **i32)
    bin_atoms = torch.empty(N, **i32)
    call("face_nbr_bin", ptr(pos64), N, ptr(inv_d), nb_arr, ptr(bin_of), ptr(wrap), ptr(bin_count), ptr(bin_start),
         ptr(bin_fill), ptr(bin_atoms), st)
    counts = torch.empty(N, **i32)
    call("face_nbr_count", ptr(pos64), N, None, None, ptr(cell_d), None, None, float(rc), nb_arr, ptr(bin_of),
         ptr(wrap), ptr(bin_start), ptr(bin_atoms), ptr(counts), st)
    row_ptr = torch.zeros(N + 1, **i32)
    row_ptr[1:] = torch.cumsum(counts, 0)
    E = int(row_ptr[-1])
    key = torch.empty(E, dtype=torch.int64, device=dev)
    col = torch.empty(E, **i32)
    S = torch.empty(E, 3, **i32)
    shift = torch.empty(E, 3, dtype=torch.float32, device=dev)
    overflow = torch.zeros(1, **i32)
    call("face_nbr_fill", ptr(pos64), N, None, None, ptr(cell_d), None, None, float(rc), nb_arr, ptr(bin_of),
         ptr(wrap), ptr(bin_start), ptr(bin_atoms), ptr(row_ptr), ptr(key), ptr(col), ptr(S), ptr(shift),
         ptr(overflow), st)
    return counts, row_ptr, col, S, shift, overflow


def _build_small(pos64, sizes, cells, pbcs, rc, dev, st):
    """CSR rows for a batch of structures with the all-pairs generator."""
    N = pos64.shape[0]
    nstr = len(sizes)
    i32 = dict(dtype=torch.int32, device=dev)
    sp = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    struct_ptr = torch.as_tensor(sp, **i32)
    atom_struct = torch.as_tensor(np.repeat(np.arange(nstr, dtype=np.int32), sizes), **i32)
    cell_d = torch.as_tensor(np.stack(cells).reshape(nstr, 9), dtype=torch.float64, device=dev)
    inv_d = torch.as_tensor(np.stack([_inv_cell(c, p) for c, p in zip(cells, pbcs)]).reshape(nstr, 9),
                            dtype=torch.float64, device=dev)
    pbc_d = torch.as_tensor(np.stack(pbcs).astype(np.int32), **i32)
    counts = torch.empty(N, **i32)
    call("face_nbr_count", ptr(pos64), N, ptr(atom_struct), ptr(struct_ptr), ptr(cell_d), ptr(inv_d), ptr(pbc_d),
         float(rc), None, None, None, None, None, ptr(counts), st)
    row_ptr = torch.zeros(N + 1, **i32)
    row_ptr[1:] = torch.cumsum(counts, 0)
    E = int(row_ptr[-1])
    col = torch.empty(E, **i32)
    S = torch.empty(E, 3, **i32)
    shift = torch.empty(E, 3, dtype=torch.float32, device=dev)
    overflow = torch.zeros(1, **i32)
    call("face_nbr_fill", ptr(pos64), N, ptr(atom_struct), ptr(struct_ptr), ptr(cell_d), ptr(inv_d), ptr(pbc_d),
         float(rc), None, None, None, None, None, ptr(row_ptr), None, ptr(col), ptr(S), ptr(shift), ptr(overflow), st)
    return counts, row_ptr, col, S, shift, overflow


def _check_image_span(pos, cell, pbc, rc):
    """Refuses inputs whose image search would be unbounded (non-finite or absurdly far
    unwrapped coordinates) before any kernel walks it."""
    if not np.isfinite(pos).all():
        raise ValueError("positions must be finite")
    if pbc.any():
        inv = np.linalg.inv(cell)
        f = pos @ inv
        span = (f.max(0) - f.min(0)) + 2 * rc * np.linalg.norm(inv, axis=0)
        if (span[pbc] > 256).any():
            raise ValueError("periodic structure spans more than 256 cells: wrap the positions first")


def build_graph(structures, rc, device="cuda", dtype=torch.float32, method="auto"):
    """Pair lists of a batch of structures on the GPU -> CSR Graph.

    structures: list of dicts {'pos','Z','cell','pbc'} or ASE-like objects.
    method: "auto" (cell list for structures above CELL_LIST_MIN_ATOMS atoms that are periodic
    on every axis, all-pairs otherwise), "cell" (cell list for every structure; each must be
    periodic on every axis) or "small" (all-pairs for every structure).
    """
    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError("build_graph needs a HIP device; there is no CPU path")
    if method not in ("auto", "cell", "small"):
        raise ValueError(method)
    parts = [_as_struct(s) for s in structures]
    for p in parts:
        _check_image_span(p[0], p[2], p[3], rc)
    sizes = [len(p[0]) for p in parts]
    nstr = len(parts)
    pos_np = np.concatenate([p[0] for p in parts]) if parts else np.zeros((0, 3))
    Z_np = np.concatenate([p[1] for p in parts]) if parts else np.zeros(0, np.int64)
    N = len(pos_np)
    pos64 = torch.as_tensor(pos_np, dtype=torch.float64, device=dev)
    st = _lib.stream_of(pos64)
    if method == "cell":
        if not all(p[3].all() for p in parts):
            raise ValueError("method='cell' needs structures periodic on every axis")
        big = list(range(nstr))
    elif method == "small":
        big = []
    else:
        big = [k for k, p in enumerate(parts) if sizes[k] > CELL_LIST_MIN_ATOMS and p[3].all()]
    i32 = dict(dtype=torch.int32, device=dev)
    if not big:
        counts, row_ptr, col, S, shift, overflow = _build_small(pos64, sizes, [p[2] for p in parts],
                                                                [p[3] for p in parts], rc, dev, st)
    else:
        # every structure separately (cell list where it applies), then stitched with offsets
        off = np.concatenate([[0], np.cumsum(sizes)])
        pieces = []
        for k, (p, n) in enumerate(zip(parts, sizes)):
            sl = pos64[off[k]:off[k] + n]
            if k in big:
                pieces.append(_build_one_cell_list(sl.contiguous(), p[2], rc, dev, st))
            else:
                pieces.append(_build_small(sl.contiguous(), [n], [p[2]], [p[3]], rc, dev, st))
        counts = torch.cat([q[0] for q in pieces])
        col = torch.cat([q[2] + int(off[k]) for k, q in enumerate(pieces)])
        S = torch.cat([q[3] for q in pieces])
        shift = torch.cat([q[4] for q in pieces])
        overflow = sum(q[5] for q in pieces)
        row_ptr = torch.zeros(N + 1, **i32)
        row_ptr[1:] = torch.cumsum(counts, 0)
    E = col.shape[0]
    rev = torch.empty(E, **i32)
    missing = torch.zeros(1, **i32)
    call("face_nbr_rev", ptr(row_ptr), ptr(col), ptr(S), N, ptr(rev), ptr(missing), st)
    if int(overflow.item()) != 0:
        raise RuntimeError("pair-list build: a row overflowed its counted size")
    if int(missing.item()) != 0:
        raise RuntimeError("pair-list build: pair list is not symmetric")
    max_row = int(counts.max()) if N else 0
    recv = torch.repeat_interleave(torch.arange(N, device=dev, dtype=torch.int32), counts.long(), output_size=E)
    batch = torch.as_tensor(np.repeat(np.arange(nstr), sizes), dtype=torch.long, device=dev)
    struct_ptr = torch.as_tensor(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32), **i32)
    return Graph(pos64.to(dtype), torch.as_tensor(Z_np, dtype=torch.long, device=dev), batch, nstr, struct_ptr,
                 row_ptr, col, recv, shift.to(dtype), rev, max_row, S)


def padded_view(graph):
    """Padded-dense tensors of face/neighbors.py:27-33 from a CSR graph: nbr (N,M) int64
    (padding -> first atom of the structure), shift (N,M,3), mask (N,M) bool."""
    N, M = graph.N, graph.max_row
    dev = graph.pos.device
    nbr = torch.empty(N, M, dtype=torch.long, device=dev)
    sh = torch.empty(N, M, 3, dtype=torch.float32, device=dev)
    mask = torch.empty(N, M, dtype=torch.uint8, device=dev)
    atom_struct = graph.batch.to(torch.int32)
    call("face_nbr_padded", ptr(graph.row_ptr), ptr(graph.col), ptr(graph.shift), ptr(atom_struct),
         ptr(graph.struct_ptr), N, M, ptr(nbr), ptr(sh), ptr(mask), _lib.stream_of(sh))
    return nbr, sh, mask.bool()


def padded_graph(atoms_list, rc, device="cuda", dtype=torch.float32, skin=0.0):
    """face/neighbors.py:7-37 signature: padded-dense graph dict, built on the GPU.

    Keys pos, Z, nbr, shift, mask, batch as in the reference, plus "nstr" and "csr" (the
    Graph the face_amd model consumes directly)."""
    g = build_graph(atoms_list, rc + skin, device, dtype)
    nbr, sh, mask = padded_view(g)
    return {"pos": g.pos, "Z": g.Z, "nbr": nbr, "shift": sh.to(dtype), "mask": mask, "batch": g.batch,
            "nstr": g.nstr, "csr": g}


def graph_from_padded(g):
    """CSR Graph from a reference-layout padded dict (pos, Z, nbr, shift, mask, batch)."""
    pos, nbr, mask, shift = g["pos"], g["nbr"], g["mask"], g["shift"]
    dev = pos.device
    N = pos.shape[0]
    i32 = dict(dtype=torch.int32, device=dev)
    counts = mask.sum(1).to(torch.int32)
    row_ptr = torch.zeros(N + 1, **i32)
    row_ptr[1:] = torch.cumsum(counts, 0)
    ii, mm = mask.nonzero(as_tuple=True)                           # row-major = receiver grouped
    col = nbr[ii, mm].to(torch.int32)
    sh = shift[ii, mm].float().contiguous()
    E = col.shape[0]
    rev = torch.empty(E, **i32)
    missing = torch.zeros(1, **i32)
    call("face_nbr_rev_shift", ptr(row_ptr), ptr(col), ptr(sh), N, ptr(rev), ptr(missing), _lib.stream_of(sh))
    batch = g["batch"]
    # per-structure energies are sums over contiguous atom ranges (struct_ptr), so the atoms of
    # each structure must be contiguous and in structure order: checked with the same host read
    unsorted = (batch[1:] < batch[:-1]).sum().to(torch.int32).view(1) if N > 1 else torch.zeros_like(missing)
    flags = torch.cat([missing, unsorted]).tolist()
    if flags[0] != 0:
        raise RuntimeError("padded graph is not symmetric: the force scatter needs every reverse pair")
    if flags[1] != 0:
        raise ValueError("padded graph: 'batch' must be non-decreasing (the atoms of each structure contiguous, "
                         "structures in order)")
    nstr = int(g["nstr"]) if "nstr" in g else int(batch.max()) + 1
    sizes = torch.bincount(batch, minlength=nstr)
    struct_ptr = torch.zeros(nstr + 1, **i32)
    struct_ptr[1:] = torch.cumsum(sizes, 0)
    return Graph(pos, g["Z"], batch, nstr, struct_ptr, row_ptr, col, ii.to(torch.int32), sh, rev,
                 int(counts.max()) if N else 0)
