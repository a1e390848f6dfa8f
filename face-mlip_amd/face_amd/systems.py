"""Seeded synthetic systems of the five benchmark workloads.

Geometry streams: numpy SeedSequence(0) spawned into five children, child k drives
workload k, so each workload is reproducible on its own. Structures are dicts
{'pos' (n,3) fp64, 'Z' (n,), 'cell' (3,3), 'pbc' (3,)} accepted by neighbors.build_graph.

  molecules(n_mol)        C9H8O4 molecules in the rMD17 aspirin atom order, 21 atoms drawn
                          uniformly in a 3.5 A ball with >= 1.0 A separation, then N(0, 0.05^2)
                          jitter; each its own non-periodic structure
  fcc(a, n, sigma)        FCC lattice, n^3 conventional cells, N(0, sigma^2) displacement,
                          wrapped into the cubic box (Ag, Z = 47)
  liquid(N, rho, dmin)    H:C:O = 8:9:4 by random sequential addition at number density rho
                          with minimum-image separation dmin in a cubic periodic box
"""
import math

import numpy as np

ASPIRIN_Z = np.array([6, 6, 6, 6, 6, 6, 6, 8, 8, 8, 6, 6, 8, 1, 1, 1, 1, 1, 1, 1, 1])


def stream(k):
    return np.random.default_rng(np.random.SeedSequence(0).spawn(5)[k])


def molecules(n_mol, rng, radius=3.5, dmin=1.0, jitter=0.05):
    out = []
    for _ in range(n_mol):
        pts = []
        while len(pts) < len(ASPIRIN_Z):
            x = rng.uniform(-radius, radius, 3)
            if x @ x > radius * radius:
                continue
            if pts and np.min(np.linalg.norm(np.asarray(pts) - x, axis=1)) < dmin:
                continue
            pts.append(x)
        pos = np.asarray(pts) + rng.normal(0.0, jitter, (len(pts), 3))
        out.append({"pos": pos, "Z": ASPIRIN_Z.copy(), "cell": np.zeros((3, 3)), "pbc": np.zeros(3, bool)})
    return out


def fcc(a, n, sigma, rng, Z=47):
    basis = np.array([[0, 0, 0], [0.5, 0.5, 0], [0.5, 0, 0.5], [0, 0.5, 0.5]])
    grid = np.array([[i, j, k] for i in range(n) for j in range(n) for k in range(n)], dtype=np.float64)
    pos = ((grid[:, None, :] + basis[None]) * a).reshape(-1, 3)
    L = a * n
    pos = np.mod(pos + rng.normal(0.0, sigma, pos.shape), L)
    return {"pos": pos, "Z": np.full(len(pos), Z), "cell": np.eye(3) * L, "pbc": np.ones(3, bool)}


def liquid_counts(N):
    """H, C, O counts for ratio 8:9:4, rounded, adjusted so they sum to N."""
    c = [round(N * f / 21) for f in (8, 9, 4)]
    c[1] += N - sum(c)
    return c


def liquid(N, rng, rho=0.10, dmin=0.9):
    L = (N / rho) ** (1.0 / 3.0)
    nc = max(1, int(L // dmin))
    h = L / nc
    cells = {}
    pos = np.empty((N, 3))
    k = 0
    d2 = dmin * dmin
    while k < N:
        x = rng.random(3) * L
        ci = tuple(int(v // h) % nc for v in x)
        ok = True
        for dx in (-1, 0, 1):
            for dy in (-1, 0, 1):
                for dz in (-1, 0, 1):
                    for j in cells.get(((ci[0] + dx) % nc, (ci[1] + dy) % nc, (ci[2] + dz) % nc), ()):
                        d = pos[j] - x
                        d -= L * np.round(d / L)
                        if d @ d < d2:
                            ok = False
                            break
                    if not ok:
                        break
                if not ok:
                    break
            if not ok:
                break
        if ok:
            pos[k] = x
            cells.setdefault(ci, []).append(k)
            k += 1
    nH, nC, nO = liquid_counts(N)
    Z = rng.permutation(np.concatenate([np.full(nH, 1), np.full(nC, 6), np.full(nO, 8)]))
    return {"pos": pos, "Z": Z, "cell": np.eye(3) * L, "pbc": np.ones(3, bool)}


# ----------------------------------------------------------------------------- workloads
# name -> (structures builder, model kwargs, elements)
FLAGSHIP = dict(n_basis=8, n_passes=2, radial_hidden=64, K_dir=16, norm="layer", transport=True, eqmsg=True,
                factor=True)


def workload(k, n_atoms=None):
    """(structures, model kwargs, elements, description) of benchmark workload k (0..4).

    n_atoms overrides the size for bounded samples: the atom count of the liquids (3, 4), or
    n_atoms // 21 molecules of the molecule batches (0, 1; the first molecules of the full batch)."""
    rng = stream(k)
    if k in (0, 1):
        n_full = 64 if k == 0 else 512
        n_mol = n_full if n_atoms is None else max(1, min(n_full, n_atoms // len(ASPIRIN_Z)))
        mols = molecules(n_mol, rng)
        if k == 0:
            return mols, dict(FLAGSHIP, C=96, B=16, K=32, rc=4.5), [1, 6, 8], \
                f"{n_mol} x C9H8O4 molecules, FACE C96 B16 K32 rc4.5"
        return mols, dict(FLAGSHIP, C=160, B=16, K=32, rc=4.5, cp=True), [1, 6, 8], \
            f"{n_mol} x C9H8O4 molecules, FACE-CP C160 B16 rc4.5"
    if k == 2:
        return [fcc(4.09, 6, 0.1, rng)], dict(FLAGSHIP, C=96, B=16, K=32, rc=4.5), [47], \
            "FCC Ag 6x6x6 (864 atoms), FACE C96 B16 K32 rc4.5"
    if k == 3:
        N = n_atoms or 24000
        return [liquid(N, rng)], dict(FLAGSHIP, C=160, B=16, K=32, rc=5.0, cp=True), [1, 6, 8], \
            f"H:C:O 8:9:4 liquid, {N} atoms, rho 0.10, FACE-CP C160 B16 rc5.0"
    if k == 4:
        N = n_atoms or 100000
        return [liquid(N, rng)], dict(FLAGSHIP, C=256, B=16, K=64, rc=5.5), [1, 6, 8], \
            f"H:C:O 8:9:4 liquid, {N} atoms, rho 0.10, FACE C256 B16 K64 rc5.5"
    raise ValueError(k)
