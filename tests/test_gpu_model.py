"""Model-level parity on the GPU: energies within 1e-5 relative and forces within
1e-4 x RMS(F) max-abs of the reference torch path (golden vectors written from the
reference itself) and of the CPU oracle at benchmark shapes."""
import os
import sys

import numpy as np
import pytest
import torch

from golden.cases import BIG_CASES, SMALL_CASES

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
E_TOL, F_TOL = 1e-5, 1e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def product_model(kw, elements, seed=0):
    from face_amd import model as fm
    torch.manual_seed(seed)
    m = fm.FACE(elements, **kw)
    fm.unit_parameterise(m)
    return m.cuda().eval()


def check(E, F, Eg, Fg):
    E, F = np.asarray(E, np.float64), np.asarray(F, np.float64)
    dE = np.abs(E - Eg).max() / np.abs(Eg).max()
    rms = np.sqrt((np.asarray(Fg, np.float64) ** 2).mean())
    dF = np.abs(F - Fg).max() / rms
    assert dE <= E_TOL and dF <= F_TOL, (dE, dF)
    return dE, dF


def golden_graph(d):
    t = lambda k, dt=None: torch.as_tensor(d[k], device="cuda", dtype=dt)
    return {"pos": t("pos", torch.float32), "Z": t("Z"), "nbr": t("nbr"), "shift": t("shift", torch.float32),
            "mask": t("mask"), "batch": t("batch")}


@pytest.mark.parametrize("name", list(SMALL_CASES) + list(BIG_CASES))
def test_energy_forces_match_reference_golden(name):
    kw, el, _ = (SMALL_CASES if name in SMALL_CASES else BIG_CASES)[name]
    say("golden", name)
    d = np.load(os.path.join(GOLD, f"{name}_f32.npz"))
    m = product_model(kw, el)
    o = m(golden_graph(d))
    dE, dF = check(o["energy"].detach().cpu(), o["forces"].detach().cpu(), d["energy"], d["forces"])
    say(f"  dE/E {dE:.2e}  max|dF|/rms {dF:.2e}")
    # a second, freshly built dict of the same structures (its CSR graph built again): the same
    # forces bit for bit (fixed summation order, no atomics)
    o2 = m(golden_graph(d))
    assert torch.equal(o["forces"], o2["forces"])               # bitwise reproducible


def test_gpu_graph_path_equals_padded_path():
    from face_amd import systems
    from face_amd.neighbors import padded_graph, build_graph
    say("graph paths")
    kw, el, _ = SMALL_CASES["small_flag_mol"]
    m = product_model(kw, el)
    sts = systems.molecules(3, np.random.default_rng(2))
    g = padded_graph(sts, kw["rc"])
    o1 = m({k: g[k] for k in ("pos", "Z", "nbr", "shift", "mask", "batch")})
    o2 = m(g)
    o3 = m(build_graph(sts, kw["rc"]))
    for o in (o2, o3):
        assert torch.allclose(o["energy"], o1["energy"], rtol=1e-6, atol=0)
        assert (o["forces"] - o1["forces"]).abs().max() <= 1e-5 * o1["forces"].abs().max()


def _oracle_EF(structures, kw, el):
    from oracle import model as om
    from oracle.neighbors import padded_graph as opad
    torch.manual_seed(0)
    m = om.FACE(el, **kw)
    om.unit_parameterise(m)
    g = opad(structures, kw["rc"])
    o = m({k: g[k] for k in ("pos", "Z", "nbr", "shift", "mask", "batch")})
    return o["energy"].detach().numpy(), o["forces"].detach().numpy()


@pytest.mark.parametrize("k,n_atoms,n_mol", [(0, None, None), (1, None, 48), (2, None, None), (3, 1500, None),
                                             (4, 1200, None)])
def test_workload_shapes_match_oracle(k, n_atoms, n_mol):
    """Benchmark models (C96/C160/C256, seed 0) on the benchmark recipes; liquids and the CP
    molecule batch are cut to sizes the CPU oracle finishes in seconds."""
    from face_amd import systems
    from face_amd.neighbors import build_graph
    sts, kw, el, desc = systems.workload(k, n_atoms=n_atoms)
    if n_mol:
        sts = sts[:n_mol]
    say("workload", k, desc, "atoms", sum(len(s["pos"]) for s in sts))
    m = product_model(kw, el)
    o = m(build_graph(sts, kw["rc"]))
    Eo, Fo = _oracle_EF(sts, kw, el)
    dE, dF = check(o["energy"].detach().cpu(), o["forces"].detach().cpu(), Eo, Fo)
    say(f"  dE/E {dE:.2e}  max|dF|/rms {dF:.2e}")


@pytest.mark.parametrize("k,n_atoms", [(3, 1500), (2, None)])
def test_workload_matches_oracle_with_tuned_library_gemms(k, n_atoms, tmp_path):
    """The benchmark's setting for the GEMMs left to the libraries (PyTorch TunableOp picking among
    fp32 hipBLASLt / rocBLAS solutions, numerical check on): same parity bar as above."""
    import torch.cuda.tunable as tun
    from face_amd import systems
    from face_amd.neighbors import build_graph
    sts, kw, el, desc = systems.workload(k, n_atoms=n_atoms)
    say("tuned library GEMMs", k, desc)
    tun.enable(True)
    tun.set_filename(str(tmp_path / "tunableop.csv"))
    tun.set_numerical_check_tolerances(True, 1e-5, 1e-5)
    try:
        m = product_model(kw, el)
        g = build_graph(sts, kw["rc"])
        m(g)                                                     # tunes every GEMM shape
        o = m(g)
    finally:
        tun.enable(False)
    Eo, Fo = _oracle_EF(sts, kw, el)
    dE, dF = check(o["energy"].detach().cpu(), o["forces"].detach().cpu(), Eo, Fo)
    say(f"  dE/E {dE:.2e}  max|dF|/rms {dF:.2e}")


@pytest.mark.parametrize("name", ["small_flag_box", "small_cp_mol", "cfg2_flag_ag", "cfg3_cp_c160"])
def test_compiled_radial_matches_oracle(name):
    """FACE.compile_radial() (face/model.py:644-655; the reference calculator's CUDA setting): tables
    built on the GPU (fp64, stored fp32), splines evaluated by the HIP kernel, against the oracle
    model in fp64 with its own tables (reverse-mode derivatives as the reference builds them),
    stored in fp32 as well: same hot-path bar as the MLP path."""
    from oracle import model as om
    kw, el, _ = (SMALL_CASES if name in SMALL_CASES else BIG_CASES)[name]
    say("compiled radial", name)
    d = np.load(os.path.join(GOLD, f"{name}_f32.npz"))
    m = product_model(kw, el).compile_radial()
    o = m(golden_graph(d))
    torch.manual_seed(0)
    mo = om.FACE(el, **kw)
    om.unit_parameterise(mo)
    mo = mo.double().eval().compile_radial(store_dtype=torch.float32)
    t = lambda k, dt=None: torch.as_tensor(d[k], dtype=dt)
    g = {"pos": t("pos", torch.float64), "Z": t("Z"), "nbr": t("nbr"), "shift": t("shift", torch.float64),
         "mask": t("mask"), "batch": t("batch")}
    oo = mo(g)
    dE, dF = check(o["energy"].detach().cpu(), o["forces"].detach().cpu(), oo["energy"].detach().numpy(),
                   oo["forces"].detach().numpy())
    say(f"  dE/E {dE:.2e}  max|dF|/rms {dF:.2e}")
    # back to the radial MLP: the golden reference values again
    m.compile_radial(on=False)
    o2 = m(golden_graph(d))
    check(o2["energy"].detach().cpu(), o2["forces"].detach().cpu(), d["energy"], d["forces"])


@pytest.mark.parametrize("cp,compiled", [(False, False), (True, False), (False, True), (True, True)])
def test_isolated_atoms_and_empty_rows(cp, compiled):
    """Two molecules and two far-away single atoms (rows without pairs: their densities are zero,
    their energies the readout of the embedding alone) in one batch, against the oracle."""
    from face_amd import systems
    from face_amd.neighbors import build_graph
    from oracle import model as om
    from oracle.neighbors import padded_graph as opad
    say("isolated atoms", cp, compiled)
    sts = systems.molecules(2, np.random.default_rng(11))
    for z, p in ((8, (40.0, 0.0, 0.0)), (1, (0.0, 45.0, 3.0))):
        sts.append({"pos": np.array([p]), "Z": np.array([z]), "cell": np.zeros((3, 3)), "pbc": np.zeros(3, bool)})
    kw = dict(C=32, transport=True, eqmsg=True, factor=True, B=16, K=32, rc=4.5, cp=cp)
    m = product_model(kw, [1, 6, 8])
    if compiled:
        m.compile_radial()
    o = m(build_graph(sts, kw["rc"]))
    torch.manual_seed(0)
    mo = om.FACE([1, 6, 8], **kw)
    om.unit_parameterise(mo)
    mo = mo.double().eval()
    if compiled:
        mo.compile_radial(store_dtype=torch.float32)
    g = opad(sts, kw["rc"], dtype=torch.float64)
    oo = mo({k: g[k] for k in ("pos", "Z", "nbr", "shift", "mask", "batch")})
    check(o["energy"].detach().cpu(), o["forces"].detach().cpu(), oo["energy"].detach().numpy(),
          oo["forces"].detach().numpy())
    assert float(o["forces"][-2:].abs().max()) == 0.0                 # no pairs: no force


def test_compiled_radial_close_to_mlp_model():
    """face/tests/test_kernels.py:38-54 (check_spline): perturbed flagship C32 model, compiled radial
    against the radial MLP on the same structures: |dE| < 1e-5 eV/atom, rel ||dF|| < 1e-3."""
    from face_amd import systems
    from face_amd.neighbors import build_graph
    say("compiled vs MLP")
    kw = dict(C=32, transport=True, eqmsg=True, factor=True, B=16, K=32, rc=5.0)
    m = product_model(kw, [1, 6, 8])
    g0 = torch.Generator(device="cuda").manual_seed(0)
    with torch.no_grad():
        for p in m.parameters():
            p.add_(0.05 * torch.randn(p.shape, generator=g0, device="cuda"))
    sts, _, _, _ = systems.workload(3, n_atoms=400)
    g = build_graph(sts, kw["rc"])
    o1 = m(g)
    o2 = m.compile_radial()(g)
    m.compile_radial(on=False)
    dE = (o1["energy"] - o2["energy"]).abs().item() / g.N
    dF = ((o1["forces"] - o2["forces"]).norm() / o1["forces"].norm()).item()
    say(f"  |dE| {dE:.1e} eV/atom  rel |dF| {dF:.1e}")
    assert dE < 1e-5 and dF < 1e-3, (dE, dF)


def test_forces_are_minus_energy_gradient_fd():
    """Central differences of the GPU energy (fp32, h = 1e-2 A on a smooth small model)."""
    from face_amd.neighbors import build_graph
    from face_amd import systems
    say("finite differences")
    kw, el, _ = SMALL_CASES["small_flag_mol"]
    m = product_model(kw, el)
    st = systems.molecules(1, np.random.default_rng(12))
    o = m(build_graph(st, kw["rc"]))
    F = o["forces"].detach().cpu().numpy()
    h = 1e-2
    for i, c in [(0, 0), (5, 1), (17, 2)]:
        vals = []
        for sgn in (1, -1):
            s2 = [dict(st[0], pos=st[0]["pos"].copy())]
            s2[0]["pos"][i, c] += sgn * h
            vals.append(m(build_graph(s2, kw["rc"]), forces=False)["energy"].item())
        fd = -(vals[0] - vals[1]) / (2 * h)
        assert abs(fd - F[i, c]) < 2e-3 * (1 + abs(F[i, c])), (fd, F[i, c])


@pytest.mark.parametrize("case", ["small_flag_mol", "cfg2", "cfg3_compiled"])
def test_graph_replay_matches_eager(case):
    """HIP-graph replays with new positions, eager work in between, every replay checked.
    cfg3_compiled: the CP liquid (cut to 1000 atoms) with compiled radial tables, whose size
    (193 MB) makes each step sort the edges by table cell inside the captured graph."""
    from face_amd import systems
    from face_amd.neighbors import build_graph
    from face_amd.runner import StepGraph
    say("graph replay", case)
    if case == "cfg2":
        sts, kw, el, _ = systems.workload(2)
    elif case == "cfg3_compiled":
        sts, kw, el, _ = systems.workload(3, n_atoms=1000)
    else:
        kw, el, _ = SMALL_CASES[case]
        sts = systems.molecules(4, np.random.default_rng(3))
    m = product_model(kw, el)
    if case == "cfg3_compiled":
        from face_amd import ops
        m.compile_radial()
        assert ops.spline_wants_order(m.blocks[0].spline.T)
    g = build_graph(sts, kw["rc"])
    run = StepGraph(m, g)
    gen = torch.Generator(device="cuda").manual_seed(0)
    for k in range(4):
        pos = g.pos + 0.01 * torch.randn(g.pos.shape, device="cuda", generator=gen)
        E1, F1 = run(pos)
        E1, F1 = E1.clone(), F1.clone()
        o = m(g.with_pos(pos.clone()))                         # eager work between replays
        torch.cuda.synchronize()
        assert torch.allclose(E1, o["energy"], rtol=1e-6, atol=0), (k, E1, o["energy"])
        assert (F1 - o["forces"]).abs().max() <= 1e-5 * o["forces"].abs().max(), k


def _repad(g, M):
    """A padded dict (oracle layout) widened to M slots: extra slots masked, pointing at the
    structure's first atom with zero shift (face/neighbors.py:27-32), moved to the GPU."""
    N, M0 = g["nbr"].shape
    nbr = torch.empty(N, M, dtype=torch.long)
    starts = torch.cat([torch.zeros(1, dtype=torch.long), torch.cumsum(torch.bincount(g["batch"]), 0)[:-1]])
    first = starts[g["batch"]]
    nbr[:] = first[:, None]
    nbr[:, :M0] = g["nbr"]
    sh = torch.zeros(N, M, 3)
    sh[:, :M0] = g["shift"]
    mk = torch.zeros(N, M, dtype=torch.bool)
    mk[:, :M0] = g["mask"]
    c = lambda t: t.to("cuda")
    return {"pos": c(g["pos"]), "Z": c(g["Z"]), "nbr": c(nbr), "shift": c(sh), "mask": c(mk), "batch": c(g["batch"])}


def _crossing_variant(sts, rc, rng):
    """A copy of the structures in which one pair of molecule 0 moves from just inside rc to just
    outside it, and one hydrogen becomes an oxygen."""
    s2 = [dict(s, pos=s["pos"].copy(), Z=s["Z"].copy()) for s in sts]
    p = s2[0]["pos"]
    d = np.linalg.norm(p[:, None] - p[None], axis=-1)
    i, j = np.argwhere((d > rc - 0.6) & (d < rc))[0]
    u = (p[j] - p[i]) / d[i, j]
    p[j] += (rc + 0.02 - d[i, j]) * u
    h = np.nonzero(s2[1]["Z"] == 1)[0][0]
    s2[1]["Z"][h] = 8
    return s2


def test_fresh_same_shape_padded_dicts_are_not_confused():
    """The reference calculator builds a new padded dict on every call (face/calculator.py:52). Two
    same-shape dicts built one after the other, the first freed in between, that differ in one pair
    crossing rc and in one species, each match the oracle; then a short MD-like loop of fresh dicts
    with moving atoms."""
    from face_amd import systems
    from oracle.neighbors import padded_graph as opad
    say("fresh padded dicts")
    kw = dict(C=32, transport=True, eqmsg=True, factor=True, B=16, K=32, rc=4.5)
    el = [1, 6, 8]
    rng = np.random.default_rng(21)
    sts_a = systems.molecules(2, rng)
    sts_b = _crossing_variant(sts_a, kw["rc"], rng)
    ga, gb = opad(sts_a, kw["rc"]), opad(sts_b, kw["rc"])
    M = max(ga["nbr"].shape[1], gb["nbr"].shape[1]) + 1
    assert int(ga["mask"].sum()) != int(gb["mask"].sum())             # a pair crossed rc
    m = product_model(kw, el)
    da = _repad(ga, M)
    oa = m(da)
    check(oa["energy"].detach().cpu(), oa["forces"].detach().cpu(), *_oracle_EF(sts_a, kw, el))
    shapes = {k: tuple(v.shape) for k, v in da.items()}
    del da
    db = _repad(gb, M)
    assert {k: tuple(v.shape) for k, v in db.items()} == shapes
    ob = m(db)
    Eb, Fb = _oracle_EF(sts_b, kw, el)
    dE, dF = check(ob["energy"].detach().cpu(), ob["forces"].detach().cpu(), Eb, Fb)
    say(f"  second dict: dE/E {dE:.2e}  max|dF|/rms {dF:.2e}")
    del db
    # MD-like loop: fresh dict per step, atoms moving by up to 0.15 A per step
    sts = sts_b
    for step in range(4):
        sts = [dict(s, pos=s["pos"] + rng.normal(0, 0.08, s["pos"].shape)) for s in sts]
        gs = opad(sts, kw["rc"])
        if gs["nbr"].shape[1] > M:
            M = gs["nbr"].shape[1]
        o = m(_repad(gs, M))
        dE, dF = check(o["energy"].detach().cpu(), o["forces"].detach().cpu(), *_oracle_EF(sts, kw, el))
        say(f"  step {step}: dE/E {dE:.2e}  max|dF|/rms {dF:.2e}")


def test_padded_dict_changed_in_place_is_rebuilt():
    """The same dict object with its topology edited in place (mask cleared for a pair and its
    reverse): the graph is rebuilt (version counters), matching a fresh dict."""
    from face_amd import systems
    from oracle.neighbors import padded_graph as opad
    say("in-place edited padded dict")
    kw = dict(C=32, transport=True, eqmsg=True, factor=True, B=16, K=32, rc=4.5)
    m = product_model(kw, [1, 6, 8])
    sts = systems.molecules(2, np.random.default_rng(5))
    g = opad(sts, kw["rc"])
    d = _repad(g, g["nbr"].shape[1])
    m(d)
    mk = g["mask"].clone()
    i, s = map(int, torch.nonzero(mk)[0])
    j = int(g["nbr"][i, s])
    mk[i, s] = False
    s2 = int(torch.nonzero((g["nbr"][j] == i) & mk[j])[0])
    mk[j, s2] = False
    d["mask"].copy_(mk.cuda())
    o1 = m(d)
    o2 = m(dict(d, mask=d["mask"].clone()))
    assert torch.equal(o1["forces"], o2["forces"])


def test_workload4_full_size_properties():
    """The 100,000-atom C256 B16 K64 box at full size (6.9 M pairs): finite energy and forces, net
    force zero to rounding (translation invariance: every pair term enters two atoms with
    opposite signs), and HIP-graph replay equal to the eager step."""
    from face_amd import systems
    from face_amd.neighbors import build_graph
    from face_amd.runner import StepGraph
    sts, kw, el, desc = systems.workload(4)
    say("full size", desc)
    g = build_graph(sts, kw["rc"])
    say(f"  N {g.N} E {g.E} max_row {g.max_row}")
    assert g.N == 100000 and g.E > 6_000_000
    m = product_model(kw, el)
    o = m(g.with_pos(g.pos.clone()))
    E, F = o["energy"].detach(), o["forces"].detach()
    assert torch.isfinite(E).all() and torch.isfinite(F).all()
    rms = F.double().pow(2).mean().sqrt()
    net = F.double().sum(0).abs().max()
    say(f"  E {E.item():.6e}  rms(F) {rms.item():.4e}  max|sum F| {net.item():.3e}")
    assert net <= 1e-3 * rms, (net, rms)
    run = StepGraph(m, g)
    E1, F1 = run(g.pos)
    torch.cuda.synchronize()
    assert torch.allclose(E1, E, rtol=1e-6, atol=0), (E1, E)
    assert (F1 - F).abs().max() <= 1e-5 * F.abs().max()
    nodes = run.node_counts()
    say(f"  graph nodes {nodes}")
    assert nodes and nodes.get("kernel", 0) > 0 and nodes.get("memset", 0) == 0


def _rotation(rng):
    q, r = np.linalg.qr(rng.standard_normal((3, 3)))
    q = q * np.sign(np.diag(r))
    return q * np.sign(np.linalg.det(q))


def _ef(m, sts, rc):
    from face_amd.neighbors import build_graph
    g = build_graph(sts, rc)
    o = m(g.with_pos(g.pos.clone()))
    return g, o["energy"].detach().double(), o["forces"].detach().double()


def _assert_close(E2, F2, E, F, what):
    """The hot-path tolerances: energies within 1e-5 relative, forces within 1e-4 x RMS(F)."""
    rms = F.pow(2).mean().sqrt()
    dE = ((E2 - E).abs() / E.abs().clamp_min(1e-30)).max().item()
    dF = ((F2 - F).abs().max() / rms).item()
    say(f"  {what}: dE/E {dE:.2e}  max|dF|/rms {dF:.2e}")
    assert dE <= E_TOL and dF <= F_TOL, (what, dE, dF)


@pytest.mark.parametrize("k", [1, 3])
def test_workload_full_size_properties(k):
    """The 512-molecule FACE-CP C160 batch (10,752 atoms) and the 24,000-atom FACE-CP C160 liquid
    (1.25 M pairs) at full size, the systems the benchmark times, through the symmetry checks of
    the reference's tests/test_symmetry.py:24-46 at the hot-path tolerances: finite energies and
    forces; zero net force per structure (every pair term enters two atoms with opposite signs);
    rotation + translation of every structure (molecules) or of atoms and cell together (periodic
    box, positions wrapped back) gives the same energies and rotated forces; a permutation of the
    atoms gives the same energies and permuted forces; a second eager call is bitwise equal; the
    HIP-graph replay equals the eager step."""
    from face_amd import systems
    from face_amd.runner import StepGraph
    sts, kw, el, desc = systems.workload(k)
    say("full size", desc)
    m = product_model(kw, el)
    g, E, F = _ef(m, sts, kw["rc"])
    say(f"  N {g.N} E {g.E} max_row {g.max_row}")
    assert g.N == (10752 if k == 1 else 24000) and g.E > (150_000 if k == 1 else 1_200_000)
    assert torch.isfinite(E).all() and torch.isfinite(F).all()
    rms = F.pow(2).mean().sqrt()
    batch = g.batch.long()
    net = torch.zeros(len(sts), 3, dtype=torch.float64, device=F.device).index_add_(0, batch, F)
    say(f"  E[0] {E[0].item():.6e}  rms(F) {rms.item():.4e}  max|sum F| per structure {net.abs().max().item():.3e}")
    assert net.abs().max() <= 1e-3 * rms
    # bitwise reproducible: a second eager call
    _, E1, F1 = _ef(m, sts, kw["rc"])
    assert torch.equal(E1, E) and torch.equal(F1, F)
    # rotation + translation (+ wrap into the rotated cell for the periodic box)
    rng = np.random.default_rng(11 + k)
    Q = _rotation(rng)
    rot = []
    for s in sts:
        p = s["pos"] @ Q.T + rng.standard_normal(3)
        cell = s["cell"] @ Q.T
        if s["pbc"].any():
            frac = p @ np.linalg.inv(cell)
            p = (frac - np.floor(frac)) @ cell
        rot.append(dict(s, pos=p, cell=cell))
    _, E2, F2 = _ef(m, rot, kw["rc"])
    Qt = torch.tensor(Q.T, dtype=torch.float64, device=F.device)
    _assert_close(E2, F2, E, F @ Qt, "rotation + translation")
    # permutation of the atoms of every structure
    perms = [rng.permutation(len(s["pos"])) for s in sts]
    per = [dict(s, pos=s["pos"][p], Z=np.asarray(s["Z"])[p]) for s, p in zip(sts, perms)]
    _, E3, F3 = _ef(m, per, kw["rc"])
    off = np.cumsum([0] + [len(s["pos"]) for s in sts[:-1]])
    idx = torch.tensor(np.concatenate([o + p for o, p in zip(off, perms)]), device=F.device)
    _assert_close(E3, F3, E, F[idx], "permutation")
    # HIP-graph replay of the step
    run = StepGraph(m, g)
    for _ in range(2):
        Er, Fr = run(g.pos)
        torch.cuda.synchronize()
        assert torch.allclose(Er.double(), E, rtol=1e-6, atol=0), (Er, E)
        assert (Fr.double() - F).abs().max() <= 1e-5 * F.abs().max()
    nodes = run.node_counts()
    say(f"  graph nodes {nodes}")
    assert nodes and nodes.get("kernel", 0) > 0 and nodes.get("memset", 0) == 0


@pytest.mark.parametrize("fused", [True, False])
def test_factor_density_mix_routes_match_oracle(fused, monkeypatch):
    """The factorised passes with the fused density + mix kernels and with the unfused route
    (density written, row GEMM), on the 64-molecule flagship workload cut to 16 molecules,
    against the oracle."""
    from face_amd import ops, systems
    from face_amd.neighbors import build_graph
    monkeypatch.setattr(ops, "DENSITY_MIX_MAX_ATOMS", 1 << 30 if fused else 0)
    sts, kw, el, desc = systems.workload(0)
    sts = sts[:16]
    say("density+mix route", fused, desc)
    m = product_model(kw, el)
    o = m(build_graph(sts, kw["rc"]))
    Eo, Fo = _oracle_EF(sts, kw, el)
    dE, dF = check(o["energy"].detach().cpu(), o["forces"].detach().cpu(), Eo, Fo)
    say(f"  dE/E {dE:.2e}  max|dF|/rms {dF:.2e}")


@pytest.mark.parametrize("k,n_atoms,n_mol", [(0, None, 16), (3, 1500, None)])
def test_row_gemm_readout_route_matches_oracle(k, n_atoms, n_mol, monkeypatch):
    """The opt-in readout on the row GEMM (LayerNorm and the out MLP with SiLU on load, the gate
    row and the residual in the same launches) against the oracle, flagship and CP workloads."""
    from face_amd import model as fm, systems
    from face_amd.neighbors import build_graph
    monkeypatch.setattr(fm, "READOUT_ROW_GEMM", True)
    sts, kw, el, desc = systems.workload(k, n_atoms=n_atoms)
    if n_mol:
        sts = sts[:n_mol]
    say("row-GEMM readout", desc)
    m = product_model(kw, el)
    o = m(build_graph(sts, kw["rc"]))
    Eo, Fo = _oracle_EF(sts, kw, el)
    dE, dF = check(o["energy"].detach().cpu(), o["forces"].detach().cpu(), Eo, Fo)
    say(f"  dE/E {dE:.2e}  max|dF|/rms {dF:.2e}")


def test_workload4_lds_backward_matches_oracle(monkeypatch):
    """The C256 B16 K64 model with the factor-density backward that stages each atom's G in LDS (the
    route taken above 64 atoms per CU, forced here on a 1,200-atom box of the same recipe) against
    the oracle."""
    from face_amd import systems
    from face_amd.neighbors import build_graph
    monkeypatch.setenv("FACE_DENSITY_BWD_LDS", "1")
    sts, kw, el, desc = systems.workload(4, n_atoms=1200)
    say("lds backward", desc)
    m = product_model(kw, el)
    o = m(build_graph(sts, kw["rc"]))
    Eo, Fo = _oracle_EF(sts, kw, el)
    dE, dF = check(o["energy"].detach().cpu(), o["forces"].detach().cpu(), Eo, Fo)
    say(f"  dE/E {dE:.2e}  max|dF|/rms {dF:.2e}")
