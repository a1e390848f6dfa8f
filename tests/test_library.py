"""CPU checks of the boundary: the C-ABI library loads and exports every declared entry point,
the host-side model mirror constructs the reference's seeded weights. No GPU calls."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

from golden.cases import BIG_CASES, SMALL_CASES

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = os.path.join(REPO, "tests", "golden")


def header_symbols():
    src = open(os.path.join(REPO, "include", "face_hip.h")).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+(face_\w+)\s*\(", src, re.M)))


def test_header_declares_the_boundary():
    names = header_symbols()
    for n in ["face_density_fwd", "face_density_bwd", "face_cp_density_fwd", "face_cp_density_bwd",
              "face_node_fwd", "face_node_bwd", "face_nbr_count", "face_nbr_fill", "face_nbr_rev",
              "face_edge_geom_fwd", "face_edge_geom_bwd", "face_force_scatter"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    from face_amd import _lib
    L = ctypes.CDLL(_lib.LIB_PATH)
    for n in header_symbols():
        assert hasattr(L, n), n
    assert set(header_symbols()) == set(_lib.exported_symbols())


def test_library_metadata_without_gpu():
    from face_amd import _lib
    L = _lib.lib()
    assert L.face_hip_abi_version() == _lib.ABI_VERSION
    assert b"invalid argument" in L.face_hip_error_string(-1)
    assert b"capacity" in L.face_hip_error_string(-3)


def test_host_rejects_bad_shapes_before_launch():
    from face_amd import _lib
    L = _lib.lib()
    # negative sizes / unsupported monomial counts are refused without touching the device
    assert L.face_density_fwd(None, 16, None, 32, None, None, 20, 7, None, 10, 4, 16, 32, None, 1, 1, None) == -1
    assert L.face_cp_density_bwd(None, 4, None, None, 1, None, None, 20, None, 1, 1, 1, 300, None, 1, 1, None, 0,
                                 None, 0, None, 0, None, None) == -1
    assert L.face_density_fwd(None, 16, None, 32, None, None, 20, 20, None, 0, 4, 16, 32, None, 1, 1, None) == 0
    # a rank-block descriptor with a missing block is refused
    assert L.face_density_fwd(1, 16, 1, 32, None, 1, 20, 20, None, 5, 4, 16, 32, None, 1, 1, None) == -1


def test_spline_entry_points_reject_bad_arguments():
    from face_amd import _lib
    L = _lib.lib()
    # E, P, G, F, dr, nb out of range are refused before any launch; an empty edge list is a no-op
    args = lambda E, P, G, F, dr, nb: (None, None, E, None, None, P, G, F, dr, None, nb, None, None, F, None, F, None)
    assert L.face_radial_spline_fwd(*args(10, 3, 1, 16, 0.1, 16)) == -1          # G < 2
    assert L.face_radial_spline_fwd(*args(10, 3, 64, 16, 0.0, 16)) == -1         # dr <= 0
    assert L.face_radial_spline_fwd(*args(10, 3, 64, 16, 0.1, 17)) == -1         # nb > F
    assert L.face_radial_spline_fwd(*args(-1, 3, 64, 16, 0.1, 16)) == -1
    assert L.face_radial_spline_fwd(*args(10, 3, 64, 16, 0.1, 16)) == -1         # NULL operands
    assert L.face_radial_spline_fwd(*args(0, 3, 64, 16, 0.1, 16)) == 0
    assert L.face_radial_spline_order(None, None, 10, 1 << 16, 1 << 16, 0.1, None, None, None) == -1
    assert L.face_radial_spline_order(None, None, 0, 3, 64, 0.1, None, None, None) == 0


def test_compiled_tables_equal_the_oracle_build():
    """FACE.compile_radial() on the CPU (float64 evaluation, float32 storage, forward-mode dT)
    against the oracle's build (the reference's reverse-mode per-column dT, float64) rounded to
    float32: T identical, dT within a float32 rounding step."""
    from face_amd import model as fm
    from oracle import model as om
    kw, el, _ = SMALL_CASES["small_cp_mol"]
    torch.manual_seed(0)
    m = fm.unit_parameterise(fm.FACE(el, **kw)).eval().compile_radial(n_grid=300)
    torch.manual_seed(0)
    mo = om.unit_parameterise(om.FACE(el, **kw)).double().eval().compile_radial(n_grid=300,
                                                                                 store_dtype=torch.float32)
    for b, bo in zip(m.blocks, mo.blocks):
        assert b.spline.T.dtype == torch.float32 and b.spline.dr == bo.spline.dr
        assert torch.equal(b.spline.T.double(), bo.spline.T)
        d = (b.spline.dT.double() - bo.spline.dT).abs()
        assert bool((d <= 1.2e-7 * bo.spline.dT.abs() + 1e-30).all())


def test_cpu_tensors_are_refused():
    from face_amd.kernels import factor_density
    with pytest.raises(RuntimeError, match="no CPU path"):
        factor_density(torch.zeros(2, 3, 4), torch.zeros(2, 3, 5), torch.zeros(2, 3, 20))


@pytest.mark.parametrize("name", list(SMALL_CASES))
def test_product_model_is_seed_faithful(name):
    from face_amd import model as fm
    kw, el, _ = SMALL_CASES[name]
    d = np.load(os.path.join(GOLD, f"{name}_f32.npz"))
    torch.manual_seed(0)
    m = fm.FACE(el, **kw)
    fm.unit_parameterise(m)
    sd = m.state_dict()
    assert list(sd.keys()) == list(d["state_keys"])
    for k, v in sd.items():
        assert np.array_equal(v.numpy(), d["state/" + k]), k


@pytest.mark.parametrize("name", list(BIG_CASES))
def test_product_model_checksums_at_benchmark_widths(name):
    from face_amd import model as fm
    kw, el, _ = BIG_CASES[name]
    d = np.load(os.path.join(GOLD, f"{name}_f32.npz"))
    torch.manual_seed(0)
    m = fm.FACE(el, **kw)
    fm.unit_parameterise(m)
    for k, v in m.state_dict().items():
        assert np.array_equal(v.double().numpy().reshape(-1)[:4], d["head/" + k]), k


def test_synthetic_workloads_follow_the_recipes():
    from face_amd import systems
    mols, kw, el, _ = systems.workload(0)
    assert len(mols) == 64 and all(len(m["pos"]) == 21 for m in mols)
    for m in mols[:8]:
        p = m["pos"]
        d = np.linalg.norm(p[:, None] - p[None], axis=-1) + np.eye(21) * 9
        assert d.min() > 1.0 - 0.5 and np.linalg.norm(p, axis=1).max() < 3.5 + 0.3
    (fcc,), kw2, el2, _ = systems.workload(2)
    assert len(fcc["pos"]) == 864 and el2 == [47] and abs(fcc["cell"][0, 0] - 24.54) < 1e-9
    (liq,), kw3, _, _ = systems.workload(3, n_atoms=3000)
    assert len(liq["pos"]) == 3000 and kw3["cp"] and kw3["C"] == 160
    L = liq["cell"][0, 0]
    assert abs(3000 / L ** 3 - 0.10) < 1e-9
    assert systems.liquid_counts(24000) == [9143, 10286, 4571]
    assert systems.liquid_counts(100000) == [38095, 42857, 19048]


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus N > 1 exits with status 2 and says why, before any
    device work."""
    import subprocess
    import sys
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300, cwd=REPO)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_bench_roofline_sums_labels_of_one_kernel():
    """The bench's roofline kernel is chosen per kernel family (labels that launch the same kernel
    summed), and its fraction is the sum of the launches' floors (bytes at 8 TB/s or flops at the
    fp32 MFMA peak, whichever binds) over their measured time."""
    import bench
    kern = {
        "cp_radial_bwd": {"family": "cp_radial_bwd", "launches_per_step": 1.0, "ms_per_step": 1.0,
                          "alg_bytes": 4.0e9, "alg_flops": None},
        "cp_radial_bwd_tab": {"family": "cp_radial_bwd", "launches_per_step": 1.0, "ms_per_step": 1.0,
                              "alg_bytes": 4.0e9, "alg_flops": None},
        "radial_head": {"family": "edge_linear_fwd", "launches_per_step": 1.0, "ms_per_step": 1.5,
                        "alg_bytes": 1.0e9, "alg_flops": 1.573e11},
    }
    fam = bench.family_stats(kern)
    assert fam["cp_radial_bwd"]["launches_per_step"] == 2.0 and fam["cp_radial_bwd"]["ms_per_step"] == 2.0
    r = bench.roofline_of(fam, "none")
    assert r["kernel"] == "cp_radial_bwd" and r["bound"] == "hbm" and r["unit"] == "GB/s"
    assert abs(r["frac"] - 0.5) < 1e-12 and abs(r["achieved"] - 4000.0) < 1e-6      # 4 GB per 1 ms launch
    assert abs(fam["edge_linear_fwd"]["frac"] - 1.0 / 1.5) < 1e-12                   # 1 ms MFMA floor
    assert fam["edge_linear_fwd"]["bound"] == "mfma"


def test_bench_labels_map_to_kernel_families():
    import bench
    for lab, fam in bench.KERNEL_FAMILY.items():
        assert fam in bench.FAMILY_KERNELS, lab


def _stub_run(bench, N, E, ms, desc):
    """A run_gpu result as the bench builds it, from made-up per-label figures."""
    kern = {
        "mix_fwd": {"family": "rows_gemm", "launches_per_step": 2.0, "ms_per_step": 0.5 * ms,
                    "alg_bytes": None, "alg_flops": 3.0e10, "avg_us": 250.0 * ms},
        "cp_fwd": {"family": "cp_density_fwd", "launches_per_step": 1.0, "ms_per_step": 0.1 * ms,
                   "alg_bytes": 4.5e9, "alg_flops": None, "avg_us": 100.0 * ms},
        "force_scatter": {"family": "force_scatter", "launches_per_step": 1.0, "ms_per_step": 0.001 * ms,
                          "alg_bytes": 2.0e7, "alg_flops": None, "avg_us": 1.0 * ms},
    }
    fam = bench.family_stats(kern)
    return {"N": N, "E": E, "max_row": 78, "ms_per_step": ms, "ms_min": ms * 0.99, "ms_max": ms * 1.01,
            "rounds": 7, "atom_steps_per_s": N / ms * 1e3, "kernels": kern, "families": fam,
            "roofline": bench.roofline_of(fam, "none"), "pairlist_ms": 5.9, "desc": desc, "kw": {},
            "mode": "hipgraph", "graph_nodes": {"kernel": 79, "memcpy": 1}, "eager_ms_per_step": ms * 1.05,
            "peak_mem_gb": 16.4}


def test_bench_line_is_compact_strict_json():
    """The one stdout line parses as strict JSON (no NaN / Infinity), stays under the size bound
    with all seven workload records, carries the contract keys, a roofline and a CPU baseline,
    and names the workload only in its config (no model hyper-parameters)."""
    import json
    import bench
    desc = "H:C:O 8:9:4 liquid, 24000 atoms, rho 0.10, FACE-CP C160 B16 rc5.0, compiled radial (4096-point splines)"
    main = _stub_run(bench, 24000, 1249484, 18.3, desc)
    results = {(k, c): _stub_run(bench, 1000 * (k + 1), 20000 * (k + 1), 1.0 + k, desc)
               for k, c in [(0, False), (1, False), (2, False), (4, False), (2, True), (3, True)]}
    sample = ("the whole system (24000 atoms, FACE-CP C160 B16 rc5.0), oracle torch path (unfused, as the "
              "reference's torch path), fp32, median of 2 single E+F calls after 1 warm-up (17.5 s), "
              "torch.set_num_threads(16)")
    cpu = {k: {"value": 1392.0 + k, "unit": "atom-steps/s", "cores": 16, "kind": "port", "sample": sample}
           for k in (0, 1, 2, 3, 4)}
    steps = bench.timed_steps(20)
    assert steps == 35 and bench.timed_steps(36) == 40 and bench.timed_steps(1) == 35
    line = bench.bench_line(main, results, cpu, 3, steps, 20, 5, True)
    s = json.dumps(line, separators=(",", ":"), allow_nan=False)
    assert "\n" not in s and len(s) < bench.LINE_MAX_CHARS, len(s)
    d = json.loads(s)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in d, key
    assert d["n_gpus"] == 1 and d["steps"] == 35 and d["steps_requested"] == 20 and d["dtype"] == "f32"
    assert abs(d["value"] - 24000 / 18.3 * 1e3) / d["value"] < 1e-5
    assert "potential" not in d["config"] and d["config"]["workload"] == desc
    r = d["roofline"]
    assert r["kernel"] == "rows_gemm" and r["bound"] == "mfma" and r["unit"] == "TFLOP/s"
    assert abs(r["achieved"] - r["frac"] * r["peak"]) / r["achieved"] < 1e-3
    assert d["cpu_baseline"]["cores"] == 16 and d["cpu_baseline"]["kind"] == "port"
    assert set(d["also"]) == {"workload0", "workload1", "workload2", "workload4", "workload2_compiled_radial",
                              "workload3_compiled_radial"}
    w = d["also"]["workload1"]
    assert w["cpu_baseline"] == 1393.0 and w["roofline"]["kernel"] == "rows_gemm"
    assert "force_scatter" in w["hbm"] and "cp_density_fwd" in w["hbm"]
    assert "cpu_baseline" not in d["also"]["workload3_compiled_radial"]


def test_probe_dispatches_are_labelled_by_call_markers():
    """Counter records of a probe run (one record per counter of a dispatch) are labelled by the
    marker launched after every library call: the dispatches between two markers belong to one
    call, whatever kernels it launched, and the start marker's own records do not shift them."""
    import bench
    mark = "void face::force_scatter_kernel<16>(float const*)"
    seq = [("face::edge_geom_fwd_kernel(float)", 1), (mark, 2), ("face::edge_geom_fwd_kernel(float)", 3), (mark, 4),
           ("void face::rows_gemm_kc_kernel<16>(x)", 5), ("void face::rows_gemm_kernel<8, 16, false, 1>(x)", 6),
           (mark, 7), ("face::node_ln_fwd_kernel(x)", 8), (mark, 9), ("__amd_rocclr_copyBuffer", 10)]
    rows = [{"Kernel_Name": n, "Dispatch_Id": str(i), "Counter_Name": c} for n, i in seq for c in ("A", "B", "C")]
    recs = bench._after_mark(rows)
    disp = {}
    for r in recs:
        disp.setdefault(r["Dispatch_Id"], r)
    labs = [(lab, int(r["Dispatch_Id"])) for lab, r in bench._label_dispatches(list(disp.values()), ["edge_fwd",
                                                                                                      "mix_fwd",
                                                                                                      "node_ln_fwd"],
                                                                             "t")]
    assert labs == [("edge_fwd", 3), ("mix_fwd", 5), ("mix_fwd", 6), ("node_ln_fwd", 8)], labs
