"""Energy + forces throughput of the FACE hot path on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload 3] [--also 2] [--compiled 2,3] [--no-cpu]

A step is one energy + forces evaluation of the whole synthetic system with its pair list
already resident in HBM (the pair-list build is timed separately, as the reference excludes
it from its timings). Workloads (face_amd.systems.workload):
  0  64 x C9H8O4 molecules, FACE C96 B16 K32 rc 4.5
  1  512 x C9H8O4 molecules, FACE-CP C160 rc 4.5
  2  FCC Ag 6x6x6 = 864 atoms, FACE C96 B16 K32 rc 4.5
  3  24,000-atom H:C:O liquid, FACE-CP C160 rc 5.0            (headline `value`)
  4  100,000-atom H:C:O liquid, FACE C256 B16 K64 rc 5.5
Prints ONE JSON line; progress goes to stderr.
"""
import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for p in (REPO, os.path.join(REPO, "face-mlip_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import numpy as np  # noqa: E402
import torch  # noqa: E402

METRIC = "atom-steps/s (E+F, fp32) at 864 & 24k atoms; density-kernel HBM GB/s"
HBM_PEAK_GBS = 8000.0
TIMED = ["density_fwd20", "density_bwd20", "cp_fwd", "cp_fwd_tab", "cp_bwd", "cp_bwd_tab", "cp_radial_bwd",
         "cp_radial_bwd_tab", "transport_fwd", "transport_bwd", "dir_fwd",
         "dir_bwd", "node_fwd", "node_bwd", "edge_fwd", "edge_bwd", "force_scatter", "gather_bwd", "radial_fwd",
         "radial_bwd", "radial_head", "edge_msg_fwd", "edge_msg_bwd", "mix_fwd", "mix_bwd", "tmix_bwd", "proj_fwd",
         "proj_bwd", "eq_gate_fwd", "eq_gate_bwd", "ln_fwd", "ln_bwd", "spline_order",
         "spline_fwd", "spline_bwd"]
MFMA_PEAK_TFS = 157.3                   # MI355X dense fp32 MFMA


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def algorithmic_bytes(label, g, kw):
    """Bytes per launch: every operand of the kernel's interface read once, every output written
    once, fp32 / int32 (valid pairs E only)."""
    E, N = g.E, g.N
    B, C = kw["B"], kw["C"]
    K = C if kw.get("cp") else kw["K"]
    Kt = 18 * kw["K_dir"]                 # transport table: 9 components x 2Kd channels
    if label == "density_fwd20":
        return 4 * (E * (B + K + 20) + 20 * N * B * K)
    if label == "density_bwd20":
        return 4 * (2 * E * (B + K + 20) + 20 * N * B * K)
    if label == "transport_fwd":          # phi, u, gathered V|M of Kd channels in; 18 sums per (b, kd) out
        return 4 * (E * (B + 3 + Kt // 2) + 18 * N * B * kw["K_dir"])
    if label == "transport_bwd":          # + upstream sums; dphi, du, per-edge table gradient out
        return 4 * (E * (B + 3 + Kt // 2) + 18 * N * B * kw["K_dir"] + E * (B + 3 + Kt // 2))
    if label.startswith("cp_fwd"):          # the CP pooling drop-in: R (4C), msg (C), Y (20) per edge in
        return 4 * (E * (5 * C + 20) + 20 * N * C)
    if label.startswith(("cp_bwd", "cp_radial_bwd")):   # + dR, dmsg, dY per edge out (fused or not)
        return 4 * (2 * E * (5 * C + 20) + 20 * N * C)
    if label == "node_fwd":
        return 4 * 67 * N * C           # 47 in; 8 invariants + V (3) + full Mf (9) out
    if label == "node_bwd":
        return 4 * 114 * N * C          # 47 in, 20 upstream, 47 out
    if label == "edge_fwd":
        return 4 * E * (11 + 29)
    if label == "edge_bwd":
        return 4 * E * (11 + 29 + 3)
    if label == "force_scatter":
        return 4 * (3 * E + E + 3 * N)
    if label.startswith("spline_"):     # r, pair, env in, F columns out (in); both tables read once
        F = kw.get("B", 16) + (4 * C if kw.get("cp") else 0)
        n_el = kw.get("n_elem", 3)
        tables = 8 * n_el * n_el * kw.get("n_grid", 4096) * F
        return 4 * E * (3 + F) + tables + (8 * E if label == "spline_bwd" else 0)
    H, nb = kw.get("radial_hidden", 64), kw.get("n_basis", 8)
    if label == "radial_fwd":           # rb, pair, env in; phi (and h2 in CP mode) out
        return 4 * E * (nb + 2 + B + (H if kw.get("cp") else 0))
    if label == "radial_bwd":           # + upstream phi (and h2) gradients; d rb, d env out
        return 4 * E * (nb + 2 + B + (H if kw.get("cp") else 0) + nb + 1)
    if label == "radial_head":          # h2 in, R (E, 4C) out
        return 4 * E * (H + 4 * C)
    Kd4 = 4 * kw["K_dir"]
    if label == "edge_msg_fwd":         # d, col in; message (E, K) out (the gathered node table: N rows)
        return 4 * (E * (Kd4 + 1 + K) + N * K)
    if label == "edge_msg_bwd":         # upstream (E, K), rev in; d d (E, 4Kd) and the table gradient out
        return 4 * (E * (K + 1 + Kd4) + N * K)
    return None


def interface_bytes(label, g, kw):
    """Bytes the CP launches' own interfaces move (each operand read once, each output written
    once): the envelope, node-table messages gathered through col (N x C + E) under the "_tab"
    labels, and for the fused backward W_cp in and d h2 (E x H) out instead of dR. None for the
    other labels (their algorithmic figure is their interface)."""
    E, N, C = g.E, g.N, kw["C"]
    if not label.startswith("cp_"):
        return None
    msg = N * C + E if label.endswith("_tab") else E * C
    ins = E * (4 * C + 1 + 20) + msg + 20 * N * C
    if label.startswith("cp_fwd"):
        return 4 * ins
    H = kw.get("radial_hidden", 64)
    if label.startswith("cp_radial_bwd"):
        return 4 * (ins + 4 * C * H + E * (H + C + 20 + 1))
    return 4 * (ins + E * (4 * C + C + 20 + 1))


def algorithmic_flops(label, g, kw):
    """Matrix-product flops per launch: the row GEMMs (the four ranks, 20 monomial rows per atom,
    of one mix pass or of one moment set of the proj: output widths C, 3C, 3C, 2C), the radial
    head (E x H by H x 4C), and the fused CP radial backward (d h2 = dR W_cp, E x 4C by 4C x H,
    plus the two 20-monomial contractions per edge and channel)."""
    N, E, C = g.N, g.E, kw["C"]
    H = kw.get("radial_hidden", 64)
    cin = C if kw.get("cp") else kw["B"] * kw["K"]
    if label in ("mix_fwd", "mix_bwd"):
        return 2 * 20 * N * cin * C
    if label in ("proj_fwd", "proj_bwd"):
        return 2 * N * C * (C + 3 * 3 * C + 6 * 3 * C + 10 * 2 * C)
    if label == "tmix_bwd":             # (3 + 6) N rows of C -> B * 2 K_dir transport columns
        return 2 * 9 * N * C * kw["B"] * 2 * kw["K_dir"]
    if label == "radial_head":
        return 2 * E * H * 4 * C
    if label.startswith("cp_radial_bwd"):
        return 2 * E * (4 * C * H + 2 * 20 * C)
    return None


def model_for(kw, el):
    from face_amd import model as fm
    torch.manual_seed(0)
    m = fm.FACE(el, **kw)
    fm.unit_parameterise(m)
    return m.cuda().eval()


def run_gpu(k, steps, warmup, use_graph=True, compiled_radial=False):
    from face_amd import _lib, systems
    from face_amd.neighbors import build_graph
    sts, kw, el, desc = systems.workload(k)
    if compiled_radial:
        desc += ", compiled radial (4096-point splines)"
    log(f"[bench] workload {k}: {desc}")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g = build_graph(sts, kw["rc"])
    torch.cuda.synchronize()
    t_nbr = time.perf_counter() - t0
    log(f"[bench]   pair list: N={g.N} E={g.E} max_row={g.max_row} ({t_nbr * 1e3:.1f} ms incl. host staging)")
    m = model_for(kw, el)
    if compiled_radial:
        m.compile_radial()
        kw = dict(kw, n_elem=len(el), n_grid=4096)

    def step():
        return m(g.with_pos(g.pos.clone()))["forces"]

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    log(f"[bench]   warm-up done ({warmup} steps)")
    torch.cuda.reset_peak_memory_stats()
    # eager pass: HIP events around every hot-kernel launch (kernel durations)
    timers = _lib.time_calls(TIMED)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    dt_eager = time.perf_counter() - t0
    _lib.stop_timing()
    peak_gb = torch.cuda.max_memory_allocated() / 1e9
    log(f"[bench]   eager: {1e3 * dt_eager / steps:.3f} ms/step, peak device memory {peak_gb:.2f} GB")
    dt = dt_eager
    mode = "eager"
    if use_graph:
        # HIP-graph replay of the whole E+F step, positions copied into the static input
        from face_amd.runner import StepGraph
        run = StepGraph(m, g)
        pos = g.pos.clone()
        for _ in range(warmup):
            run(pos)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            run(pos)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        mode = "hipgraph"
        log(f"[bench]   graph replay: {1e3 * dt / steps:.3f} ms/step")
        del run
    kern = {}
    for label, evs in timers.items():
        if not evs:
            continue
        ms = [s.elapsed_time(e) for s, e in evs]
        avg_us = 1e3 * float(np.mean(ms))
        byts = algorithmic_bytes(label, g, kw)
        fl = algorithmic_flops(label, g, kw)
        ib = interface_bytes(label, g, kw)
        kern[label] = {"launches_per_step": len(evs) / steps, "avg_us": avg_us,
                       "ms_per_step": float(np.sum(ms)) / steps,
                       "alg_bytes": byts, "alg_flops": fl, "GBps": (byts / (avg_us * 1e-6) / 1e9) if byts else None,
                       "GBps_interface": (ib / (avg_us * 1e-6) / 1e9) if ib else None,
                       "TFLOPs": (fl / (avg_us * 1e-6) / 1e12) if fl else None}
    ms_step = 1e3 * dt / steps
    log(f"[bench]   {ms_step:.3f} ms/step, {g.N * steps / dt:.0f} atom-steps/s")
    return {"N": g.N, "E": g.E, "ms_per_step": ms_step, "atom_steps_per_s": g.N * steps / dt, "kernels": kern,
            "pairlist_ms": 1e3 * t_nbr, "desc": desc, "kw": kw, "mode": mode,
            "eager_ms_per_step": 1e3 * dt_eager / steps, "peak_mem_gb": peak_gb}


def pmc_probe(k, steps=2, copy_floats=1 << 28):
    """Short run for hardware-counter passes: a few eager E+F steps of workload k, then a plain
    device-to-device copy of a known size, whose FETCH_SIZE / WRITE_SIZE readings calibrate the
    counters (bytes known / counter reading). The JSON line lists the library calls in launch
    order, which assigns the profiler's dispatches to call labels."""
    from face_amd import systems
    from face_amd.neighbors import build_graph
    sts, kw, el, desc = systems.workload(k)
    g = build_graph(sts, kw["rc"])
    m = model_for(kw, el)
    from face_amd import _lib
    order = _lib.record_order(True)
    for _ in range(steps):
        m(g.with_pos(g.pos.clone()))["forces"]
    torch.cuda.synchronize()
    _lib.record_order(False)
    src = torch.ones(copy_floats, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    out = {"probe": desc, "steps": steps, "copy_bytes_read": 4 * copy_floats, "copy_bytes_written": 4 * copy_floats,
           "alg_bytes": {lab: algorithmic_bytes(lab, g, kw) for lab in TIMED},
           "interface_bytes": {lab: interface_bytes(lab, g, kw) for lab in TIMED},
           "alg_flops": {lab: algorithmic_flops(lab, g, kw) for lab in TIMED}, "order": order}
    print(json.dumps(out), flush=True)


def measured_traffic(label):
    """HBM bytes per launch of a labelled kernel from the committed counter summary, or None."""
    path = os.path.join(REPO, "profiles", "traffic_liquid24k_cp160.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        parts = [x.strip() for x in line.strip().strip("|").split("|")]
        if len(parts) >= 6 and parts[0] == label:
            try:
                return float(parts[5])
            except ValueError:
                return None
    return None


def run_cpu(k, n_atoms, rounds=5, warm=2):
    """The CPU oracle (pure-torch restatement of the reference path) on a bounded sample."""
    from face_amd import systems
    from oracle import model as om
    from oracle.neighbors import padded_graph as opad
    cores = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(cores)
    sts, kw, el, desc = systems.workload(k, n_atoms=n_atoms)
    if n_atoms and k in (0, 1):
        sts = sts[:max(1, n_atoms // 21)]
    torch.manual_seed(0)
    m = om.unit_parameterise(om.FACE(el, **kw)).eval()
    g = opad(sts, kw["rc"])
    gg = {kk: g[kk] for kk in ("pos", "Z", "nbr", "shift", "mask", "batch")}
    N = gg["pos"].shape[0]
    for _ in range(warm):
        m(dict(gg, pos=gg["pos"].clone()))
    t0 = time.perf_counter()
    for _ in range(rounds):
        m(dict(gg, pos=gg["pos"].clone()))
    dt = time.perf_counter() - t0
    return {"value": N * rounds / dt, "unit": "atom-steps/s", "cores": cores, "kind": "port",
            "sample": f"{N}-atom sample of the same recipe and model ({desc.split(',')[-1].strip()}), "
                      f"oracle torch path, {rounds} timed E+F calls after {warm} warm-ups, "
                      f"torch.set_num_threads({cores})"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", type=int, default=3)
    ap.add_argument("--also", default="2", help="comma list of extra workloads reported under 'also'")
    ap.add_argument("--compiled", default="2,3",
                    help="comma list of workloads also run with compile_radial() (the reference calculator's "
                         "CUDA setting), reported under 'also'")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-atoms", type=int, default=1500)
    ap.add_argument("--eager", action="store_true", help="time eager steps instead of HIP-graph replays")
    ap.add_argument("--pmc-probe", action="store_true", help="short run for rocprofv3 --pmc passes")
    ap.add_argument("--no-tunable", action="store_true",
                    help="library GEMMs with hipBLASLt's default solutions instead of PyTorch TunableOp")
    a = ap.parse_args()
    if a.gpus != 1:
        print("bench.py measures one GPU only: there is no multi-GPU path in this library (the pair list "
              "would shard by spatial domain with halo atoms; nothing here runs it). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(2)
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    torch.set_float32_matmul_precision("highest")
    tunable = not a.no_tunable and not a.pmc_probe
    if tunable:
        # the GEMMs left to the libraries: solutions timed in the warm-up steps (face_amd.runner)
        from face_amd.runner import tune_library_gemms
        tune_library_gemms()
    if a.pmc_probe:
        pmc_probe(a.workload)
        return
    main_run = run_gpu(a.workload, a.steps, a.warmup, not a.eager)
    also = {}
    runs = [(int(x), False) for x in a.also.split(",") if x.strip() and int(x) != a.workload]
    runs += [(int(x), True) for x in a.compiled.split(",") if x.strip()]
    for k, comp in runs:
        r = run_gpu(k, a.steps, a.warmup, not a.eager, compiled_radial=comp)
        also[f"workload{k}" + ("_compiled_radial" if comp else "")] = {
            "desc": r["desc"], "atoms": r["N"], "pairs": r["E"], "atom_steps_per_s": r["atom_steps_per_s"],
            "ms_per_step": r["ms_per_step"], "pairlist_ms": r["pairlist_ms"], "mode": r["mode"],
            "eager_ms_per_step": r["eager_ms_per_step"],
            "kernels": {kk: {"avg_us": v["avg_us"], "GBps": v["GBps"], "TFLOPs": v["TFLOPs"]}
                        for kk, v in r["kernels"].items()}}
    kern = main_run["kernels"]
    known = {k: v for k, v in kern.items() if v["alg_bytes"] or v["alg_flops"]}
    dom = max(known, key=lambda k: known[k]["ms_per_step"]) if known else None
    roofline = None
    if dom:
        # the bound is the larger of the two floors: algorithmic bytes at peak HBM bandwidth and
        # algorithmic flops at the dense fp32 MFMA peak
        v = known[dom]
        t_hbm = (v["alg_bytes"] or 0) / (HBM_PEAK_GBS * 1e9)
        t_mfma = (v["alg_flops"] or 0) / (MFMA_PEAK_TFS * 1e12)
        if t_mfma > t_hbm:
            bound, ach, peak, unit = "mfma", v["TFLOPs"], MFMA_PEAK_TFS, "TFLOP/s"
        else:
            bound, ach, peak, unit = "hbm", v["GBps"], HBM_PEAK_GBS, "GB/s"
        roofline = {"kernel": dom, "bound": bound, "achieved": ach, "peak": peak, "unit": unit, "frac": ach / peak,
                    "traffic": measured_traffic(dom) if a.workload == 3 else None,
                    "alg_bytes_per_launch": v["alg_bytes"], "alg_flops_per_launch": v["alg_flops"],
                    "GBps": v["GBps"], "TFLOPs": v["TFLOPs"], "avg_launch_us": v["avg_us"]}
    cpu = None
    if not a.no_cpu:
        log("[bench] cpu baseline ...")
        cpu = run_cpu(a.workload, a.cpu_atoms)
        log(f"[bench]   cpu {cpu['value']:.1f} atom-steps/s on {cpu['cores']} cores")
    kw = main_run["kw"]
    out = {
        "metric": METRIC, "value": main_run["atom_steps_per_s"], "unit": "atom-steps/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": main_run["ms_per_step"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": main_run["desc"], "atoms": main_run["N"], "pairs": main_run["E"],
                   "model": {k: kw[k] for k in ("C", "B", "K", "rc") if k in kw} | {"cp": bool(kw.get("cp"))},
                   "weights": "random init, torch.manual_seed(0) + unit_parameterise", "parallelism": "single GPU",
                   "library_gemms": ("fp32 hipBLASLt/rocBLAS, solutions picked by PyTorch TunableOp in the warm-up"
                                     if tunable else "fp32 hipBLASLt default solutions"),
                   "step": main_run["mode"], "eager_ms_per_step": main_run["eager_ms_per_step"],
                   "peak_mem_gb": main_run["peak_mem_gb"]},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": {k: {"avg_us": v["avg_us"], "launches_per_step": v["launches_per_step"], "GBps": v["GBps"],
                        "GBps_interface": v["GBps_interface"],
                        "frac_hbm": (v["GBps"] / HBM_PEAK_GBS) if v["GBps"] else None,
                        "TFLOPs": v["TFLOPs"], "frac_mfma": (v["TFLOPs"] / MFMA_PEAK_TFS) if v["TFLOPs"] else None}
                    for k, v in kern.items()},
        "pairlist_ms": main_run["pairlist_ms"],
        "also": also,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
