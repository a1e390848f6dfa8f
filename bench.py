"""Energy + forces throughput of the FACE hot path on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload 3] [--also 0,1,2,4] [--compiled 2,3]
                [--no-cpu] [--cpu-budget S]

A step is one energy + forces evaluation of the whole synthetic system with its pair list
already resident in HBM (the pair-list build is timed separately, as the reference excludes
it from its timings, tools/bench.py:4). Workloads (face_amd.systems.workload):
  0  64 x C9H8O4 molecules, FACE C96 B16 K32 rc 4.5
  1  512 x C9H8O4 molecules, FACE-CP C160 rc 4.5
  2  FCC Ag 6x6x6 = 864 atoms, FACE C96 B16 K32 rc 4.5
  3  24,000-atom H:C:O liquid, FACE-CP C160 rc 5.0            (headline `value`)
  4  100,000-atom H:C:O liquid, FACE C256 B16 K64 rc 5.5
Timing follows the reference's protocol (tools/bench_review.py:53-69): W warm-up steps, then
rounds of 5 calls, each round bracketed by torch.cuda.synchronize(); ms/step is the median
over the rounds (min and max reported beside it). At least 7 rounds are timed whatever K is
(K is raised to whole rounds, >= 35 steps); the line's `steps` is the number actually timed.
Prints ONE compact JSON line (a few KB: headline, roofline, CPU baseline, one short record per
other workload); progress and the per-label / per-family detail ([bench-detail] lines) go to
stderr, and to --detail-out FILE when given.

Profile summaries (text under profiles/) are written by the summary modes from rocprofv3 output:
  --pmc-probe                       short eager run for `rocprofv3 --pmc` passes (one counter each)
  --pmc-summary FETCH_DIR WRITE_DIR  HBM traffic per call label / kernel family from the two passes
  --trace-summary STATS_CSV          per-workload kernel-time summary of a `rocprofv3 --kernel-trace
                                    --stats` run (the timed replays between each workload's two marks)
"""
import argparse
import json
import math
import os
import statistics
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
MFMA_PEAK_TFS = 157.3                   # MI355X dense fp32 MFMA
CALLS_PER_ROUND = 5
TAGS = {0: "mol64_c96", 1: "mol512_cp160", 2: "fcc864_c96", 3: "liquid24k_cp160", 4: "liquid100k_c256"}

# call label -> kernel family (the kernel function the label's entry point launches; labels that
# launch the same kernel are summed when the dominant kernel is chosen)
KERNEL_FAMILY = {
    "density_fwd20": "density_fwd", "density_bwd20": "density_bwd",
    "density_mix_fwd": "density_mix_fwd", "density_mix_bwd": "density_mix_bwd",
    "cp_fwd": "cp_density_fwd", "cp_fwd_tab": "cp_density_fwd",
    "cp_bwd": "cp_density_bwd", "cp_bwd_tab": "cp_density_bwd",
    "cp_radial_fwd": "cp_radial_fwd", "cp_radial_fwd_tab": "cp_radial_fwd",
    "cp_radial_bwd": "cp_radial_bwd", "cp_radial_bwd_tab": "cp_radial_bwd",
    "transport_fwd": "transport_fwd", "transport_bwd": "transport_bwd",
    "dir_fwd": "dir_feats_fwd", "dir_bwd": "dir_feats_bwd",
    "node_fwd": "node_fwd", "node_bwd": "node_bwd", "node_ln_fwd": "node_ln_fwd", "node_ln_bwd": "node_ln_bwd",
    "edge_fwd": "edge_geom_fwd", "edge_bwd": "edge_geom_bwd", "force_scatter": "force_scatter",
    "gather_bwd": "gather_rows_bwd", "radial_fwd": "radial_fwd", "radial_bwd": "radial_bwd",
    "radial_head": "edge_linear_fwd", "edge_msg_fwd": "edge_linear_fwd", "edge_msg_bwd": "edge_linear_bwd",
    "mix_fwd": "rows_gemm", "mix_bwd": "rows_gemm", "tmix_bwd": "rows_gemm", "mix_tmix_bwd": "rows_gemm",
    "proj_fwd": "rows_gemm",
    "proj_bwd": "rows_gemm", "readout_in": "rows_gemm", "readout_hid": "rows_gemm", "readout_out": "rows_gemm",
    "readout_in_bwd": "rows_gemm", "readout_hid_bwd": "rows_gemm", "readout_out_bwd": "rows_gemm",
    "table_linear_fwd": "rows_gemm", "table_linear_bwd": "rows_gemm",
    "eq_gate_fwd": "eq_gate_fwd", "eq_gate_bwd": "eq_gate_bwd",
    "ln_fwd": "layer_norm_fwd", "ln_bwd": "layer_norm_bwd", "spline_order": "spline_order",
    "spline_fwd": "radial_spline_fwd", "spline_bwd": "radial_spline_bwd",
}
# kernel family -> kernel functions of libface_hip.so it stands for (rocprofv3 names, namespace face)
FAMILY_KERNELS = {
    "density_fwd": ["density_fwd_row_kernel", "density_fwd_kernel"],
    "density_bwd": ["density_bwd_split_kernel", "density_bwd_mfma_kernel", "density_bwd_lds_kernel",
                    "density_bwd_kernel"],
    "density_mix_fwd": ["density_mix_fwd_kernel"], "density_mix_bwd": ["density_mix_bwd_kernel"],
    "cp_density_fwd": ["cp_density_fwd_wave_kernel", "cp_density_fwd_kernel"],
    "cp_density_bwd": ["cp_density_bwd_mfma_kernel", "cp_density_bwd_kernel"],
    "cp_radial_fwd": ["cp_radial_fwd_kernel"],
    "cp_radial_bwd": ["cp_radial_bwd_res_kernel", "cp_radial_bwd_lds_kernel"],
    "transport_fwd": ["transport_fwd_kernel"],
    "transport_bwd": ["transport_bwd_mfma_kernel", "transport_bwd_kernel", "transport_table_grad_kernel"],
    "dir_feats_fwd": ["dir_feats_fwd_kernel"], "dir_feats_bwd": ["dir_feats_bwd_edge_kernel",
                                                                 "dir_feats_bwd_node_kernel"],
    "node_fwd": ["node_fwd_kernel"], "node_bwd": ["node_bwd_kernel"],
    "node_ln_fwd": ["node_ln_fwd_kernel"], "node_ln_bwd": ["node_ln_bwd_kernel"],
    "edge_geom_fwd": ["edge_geom_fwd_kernel"], "edge_geom_bwd": ["edge_geom_bwd_seg_kernel", "edge_geom_bwd_kernel"],
    "force_scatter": ["force_scatter_rows_kernel", "force_scatter_kernel"],
    "gather_rows_bwd": ["gather_rows_bwd_kernel"],
    "radial_fwd": ["radial_fwd_kernel"], "radial_bwd": ["radial_bwd_kernel"],
    "edge_linear_fwd": ["edge_linear_fwd_kernel"], "edge_linear_bwd": ["edge_linear_bwd_kernel"],
    "rows_gemm": ["rows_gemm_kernel", "rows_gemm_kc_kernel"], "eq_gate_fwd": ["eq_gate_fwd_kernel"], "eq_gate_bwd": ["eq_gate_bwd_kernel"],
    "layer_norm_fwd": ["layer_norm_fwd_kernel"], "layer_norm_bwd": ["layer_norm_bwd_kernel"],
    "spline_order": ["spline_zero_kernel", "spline_count_kernel", "spline_scan_kernel", "spline_place_kernel"],
    "radial_spline_fwd": ["radial_spline_fwd_kernel", "radial_spline_run_fwd_kernel"],
    "radial_spline_bwd": ["radial_spline_bwd_kernel", "radial_spline_run_bwd_kernel"],
}
TIMED = list(KERNEL_FAMILY)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ----------------------------------------------------------------------------- algorithmic figures
def split_label(label):
    """(base label, n) of a call label "base*n": one launch doing the work of n calls of base
    (passes or moment sets merged into one launch)."""
    base, _, n = label.partition("*")
    return base, int(n) if n else 1


def family_of(label):
    return KERNEL_FAMILY.get(split_label(label)[0])


def algorithmic_bytes(label, g, kw):
    """Bytes per launch: every operand of the kernel's interface read once, every output written
    once, fp32 / int32 (valid pairs E only); a merged launch (label "base*n") counts the inputs
    its n units share once."""
    E, N = g.E, g.N
    label, units = split_label(label)
    if label.startswith("radial_") and units > 1:     # rb, pair, env shared by the passes
        H, nb = kw.get("radial_hidden", 64), kw.get("n_basis", 8)
        one = algorithmic_bytes(label, g, kw)
        return one + (units - 1) * (one - 4 * E * (nb + 2))
    if units > 1:
        one = algorithmic_bytes(label, g, kw)
        return units * one if one else None
    B, C = kw["B"], kw["C"]
    K = C if kw.get("cp") else kw["K"]
    Kt = 18 * kw["K_dir"]                 # transport table: 9 components x 2Kd channels
    if label == "density_fwd20":
        return 4 * (E * (B + K + 20) + 20 * N * B * K)
    if label == "density_bwd20":
        return 4 * (2 * E * (B + K + 20) + 20 * N * B * K)
    if label == "density_mix_fwd":        # the density's drop-in figure (D counted as if written)
        return 4 * (E * (B + K + 20) + 20 * N * B * K)
    if label == "density_mix_bwd":
        return 4 * (2 * E * (B + K + 20) + 20 * N * B * K)
    if label == "transport_fwd":          # phi, u, gathered V|M of Kd channels in; 18 sums per (b, kd) out
        return 4 * (E * (B + 3 + Kt // 2) + 18 * N * B * kw["K_dir"])
    if label == "transport_bwd":          # + upstream sums; dphi, du, per-edge table gradient out
        return 4 * (E * (B + 3 + Kt // 2) + 18 * N * B * kw["K_dir"] + E * (B + 3 + Kt // 2))
    if label.startswith("cp_fwd"):          # the CP pooling drop-in: R (4C), msg (C), Y (20) per edge in
        return 4 * (E * (5 * C + 20) + 20 * N * C)
    if label.startswith("cp_radial_fwd"):   # the fused radial head + pooling: h2 (H) in, R (4C) out once,
        H = kw.get("radial_hidden", 64)   # msg (C), Y (20), env per edge in, A out (R is not read back)
        return 4 * (E * (H + 4 * C + C + 21) + 20 * N * C)
    if label.startswith(("cp_bwd", "cp_radial_bwd")):   # + dR, dmsg, dY per edge out (fused or not)
        return 4 * (2 * E * (5 * C + 20) + 20 * N * C)
    if label == "node_fwd":
        return 4 * 67 * N * C           # 47 in; 8 invariants + V (3) + full Mf (9) out
    if label == "node_bwd":
        return 4 * 114 * N * C          # 47 in, 20 upstream, 47 out
    if label == "node_ln_fwd":          # 47 + P0 in; the normalised row (9), V (3), full Mf (9) out
        return 4 * 69 * N * C
    if label == "node_ln_bwd":          # 47 + P0 in, 9 + 12 upstream, 47 + P0 out
        return 4 * 117 * N * C
    if label == "edge_fwd":
        return 4 * E * (11 + 29)
    if label == "edge_bwd":
        # geometry in, dL/dvec out, and every reader's gradient of Y, rb (or r), the envelope read
        # once (the model hands each reader its own view: pass t reads Y once more when
        # directional, t >= 1, the envelope once more in CP form; at most 4 buffers per input)
        P = kw.get("n_passes", 2)
        nY, nE = min(4, 2 * P - 1), min(4, P * (1 + int(bool(kw.get("cp")))))
        nR = min(4, P)
        radial = nR * (1 if kw.get("compiled") else kw.get("n_basis", 8))
        return 4 * E * (11 + 3 + 20 * nY + radial + nE)
    if label == "force_scatter":
        return 4 * (3 * E + E + 3 * N)
    if label.startswith("spline_") and label != "spline_order":   # r, pair, env in, F columns out; tables once
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
    if label == "eq_gate_fwd":          # V (3), Ms (6), gate row (2) in; Vo, Mo (9) out per (atom, channel)
        return 4 * 20 * N * C
    if label == "eq_gate_bwd":          # + upstream (9); dV, dMs (9), gate-row gradient (2) out
        return 4 * 31 * N * C
    if label == "dir_fwd":              # the 9 used monomials, col, the directional half of V|M (9 Kd per
        return 4 * (E * (9 + 1 + Kd4) + 9 * N * kw["K_dir"])  # node) in; d (E, 4 Kd) out
    if label == "dir_bwd":              # gd, 9 monomials, col + rev, tables in; gY (20), table grads out
        return 4 * (E * (Kd4 + 9 + 2 + 20) + 18 * N * kw["K_dir"])
    # row GEMMs: the rows read once, the weights once, the outputs written once (no initial sums)
    cin = C if kw.get("cp") else B * kw["K"]
    T = B * 2 * kw["K_dir"]             # transport columns
    if label in ("mix_fwd", "mix_bwd"):   # 20 N rows, cin <-> C, one weight per rank
        return 4 * (20 * N * (cin + C) + 4 * cin * C)
    if label in ("proj_fwd", "proj_bwd"):  # 20 N rows of C <-> N (C + 9C + 18C + 20C); weights 9 C^2
        return 4 * (20 * N * C + 48 * N * C + 9 * C * C)
    if label == "tmix_bwd":             # 9 N rows, C -> T
        return 4 * (9 * N * (C + T) + C * T)
    if label == "mix_tmix_bwd":
        return algorithmic_bytes("mix_bwd", g, kw) + algorithmic_bytes("tmix_bwd", g, kw)
    if label in ("table_linear_fwd", "table_linear_bwd"):   # (3 + 6) N rows, C <-> 2 K_dir, two weights
        return 4 * (9 * N * (C + 2 * kw["K_dir"]) + 2 * C * 2 * kw["K_dir"])
    if label == "ln_fwd":               # row of 9C in and out (+ mean, rstd)
        return 4 * (2 * 9 * C + 2) * N
    if label == "ln_bwd":
        return 4 * (3 * 9 * C + 2) * N
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
    if label.startswith("cp_radial_fwd"):     # h2 and W_cp in instead of R; R written once
        return 4 * (E * (H + 1 + 20) + msg + 4 * C * H + E * 4 * C + 20 * N * C)
    if label.startswith("cp_radial_bwd"):
        return 4 * (ins + 4 * C * H + E * (H + C + 20 + 1))
    return 4 * (ins + E * (4 * C + C + 20 + 1))


def algorithmic_flops(label, g, kw):
    """Matrix-product flops per launch: the row GEMMs (the four ranks, 20 monomial rows per atom,
    of one mix pass or of one moment set of the proj: output widths C, 3C, 3C, 2C), the radial
    head (E x H by H x 4C), the pass message's d W_d^T (E x 4Kd by 4Kd x K) and its input
    gradient, the fused CP radial backward (d h2 = dR W_cp, E x 4C by 4C x H, plus the two
    20-monomial contractions per edge and channel), and the factor density's per-monomial
    products (2 E 20 B K forward; two such in the backward, plus the 2 E 20 B of dphi and dY), and the radial MLP of each pass (nb ->
    H -> H -> B per edge; the backward recomputes the hidden layers instead of reading them)."""
    label, units = split_label(label)
    if units > 1:
        one = algorithmic_flops(label, g, kw)
        return units * one if one else None
    N, E, C = g.N, g.E, kw["C"]
    H = kw.get("radial_hidden", 64)
    cin = C if kw.get("cp") else kw["B"] * kw["K"]
    K = C if kw.get("cp") else kw["K"]
    if label in ("mix_fwd", "mix_bwd"):
        return 2 * 20 * N * cin * C
    if label in ("proj_fwd", "proj_bwd"):
        return 2 * N * C * (C + 3 * 3 * C + 6 * 3 * C + 10 * 2 * C)
    if label == "tmix_bwd":             # (3 + 6) N rows of C -> B * 2 K_dir transport columns
        return 2 * 9 * N * C * kw["B"] * 2 * kw["K_dir"]
    if label in ("table_linear_fwd", "table_linear_bwd"):   # (3 + 6) N rows, C <-> nt K_dir
        return 2 * 9 * N * C * 2 * kw["K_dir"]
    if label == "mix_tmix_bwd":         # both in one launch
        return algorithmic_flops("mix_bwd", g, kw) + algorithmic_flops("tmix_bwd", g, kw)
    if label == "radial_head":
        return 2 * E * H * 4 * C
    if label in ("edge_msg_fwd", "edge_msg_bwd"):
        return 2 * E * 4 * kw["K_dir"] * K
    if label.startswith("cp_radial_bwd"):
        return 2 * E * (4 * C * H + 2 * 20 * C)
    if label.startswith("cp_radial_fwd"):     # R = h2 W^T (E x H by H x 4C), then the 20-monomial pooling
        return 2 * E * (4 * C * H + 20 * C)
    nb, B = kw.get("n_basis", 8), kw["B"]
    if label == "radial_fwd":           # per pass: nb -> H -> H -> B (phi; h2 is the second layer)
        return 2 * E * (nb * H + H * H + H * B)
    if label == "radial_bwd":           # the two hidden layers recomputed, then B -> H -> H -> nb
        return 2 * E * (nb * H + H * H) + 2 * E * (B * H + H * H + H * nb)
    # readout (per launch, averaged over the passes: the gate row only where a pass has
    # equivariant outputs, i.e. all passes but the last with eqmsg)
    gate = (kw.get("n_passes", 2) - 1) / kw.get("n_passes", 2) if kw.get("eqmsg") else 0.0
    if label == "readout_in":
        return 2 * N * 10 * C * 2 * C + gate * 2 * N * 9 * C * 2 * C
    if label in ("readout_hid", "readout_hid_bwd"):
        return 2 * N * 2 * C * 2 * C
    if label in ("readout_out", "readout_out_bwd"):
        return 2 * N * 2 * C * (C + 16)
    if label == "readout_in_bwd":
        return 2 * N * 2 * C * 10 * C + gate * 2 * N * 2 * C * 9 * C
    if label == "density_fwd20":
        return 2 * E * 20 * kw["B"] * kw["K"]
    if label == "density_bwd20":         # S = msg G_x^T and dmsg = (Y_x phi) G_x; dphi, dY from S
        return 2 * 2 * E * 20 * kw["B"] * kw["K"] + 2 * 2 * E * 20 * kw["B"]
    if label == "density_mix_fwd":        # density products + the four mixes (20 rows per atom)
        return 2 * E * 20 * kw["B"] * kw["K"] + 2 * 20 * N * cin * C
    if label == "density_mix_bwd":
        return 2 * 2 * E * 20 * kw["B"] * kw["K"] + 2 * 2 * E * 20 * kw["B"] + 2 * 20 * N * cin * C
    return None


def floor_us(byts, fl):
    """(time floor in us, binding bound) of one launch: bytes at peak HBM, flops at the fp32 MFMA peak."""
    t_hbm = (byts or 0) / (HBM_PEAK_GBS * 1e9) * 1e6
    t_mfma = (fl or 0) / (MFMA_PEAK_TFS * 1e12) * 1e6
    return (t_mfma, "mfma") if t_mfma > t_hbm else (t_hbm, "hbm")


# ----------------------------------------------------------------------------- GPU runs
def model_for(kw, el):
    from face_amd import model as fm
    torch.manual_seed(0)
    m = fm.FACE(el, **kw)
    fm.unit_parameterise(m)
    return m.cuda().eval()


def timed_rounds(fn, steps, calls=CALLS_PER_ROUND):
    """Per-step seconds of each round of `calls` calls (the last round shorter when steps is not a
    multiple), every round bracketed by torch.cuda.synchronize()."""
    out, left = [], steps
    while left > 0:
        c = min(calls, left)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(c):
            fn()
        torch.cuda.synchronize()
        out.append((time.perf_counter() - t0) / c)
        left -= c
    return out


def label_stats(timers, steps, g, kw):
    kern = {}
    for label, evs in timers.items():
        if not evs:
            continue
        ms = [s.elapsed_time(e) for s, e in evs]
        avg_us = 1e3 * float(np.mean(ms))
        byts = algorithmic_bytes(label, g, kw)
        fl = algorithmic_flops(label, g, kw)
        ib = interface_bytes(label, g, kw)
        fus, bound = floor_us(byts, fl)
        kern[label] = {"family": family_of(label), "launches_per_step": len(evs) / steps, "avg_us": avg_us,
                       "ms_per_step": float(np.sum(ms)) / steps, "alg_bytes": byts, "alg_flops": fl,
                       "GBps": (byts / (avg_us * 1e-6) / 1e9) if byts else None,
                       "GBps_interface": (ib / (avg_us * 1e-6) / 1e9) if ib else None,
                       "TFLOPs": (fl / (avg_us * 1e-6) / 1e12) if fl else None,
                       "bound": bound if (byts or fl) else None,
                       "frac": (fus / avg_us) if (byts or fl) else None}
    return kern


def family_stats(kern):
    """Per kernel family: launches, time, algorithmic bytes / flops per launch, and the roofline
    fraction = sum of the launches' floors / their measured time."""
    fam = {}
    for label, v in kern.items():
        f = fam.setdefault(v["family"] or label, {"labels": [], "launches_per_step": 0.0, "ms_per_step": 0.0,
                                                  "bytes_per_step": 0.0, "flops_per_step": 0.0,
                                                  "floor_ms_per_step": 0.0, "floor_hbm": 0.0, "floor_mfma": 0.0,
                                                  "known": False})
        f["labels"].append(label)
        n = v["launches_per_step"]
        f["launches_per_step"] += n
        f["ms_per_step"] += v["ms_per_step"]
        f["bytes_per_step"] += n * (v["alg_bytes"] or 0)
        f["flops_per_step"] += n * (v["alg_flops"] or 0)
        if v["alg_bytes"] or v["alg_flops"]:
            fus, bound = floor_us(v["alg_bytes"], v["alg_flops"])
            f["floor_ms_per_step"] += n * fus * 1e-3
            f["floor_" + bound] += n * fus * 1e-3
            f["known"] = True
    for k, f in fam.items():
        n = f["launches_per_step"]
        f["avg_us"] = 1e3 * f["ms_per_step"] / n
        f["alg_bytes_per_launch"] = f["bytes_per_step"] / n if f["bytes_per_step"] else None
        f["alg_flops_per_launch"] = f["flops_per_step"] / n if f["flops_per_step"] else None
        f["frac"] = f["floor_ms_per_step"] / f["ms_per_step"] if f["known"] else None
        f["bound"] = ("mfma" if f["floor_mfma"] > f["floor_hbm"] else "hbm") if f["known"] else None
        f["kernels"] = FAMILY_KERNELS.get(k, [k])
    return fam


def roofline_of(fam, tag):
    """The roofline object of the kernel family with the largest time per step (families without
    an algorithmic figure are skipped): achieved = frac x peak of its binding bound."""
    known = {k: v for k, v in fam.items() if v["known"]}
    if not known:
        return None
    dom = max(known, key=lambda k: known[k]["ms_per_step"])
    v = known[dom]
    if v["bound"] == "mfma":
        peak, unit = MFMA_PEAK_TFS, "TFLOP/s"
    else:
        peak, unit = HBM_PEAK_GBS, "GB/s"
    return {"kernel": dom, "kernels": v["kernels"], "labels": v["labels"], "bound": v["bound"],
            "achieved": v["frac"] * peak, "peak": peak, "unit": unit, "frac": v["frac"],
            "traffic": measured_traffic(tag, v["labels"]),
            "alg_bytes_per_launch": v["alg_bytes_per_launch"], "alg_flops_per_launch": v["alg_flops_per_launch"],
            "avg_launch_us": v["avg_us"], "launches_per_step": v["launches_per_step"],
            "GBps": (v["alg_bytes_per_launch"] / (v["avg_us"] * 1e-6) / 1e9) if v["alg_bytes_per_launch"] else None,
            "TFLOPs": (v["alg_flops_per_launch"] / (v["avg_us"] * 1e-6) / 1e12) if v["alg_flops_per_launch"]
            else None}


_SPIN_PER_S = None


def spin_cycles(seconds):
    """Argument of torch.cuda._sleep for a device spin of about `seconds` (rate measured once)."""
    global _SPIN_PER_S
    if _SPIN_PER_S is None:
        n = 1 << 22
        torch.cuda._sleep(n)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        torch.cuda._sleep(4 * n)
        e.record()
        torch.cuda.synchronize()
        _SPIN_PER_S = 4 * n / (s.elapsed_time(e) * 1e-3)
    return int(seconds * _SPIN_PER_S)


def trace_mark():
    """One launch of a kernel the model never runs (the gather form of the force scatter, on one
    atom), outside any timed region: in a kernel trace, the dispatches between two marks are
    exactly the timed replays of one workload."""
    from face_amd import _lib
    torch.cuda.synchronize()
    z = torch.zeros(2, dtype=torch.int32, device="cuda")
    mark = torch.empty(1, 3, device="cuda")
    _lib.call("face_force_scatter", _lib.ptr(mark), _lib.ptr(z), _lib.ptr(z), 1, 1.0, _lib.ptr(mark),
              _lib.stream_of(mark))
    torch.cuda.synchronize()


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
        kw = dict(kw, n_elem=len(el), n_grid=4096, compiled=True)

    def step():
        return m(g.with_pos(g.pos.clone()))["forces"]

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    log(f"[bench]   warm-up done ({warmup} steps)")
    torch.cuda.reset_peak_memory_stats()
    eager = timed_rounds(step, min(steps, 2 * CALLS_PER_ROUND))
    peak_gb = torch.cuda.max_memory_allocated() / 1e9
    log(f"[bench]   eager: {1e3 * statistics.median(eager):.3f} ms/step, peak device memory {peak_gb:.2f} GB")
    # eager steps with HIP events around every hot-kernel launch (kernel durations), recorded on
    # torch's current stream, the stream every entry point launches on. Where the host sets the
    # pace (its enqueue time per step above half the eager step time: the small systems), a start
    # event fires while the GPU waits for the launch and the wait counts as kernel time: there
    # each step is queued behind a device spin longer than the host takes to enqueue it, so its
    # launches run back to back (864 atoms: density forward 17.5 -> 15.4 us by events, 12.6-13.4
    # us in the kernel trace). Where the GPU sets the pace the host runs ahead anyway and the steps
    # run as they come (the spin there raised the 24k row-GEMM average from 409 to 462 us against
    # 404 us in the trace; under a profiler the host enqueues a 24k step in 7 of its 18 ms).
    t0 = time.perf_counter()
    step()
    t_host = time.perf_counter() - t0
    spin = spin_cycles(2.0 * t_host + 2e-3) if t_host > 0.5 * statistics.median(eager) else 0
    torch.cuda.synchronize()
    timers = _lib.time_calls(TIMED)
    for _ in range(steps):
        if spin:
            torch.cuda._sleep(spin)
        step()
    torch.cuda.synchronize()
    _lib.stop_timing()
    log(f"[bench]   instrumented: {steps} steps" + (f", each queued behind a {1e3 * (2.0 * t_host + 2e-3):.1f} ms "
                                                     f"device spin" if spin else f" (host enqueue {1e3 * t_host:.1f} ms "
                                                     f"per step: no spin)"))
    rounds, mode, nodes = eager, "eager", None
    if use_graph:
        # HIP-graph replay of the whole E+F step, positions copied into the static input
        from face_amd.runner import StepGraph
        run = StepGraph(m, g)
        nodes = run.node_counts()
        pos = g.pos.clone()
        for _ in range(warmup):
            run(pos)
        trace_mark()
        rounds = timed_rounds(lambda: run(pos), steps)
        trace_mark()
        mode = "hipgraph"
        del run
    ms = [1e3 * x for x in rounds]
    ms_step = statistics.median(ms)
    log(f"[bench]   {mode}: {ms_step:.3f} ms/step (median of {len(ms)} rounds; {min(ms):.3f}-{max(ms):.3f}), "
        f"{g.N / ms_step * 1e3:.0f} atom-steps/s; graph nodes {nodes}")
    kern = label_stats(timers, steps, g, kw)
    fam = family_stats(kern)
    # the density route the step took (labels of the launches it made)
    if any(lab.startswith("density_mix") for lab in kern):
        route = "fused factor density + mix (density_mix)"
    elif any(lab.startswith("density_fwd") for lab in kern):
        route = "factor density written, then the row-GEMM mix"
    elif any(lab.startswith("cp_") for lab in kern):
        route = "CP pooling written, then the row-GEMM mix"
    else:
        route = None
    tag = TAGS[k] + ("_compiled" if compiled_radial else "")
    out = {"N": g.N, "E": g.E, "max_row": g.max_row, "ms_per_step": ms_step, "ms_min": min(ms), "ms_max": max(ms),
           "rounds": len(ms), "atom_steps_per_s": g.N / ms_step * 1e3, "kernels": kern, "families": fam,
           "roofline": roofline_of(fam, tag), "pairlist_ms": 1e3 * t_nbr, "desc": desc, "kw": kw, "mode": mode,
           "graph_nodes": nodes, "eager_ms_per_step": 1e3 * statistics.median(eager), "peak_mem_gb": peak_gb,
           "route": route}
    del m, g
    torch.cuda.empty_cache()
    return out


# ----------------------------------------------------------------------------- CPU baseline
# CPU samples of the default run: None = the whole system, otherwise the atom count of a sample of
# the same recipe. The whole 100,000-atom C256 K64 box is not run: the unfused torch path
# materialises phi (x) msg of 100,000 x 101 x 1024 floats (41 GB) plus its autograd buffers and one
# call takes minutes; a 10,000-atom box of the same recipe stands for it (reported per atom).
# --cpu-full runs it whole.
CPU_SAMPLE = {0: None, 1: None, 2: None, 3: None, 4: 10000}


def run_cpu(k, budget_s=10.0, full=False):
    """The CPU oracle (the pure-torch restatement of the reference's torch path, unfused density
    bmm and broadcast node algebra, autograd forces) on the workload's system or a bounded
    sample of it: one warm-up call, then as many single-call rounds as fit the budget (2..7),
    median reported. The padded pair list comes from the GPU build (bit-exact with the oracle's
    pair list); like the reference's timings it is outside the timed region."""
    from face_amd import systems
    from face_amd.neighbors import build_graph, padded_view
    from oracle import model as om
    cores = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(cores)
    n_atoms = None if full else CPU_SAMPLE.get(k)
    sts, kw, el, desc = systems.workload(k, n_atoms=n_atoms)
    g = build_graph(sts, kw["rc"])
    nbr, sh, mask = padded_view(g)
    gg = {"pos": g.pos.cpu(), "Z": g.Z.cpu(), "nbr": nbr.cpu(), "shift": sh.cpu(), "mask": mask.cpu(),
          "batch": g.batch.cpu()}
    N = g.N
    del g, nbr, sh, mask
    torch.manual_seed(0)
    m = om.unit_parameterise(om.FACE(el, **kw)).eval()

    def call():
        t0 = time.perf_counter()
        m(dict(gg, pos=gg["pos"].clone()))
        return time.perf_counter() - t0

    t_warm = call()
    rounds = int(max(2, min(7, budget_s // max(t_warm, 1e-3))))
    ts = [call() for _ in range(rounds)]
    med = statistics.median(ts)
    what = "the whole system" if n_atoms is None else f"a {N}-atom sample of the same recipe"
    return {"value": N / med, "unit": "atom-steps/s", "cores": cores, "kind": "port",
            "ms_per_step": 1e3 * med, "ms_min": 1e3 * min(ts), "ms_max": 1e3 * max(ts),
            "sample": f"{what} ({N} atoms, {desc.split(',')[-1].strip()}), oracle torch path (unfused, as the "
                      f"reference's torch path), fp32, median of {rounds} single E+F calls after 1 warm-up "
                      f"({t_warm:.1f} s), torch.set_num_threads({cores}); bounded to ~{budget_s:.0f} s of CPU "
                      f"work instead of the planned 3 warm-ups + 7 x 5 calls"}


# ----------------------------------------------------------------------------- profiler helpers
def pmc_probe(k, steps=2, copy_floats=1 << 28):
    """Short run for hardware-counter passes: a few eager E+F steps of workload k, then a plain
    device-to-device copy of a known size, whose FETCH_SIZE / WRITE_SIZE readings calibrate the
    counters (bytes known / counter reading). The JSON line lists the library calls in launch
    order, which assigns the profiler's dispatches to call labels."""
    from face_amd import _lib, systems
    from face_amd.neighbors import build_graph
    sts, kw, el, desc = systems.workload(k)
    g = build_graph(sts, kw["rc"])
    m = model_for(kw, el)
    # one step first, so that the row GEMM's launch shapes are timed and cached; then a marker
    # launch (the gather form of the force scatter, which the model does not use) whose dispatch
    # separates that step's (and the shape timing's) dispatches from the recorded steps'
    m(g.with_pos(g.pos.clone()))["forces"]
    trace_mark()
    # a marker after every library call: the dispatches between two markers are one call's
    L = _lib.lib()
    z = torch.zeros(2, dtype=torch.int32, device="cuda")
    mark = torch.empty(1, 3, device="cuda")
    st = _lib.stream_of(mark)

    def after_call():
        L.face_force_scatter(_lib.ptr(mark), _lib.ptr(z), _lib.ptr(z), 1, 1.0, _lib.ptr(mark), st)

    order = _lib.record_order(True, after=after_call)
    for _ in range(steps):
        m(g.with_pos(g.pos.clone()))["forces"]
    torch.cuda.synchronize()
    _lib.record_order(False)
    src = torch.ones(copy_floats, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    labs = sorted(set(TIMED) | {lab for lab in order if family_of(lab)})
    out = {"probe": desc, "workload": k, "steps": steps, "copy_bytes_read": 4 * copy_floats,
           "copy_bytes_written": 4 * copy_floats,
           "alg_bytes": {lab: algorithmic_bytes(lab, g, kw) for lab in labs},
           "interface_bytes": {lab: interface_bytes(lab, g, kw) for lab in labs},
           "alg_flops": {lab: algorithmic_flops(lab, g, kw) for lab in labs}, "order": order}
    print(json.dumps(out), flush=True)


PROBE_MARK = "force_scatter_kernel"


def _after_mark(rows):
    """Dispatch records (sorted by Dispatch_Id; one per counter of a dispatch) after the probe's
    first marker launch (the one between the untimed first step and the recorded steps)."""
    ids = [int(r["Dispatch_Id"]) for r in rows if _kernel_base(r["Kernel_Name"]) == PROBE_MARK]
    return [r for r in rows if int(r["Dispatch_Id"]) > ids[0]] if ids else rows


def _label_dispatches(rows, order, what):
    """(label, record) for the library dispatches of a probe run, in order. The probe launches a
    marker after every library call of the recorded steps, so the dispatches between marker i-1
    and marker i are exactly those of call i (one call may launch several kernels); the
    dispatches after the last call's marker get label None."""
    out, seg, marks = [], 0, 0
    for r in rows:
        if "face::" not in r["Kernel_Name"]:
            continue
        if _kernel_base(r["Kernel_Name"]) == PROBE_MARK:
            seg += 1
            marks += 1
            continue
        out.append((order[seg] if seg < len(order) else None, r))
    if marks < len(order):
        sys.exit(f"{what}: {marks} call markers for {len(order)} recorded calls")
    return out


def _kernel_base(name):
    """Kernel function name of a profiler kernel name ("void face::foo<...>(...)" -> "foo")."""
    n = name.replace("void ", "")
    if "face::" in n:
        n = n.split("face::", 1)[1]
    for stop in "<( ":
        n = n.split(stop, 1)[0]
    return n


def pmc_summary(fetch_dir, write_dir, probe_log, out_path):
    """HBM traffic per call label and per kernel family from two `rocprofv3 --pmc` passes over
    `bench.py --pmc-probe` (FETCH_SIZE, WRITE_SIZE; counter CSVs in the two directories), scaled by
    what the same counters read for the probe's 1 GiB device copy. Writes a markdown summary."""
    import collections
    import csv
    import glob
    rows = {}
    for C, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        f = sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True))
        if not f:
            sys.exit(f"no counter_collection.csv under {d}")
        rows[C] = _after_mark(sorted(csv.DictReader(open(f[0])), key=lambda r: int(r["Dispatch_Id"])))
    probe = [json.loads(x) for x in open(probe_log) if x.startswith('{"probe"')][0]
    cb = probe["copy_bytes_read"]
    scale = {}
    for C in rows:
        cp = sorted((r for r in rows[C] if "copyBuffer" in r["Kernel_Name"]), key=lambda r: -float(r["Counter_Value"]))
        scale[C] = cb / (1024 * sum(float(r["Counter_Value"]) for r in cp[:3]) / 3)
    order = probe["order"]
    acc = {C: collections.defaultdict(float) for C in rows}
    names = collections.defaultdict(set)
    calls = collections.Counter(lab for lab in order)
    for C, rs in rows.items():
        for lab, r in _label_dispatches(rs, order, C):
            if lab is None:
                continue
            acc[C][lab] += float(r["Counter_Value"])
            names[lab].add(r["Kernel_Name"].replace("void ", "").split("(")[0].replace("face::", ""))
    k = probe.get("workload", 3)
    out = [f"# HBM traffic per launch: {probe['probe']}\n\n",
           "Commands (repo root, MI355X, ROCm 7.2; OUT is the output directory), one counter per pass, "
           "then the summary:\n\n```\n"]
    for C in ("FETCH_SIZE", "WRITE_SIZE"):
        out.append(f"rocprofv3 --pmc {C} --kernel-include-regex 'face::|copy' --output-format csv "
                   f"-d $OUT/pmc_{C}_w{k} -o p -- python -u bench.py --pmc-probe --workload {k} "
                   f"> $OUT/pmc_{C}_w{k}.log\n")
    out.append(f"python bench.py --pmc-summary $OUT/pmc_FETCH_SIZE_w{k} $OUT/pmc_WRITE_SIZE_w{k} "
               f"$OUT/pmc_FETCH_SIZE_w{k}.log {out_path}\n```\n\n")
    out.append("`bench.py --pmc-probe` runs one eager E+F step (the row GEMM's launch shapes are timed there) "
               "and a marker launch, then 2 recorded eager E+F steps with a marker launch after every library "
               "call, then three device-to-device copies of 1 GiB; only dispatches after the first marker are "
               "counted. Its JSON line lists the library calls of the recorded steps in launch order: the "
               "dispatches between two markers belong to one call (a call may launch several kernels).\n\n")
    out.append(f"Calibration on the 1 GiB copy: bytes = FETCH_SIZE x 1024 x {scale['FETCH_SIZE']:.4f} and "
               f"WRITE_SIZE x 1024 x {scale['WRITE_SIZE']:.4f}.\n\n")
    out.append("traffic = scaled FETCH + scaled WRITE per call (kernels of one call summed); alg = algorithmic "
               "bytes of the label (operands of the drop-in read once, outputs written once).\n\n")
    out.append("| label | family | kernels | calls | traffic bytes/call | alg bytes/call | traffic/alg |\n"
               "|---|---|---|---:|---:|---:|---:|\n")
    tracked = [lab for lab in sorted(calls, key=lambda x: (list(KERNEL_FAMILY).index(split_label(x)[0])
                                                             if family_of(x) else 1 << 30, x)) if family_of(lab)]
    fam_t = collections.defaultdict(lambda: [0.0, 0.0, 0])
    for lab in tracked:
        n = calls[lab]
        t = (acc["FETCH_SIZE"][lab] * 1024 * scale["FETCH_SIZE"] + acc["WRITE_SIZE"][lab] * 1024 *
             scale["WRITE_SIZE"]) / n
        alg = probe["alg_bytes"].get(lab)
        fam = family_of(lab)
        fam_t[fam][0] += t * n
        fam_t[fam][1] += (alg or 0) * n
        fam_t[fam][2] += n
        out.append(f"| {lab} | {fam} | {' + '.join(sorted(names[lab])) or '-'} | {n} | {t:.0f} | "
                   f"{alg if alg else '-'} | {f'{t / alg:.3f}' if alg else '-'} |\n")
    out.append("\nPer kernel family (the bench's roofline unit):\n\n| family | calls | traffic bytes/launch | "
               "alg bytes/launch | traffic/alg |\n|---|---:|---:|---:|---:|\n")
    for fam, (t, a, n) in fam_t.items():
        out.append(f"| {fam} | {n} | {t / n:.0f} | {a / n if a else '-'} | {f'{t / a:.3f}' if a else '-'} |\n")
    # register / scratch footprint of every library kernel of the run (same dispatch records):
    # Scratch_Size is the per-lane private segment, non-zero when registers spill
    res = {}
    for r in rows["FETCH_SIZE"]:
        if "face::" in r["Kernel_Name"]:
            nm = r["Kernel_Name"].replace("void ", "").split("(")[0].replace("face::", "")
            res[nm] = (r.get("VGPR_Count"), r.get("Accum_VGPR_Count"), r.get("SGPR_Count"), r.get("LDS_Block_Size"),
                       r.get("Scratch_Size"), r.get("Workgroup_Size"))
    out.append("\nKernel resources (dispatch records of the same run; scratch = per-lane private segment "
               "bytes, non-zero when registers spill):\n\n| kernel | VGPR | AGPR | SGPR | LDS bytes | scratch | "
               "workgroup |\n|---|---:|---:|---:|---:|---:|---:|\n")
    for nm, v in sorted(res.items()):
        out.append(f"| `{nm}` | " + " | ".join(str(x) for x in v) + " |\n")
    open(out_path, "w").write("".join(out))
    print("".join(out))


SQ_PASSES = [
    "SQ_WAVES SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY SQ_ACTIVE_INST_ANY SQ_LEVEL_WAVES "
    "SQ_VALU_MFMA_BUSY_CYCLES",
    "SQ_INSTS_MFMA SQ_INSTS_VALU SQ_INSTS_LDS SQ_INSTS_VMEM_RD SQ_INSTS_VMEM_WR SQ_ACTIVE_INST_VALU "
    "SQ_ACTIVE_INST_VMEM SQ_ACTIVE_INST_LDS",
    "SQ_LDS_BANK_CONFLICT SQ_WAIT_INST_LDS SQ_INST_LEVEL_VMEM SQ_INSTS_SALU SQ_INST_CYCLES_VMEM_RD "
    "SQ_INST_CYCLES_VMEM_WR SQ_LDS_IDX_ACTIVE SQ_CYCLES",
]


def _out_rel(path):
    """A path of the run's output directory written as $OUT/... (the summaries' commands name the
    output directory OUT); paths under profiles/ are kept."""
    path = str(path)
    if path.startswith("profiles/") or "/" not in path:
        return path
    return "$OUT/" + path.split("/", 1)[1]


def sq_summary(out_path, title, probe_args, *dirs):
    """Per-kernel SQ counter summary of `rocprofv3 --pmc` passes (SQ_PASSES, one directory each) over
    `bench.py --pmc-probe ...`: wave occupancy and wait fractions, instruction mix and MFMA busy
    cycles per dispatch. mfma_util = SQ_VALU_MFMA_BUSY_CYCLES (= MFMA instructions x their busy
    cycles, summed over SIMDs) / (1024 SIMDs x the dispatch's duration x 2.4 GHz): the share of the
    matrix-core cycles of the whole device the kernel kept busy."""
    import collections
    import csv
    import glob
    # rows keyed by call label for the kernels that serve labels (each pass is its own process, whose
    # row GEMM may pick other launch shapes, i.e. other kernel instances, for the same call), else by
    # kernel; each pass's probe JSON line (the .log beside its directory) gives the call order
    data = collections.defaultdict(lambda: collections.defaultdict(list))
    for d in dirs:
        f = sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True))
        if not f:
            sys.exit(f"no counter_collection.csv under {d}")
        recs = _after_mark(sorted(csv.DictReader(open(f[0])), key=lambda r: int(r["Dispatch_Id"])))
        log = d.rstrip("/") + ".log"
        order = []
        if os.path.exists(log):
            probes = [json.loads(x) for x in open(log) if x.startswith('{"probe"')]
            order = probes[0]["order"] if probes else []
        # a dispatch carries one record per counter: label the dispatches, then their records
        disp = {}
        for r in recs:
            disp.setdefault(r["Dispatch_Id"], r)
        labels = {r["Dispatch_Id"]: lab for lab, r in _label_dispatches(list(disp.values()), order, d)}
        for r in recs:
            lab = labels.get(r["Dispatch_Id"])
            k = f"{lab} ({_kernel_base(r['Kernel_Name'])})" if lab else \
                r["Kernel_Name"].split("(")[0].replace("void ", "").replace("face::", "")
            data[k][r["Counter_Name"]].append(float(r["Counter_Value"]))
            data[k]["_dur_ns"].append(float(r["End_Timestamp"]) - float(r["Start_Timestamp"]))
    out = [f"# SQ counters: {title}\n\nCommands (repo root, MI355X, ROCm 7.2; OUT is the output directory), one "
           "pass per counter group:\n\n```\n"]
    for P, d in zip(SQ_PASSES, dirs):
        out.append(f"rocprofv3 --pmc {P} --kernel-include-regex 'face::' --output-format csv "
                   f"-d {_out_rel(d)} -o p -- python -u bench.py --pmc-probe {probe_args}\n")
    out.append(f"python bench.py --sq-summary {_out_rel(out_path)} '{title}' '{probe_args}' "
               + " ".join(_out_rel(d) for d in dirs) + "\n```\n\n")
    out.append("Per dispatch averages. wave-cycle fractions: time a wave spends waiting on anything / on "
               "s_waitcnt / issuing. mfma_util: SQ_VALU_MFMA_BUSY_CYCLES over (1024 SIMDs x duration x 2.4 GHz).\n\n"
               "| kernel | dispatches | waves | us | wait_any | wait_inst | active | mfma insts | "
               "mfma_util | valu insts | lds insts | vmem rd | vmem wr | lds bank conflicts |\n"
               "|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|\n")
    for k, d in sorted(data.items(), key=lambda kv: -sum(kv[1].get("_dur_ns", [0]))):
        m = {c: sum(v) / len(v) for c, v in d.items()}
        wc = m.get("SQ_WAVE_CYCLES", 0) or 1
        dur = m.get("_dur_ns", 0) or 1
        g = lambda c: m.get(c, float("nan"))
        out.append(f"| `{k[:70]}` | {len(d.get('SQ_WAVES', []))} | {g('SQ_WAVES'):.0f} | {dur / 1e3:.1f} | "
                   f"{g('SQ_WAIT_ANY') / wc:.2f} | {g('SQ_WAIT_INST_ANY') / wc:.2f} | {g('SQ_ACTIVE_INST_ANY') / wc:.2f} | "
                   f"{g('SQ_INSTS_MFMA'):.3g} | {g('SQ_VALU_MFMA_BUSY_CYCLES') / (1024 * 2.4 * dur):.3f} | "
                   f"{g('SQ_INSTS_VALU'):.3g} | {g('SQ_INSTS_LDS'):.3g} | {g('SQ_INSTS_VMEM_RD'):.3g} | "
                   f"{g('SQ_INSTS_VMEM_WR'):.3g} | {g('SQ_LDS_BANK_CONFLICT'):.3g} |\n")
    open(out_path, "w").write("".join(out))
    print("".join(out))


def measured_traffic(tag, labels):
    """HBM bytes per launch of a kernel family (its labels' calls) from the committed counter
    summary of the workload (profiles/traffic_<tag>.md), or None."""
    path = os.path.join(REPO, "profiles", f"traffic_{tag}.md")
    if not os.path.exists(path):
        return None
    tot = n = 0.0
    for line in open(path):
        parts = [x.strip() for x in line.strip().strip("|").split("|")]
        if len(parts) == 7 and parts[0] in labels:
            try:
                tot += float(parts[4]) * int(parts[3])
                n += int(parts[3])
            except ValueError:
                return None
    return tot / n if n else None


def trace_summary(stats_csv, bench_log, out_path, title):
    """Kernel-time summary of a `rocprofv3 --kernel-trace --stats` run of bench.py, per workload:
    the dispatches between the two trace marks of each workload (exactly its timed HIP-graph
    replays) grouped by library kernel family, per step, beside the bench's HIP-event figures of
    the same run; then the library kernels' register / LDS / scratch footprint. BENCH_LOG is the
    run's stdout + stderr (its JSON line and its [bench] / [bench-detail] lines)."""
    import csv
    lines = open(bench_log).read().splitlines()
    d = [json.loads(x) for x in lines if x.startswith('{"metric"')][0]
    detail = {}
    for x in lines:
        if x.startswith("[bench-detail] "):
            key, _, js = x[len("[bench-detail] "):].partition(" ")
            detail[key] = json.loads(js)
    order = []                          # workload keys in run order
    for x in lines:
        if x.startswith("[bench] workload "):
            k = x.split()[2].rstrip(":")
            order.append(f"workload{k}" + ("_compiled_radial" if "compiled radial" in x else ""))
    trace_csv = stats_csv.replace("kernel_stats.csv", "kernel_trace.csv")
    rows = sorted(csv.DictReader(open(trace_csv)), key=lambda r: int(r["Dispatch_Id"]))
    marks = [i for i, r in enumerate(rows) if _kernel_base(r["Kernel_Name"]) == PROBE_MARK]
    base_fam = {kn: fam for fam, kns in FAMILY_KERNELS.items() for kn in kns}
    steps = d["steps"]
    out = [f"# Kernel-time summary: {title}\n\nCommand (repo root, MI355X, ROCm 7.2; OUT is the output "
           f"directory):\n\n```\n"
           f"rocprofv3 --kernel-trace --stats --output-format csv -d {_out_rel(os.path.dirname(stats_csv))} -o bench "
           f"-- python -u bench.py {d.get('_argv', '')}\n"
           f"python bench.py --trace-summary {_out_rel(stats_csv)} <bench stdout+stderr> {_out_rel(out_path)} "
           f"'<title>'\n```\n\n"
           f"Each workload's section covers only the dispatches between its two trace marks: the {steps} timed "
           f"HIP-graph replays of the E+F step (warm-ups, the instrumented eager steps and TunableOp's tuning "
           f"fall outside). Per-step figures divide by {steps}. \"bench us\" is the HIP-event average per launch "
           f"of the same run's instrumented eager steps.\n\n"]
    if len(marks) != 2 * len(order):
        out.append(f"**{len(marks)} trace marks for {len(order)} workloads: sections not attributable.**\n")
        order = []
    for w, key in enumerate(order):
        sel = rows[marks[2 * w] + 1:marks[2 * w + 1]]
        rec = detail.get(key, {})
        tot_ns = sum(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in sel)
        ms_step = rec.get("ms_per_step")
        out.append(f"## {key}: {rec.get('desc', '')}\n\n{len(sel) / steps:.0f} dispatches per step, kernel "
                   f"time {tot_ns / 1e6 / steps:.3f} ms per step"
                   + (f" against {ms_step:.3f} ms per replayed step by the bench's clock" if ms_step else "")
                   + ".\n\n| family / kernel | per step | trace avg us | bench us | us per step | % of kernel time |\n"
                   "|---|---:|---:|---:|---:|---:|\n")
        grp = {}
        for r in sel:
            b = _kernel_base(r["Kernel_Name"])
            name = base_fam.get(b) if "face::" in r["Kernel_Name"] else None
            name = name or ("lib: " + r["Kernel_Name"].replace("|", "/")[:70])
            gk = grp.setdefault(name, [0, 0])
            gk[0] += 1
            gk[1] += int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        fams = rec.get("families", {})
        for name, (c, t) in sorted(grp.items(), key=lambda kv: -kv[1][1]):
            bus = fams.get(name, {}).get("avg_us")
            out.append(f"| `{name}` | {c / steps:.2f} | {t / c / 1e3:.1f} | "
                       + (f"{bus:.1f}" if bus else "") + f" | {t / steps / 1e3:.1f} | {100 * t / tot_ns:.1f} |\n")
        rf = rec.get("roofline")
        if rf and rf["kernel"] in grp:
            c, t = grp[rf["kernel"]]
            out.append(f"\nRoofline family `{rf['kernel']}` ({rf['bound']}): trace average {t / c / 1e3:.1f} us per "
                       f"launch against the bench's {rf['avg_launch_us']:.1f} us; bench fraction "
                       f"{rf['frac']:.3f} of {rf['peak']} {rf['unit']}.\n")
        out.append("\n")
    res = {}
    for x in rows:
        if "face::" in x["Kernel_Name"]:
            nm = x["Kernel_Name"].replace("void ", "").split("(")[0].replace("face::", "")
            res[nm] = (x.get("VGPR_Count"), x.get("Accum_VGPR_Count"), x.get("SGPR_Count"),
                       x.get("LDS_Block_Size"), x.get("Scratch_Size"))
    out.append("## Library kernels' resources\n\nDispatch records of the same run; scratch = per-lane private "
               "segment bytes, non-zero when registers spill.\n\n| kernel | VGPR | AGPR | SGPR | LDS bytes | "
               "scratch |\n|---|---:|---:|---:|---:|---:|\n")
    for nm, v in sorted(res.items()):
        out.append(f"| `{nm}` | " + " | ".join(str(t) for t in v) + " |\n")
    open(out_path, "w").write("".join(out))
    print("".join(out)[:3000])


# ----------------------------------------------------------------------------- main
MIN_ROUNDS = 7                          # the reference's protocol: >= 7 rounds of 5 calls
LINE_MAX_CHARS = 8000                   # the one stdout line stays a few KB (per-label detail -> stderr)
DENSITY_FAMILIES = ("density_fwd", "density_bwd", "cp_density_fwd", "cp_radial_fwd", "cp_radial_bwd",
                    "cp_density_bwd", "density_mix_fwd", "density_mix_bwd")


def timed_steps(requested):
    """Steps actually timed: the requested count, raised to whole rounds and to at least
    MIN_ROUNDS rounds of CALLS_PER_ROUND calls."""
    rounds = max(MIN_ROUNDS, -(-requested // CALLS_PER_ROUND))
    return rounds * CALLS_PER_ROUND


def workload_record(r, cpu=None):
    """Full per-workload record (every label and family): written to stderr, not the stdout line."""
    return {"desc": r["desc"], "atoms": r["N"], "pairs": r["E"], "max_row": r["max_row"],
            "atom_steps_per_s": r["atom_steps_per_s"], "ms_per_step": r["ms_per_step"], "ms_min": r["ms_min"],
            "ms_max": r["ms_max"], "rounds": r["rounds"], "pairlist_ms": r["pairlist_ms"], "mode": r["mode"],
            "eager_ms_per_step": r["eager_ms_per_step"], "peak_mem_gb": r["peak_mem_gb"],
            "graph_nodes": r["graph_nodes"], "roofline": r["roofline"], "cpu_baseline": cpu,
            "kernels": {k: {"avg_us": v["avg_us"], "launches_per_step": v["launches_per_step"], "GBps": v["GBps"],
                            "TFLOPs": v["TFLOPs"], "bound": v["bound"], "frac": v["frac"]}
                        for k, v in r["kernels"].items()},
            "families": {k: {"ms_per_step": v["ms_per_step"], "launches_per_step": v["launches_per_step"],
                             "avg_us": v["avg_us"], "bound": v["bound"], "frac": v["frac"]}
                         for k, v in r["families"].items()}}


def _r(x, nd=4):
    """Round a figure for the compact line (None stays None)."""
    if x is None:
        return None
    return float(f"{x:.{nd}g}")


def compact_roofline(rf):
    """The roofline object of the stdout line: the dominant kernel family's bound, achieved /
    peak, fraction and counter traffic per launch, with the per-launch figures it comes from."""
    if rf is None:
        return None
    out = {"kernel": rf["kernel"], "bound": rf["bound"], "achieved": _r(rf["achieved"]), "peak": rf["peak"],
           "unit": rf["unit"], "frac": _r(rf["frac"]), "traffic": _r(rf["traffic"]),
           "avg_launch_us": _r(rf["avg_launch_us"]), "launches_per_step": _r(rf["launches_per_step"])}
    if rf.get("alg_flops_per_launch"):
        out["alg_flops_per_launch"] = _r(rf["alg_flops_per_launch"])
    if rf.get("alg_bytes_per_launch"):
        out["alg_bytes_per_launch"] = _r(rf["alg_bytes_per_launch"])
    return out


def compact_cpu(cpu):
    if cpu is None:
        return None
    return {"value": _r(cpu["value"]), "unit": cpu["unit"], "cores": cpu["cores"], "kind": cpu["kind"],
            "sample": cpu["sample"]}


def hot_path_kernels(r):
    """HBM fraction of the density kernels and of the force scatter (the kernels the target is
    quoted on): per family present, the fraction of 8 TB/s its algorithmic bytes reach, and for a
    family whose binding floor is its matrix work (the fused CP kernels, the factor density at
    100k atoms) also its fraction of the fp32 MFMA peak. The force backward is also given as one
    unit, the edge backward (which writes every edge's dL/dvec into its reverse edge's slot) and
    the row scatter that completes it: their bytes over their time."""
    out = {}
    for fam_name in DENSITY_FAMILIES + ("force_scatter",):
        f = r["families"].get(fam_name)
        if not f or not f.get("alg_bytes_per_launch"):
            continue
        gbs = f["alg_bytes_per_launch"] / (f["avg_us"] * 1e-6) / 1e9
        out[fam_name] = {"us": _r(f["avg_us"]), "GBps": _r(gbs), "hbm_frac": _r(gbs / HBM_PEAK_GBS, 3)}
        if f.get("bound") == "mfma" and f.get("alg_flops_per_launch"):
            tfs = f["alg_flops_per_launch"] / (f["avg_us"] * 1e-6) / 1e12
            out[fam_name]["mfma_frac"] = _r(tfs / MFMA_PEAK_TFS, 3)
    fe, fs = r["families"].get("edge_geom_bwd"), r["families"].get("force_scatter")
    if fe and fs and fe.get("alg_bytes_per_launch") and fs.get("alg_bytes_per_launch"):
        byts = fe["bytes_per_step"] + fs["bytes_per_step"]
        ms = fe["ms_per_step"] + fs["ms_per_step"]
        gbs = byts / (ms * 1e-3) / 1e9
        out["force_bwd"] = {"us": _r(1e3 * ms), "GBps": _r(gbs), "hbm_frac": _r(gbs / HBM_PEAK_GBS, 3)}
    return out


def compact_workload(r, cpu=None):
    """One workload's entry under 'also' in the stdout line."""
    rf = r["roofline"]
    out = {"workload": r["desc"], "atoms": r["N"], "pairs": r["E"], "ms_per_step": _r(r["ms_per_step"]),
           "value": _r(r["atom_steps_per_s"]), "rounds": r["rounds"],
           "roofline": None if rf is None else {"kernel": rf["kernel"], "bound": rf["bound"],
                                                "frac": _r(rf["frac"], 3)},
           "hbm": hot_path_kernels(r)}
    if r.get("route"):
        out["route"] = r["route"]
    if cpu is not None:
        out["cpu_baseline"] = _r(cpu["value"])
    return out


def bench_line(main_run, results, cpu, workload, steps, steps_requested, warmup, tunable):
    """The one JSON line bench.py prints: the headline workload's throughput, its roofline and CPU
    baseline, and a compact record per other workload. Everything per label goes to stderr."""
    also = {}
    for (k, comp), r in results.items():
        also[f"workload{k}" + ("_compiled_radial" if comp else "")] = compact_workload(r, None if comp else
                                                                                         cpu.get(k))
    return {
        "metric": METRIC, "value": _r(main_run["atom_steps_per_s"], 6), "unit": "atom-steps/s", "n_gpus": 1,
        "steps": steps, "steps_requested": steps_requested, "warmup": warmup,
        "ms_per_step": _r(main_run["ms_per_step"], 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": main_run["desc"], "atoms": main_run["N"], "pairs": main_run["E"],
                   "parallelism": "single GPU", "step": main_run["mode"],
                   "timing": f"median of {main_run['rounds']} rounds of {CALLS_PER_ROUND} calls after {warmup} "
                             f"warm-ups (tools/bench_review.py:53-69)",
                   "ms_min": _r(main_run["ms_min"]), "ms_max": _r(main_run["ms_max"]),
                   "library_gemms": "TunableOp" if tunable else "default", "graph_nodes": main_run["graph_nodes"],
                   "peak_mem_gb": _r(main_run["peak_mem_gb"], 3)},
        "roofline": compact_roofline(main_run["roofline"]),
        "cpu_baseline": compact_cpu(cpu.get(workload)),
        "hbm": hot_path_kernels(main_run),
        "also": also,
        "_argv": " ".join(sys.argv[1:]),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=35, help="timed steps (rounds of 5 calls)")
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", type=int, default=3)
    ap.add_argument("--also", default="0,1,2,4", help="comma list of extra workloads reported under 'also'")
    ap.add_argument("--compiled", default="2,3",
                    help="comma list of workloads also run with compile_radial() (the reference calculator's "
                         "CUDA setting), reported under 'also'")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of timed CPU calls per workload")
    ap.add_argument("--cpu-full", action="store_true", help="CPU baselines on the whole systems (slow)")
    ap.add_argument("--eager", action="store_true", help="time eager steps instead of HIP-graph replays")
    ap.add_argument("--pmc-probe", action="store_true", help="short run for rocprofv3 --pmc passes")
    ap.add_argument("--pmc-summary", nargs=4, metavar=("FETCH_DIR", "WRITE_DIR", "PROBE_LOG", "OUT"))
    ap.add_argument("--trace-summary", nargs=4, metavar=("STATS_CSV", "BENCH_LOG", "OUT", "TITLE"))
    ap.add_argument("--sq-summary", nargs="+", metavar="OUT TITLE PROBE_ARGS DIR",
                    help="OUT TITLE PROBE_ARGS DIR1 [DIR2 DIR3]: SQ counter summary of rocprofv3 --pmc passes")
    ap.add_argument("--detail-out", default=None, help="also write the per-label detail of every workload here")
    ap.add_argument("--no-tunable", action="store_true",
                    help="library GEMMs with hipBLASLt's default solutions instead of PyTorch TunableOp")
    a = ap.parse_args()
    if a.pmc_summary:
        pmc_summary(*a.pmc_summary)
        return
    if a.trace_summary:
        trace_summary(*a.trace_summary)
        return
    if a.sq_summary:
        sq_summary(*a.sq_summary)
        return
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
    steps = timed_steps(a.steps)
    if steps != a.steps:
        log(f"[bench] timing {steps} steps ({steps // CALLS_PER_ROUND} rounds of {CALLS_PER_ROUND} calls; "
            f"{a.steps} requested): at least {MIN_ROUNDS} rounds per workload")
    main_run = run_gpu(a.workload, steps, a.warmup, not a.eager)
    runs = [(int(x), False) for x in a.also.split(",") if x.strip() and int(x) != a.workload]
    runs += [(int(x), True) for x in a.compiled.split(",") if x.strip()]
    results = {}
    for k, comp in runs:
        results[(k, comp)] = run_gpu(k, steps, a.warmup, not a.eager, compiled_radial=comp)
    cpu = {}
    if not a.no_cpu:
        for k in [a.workload] + [k for k, comp in runs if not comp]:
            log(f"[bench] cpu baseline, workload {k} ...")
            cpu[k] = run_cpu(k, a.cpu_budget, a.cpu_full)
            log(f"[bench]   cpu {cpu[k]['value']:.1f} atom-steps/s on {cpu[k]['cores']} cores ({cpu[k]['sample']})")
    # per-label and per-family detail of every workload: stderr (and a file when asked)
    detail = {f"workload{a.workload}": workload_record(main_run, cpu.get(a.workload))}
    for (k, comp), r in results.items():
        detail[f"workload{k}" + ("_compiled_radial" if comp else "")] = workload_record(r, None if comp
                                                                                        else cpu.get(k))
    for key, rec in detail.items():
        log(f"[bench-detail] {key} " + json.dumps(rec))
    if a.detail_out:
        with open(a.detail_out, "w") as f:
            json.dump(detail, f, indent=1)
    line = bench_line(main_run, results, cpu, a.workload, steps, a.steps, a.warmup, tunable)
    print(json.dumps(line, separators=(",", ":")), flush=True)


if __name__ == "__main__":
    main()
