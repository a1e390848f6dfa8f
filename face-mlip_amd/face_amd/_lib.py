"""ctypes binding of libface_hip.so (the C-ABI declared in include/face_hip.h).

The library is loaded once, lazily; a missing or unloadable library raises at the first call
(there is no fallback path). Every entry point returns an int status that is turned into a
RuntimeError carrying face_hip_error_string().
"""
import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("FACE_HIP_LIB", os.path.join(_HERE, "libface_hip.so"))
_lib = None
_lock = threading.Lock()

P = ctypes.c_void_p
I32 = ctypes.c_int32
I64 = ctypes.c_int64
F32 = ctypes.c_float
F64 = ctypes.c_double

_SIGS = {
    "face_hip_error_string": (ctypes.c_char_p, [ctypes.c_int]),
    "face_hip_abi_version": (ctypes.c_int, []),
    "face_density_fwd": (ctypes.c_int, [P, I32, P, I32, P, P, I32, I32, P, I64, I32, I32, I32, P, I64, I64, P]),
    "face_density_bwd": (ctypes.c_int, [P, I32, P, I32, P, P, I32, I32, P, I64, I32, I32, I32, I32, P, I64, I64, P,
                                        I32, P, I32, P, I32, P]),
    "face_density_mix_fwd": (ctypes.c_int, [P, I32, P, I32, P, P, I32, P, I64, I32, I32, I32, P, I64, P, I64, I64, P,
                                            I32, P, I32, P]),
    "face_density_mix_bwd": (ctypes.c_int, [P, I32, P, I32, P, P, I32, P, I64, I32, I32, I32, P, I64, P, I64, I64, P,
                                            I32, P, P, I32, P, I32, P, I32, P]),
    "face_cp_density_fwd": (ctypes.c_int, [P, I32, P, P, I32, P, P, I32, P, I64, I32, I32, P, I64, I64, P]),
    "face_cp_density_bwd": (ctypes.c_int, [P, I32, P, P, I32, P, P, I32, P, I64, I32, I32, I32, P, I64, I64, P, I32,
                                           P, I32, P, I32, P, P]),
    "face_node_fwd": (ctypes.c_int, [P, P, P, P, P, P, P, P, P, P, I32, I64, I32, I32, P]),
    "face_node_bwd": (ctypes.c_int, [P, P, P, P, P, P, P, P, P, P, I32, P, P, P, P, I64, I32, I32, P]),
    "face_node_ln_fwd": (ctypes.c_int, [P, P, P, I64, P, P, P, P, F32, P, I64, P, P, P, P, P, I32, I64, I32, I32, P]),
    "face_node_ln_bwd": (ctypes.c_int, [P, P, P, I64, P, P, P, P, I64, P, P, P, P, P, I32, P, P, P, I64, P, P, I64,
                                        I32, I32, P]),
    "face_nbr_bin": (ctypes.c_int, [P, I64, P, P, P, P, P, P, P, P, P]),
    "face_nbr_count": (ctypes.c_int, [P, I64, P, P, P, P, P, F64, P, P, P, P, P, P, P]),
    "face_nbr_fill": (ctypes.c_int, [P, I64, P, P, P, P, P, F64, P, P, P, P, P, P, P, P, P, P, P, P]),
    "face_nbr_rev": (ctypes.c_int, [P, P, P, I64, P, P, P]),
    "face_nbr_rev_shift": (ctypes.c_int, [P, P, P, I64, P, P, P]),
    "face_nbr_padded": (ctypes.c_int, [P, P, P, P, P, I64, I32, P, P, P, P]),
    "face_edge_geom_fwd": (ctypes.c_int, [P, P, P, P, P, I64, P, I32, F32, F32, P, P, P, P, P]),
    "face_edge_geom_bwd": (ctypes.c_int, [P, P, P, P, P, I64, P, I32, F32, F32, P, P, P, P, P, P]),
    "face_dir_feats_fwd": (ctypes.c_int, [P, I64, I64, P, I64, I64, I32, P, P, P, I64, P, P]),
    "face_dir_feats_bwd": (ctypes.c_int, [P, I64, I64, P, I64, I64, I32, P, P, P, P, P, P, I64, I64, P, P, P, P]),
    "face_transport_fwd": (ctypes.c_int, [P, I32, I32, P, I64, I64, P, I64, I64, I32, P, I32, P, P, I64, F32, P, P,
                                          P]),
    "face_transport_bwd": (ctypes.c_int, [P, I32, I32, P, I64, I64, P, I64, I64, I32, P, I32, P, P, P, I64, I32, F32,
                                          P, P, P, I32, P, P, P, P, P]),
    "face_gather_rows": (ctypes.c_int, [P, I32, P, I64, I32, P, I32, P]),
    "face_gather_rows_bwd": (ctypes.c_int, [P, I32, P, P, I64, I32, P, I32, P]),
    "face_segment_sum": (ctypes.c_int, [P, I32, P, I64, I32, P, I32, P]),
    "face_atom_energy_fwd": (ctypes.c_int, [P, P, P, P, I32, P, I64, P, P, P]),
    "face_atom_energy_bwd": (ctypes.c_int, [P, P, P, P, I64, P, P]),
    "face_force_scatter": (ctypes.c_int, [P, P, P, I64, F32, P, P]),
    "face_edge_geom_bwd_seg": (ctypes.c_int, [P, P, P, P, P, I64, P, I32, F32, F32, P, P, P, P, P, P, P]),
    "face_force_scatter_rows": (ctypes.c_int, [P, P, P, I64, I32, F32, P, P]),
    "face_cp_radial_fwd": (ctypes.c_int, [P, I32, I32, P, P, P, P, I32, P, P, I32, P, I64, I64, I32, P, I64, I64, P,
                                           I32, P]),
    "face_cp_radial_bwd": (ctypes.c_int, [P, I32, P, P, I32, P, P, I32, P, I64, I32, I32, P, I64, I64, P, I32, P, I32,
                                          P, I32, P, I32, P, P]),
    "face_radial_fwd": (ctypes.c_int, [P, I32, I32, P, P, I64, P, P, P, I32, I32, P, P, P, P, I32, P, I32, P, I32, P]),
    "face_radial_bwd": (ctypes.c_int, [P, I32, I32, P, P, I64, P, P, P, I32, I32, P, P, P, P, I32, P, I32, P, P, I32,
                                       P, I32, P, P]),
    "face_radial_fwd_sets": (ctypes.c_int, [P, I32, I32, P, P, I64, I32, P, I32, I32, I32, P, I32, P, I32, P]),
    "face_radial_bwd_sets": (ctypes.c_int, [P, I32, I32, P, P, I64, I32, P, I32, I32, I32, P, I32, P, P, I32, P, I32,
                                            P, P]),
    "face_radial_spline_fwd": (ctypes.c_int, [P, P, I64, P, P, I32, I32, I32, F32, P, I32, P, P, I32, P, I32, P]),
    "face_radial_spline_bwd": (ctypes.c_int, [P, P, I64, P, P, I32, I32, I32, F32, P, I32, P, P, I32, P, I32, P,
                                              P, P]),
    "face_radial_spline_order": (ctypes.c_int, [P, P, I64, I32, I32, F32, P, P, P]),
    "face_radial_spline_order_noalloc": (ctypes.c_int, [P, P, I64, I32, I32, F32, P, P]),
    "face_edge_linear_fwd": (ctypes.c_int, [P, I32, I64, I32, P, P, I32, P, I32, P, P, I32, P]),
    "face_edge_linear_bwd": (ctypes.c_int, [P, I32, I32, P, I32, P, P, I64, P, I32, P, I32, P]),
    "face_rows_linear": (ctypes.c_int, [P, I32, I32, P, P, I32, I32, P, I64, P]),
    "face_eq_gate_fwd": (ctypes.c_int, [P, P, P, I64, I32, P, P, P]),
    "face_eq_gate_bwd": (ctypes.c_int, [P, P, P, P, P, I64, I32, P, P, P, P]),
    "face_layer_norm_fwd": (ctypes.c_int, [P, I64, I32, P, P, ctypes.c_float, P, P, P, P]),
    "face_layer_norm_bwd": (ctypes.c_int, [P, P, I64, I32, P, P, P, P, P]),
}

ABI_VERSION = 24


class LinProblem(ctypes.Structure):
    """face_lin_problem of include/face_hip.h."""
    _fields_ = [("x", ctypes.c_void_p), ("ld_x", ctypes.c_int64), ("m", ctypes.c_int64), ("w", ctypes.c_void_p),
                ("ld_w", ctypes.c_int64), ("y", ctypes.c_void_p), ("ld_y", ctypes.c_int64), ("n", ctypes.c_int32),
                ("k", ctypes.c_int32), ("s_off", ctypes.c_int32), ("beta", ctypes.c_float),
                ("x2", ctypes.c_void_p), ("ld_x2", ctypes.c_int64), ("k1", ctypes.c_int32), ("x_op", ctypes.c_int32),
                ("xz", ctypes.c_void_p), ("ld_xz", ctypes.c_int64), ("bias", ctypes.c_void_p),
                ("y0", ctypes.c_void_p), ("ld_y0", ctypes.c_int64), ("n_y0", ctypes.c_int32), ("pad_", ctypes.c_int32)]


def lib():
    """The loaded library (loads on first use; raises if it is missing)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise RuntimeError(f"libface_hip.so not found at {LIB_PATH}: build it with "
                                       f"`python face-mlip_amd/csrc/build.py` (or __graft_entry__.build())")
                L = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in _SIGS.items():
                    fn = getattr(L, name)
                    fn.restype = res
                    fn.argtypes = args
                if L.face_hip_abi_version() != ABI_VERSION:
                    raise RuntimeError("libface_hip.so ABI version mismatch: rebuild it")
                _lib = L
    return _lib


def exported_symbols():
    return list(_SIGS)


# Optional per-entry-point launch timing: {name: [(start_event, end_event), ...]}; events are
# recorded on torch's current stream, the stream every entry point is launched on.
_timing = None


def time_calls(names):
    """Start recording HIP events around every call of the given entry points."""
    global _timing
    _timing = {n: [] for n in names}
    return _timing


def stop_timing():
    global _timing
    t, _timing = _timing, None
    return t


# Optional call log: the label (or entry-point name) of every successful call, in call order,
# for matching a profiler's dispatch list to the calls that launched it.
_order = None
_after_call = None


def record_order(on=True, after=None):
    """Start (on) or stop logging call labels; returns the list being filled (or None). `after`
    (optional) is run after every logged call, e.g. a marker launch that separates the calls'
    dispatches in a profiler's record."""
    global _order, _after_call
    _order = [] if on else None
    _after_call = after if on else None
    return _order


def call(name, *args, label=None):
    """Call entry point `name`; raise RuntimeError on a non-zero status. `label` names the
    launch for time_calls (defaults to the entry-point name)."""
    fn = getattr(lib(), name)
    key = label or name
    # "name*n": a launch doing the work of n calls of "name" (passes or moment sets merged)
    if _timing is not None and key.split("*")[0] in _timing:
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        code = fn(*args)
        e.record()
        _timing.setdefault(key, []).append((s, e))
    else:
        code = fn(*args)
    if code != 0:
        msg = lib().face_hip_error_string(code).decode()
        raise RuntimeError(f"{name} failed: {msg} (code {code})")
    if _order is not None:
        _order.append(key)
        if _after_call is not None:
            _after_call()


FACE_ERR_UNSUPPORTED = -2


def call_status(name, *args, label=None):
    """call(), except that FACE_ERR_UNSUPPORTED (a shape the entry point's kernels cannot serve;
    nothing was launched) is returned instead of raised, for callers with another route."""
    try:
        call(name, *args, label=label)
        return 0
    except RuntimeError as err:
        if f"(code {FACE_ERR_UNSUPPORTED})" in str(err):
            return FACE_ERR_UNSUPPORTED
        raise


def ptr(t):
    """Device pointer of a tensor (or None -> NULL)."""
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t=None):
    """Raw HIP stream handle of torch's current stream on the tensor's device (the raw-handle
    query skips building a Stream object on every launch)."""
    if _raw_stream is not None:
        idx = t.device.index if (t is not None and t.device.index is not None) else torch.cuda.current_device()
        return _raw_stream(idx)
    dev = t.device if t is not None else torch.device("cuda")
    return torch.cuda.current_stream(dev).cuda_stream


def require_gpu(*ts):
    for t in ts:
        if t is not None and (not t.is_cuda):
            raise RuntimeError("face_amd kernels need tensors on a HIP device (got "
                               f"{t.device}); there is no CPU path")


def ptr_array(ts):
    return (P * len(ts))(*[ptr(t) for t in ts])


def i64_array(vals):
    return (I64 * len(vals))(*vals)


RANK_X0 = (0, 1, 4, 10)


def ranks_of_dense(t):
    """Rank-block descriptor of a reference-layout (N, NX, W) contiguous tensor."""
    N, NX, W = t.shape
    base = t.data_ptr()
    nr = 4 if NX == 20 else 2
    ptrs = [base + 4 * RANK_X0[l] * W if l < nr else None for l in range(4)]
    return (P * 4)(*ptrs), NX * W, W


def ranks_of_blocks(blocks):
    """Rank-block descriptor of per-rank (k_l, N, W) contiguous tensors (2 or 4 of them)."""
    k, N, W = blocks[0].shape
    ptrs = [b.data_ptr() for b in blocks] + [None] * (4 - len(blocks))
    return (P * 4)(*ptrs), W, N * W
