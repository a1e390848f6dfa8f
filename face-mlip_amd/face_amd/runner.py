"""Energy + forces of a fixed pair list, captured once into a HIP graph and replayed.

For a molecular-dynamics or benchmark loop the pair list (and so every tensor shape) stays
fixed between list rebuilds; only positions change. StepGraph captures the whole E+F step
(edge kernel, densities, node algebra, readout GEMMs, the autograd backward and the force
scatter) and replays it: one launch from the host per step instead of several hundred, which
is what bounds small systems (the reference replays CUDA graphs the same way in
tools/graph_bench.py:29-40).

The captured step allocates from a private pool and never synchronises with the host; new
positions are copied into the static input buffer before each replay.
"""
import ctypes
import os
import tempfile

import torch

_HIP = None


def _hip_runtime():
    """ctypes handle of the libamdhip64 that this process already loaded (torch's), found by path
    in the process maps so that no second HIP runtime is loaded."""
    global _HIP
    if _HIP is None:
        path = None
        with open("/proc/self/maps") as f:
            for line in f:
                if "libamdhip64.so" in line:
                    path = line.split()[-1]
                    break
        _HIP = ctypes.CDLL(path or "libamdhip64.so")
        _HIP.hipGraphGetNodes.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_size_t)]
        _HIP.hipGraphNodeGetType.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int)]
    return _HIP


def tune_library_gemms(results_file=None):
    """Let PyTorch TunableOp pick the solutions of the GEMMs left to the libraries (readout MLP,
    tmix forward, per-node linears): the first call of each shape times the fp32 hipBLASLt /
    rocBLAS solutions and keeps the fastest whose result matches the default one within 1e-5.
    Call before the first step (tuning runs eagerly, so before any graph capture). Process-wide;
    results go to results_file (default: a fresh temporary directory)."""
    if results_file is None:
        results_file = os.path.join(tempfile.mkdtemp(prefix="face_tunableop_"), "results.csv")
    torch.cuda.tunable.enable(True)
    torch.cuda.tunable.set_filename(results_file)
    torch.cuda.tunable.set_numerical_check_tolerances(True, 1e-5, 1e-5)


class StepGraph:
    def __init__(self, model, graph, warmup=2):
        self.model = model
        self.pos = graph.pos.detach().clone().contiguous()
        self.graph = graph.with_pos(self.pos)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self._step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        # the captured graph is kept (instantiated on the first replay) so that its nodes can be counted
        self.cg = torch.cuda.CUDAGraph(keep_graph=True)
        with torch.cuda.graph(self.cg):
            self.energy, self.forces = self._step()
        self.cg.instantiate()

    def node_counts(self):
        """{node type: count} of the captured step graph (hipGraphGetNodes / hipGraphNodeGetType of
        the HIP runtime torch loaded): "kernel" is the number of kernel launches per replayed step."""
        hip = _hip_runtime()
        g = ctypes.c_void_p(self.cg.raw_cuda_graph())
        n = ctypes.c_size_t(0)
        if hip.hipGraphGetNodes(g, None, ctypes.byref(n)) != 0:
            return None
        nodes = (ctypes.c_void_p * n.value)()
        if hip.hipGraphGetNodes(g, nodes, ctypes.byref(n)) != 0:
            return None
        names = {0: "kernel", 1: "memcpy", 2: "memset", 3: "host", 4: "graph", 5: "empty", 6: "wait_event",
                 7: "event_record"}
        out = {}
        t = ctypes.c_int(0)
        for k in range(n.value):
            if hip.hipGraphNodeGetType(ctypes.c_void_p(nodes[k]), ctypes.byref(t)) != 0:
                return None
            key = names.get(t.value, f"type{t.value}")
            out[key] = out.get(key, 0) + 1
        return out

    def _step(self):
        p = self.pos.detach().requires_grad_(True)
        o = self.model(self.graph.with_pos(p))
        return o["energy"].detach(), o["forces"].detach()

    def __call__(self, pos=None):
        """Replay with new positions (copied into the static input); returns (energy, forces),
        static output tensors overwritten by the next replay."""
        if pos is not None:
            self.pos.copy_(pos)
        self.cg.replay()
        return self.energy, self.forces
