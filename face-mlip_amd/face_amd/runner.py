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
import os
import tempfile

import torch


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
        self.cg = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.cg):
            self.energy, self.forces = self._step()

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
