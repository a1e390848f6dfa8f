"""MI355X-native FACE hot path: pair-list build, edge front-end, factor / CP density,
node invariants and force scatter as hand-written HIP kernels for gfx950, reached through
the C-ABI of libface_hip.so (include/face_hip.h).

Drop-in modules (same call signatures as the reference package `face`):
  face_amd.kernels.factor_density      <- face/kernels.py
  face_amd.node_kernel.node_algebra    <- face/node_kernel.py
  face_amd.neighbors.padded_graph      <- face/neighbors.py
  face_amd.model.FACE                  <- face/model.py (factorised passes)
"""
__all__ = ["kernels", "node_kernel", "neighbors", "model", "ops", "systems"]
