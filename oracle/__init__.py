"""CPU oracle for the FACE density / node-invariant hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package may import, call or link
anything under this directory; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it: as the reference the HIP results are compared
against, and as the timed CPU baseline -- never as the measured or shipped path.

Contents (each function cites the reference file:line it restates):
  cartesian.py   symmetric Cartesian storage, monomials, expansion  (face/cartesian.py)
  ops.py         factor density, CP density, node algebra, transport sums as textbook
                 einsums on full tensors (face/kernels.py:175-178, face/node_kernel.py:212-228,
                 face/model.py:252-264,288-291,496-502,514-533)
  model.py       the unfused FACE torch path with the reference's module construction
                 order, so torch.manual_seed(s) gives the same random-init weights
                 (face/model.py:28-77,90-339,421-534,558-590,665-695)
  neighbors.py   brute-force periodic pair list in fp64 with ASE neighbor_list semantics
                 (ase 3.29.0, called at face/neighbors.py:12), C core in neighbors.c, and the
                 padded-dense graph layout of face/neighbors.py:7-37 built from that pair list

How each part is pinned is stated in the docstring of the function.
"""
