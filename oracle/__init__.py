"""CPU oracle of the GPU-resident MD step -- TEST INFRASTRUCTURE ONLY.

A plain NumPy / PyTorch-CPU restatement of the reference's algorithms on the hot path
(neighbour list, gather-cat, segment sums, edge GEMM, Nose-Hoover chain, engine-owned
derivative, the Morse and MACE-like models), each function citing the reference file:line it
follows (paths relative to the reference repository, ICT-fushibo/fastMD). Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import it, and only as the
checker (or the timed CPU baseline), never as the product path: ``fastmd_amd`` does not import
anything from here, and its GPU entry points raise when the HIP library is missing.

How each part is pinned (beyond restating the reference's formulas):
  nl      brute-force FP64 pair sets over all images (the reference's own check,
          tests/test_fixed_capacity_boundary.py:86-102), the canonical key order, the padding
          layout, estimate_max_neighbors known answers (tests/test_ragged_builder_overflow.py:328-336)
  ops     closed forms and FP64 references (index_add_ / cat semantics)
  nhc     ASE 3.29 NoseHooverChainNVT step order (gpu_nhc.py:1165-1195), pinned by conserved-
          energy drift, time reversibility, set_temperature identity and the harmonic closed form
  models  finite differences of the energy (forces), exact-zero padding, energy invariances
"""
