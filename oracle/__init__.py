"""CPU oracle of neso's hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU (torch fp32/fp64 and numpy), the
algorithms of the reference kernels that ``neso_amd`` implements in HIP:

* ``oracle.attention`` — Flash-Attention-2 forward (closed form and the
  blockwise online-softmax loop), causal masking, both relative-position
  bias semantics, the Transformer-XL bias precompute;
* ``oracle.qmatmul`` — int4 packing / group-32 dequantisation / W4A16 matmul
  and the W8A16 (+ per-channel scale) references;
* ``oracle.inputs`` — seeded input generators: BASELINE configs and the
  reference tests' own generators.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg
of ``bench.py`` may import it, and only as the checker or as the timed CPU
baseline.  The product path (``neso_amd``) never imports or calls it and
fails loudly when its HIP library is missing.

Every function cites the reference file:line it follows.  How each is
pinned (golden vectors, closed forms, invariants, library routines) is in
``tests/test_oracle_attention.py`` and ``tests/test_oracle_qmatmul.py``.
"""
