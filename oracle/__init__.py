"""CPU restatement of the reference's GLIF_3 cell hot path: the parity checker.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package.  The product path
(``v1_glif_model_amd``) never imports, links or calls anything here and fails
loudly when its HIP library is missing.

Contents (each function cites the reference file:line it follows):

* ``glif_oracle.c`` / ``cpu.py`` -- plain-C restatement in the reference's fp32
  accumulation order: CSR build, spike compaction, synaptic-current forward and
  custom gradient, the T-step cell forward and its BPTT.
* ``dense.py`` -- numpy float64 brute force of the synaptic operator (dense
  per-receptor matrices) and the reference's own numpy CSR fallback.
* ``torch_ref.py`` -- a float64 PyTorch autograd restatement of ``V1Column.call``
  used to pin the hand-derived BPTT of ``glif_oracle.c``.

How each function is pinned (none of the reference's own tests ship with it, so
there are no reference golden vectors): see the module docstrings and
``tests/test_oracle.py``.
"""
