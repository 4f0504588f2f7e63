"""MI355X (gfx950) implementation of the GLIF_3 V1 cell hot path of
JavierGalvan9/V1_GLIF_model: the event-driven synaptic-current operator with its
custom gradient, and the fused GLIF_3 step with BPTT, as HIP kernels behind the
C ABI in include/glif.h.

Python mirror of the reference interface:
  ops.make_pre_ind_table, ops.calculate_synaptic_currents   (models.py:103-373)
  models.V1Column                                          (models.py:450-1135)
Synthetic networks of the benchmark configurations: synthetic.make_network.
"""
__version__ = "0.1.0"
