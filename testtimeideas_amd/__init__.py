"""MI355X (gfx950) grad-grad-safe attention: HIP kernels behind the
reference's ``ttt_kernels`` interface.

  testtimeideas_amd.ttt_kernels  - the reference-compatible Python surface
  testtimeideas_amd._lib         - ctypes binding of libttt_attn.so (C ABI in include/ttt_attn.h)
  testtimeideas_amd.workloads    - benchmark configurations, seeded inputs, FLOP/byte model
"""
__version__ = "0.1.0"
