"""MI355X-native EXL3 trellis decode path (dense linear + routed-MoE decode).

Python host layer over libexl3_amd.so (hand-written gfx950 HIP kernels behind a
C ABI, include/exl3_amd.h).  Submodules:
  ops        torch custom ops over the C ABI (dequant, GEMM/GEMV, MoE decode)
  synth      seeded synthetic tensors of the benchmark shapes
"""

__all__ = ["ops", "synth"]
