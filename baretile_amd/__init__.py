"""baretile for MI355X: baretile's hot path, the fused block-float matmul and the KV-cache attention, on gfx950.

Modules mirror baretile's: pci, chip, runtime, tensor, and models.llama. The kernels are HIP, in
libbaretile_amd.so (csrc/), reached through the C ABI of include/baretile_amd.h by ctypes (_lib).
"""
