"""MI355X-native token-sampling hot path of DeepSeekRPC.

Modules:
  sampling, terminal_sampling, jsonutil  drop-in replacements of the
                                         reference's sampling API
  batch                                  batched device API (rows in HBM)
  workloads                              seeded synthetic row families
  build                                  hipcc build of libdsr_sampling.so
The kernels live in csrc/ and are reached through the C ABI in
include/dsr_sampling.h.
"""
__version__ = "0.1.0"
