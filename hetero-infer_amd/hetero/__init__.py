"""MI355X-native int4 GEMV path of hetero-infer: host-side package.

  q4         ctypes binding of kernel/libq4gemv.so (the HIP library)
  cpu_model  the NumPy Qwen2 stage of the reference, driving libq4gemv.so
             through the same C-ABI as the reference's CPU kernel
  synth      seeded synthetic weights and activations
"""
