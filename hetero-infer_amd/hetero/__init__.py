"""MI355X-native int4 GEMV path of hetero-infer: host-side package.

  q4           ctypes binding of kernel/libq4gemv.so (the HIP library)
  qlinear      QLinear, the reference's 4-bit projection operator, over the
               library's C-ABI (GEMV for decode, dequant + BLAS for prompts)
  numpy_stage  a NumPy Qwen2 stage driving the library through that ABI,
               the drop-in caller of the reference's CPU kernel
  gpu_model    the device-resident decode step (one HIP graph per token)
  qwen2        Qwen2 constants and seeded random-init 4-bit weights
  shard        safetensors checkpoint shard -> HBM loader and residency
  transport    the activation wire codec on the GPU
  synth        seeded synthetic weights and activations
"""
