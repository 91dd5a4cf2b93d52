"""loractl_amd — MI355X (gfx950) kernels for loractl's quantized frozen-base
LoRA linear, behind a C ABI (include/loractl_rocm.h, libloractl_rocm.so).

Modules:
  quant     QuantBackend / quantize_linear_weight / chunking (src/quant.rs)
  fp8       e4m3fn weights and their scale sidecars (src/fp8.rs decode half)
  lora      LoraDelta and the fused quantized site op (src/lora.rs)
  adapters  LoraAdapters, build_adapters, QuantLinear, site() (src/adapters.rs,
            src/mmdit.rs:413-536)
  accuracy  RelGate / rel_deviation (src/accuracy.rs)
  device    the ctypes calls into libloractl_rocm.so (torch tensors as
            device memory, torch's current stream)

Importing the package does not load the GPU library; the first compute call
does, and raises if it is not built.
"""

__all__ = ["quant", "fp8", "lora", "adapters", "accuracy", "device"]
