"""helexa_amd: MI355X (gfx950) implementation of helexa neuron's Qwen3-Next
sparse-MoE block behind a C ABI (include/hx_moe.h, libhxmoe.so)."""
from .moe import (BF16, F16, F32, HX_DEVICE, HX_HOST, Q4_K, Q6_K, Q8_0, HxError, Qwen3_5MoeBlock, TextConfig,
                  dequantize, lib, quantize, quantize_activations, row_bytes)

__all__ = ["BF16", "F16", "F32", "HX_DEVICE", "HX_HOST", "Q4_K", "Q6_K", "Q8_0", "HxError", "Qwen3_5MoeBlock",
           "TextConfig", "dequantize", "lib", "quantize", "quantize_activations", "row_bytes"]
