// grouped-GEMM prefill kernels (MFMA) -- filled in next
