"""GPU kernels of the per-block hot path, one module per reference module
(src/qwen_image_accel/kernels/): mxfp8, epilogue, layernorm, bf16,
elementwise, attention, plus gemm for the MXFP8 matmul call site."""
