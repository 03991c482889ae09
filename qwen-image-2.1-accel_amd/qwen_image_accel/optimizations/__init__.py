"""Call sites of the hot-path kernels (reference src/qwen_image_accel/optimizations/)."""
