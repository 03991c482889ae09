"""MI355X (gfx950) implementation of Qwen-Image-2.1-Accel's per-block hot path.

The public modules keep the reference package's names
(src/qwen_image_accel/kernels/*, optimizations/mxfp8.py, profiles.py); the
arithmetic runs in hand-written HIP kernels (libqim.so, C ABI in
include/qim.h) reached through ``qwen_image_accel._native``.
"""
__version__ = "0.1.0"


def __getattr__(name):
    # Lazy like the reference (src/qwen_image_accel/__init__.py:14-17): importing
    # the package does not import torch.
    if name == "configure_pipeline":
        from qwen_image_accel.pipeline import configure_pipeline
        return configure_pipeline
    raise AttributeError(name)
