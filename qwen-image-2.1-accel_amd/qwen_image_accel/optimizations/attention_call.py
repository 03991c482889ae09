"""The attention core as the fused processors call it (outside this build).

The reference calls Diffusers' ``dispatch_attention_fn(q, k, v, attn_mask,
dropout_p=0.0, backend=..., parallel_config=...)`` with (B, S, H, D) tensors
(optimizations/fusion.py:31-34).  When Diffusers is importable that is what
runs here too, with the original processor's backend settings; otherwise
torch's scaled_dot_product_attention over the same layout, computed in fp32
and rounded back to the input dtype.

``QW21_ATTENTION_BACKEND=qim`` (no reference counterpart; default "dispatch",
the reference's behaviour) runs this build's attention core instead
(``kernels.attention.attention``, libqim's ``qim_attention``) wherever it
applies: no mask, bf16 CUDA tensors, head dim 128, packed heads.
"""
import os

import torch

BACKENDS = ("dispatch", "qim")


def _qim_applies(q, k, v, attention_mask):
    if attention_mask is not None or q.dtype != torch.bfloat16 or not q.is_cuda or q.shape[-1] != 128:
        return False
    return all(t.dtype == q.dtype and t.device == q.device and t.stride(-1) == 1 and t.stride(-2) == 128
               and t.stride(0) == t.shape[1] * t.stride(1) for t in (q, k, v))


def qim_backend(q, k, v, attention_mask=None):
    """Whether this call goes to qim_attention (QW21_ATTENTION_BACKEND=qim and
    the inputs fit it)."""
    backend = os.environ.get("QW21_ATTENTION_BACKEND", "dispatch")
    if backend not in BACKENDS:
        raise ValueError(f"QW21_ATTENTION_BACKEND={backend!r}: choose from {BACKENDS}")
    return backend == "qim" and _qim_applies(q, k, v, attention_mask)


def attention(q, k, v, attention_mask=None, processor=None):
    if qim_backend(q, k, v, attention_mask):
        from qwen_image_accel.kernels.attention import attention as qim_attention
        return qim_attention(q, k, v)
    try:
        from diffusers.models.attention_dispatch import dispatch_attention_fn
    except ImportError:
        dispatch_attention_fn = None
    if dispatch_attention_fn is not None:
        return dispatch_attention_fn(q, k, v, attn_mask=attention_mask, dropout_p=0.0,
                                     backend=getattr(processor, "_attention_backend", None),
                                     parallel_config=getattr(processor, "_parallel_config", None))
    out = torch.nn.functional.scaled_dot_product_attention(
        q.transpose(1, 2).float(), k.transpose(1, 2).float(), v.transpose(1, 2).float(),
        attn_mask=attention_mask)
    return out.transpose(1, 2).to(q.dtype)
