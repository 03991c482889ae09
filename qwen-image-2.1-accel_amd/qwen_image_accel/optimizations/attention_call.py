"""The attention core as the fused processors call it (outside this build).

The reference calls Diffusers' ``dispatch_attention_fn(q, k, v, attn_mask,
dropout_p=0.0, backend=..., parallel_config=...)`` with (B, S, H, D) tensors
(optimizations/fusion.py:31-34).  When Diffusers is importable that is what
runs here too, with the original processor's backend settings; otherwise
torch's scaled_dot_product_attention over the same layout, computed in fp32
and rounded back to the input dtype.
"""
import torch


def attention(q, k, v, attention_mask=None, processor=None):
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
