"""Replace transformer linears with MXFP8 linears backed by the CDNA4 GEMM.

Reference interface: src/qwen_image_accel/optimizations/mxfp8.py --
``MXFP8Linear`` (:19-41), ``LAYER_GROUPS`` (:46-50), ``selected_layers``
(:53-63), ``quantize_transformer`` (:66-91).  Weights are quantized once with
the same quantizer as activations.  The reference keeps ``weight_fp8`` = the
(K, N) column-major view of the row-major (N, K) codes; here the same codes are
kept once, in the GEMM's tiled layout (buffer ``weight_tiled``), so every DMA
instruction of the GEMM reads 1 KiB contiguous.  ``weight_fp8`` remains
readable (a row-major copy in the reference's view), and a state dict saved by
the reference (``weight_fp8``) loads: its codes are tiled on the way in.
``weight_scale`` is the swizzled exponents over N rows in both.
"""
import os

import torch
from torch import nn

from qwen_image_accel.kernels.gemm import mx_matmul
from qwen_image_accel.kernels.mxfp8 import Quantized, padded_rows, quantize, tile_codes, untile_codes


def _supported(k, n):
    return k % 128 == 0 and n % 256 == 0


class MXFP8Linear(nn.Module):
    """Linear whose weight is stored as MXFP8 and multiplied as MXFP8.

    Like the reference it rejects a bias unless ``allow_bias=True``; then the
    bias is added in the GEMM epilogue (the config-4 "fused bias" form)."""

    def __init__(self, linear, *, allow_bias=False):
        super().__init__()
        if linear.bias is not None and not allow_bias:
            raise ValueError("Qwen 2.1 DiT MXFP8 conversion expects bias-free linears")
        self.in_features, self.out_features = linear.in_features, linear.out_features
        weight = linear.weight.detach().to(torch.bfloat16).contiguous()
        quantized = quantize(weight, tiled=True)
        self.register_buffer("weight_tiled", quantized.values)     # (N, K) codes, tiled layout
        self.register_buffer("weight_scale", quantized.scales)
        self.register_buffer("bias", None if linear.bias is None
                             else linear.bias.detach().to(torch.bfloat16).contiguous())

    @classmethod
    def from_quantized(cls, in_features, out_features, weight_tiled, weight_scale, bias=None):
        """An ``MXFP8Linear`` holding already quantized bytes, without quantizing:
        the (N, K) E4M3 codes in the tiled layout (N padded to 128) and the
        swizzled E8M0 scales, as ``weight_tiled`` / ``weight_scale`` hold them."""
        rows = padded_rows(out_features)
        codes = weight_tiled.view(torch.float8_e4m3fn)
        scales = weight_scale.view(torch.float8_e8m0fnu).reshape(-1)
        if codes.shape != (rows, in_features) or scales.numel() != rows * in_features // 32:
            raise ValueError(f"quantized weight does not match a ({out_features}, {in_features}) linear")
        self = cls.__new__(cls)
        nn.Module.__init__(self)
        self.in_features, self.out_features = in_features, out_features
        self.register_buffer("weight_tiled", codes)
        self.register_buffer("weight_scale", scales)
        self.register_buffer("bias", bias)
        return self

    def matmul(self, activation, dtype=torch.bfloat16, **epilogue):
        """Multiply an already quantized activation; several weights can share one.

        Keyword-only epilogue arguments are those of ``kernels.gemm.mx_matmul``."""
        if dtype != torch.bfloat16:
            raise ValueError("the MXFP8 GEMM writes bfloat16")
        if self.bias is not None and "epilogue" not in epilogue:
            epilogue = dict(epilogue, epilogue="bias", bias=self.bias)
        return mx_matmul(activation, self.weight_tiled, self.weight_scale, weight_tiled=True, **epilogue)

    def forward(self, x):
        flat = x.reshape(-1, x.shape[-1])
        activation = quantize(flat if flat.is_contiguous() else flat.contiguous(), tiled=True)
        return self.matmul(activation, x.dtype).reshape(*x.shape[:-1], self.out_features)

    @property
    def weight_fp8(self):
        """The reference's view of the weight codes: (K, N) column-major (a copy)."""
        return untile_codes(self.weight_tiled).t()

    def _load_from_state_dict(self, state_dict, prefix, *args, **kwargs):
        key = prefix + "weight_fp8"
        if key in state_dict:  # a reference state dict: (K, N) view of row-major (N, K) codes
            codes = state_dict.pop(key)
            state_dict[prefix + "weight_tiled"] = tile_codes(codes.t() if codes.t().is_contiguous() else codes)
        super()._load_from_state_dict(state_dict, prefix, *args, **kwargs)


# Which of a block's linears each selection converts (reference :46-50).
LAYER_GROUPS = {
    "attention": ("attn.to_q", "attn.to_k", "attn.to_v", "attn.to_out.0"),
    "mlp": ("img_mlp.gate_layer", "img_mlp.proj", "img_mlp.out"),
}
LAYER_GROUPS["all"] = LAYER_GROUPS["attention"] + LAYER_GROUPS["mlp"]


def selected_layers(selection=None):
    """Resolve QW21_MXFP8_LAYERS: a group name or an explicit comma-separated list."""
    raw = (selection if selection is not None else os.environ.get("QW21_MXFP8_LAYERS", "all")).strip()
    if raw in LAYER_GROUPS:
        return set(LAYER_GROUPS[raw])
    names = {n.strip() for n in raw.split(",") if n.strip()}
    unknown = names - set(LAYER_GROUPS["all"])
    if unknown:
        raise ValueError(f"Unknown MXFP8 layer names {sorted(unknown)}; "
                         f"choose from {sorted(LAYER_GROUPS['all'])} or {sorted(LAYER_GROUPS)}")
    return names


def quantize_transformer(transformer, skip_blocks=None, layers=None):
    """Replace selected DiT block linears with MXFP8; everything else stays BF16.

    Blocks listed in ``QW21_MXFP8_SKIP_BLOCKS`` (default "0,31") keep every
    linear in BF16.  Returns the converted module paths."""
    raw = skip_blocks if skip_blocks is not None else os.environ.get("QW21_MXFP8_SKIP_BLOCKS", "0,31")
    skip = {int(i) for i in str(raw).split(",") if i.strip()}
    wanted = selected_layers(layers)
    converted = []
    with torch.no_grad():
        for index, block in enumerate(transformer.transformer_blocks):
            if index in skip:
                continue
            for name in sorted(wanted):
                child = block.get_submodule(name)
                if not isinstance(child, nn.Linear) or not _supported(child.in_features, child.out_features):
                    continue
                parent_name, _, leaf = name.rpartition(".")
                parent = block.get_submodule(parent_name) if parent_name else block
                setattr(parent, leaf, MXFP8Linear(child))
                converted.append(f"transformer_blocks.{index}.{name}")
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    return converted


__all__ = ["MXFP8Linear", "LAYER_GROUPS", "selected_layers", "quantize_transformer", "Quantized"]
