"""MXFP8 linears of the DiT blocks, multiplied by libqim's scaled-MFMA GEMM.

Reference interface: src/qwen_image_accel/optimizations/mxfp8.py --
``MXFP8Linear`` (:19-41), ``LAYER_GROUPS`` (:46-50), ``selected_layers``
(:53-63), ``quantize_transformer`` (:66-91), and the conversion rule
(:15-16: K and N multiples of 128).

Storage.  The weight is quantized once with the activation quantizer and kept
once, as (N, K) E4M3 codes in the GEMM's tiled layout (buffer
``weight_tiled``), plus the swizzled E8M0 scales over N rows
(``weight_scale``).  The reference keeps ``weight_fp8``, the (K, N) transpose
view of row-major codes; that view is what ``weight_fp8`` returns and what a
state dict holds, so state dicts move both ways between the reference's
module and this one: saving writes ``weight_fp8`` / ``weight_scale``,
loading accepts ``weight_fp8`` in any memory format (the (K, Np) transpose
view, or a contiguous copy of it as safetensors gives back) and tiles it.
"""
import os

import torch
from torch import nn

from qwen_image_accel.kernels.gemm import mx_matmul
from qwen_image_accel.kernels.mxfp8 import Quantized, padded_rows, quantize, tile_codes, untile_codes

CONVERTIBLE_MULTIPLE = 128  # K and N of a linear the GEMM takes


def convertible(linear):
    """Whether ``linear`` becomes an MXFP8Linear (K, N multiples of 128)."""
    return (isinstance(linear, nn.Linear) and linear.in_features % CONVERTIBLE_MULTIPLE == 0
            and linear.out_features % CONVERTIBLE_MULTIPLE == 0)


class MXFP8Linear(nn.Module):
    """A linear layer held and multiplied in MXFP8.

    A biased linear is refused (``ValueError``), as in the reference, unless
    ``allow_bias=True``, which adds the bias in the GEMM's epilogue."""

    def __init__(self, linear, *, allow_bias=False):
        super().__init__()
        if linear.bias is not None and not allow_bias:
            raise ValueError("Qwen 2.1 DiT MXFP8 conversion expects bias-free linears")
        q = quantize(linear.weight.detach().to(torch.bfloat16).contiguous(), tiled=True)
        bias = None if linear.bias is None else linear.bias.detach().to(torch.bfloat16).contiguous()
        self._hold(linear.in_features, linear.out_features, q.values, q.scales, bias)

    def _hold(self, k, n, codes, scales, bias):
        self.in_features, self.out_features = k, n
        self.register_buffer("weight_tiled", codes)
        self.register_buffer("weight_scale", scales)
        self.register_buffer("bias", bias)

    @classmethod
    def from_quantized(cls, in_features, out_features, weight_tiled, weight_scale, bias=None):
        """An ``MXFP8Linear`` over already quantized bytes (no quantization):
        (padded N, K) E4M3 codes in the tiled layout and the swizzled scales."""
        rows = padded_rows(out_features)
        codes = weight_tiled.view(torch.float8_e4m3fn)
        scales = weight_scale.view(torch.float8_e8m0fnu).reshape(-1)
        if codes.shape != (rows, in_features) or scales.numel() != rows * in_features // 32:
            raise ValueError(f"quantized weight does not match a ({out_features}, {in_features}) linear")
        self = cls.__new__(cls)
        nn.Module.__init__(self)
        self._hold(in_features, out_features, codes, scales, bias)
        return self

    def matmul(self, activation, dtype=torch.bfloat16, **epilogue):
        """``activation`` (a ``Quantized``, shared by several weights if need
        be) times the weight: (activation rows, N) of ``dtype`` (bf16, fp32 or
        fp16, like torch._scaled_mm's out_dtype).  Keyword-only epilogue
        arguments are ``kernels.gemm.mx_matmul``'s."""
        if self.bias is not None and "epilogue" not in epilogue:
            epilogue = {**epilogue, "epilogue": "bias", "bias": self.bias}
        return mx_matmul(activation, self.weight_tiled, self.weight_scale, weight_tiled=True, dtype=dtype,
                         **epilogue)

    def forward(self, x):
        lead = x.shape[:-1]
        rows = x.reshape(-1, self.in_features).contiguous()
        return self.matmul(quantize(rows, tiled=True), x.dtype).view(*lead, self.out_features)

    @property
    def weight_fp8(self):
        """The reference's view of the codes: (K, padded N), column-major (a copy)."""
        return untile_codes(self.weight_tiled).t()

    # State dicts carry the reference's keys and layout.
    def _save_to_state_dict(self, destination, prefix, keep_vars):
        super()._save_to_state_dict(destination, prefix, keep_vars)
        del destination[prefix + "weight_tiled"]
        destination[prefix + "weight_fp8"] = self.weight_fp8

    def _load_from_state_dict(self, state_dict, prefix, *args, **kwargs):
        key = prefix + "weight_fp8"
        if key in state_dict:
            codes = state_dict.pop(key)
            want = (self.in_features, padded_rows(self.out_features))
            if tuple(codes.shape) != want:
                raise ValueError(f"{key}: shape {tuple(codes.shape)}, expected (K, padded N) = {want}")
            state_dict[prefix + "weight_tiled"] = tile_codes(codes.t().contiguous())
        super()._load_from_state_dict(state_dict, prefix, *args, **kwargs)


# The block-relative paths each QW21_MXFP8_LAYERS group names (reference :46-50).
LAYER_GROUPS = {
    "attention": ("attn.to_q", "attn.to_k", "attn.to_v", "attn.to_out.0"),
    "mlp": ("img_mlp.gate_layer", "img_mlp.proj", "img_mlp.out"),
}
LAYER_GROUPS["all"] = LAYER_GROUPS["attention"] + LAYER_GROUPS["mlp"]


def selected_layers(selection=None):
    """The set of block-relative linear paths a QW21_MXFP8_LAYERS value names:
    a key of LAYER_GROUPS, or paths from LAYER_GROUPS["all"] separated by
    commas.  ``selection`` overrides the environment (default "all")."""
    spec = (os.environ.get("QW21_MXFP8_LAYERS", "all") if selection is None else selection).strip()
    if spec in LAYER_GROUPS:
        return set(LAYER_GROUPS[spec])
    requested = {part.strip() for part in spec.split(",")} - {""}
    invalid = sorted(requested.difference(LAYER_GROUPS["all"]))
    if invalid:
        raise ValueError(f"Unknown MXFP8 layer names {invalid}; "
                         f"choose from {sorted(LAYER_GROUPS['all'])} or {sorted(LAYER_GROUPS)}")
    return requested


def skipped_blocks(spec=None):
    """Block indices a QW21_MXFP8_SKIP_BLOCKS value names (default "0,31")."""
    raw = os.environ.get("QW21_MXFP8_SKIP_BLOCKS", "0,31") if spec is None else spec
    return {int(part) for part in str(raw).split(",") if part.strip()}


def conversion_plan(transformer, skip_blocks=None, layers=None):
    """The (block index, block-relative path, linear) triples
    quantize_transformer converts: the selected paths of every block not
    skipped whose module is a convertible linear, by block, paths sorted."""
    skip, paths = skipped_blocks(skip_blocks), sorted(selected_layers(layers))
    return [(i, path, block.get_submodule(path))
            for i, block in enumerate(transformer.transformer_blocks) if i not in skip
            for path in paths if convertible(block.get_submodule(path))]


def _replace(block, path, module):
    parent, _, leaf = path.rpartition(".")
    setattr(block.get_submodule(parent) if parent else block, leaf, module)


def quantize_transformer(transformer, skip_blocks=None, layers=None):
    """Swap the planned linears for MXFP8Linear (everything else stays bf16)
    and return their module paths ("transformer_blocks.<i>.<path>")."""
    plan = conversion_plan(transformer, skip_blocks, layers)
    blocks = transformer.transformer_blocks
    with torch.no_grad():
        for i, path, linear in plan:
            _replace(blocks[i], path, MXFP8Linear(linear))
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    return [f"transformer_blocks.{i}.{path}" for i, path, _ in plan]


__all__ = ["MXFP8Linear", "LAYER_GROUPS", "selected_layers", "skipped_blocks", "conversion_plan",
           "quantize_transformer", "convertible", "Quantized"]
