"""Weight-side MXFP8 formats: the SwiGLU gate/up pair as one interleaved MXFP8
weight, and pre-quantized weights persisted to a file.

The reference quantizes every MXFP8 linear when the profile is installed
(optimizations/mxfp8.py:22-30, 66-91) and runs the SwiGLU gate and value
projections as two GEMMs whose bf16 outputs ``swiglu_quantize`` reads back
(optimizations/quantized_decode.py:81-96).  Here:

* ``interleave_quantized`` builds the (2F, K) weight the GEMM's SwiGLU epilogues
  take (rows in groups of ``QIM_SWIGLU_GROUP``: gate rows, then the same up
  rows) straight from the two quantized weights.  MXFP8 scales are per row and
  32-element K block, so permuting rows of the codes and of the (unswizzled)
  scales gives exactly the bytes of quantizing the interleaved bf16 weight; no
  requantization.  The decode MLP then runs one GEMM whose epilogue writes the
  down projection's MXFP8 input (no [M, 2F] bf16 round trip).
* ``fuse_qkv`` stacks the Q, K and V projections' quantized weights into one
  (3N, K) weight: the decode path's three projection GEMMs become one.
* ``save_mxfp8`` / ``load_mxfp8`` keep every converted linear's codes (tiled
  layout), scales and bias, and the fused gate/up and QKV weights, in a
  safetensors file; loading replaces the same linears without quantizing.
"""
import json

import torch
from torch import nn

from qwen_image_accel import _native
from qwen_image_accel.kernels.mxfp8 import BLOCK, padded_rows, tile_codes, untile_codes
from qwen_image_accel.optimizations.mxfp8 import MXFP8Linear

FORMAT = "qim-mxfp8"
VERSION = 1


def unswizzle_scales(scales, rows, k):
    """Flat swizzled E8M0 bytes of a (rows, k) tensor -> (padded rows, k / 32)
    row-major (the inverse of the 128x4 layout, kernels/mxfp8.py:53-56)."""
    m, kb = padded_rows(rows), k // BLOCK
    return scales.view(torch.uint8).reshape(m // 128, kb // 4, 32, 4, 4).permute(0, 3, 2, 1, 4).reshape(m, kb)


def swizzle_scales(exponents):
    """(padded rows, k / 32) row-major E8M0 bytes -> the flat swizzled layout."""
    m, kb = exponents.shape
    return exponents.reshape(m // 128, 4, 32, kb // 4, 4).permute(0, 3, 2, 1, 4).reshape(-1).contiguous()


def _interleave_rows(a, b, group):
    f = a.shape[0]
    return torch.stack([a.reshape(f // group, group, -1), b.reshape(f // group, group, -1)], dim=1).reshape(2 * f, -1)


def interleave_quantized(gate, up, group=_native.SWIGLU_GROUP):
    """(codes, scales) of the interleaved gate/up weight from two
    ``MXFP8Linear`` s of the same (F, K) shape: the tiled codes (2F, K) and the
    swizzled scales, byte-identical to quantizing ``gemm.interleave_swiglu``
    of the two bf16 weights."""
    f, k = gate.out_features, gate.in_features
    if (up.out_features, up.in_features) != (f, k) or f % 128 or k % 128:
        raise ValueError("gate and up must both be (F, K) with F, K multiples of 128")
    codes = _interleave_rows(untile_codes(gate.weight_tiled).view(torch.uint8),
                             untile_codes(up.weight_tiled).view(torch.uint8), group)
    exps = _interleave_rows(unswizzle_scales(gate.weight_scale, f, k), unswizzle_scales(up.weight_scale, f, k), group)
    return (tile_codes(codes.view(gate.weight_tiled.dtype)).contiguous(),
            swizzle_scales(exps).view(gate.weight_scale.dtype))


def fuse_gate_up(mlp):
    """Attach the interleaved gate/up weight to a SwiGLU MLP whose gate and
    value projections are MXFP8 (``mlp._mx_gate_up``, used by the decode MLP).
    Returns whether it did.  Needs F % 256 == 0 (the SwiGLU epilogue's N) and
    bias-free projections."""
    gate, up = getattr(mlp, "gate_layer", None), getattr(mlp, "proj", None)
    if not (isinstance(gate, MXFP8Linear) and isinstance(up, MXFP8Linear)) or gate.out_features % 256:
        return False
    if gate.bias is not None or up.bias is not None:  # the SwiGLU epilogue adds no bias
        return False
    if (up.out_features, up.in_features) != (gate.out_features, gate.in_features):
        return False
    mlp._mx_gate_up = interleave_quantized(gate, up)
    return True


def fuse_qkv(attn):
    """Attach the Q, K and V projections of an attention module as one MXFP8
    weight (``attn._mx_qkv``: rows Q, then K, then V), so that the decode
    path runs one GEMM instead of three.  Needs three MXFP8 linears of the
    same (N, K) with N % 256 == 0: the tiled codes of each are whole 256-row
    super-blocks and its swizzled scales whole 128-row tiles, so both
    concatenate as flat byte arrays.  Returns whether it did."""
    ps = [getattr(attn, n, None) for n in ("to_q", "to_k", "to_v")]
    if not all(isinstance(p, MXFP8Linear) and p.bias is None for p in ps):  # one plain GEMM: no biases
        return False
    n, k = ps[0].out_features, ps[0].in_features
    if any((p.out_features, p.in_features) != (n, k) for p in ps) or n % 256:
        return False
    attn._mx_qkv = (torch.cat([p.weight_tiled for p in ps], 0), torch.cat([p.weight_scale for p in ps], 0))
    return True


_FUSED = ("_mx_gate_up", "_mx_qkv")


def _modules(transformer):
    """(path, module) over the DiT blocks, paths as quantize_transformer names
    them ("transformer_blocks.<i>.<name>")."""
    for i, block in enumerate(transformer.transformer_blocks):
        for name, m in block.named_modules():
            yield (f"transformer_blocks.{i}.{name}" if name else f"transformer_blocks.{i}"), m


def _resolve(transformer, path):
    _, i, rest = path.split(".", 2) if path.count(".") >= 2 else (*path.split("."), "")
    block = transformer.transformer_blocks[int(i)]
    return block.get_submodule(rest) if rest else block


def _set(transformer, path, module):
    parent, _, leaf = path.rpartition(".")
    setattr(_resolve(transformer, parent), leaf, module)


def save_mxfp8(transformer, path):
    """Write every ``MXFP8Linear`` of ``transformer`` (tiled codes, scales,
    bias) and every interleaved gate/up weight to a safetensors file."""
    from safetensors.torch import save_file
    tensors, layers, fused = {}, {}, []
    for name, m in _modules(transformer):
        if not isinstance(m, MXFP8Linear):
            continue
        tensors[f"{name}.codes"] = m.weight_tiled.view(torch.uint8).cpu().contiguous()
        tensors[f"{name}.scales"] = m.weight_scale.view(torch.uint8).cpu().contiguous()
        if m.bias is not None:
            tensors[f"{name}.bias"] = m.bias.cpu().contiguous()
        layers[name] = [m.in_features, m.out_features]
    for name, mod in _modules(transformer):
        for attr in _FUSED:
            w = getattr(mod, attr, None)
            if w is not None:
                tensors[f"{name}.{attr}.codes"] = w[0].view(torch.uint8).cpu().contiguous()
                tensors[f"{name}.{attr}.scales"] = w[1].view(torch.uint8).cpu().contiguous()
                fused.append(f"{name}.{attr}")
    meta = {"format": FORMAT, "version": str(VERSION), "swiglu_group": str(_native.SWIGLU_GROUP),
            "layers": json.dumps(layers), "fused": json.dumps(fused)}
    save_file(tensors, path, metadata=meta)
    return sorted(layers)


def load_mxfp8(transformer, path, device=None):
    """Replace the linears named in a ``save_mxfp8`` file by ``MXFP8Linear`` s
    holding the saved bytes (no quantization), and restore the interleaved
    gate/up weights.  Returns the converted module paths."""
    from safetensors import safe_open
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT or int(meta.get("version", -1)) != VERSION:
            raise ValueError(f"{path}: not a {FORMAT} v{VERSION} file")
        if int(meta["swiglu_group"]) != _native.SWIGLU_GROUP:
            raise ValueError(f"{path}: SwiGLU group {meta['swiglu_group']} != {_native.SWIGLU_GROUP}")
        keys = set(f.keys())
        loaded = []
        for name, (k, n) in sorted(json.loads(meta["layers"]).items()):
            old = _resolve(transformer, name)
            if not isinstance(old, (nn.Linear, MXFP8Linear)) or (old.in_features, old.out_features) != (k, n):
                raise ValueError(f"{path}: {name} is not a ({n}, {k}) linear in this model")
            dev = device if device is not None else next(old.buffers(), next(old.parameters(), None)).device
            bias = f.get_tensor(f"{name}.bias").to(dev) if f"{name}.bias" in keys else None
            new = MXFP8Linear.from_quantized(k, n, f.get_tensor(f"{name}.codes").to(dev),
                                             f.get_tensor(f"{name}.scales").to(dev), bias)
            _set(transformer, name, new)
            loaded.append(name)
        for key in json.loads(meta["fused"]):
            name, _, attr = key.rpartition(".")
            if attr not in _FUSED:
                raise ValueError(f"{path}: unknown fused weight {key}")
            mod = _resolve(transformer, name)
            ref = mod.gate_layer if attr == "_mx_gate_up" else mod.to_q
            dev = ref.weight_tiled.device
            setattr(mod, attr, (f.get_tensor(f"{key}.codes").to(dev).view(ref.weight_tiled.dtype),
                                f.get_tensor(f"{key}.scales").to(dev).view(ref.weight_scale.dtype)))
    return loaded


__all__ = ["unswizzle_scales", "swizzle_scales", "interleave_quantized", "fuse_gate_up", "fuse_qkv", "save_mxfp8",
           "load_mxfp8"]
