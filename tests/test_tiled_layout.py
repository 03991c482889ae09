"""The GEMM's tiled E4M3 code layout (include/qim.h, QIM_GEMM_A_TILED): the
torch converters against the layout's byte formula, evaluated code by code.

The layout has no reference counterpart (the reference hands row-major codes to
torch._scaled_mm); what fixes it is the header's definition, restated here as a
per-code offset and compared with ``tile_codes`` / ``untile_codes``, which
build it by reshapes and gathers.  GPU tests then hold every kernel that writes
or reads tiled codes to ``tile_codes`` of the row-major result.
"""
import numpy as np
import pytest
import torch

from qwen_image_accel.kernels import mxfp8


def tiled_offset(r, k, rows, width):
    """Byte offset of code (r, k) of a (rows, width) matrix in the tiled layout."""
    r0 = r - r % 256
    n = min(256, rows - r0)
    chunk = ((k % 64) // 16) ^ (((r >> 1) ^ (r >> 2)) & 3)
    return r0 * width + (k // 64) * n * 64 + (r - r0) * 64 + chunk * 16 + k % 16


def random_codes(rows, width, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 256, (rows, width), generator=g, dtype=torch.uint8).view(torch.float8_e4m3fn)


@pytest.mark.parametrize("rows,width", [(128, 64), (256, 128), (384, 192), (640, 128)])
def test_tile_codes_matches_the_layout_formula(rows, width):
    codes = random_codes(rows, width, rows + width)
    src = codes.view(torch.uint8).numpy()
    want = np.empty(rows * width, np.uint8)
    for r in range(rows):
        for k in range(width):
            want[tiled_offset(r, k, rows, width)] = src[r, k]
    got = mxfp8.tile_codes(codes).view(torch.uint8).reshape(-1).numpy()
    assert np.array_equal(got, want)


def test_layout_formula_is_a_permutation():
    rows, width = 384, 256
    offs = {tiled_offset(r, k, rows, width) for r in range(rows) for k in range(width)}
    assert offs == set(range(rows * width))


@pytest.mark.parametrize("rows,width", [(128, 128), (384, 3072), (4224, 256)])
def test_untile_inverts_tile(rows, width):
    codes = random_codes(rows, width, 7)
    tiled = mxfp8.tile_codes(codes)
    assert tiled.shape == codes.shape and tiled.dtype == codes.dtype
    assert torch.equal(mxfp8.untile_codes(tiled).view(torch.uint8), codes.view(torch.uint8))


def test_sixteen_row_group_is_one_contiguous_kib():
    """Each 16-row group of one 64-byte K-slab is the 1 KiB LDS image of the
    GEMM's DMA: rows in order, 16-byte chunks permuted by the row's swizzle."""
    rows, width = 256, 192
    codes = random_codes(rows, width, 3)
    tiled = mxfp8.tile_codes(codes).view(torch.uint8).reshape(-1).numpy()
    src = codes.view(torch.uint8).numpy()
    for s in range(width // 64):
        for grp in range(rows // 16):
            block = tiled[s * rows * 64 + grp * 1024:][:1024].reshape(16, 4, 16)
            for i in range(16):
                r = grp * 16 + i
                sw = ((r >> 1) ^ (r >> 2)) & 3
                for c in range(4):
                    assert np.array_equal(block[i, c ^ sw], src[r, s * 64 + c * 16:s * 64 + c * 16 + 16])


def test_bad_shapes_rejected():
    with pytest.raises(ValueError):
        mxfp8.tile_codes(random_codes(100, 128, 0))
    with pytest.raises(ValueError):
        mxfp8.tile_codes(random_codes(128, 96, 0))


def test_tiled_quantized_is_a_quantized():
    q = mxfp8.TiledQuantized(torch.empty(0), torch.empty(0), 0, torch.Size((0, 0)))
    assert isinstance(q, mxfp8.Quantized) and q.tiled and not mxfp8.Quantized(*q).tiled
    values, scales, rows, shape = q
    assert type(q._replace(rows=3)) is mxfp8.TiledQuantized
