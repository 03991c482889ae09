"""The C ABI library: it loads without a GPU, exports every symbol include/qim.h
declares, binds to torch's HIP runtime, and rejects bad arguments with the
documented status codes before touching the device."""
import ctypes
import os
import re

import pytest

from qwen_image_accel import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qim.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qim_[a-z0-9_]+)\s*\(", text)))


def test_library_built():
    assert _native.available(), "run qwen-image-2.1-accel_amd/build_native.py (or __graft_entry__.build())"


def test_every_declared_symbol_is_exported():
    names = declared_functions()
    assert len(names) >= 14
    handle = ctypes.CDLL(_native.LIB_PATH)
    missing = [n for n in names if not hasattr(handle, n)]
    assert not missing, missing
    assert set(names) <= set(_native.SIGNATURES)


def test_single_hip_runtime():
    _native.lib()
    runtimes = _native.loaded_hip_runtimes()
    assert len(runtimes) == 1, runtimes


def test_abi_version():
    assert _native.lib().qim_abi_version() == 3


@pytest.mark.parametrize("name,args,code", [
    ("qim_mx_quantize", (None, 0, 1, 128, None, None, None), _native.QIM_ERR_ARG),
    ("qim_mx_quantize", (16, 128, 1, 100, 16, 16, None), _native.QIM_ERR_SHAPE),
    ("qim_mx_quantize", (17, 128, 1, 128, 16, 16, None), _native.QIM_ERR_LAYOUT),
    ("qim_gated_residual", (16, 16, 16, 16, 4, 12, 4, None), _native.QIM_ERR_SHAPE),
    # modulation terms: a period of 0, a row of kind 3, D not a multiple of 8
    ("qim_modulation_values", (16, 6, 16, 0, 0, 16, None), _native.QIM_ERR_ARG),
    ("qim_modulation_values", (16, 6, 16, 0b110000, 3, 16, None), _native.QIM_ERR_ARG),
    ("qim_modulation_values", (16, 6, 12, 0b100100, 3, 16, None), _native.QIM_ERR_SHAPE),
    ("qim_modulation_values", (16, 7, 16, 0b100100, 3, 16, None), _native.QIM_ERR_SHAPE),
    # rstd sweep: no counter buffer; patterns past 2^32; a misaligned counter buffer
    ("qim_debug_rstd_sweep", (0, 16, 0.0, None, None), _native.QIM_ERR_ARG),
    ("qim_debug_rstd_sweep", (0xffffff00, 0x200, 0.0, 16, None), _native.QIM_ERR_SHAPE),
    ("qim_debug_rstd_sweep", (0, 16, 0.0, 18, None), _native.QIM_ERR_LAYOUT),
    ("qim_swiglu", (16, 8, 16, 8, 16, 4, 1, 8, None), _native.QIM_ERR_LAYOUT),
    ("qim_rms_norm", (16, 16, 16, 4, 96, 1e-6, None), _native.QIM_ERR_SHAPE),
    ("qim_adaln", (16, 16, None, None, None, 16, 1, 16392, 1, 1e-6, 0, None), _native.QIM_ERR_SHAPE),
    ("qim_adaln_quantize", (16, 16, None, None, None, 16, 16, 1, 3000, 1, 1e-6, 0, None),
     _native.QIM_ERR_SHAPE),
    ("qim_mxfp8_gemm", (16, 16, 16, 16, 4, 320, 128, 0, None, None, None, 0, 16, 320, None, None),
     _native.QIM_ERR_SHAPE),
    # an fp32 and an fp16 output at once; an fp32 output with the bias epilogue
    ("qim_mxfp8_gemm_ex", (16, 16, 16, 16, 4, 256, 128, 0, 24, None, None, None, 0, 16, 256, None, None),
     _native.QIM_ERR_ARG),
    ("qim_mxfp8_gemm_ex", (16, 16, 16, 16, 4, 256, 128, 1, 8, 16, None, None, 0, 16, 256, None, None),
     _native.QIM_ERR_ARG),
    ("qim_mxfp8_gemm", (16, 16, 16, 16, 4, 256, 128, 9, None, None, None, 0, 16, 256, None, None),
     _native.QIM_ERR_ARG),
    ("qim_mxfp8_gemm", (16, 16, 16, 16, 4, 256, 128, 2, None, None, None, 0, 16, 256, None, None),
     _native.QIM_ERR_ARG),
    ("qim_mxfp8_gemm_ex", (16, 16, 16, 16, 4, 256, 128, 0, 32, None, None, None, 0, 16, 256, None, None),
     _native.QIM_ERR_ARG),
    ("qim_mxfp8_gemm_ex", (16, 16, 16, 16, 4, 256, 128, 0, 4, None, None, None, 0, 16, 256, None, None),
     _native.QIM_ERR_ARG),
    ("qim_mx_quantize_tiled", (16, 128, 1, 100, 16, 16, None), _native.QIM_ERR_SHAPE),
    # scaled-conversion hook: exponent 255; n not a multiple of 4
    ("qim_debug_e4m3_encode_scaled", (16, 255, 16, 64, None), _native.QIM_ERR_ARG),
    ("qim_debug_e4m3_encode_scaled", (16, 127, 16, 66, None), _native.QIM_ERR_ARG),
    ("qim_qk_norm_rope_pack", (16, 16, None, None, None, 16, 16, 16, 16, 16, None, 1, 4, 3, 2, 128,
                               256, 1e-6, 1e-6, None), _native.QIM_ERR_ARG),
    # attention: head dim 64; scale 0; a workspace smaller than the problem needs; misaligned q
    ("qim_attention", (16, 3072, 16, 3072, 16, 3072, 16, 3072, 16, 1 << 40, 1, 256, 256, 24, 64, 0.1, None),
     _native.QIM_ERR_SHAPE),
    ("qim_attention", (16, 3072, 16, 3072, 16, 3072, 16, 3072, 16, 1 << 40, 1, 256, 256, 24, 128, 0.0, None),
     _native.QIM_ERR_ARG),
    ("qim_attention", (16, 3072, 16, 3072, 16, 3072, 16, 3072, 16, 1024, 1, 256, 256, 24, 128, 0.1, None),
     _native.QIM_ERR_ARG),
    ("qim_attention", (18, 3072, 16, 3072, 16, 3072, 16, 3072, 16, 1 << 40, 1, 256, 256, 24, 128, 0.1, None),
     _native.QIM_ERR_LAYOUT),
    # QKV GEMM writing V^T: null vt; seq not a multiple of 64
    ("qim_mxfp8_gemm_qk_norm_rope_vt", (16, 16, 16, 16, 4352, 256, 24, 0, 16, 16, 16, 4352, 1e-6, 1e-6, 16, 9216,
                                        None, None), _native.QIM_ERR_ARG),
    ("qim_mxfp8_gemm_qk_norm_rope_vt", (16, 16, 16, 16, 4350, 256, 24, 0, 16, 16, 16, 4350, 1e-6, 1e-6, 16, 9216,
                                        16, None), _native.QIM_ERR_SHAPE),
    # attention with V^T from the workspace (v null) needs T % 64 == 0
    ("qim_attention", (16, 3072, 16, 3072, None, 0, 16, 3072, 16, 1 << 40, 1, 256, 250, 24, 128, 0.1, None),
     _native.QIM_ERR_SHAPE),
    # attention_mxfp8: null scales; tiled 2; misaligned codes
    ("qim_attention_mxfp8", (16, 3072, 16, 3072, 16, 3072, 16, None, 1, 16, 1 << 40, 1, 256, 256, 24, 128, 0.1,
                             None), _native.QIM_ERR_ARG),
    ("qim_attention_mxfp8", (16, 3072, 16, 3072, 16, 3072, 16, 16, 2, 16, 1 << 40, 1, 256, 256, 24, 128, 0.1,
                             None), _native.QIM_ERR_ARG),
    ("qim_attention_mxfp8", (16, 3072, 16, 3072, 16, 3072, 8, 16, 1, 16, 1 << 40, 1, 256, 256, 24, 128, 0.1,
                             None), _native.QIM_ERR_LAYOUT),
    # size limits: a GEMM output stride of 2^25 elements; N * K = 2^31 code bytes; a quantizer row of 2^23
    # elements (65536 scale blocks of 128); 2^30 heads of norm + RoPE
    ("qim_mxfp8_gemm", (16, 16, 16, 16, 4, 256, 128, 0, None, None, None, 0, 16, 1 << 25, None, None),
     _native.QIM_ERR_LAYOUT),
    ("qim_mxfp8_gemm", (16, 16, 16, 16, 4, 1 << 16, 1 << 15, 0, None, None, None, 0, 16, 1 << 16, None, None),
     _native.QIM_ERR_SHAPE),
    ("qim_mx_quantize", (16, 1 << 23, 1, 1 << 23, 16, 16, None), _native.QIM_ERR_SHAPE),
    ("qim_qk_norm_rope_pack", (16, 16, None, None, None, 16, 16, 16, 16, 16, None, 1, 4, 0, 1 << 30, 128,
                               1 << 37, 1e-6, 1e-6, None), _native.QIM_ERR_SHAPE),
    # GEMM with a workspace: a misaligned workspace
    ("qim_mxfp8_gemm_ws", (16, 16, 16, 16, 4352, 4096, 12288, 0, 0, None, None, None, 0, 16, 4096, None, 8, 1 << 24,
                           None), _native.QIM_ERR_LAYOUT),
    # attention without a workspace: v required; a problem above the scratch array (S = T = 16640, 24 heads)
    ("qim_attention_noalloc", (16, 3072, 16, 3072, None, 3072, 16, 3072, 1, 256, 256, 24, 128, 0.1, None),
     _native.QIM_ERR_ARG),
    ("qim_attention_noalloc", (16, 3072, 16, 3072, 16, 3072, 16, 3072, 1, 16640, 16640, 24, 128, 0.1, None),
     _native.QIM_ERR_SHAPE),
])
def test_argument_checks_return_status(name, args, code):
    """Rejected before any launch: fake (aligned or misaligned) addresses are
    never dereferenced."""
    fn = getattr(_native.lib(), name)
    rc = fn(*args)
    assert rc == code, (rc, _native.lib().qim_last_error())
    assert _native.lib().qim_last_error()


def test_call_raises_unsupported_and_qimerror():
    with pytest.raises(_native.Unsupported):
        _native.call("qim_mx_quantize", 16, 128, 1, 100, 16, 16, None)
    with pytest.raises(_native.QimError):
        _native.call("qim_mx_quantize", None, 0, 1, 128, None, None, None)


def test_gemm_workspace_bytes():
    """The split-K tail's workspace: 64 KiB of fp32 partial sums per quarter
    tile and K-split, for the plain, bias and gated-residual epilogues when the
    last partial round is at most CUs / 2 quarter tiles (256 CUs, the value
    assumed without a GPU); splits fill one round of the CUs, at most one
    stage pair (K = 128) each and at most 8."""
    lib = _native.lib()
    part = 64 * 1024
    gr, bias, none, swq = _native.EPI_GATED_RESIDUAL, _native.EPI_BIAS, _native.EPI_NONE, _native.EPI_SWIGLU_QUANT
    # 17 x 16 = 272 tiles: a tail of 16 tiles = 64 quarters, 4 splits each
    assert lib.qim_mxfp8_gemm_ws_bytes(4352, 4096, 12288, gr) == 64 * 4 * part
    assert lib.qim_mxfp8_gemm_ws_bytes(4352, 4096, 4096, none) == 64 * 4 * part
    # K = 256 is two stage pairs: two splits
    assert lib.qim_mxfp8_gemm_ws_bytes(4352, 4096, 256, bias) == 64 * 2 * part
    # 65 x 12 = 780 tiles (2048^2 out- and down-projections): 12 tail tiles, 48 quarters, 5 splits
    assert lib.qim_mxfp8_gemm_ws_bytes(16640, 3072, 12288, gr) == 48 * 5 * part
    # no tail (204 tiles), a tail of 192 quarters (one split), a split-less epilogue, a last 128-column block,
    # and shapes the GEMM rejects
    assert lib.qim_mxfp8_gemm_ws_bytes(4352, 3072, 12288, gr) == 0
    assert lib.qim_mxfp8_gemm_ws_bytes(4352, 12288, 3072, bias) == 0
    assert lib.qim_mxfp8_gemm_ws_bytes(4352, 8192, 4096, swq) == 0
    assert lib.qim_mxfp8_gemm_ws_bytes(4352, 4224, 4096, none) == 0
    assert lib.qim_mxfp8_gemm_ws_bytes(4352, 4096, 100, none) == 0
    assert lib.qim_mxfp8_gemm_ws_bytes(0, 4096, 4096, none) == 0


def test_attention_workspace_bytes():
    """V^T tiles (16 KiB per batch, head and 64-key block), plus, when the last
    partial round of work items is split over key ranges (the work split only
    counts CUs: 256 on MI355X, also the value assumed without a GPU),
    256 x 128 bf16 normalised output rows and 256 fp32 (m, l) pairs per chunk."""
    lib = _native.lib()
    vt = lambda b, t, h: b * h * -(-t // 64) * 16384  # noqa: E731
    part = 256 * 128 * 2 + 256 * 2 * 4
    assert lib.qim_attention_workspace_bytes(1, 4352, 4352, 24, 64) == 0
    assert lib.qim_attention_workspace_bytes(0, 4352, 4352, 24, 128) == 0
    # 408 items on 256 CUs: the last 152 run as 3 chunks of 23 key blocks
    # (456 chunks, two rounds of a third of an item each).
    assert lib.qim_attention_workspace_bytes(1, 4352, 4352, 24, 128) == vt(1, 4352, 24) + 152 * 3 * part
    # 1560 items: the last 24 run as 10 chunks of 26 key blocks.
    assert lib.qim_attention_workspace_bytes(1, 16640, 16640, 24, 128) == vt(1, 16640, 24) + 24 * 10 * part
    # 16 query blocks x 16 heads = 256 items, one whole round: no split
    assert lib.qim_attention_workspace_bytes(1, 4096, 8192, 16, 128) == vt(1, 8192, 16)
    for b, s, t, h in [(1, 300, 300, 2), (2, 520, 1500, 3), (1, 8, 20000, 1), (3, 700, 4352, 40)]:
        n = lib.qim_attention_workspace_bytes(b, s, t, h, 128)
        assert n >= vt(b, t, h) and (n - vt(b, t, h)) % part == 0
