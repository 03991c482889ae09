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
    ("qim_swiglu", (16, 8, 16, 8, 16, 4, 1, 8, None), _native.QIM_ERR_LAYOUT),
    ("qim_rms_norm", (16, 16, 16, 4, 96, 1e-6, None), _native.QIM_ERR_SHAPE),
    ("qim_adaln", (16, 16, None, None, None, 16, 1, 16392, 1, 1e-6, 0, None), _native.QIM_ERR_SHAPE),
    ("qim_adaln_quantize", (16, 16, None, None, None, 16, 16, 1, 3000, 1, 1e-6, 0, None),
     _native.QIM_ERR_SHAPE),
    ("qim_mxfp8_gemm", (16, 16, 16, 16, 4, 384, 128, 0, None, None, None, 0, 16, 384, None, None),
     _native.QIM_ERR_SHAPE),
    ("qim_mxfp8_gemm", (16, 16, 16, 16, 4, 256, 128, 9, None, None, None, 0, 16, 256, None, None),
     _native.QIM_ERR_ARG),
    ("qim_mxfp8_gemm", (16, 16, 16, 16, 4, 256, 128, 2, None, None, None, 0, 16, 256, None, None),
     _native.QIM_ERR_ARG),
    ("qim_mxfp8_gemm_ex", (16, 16, 16, 16, 4, 256, 128, 0, 8, None, None, None, 0, 16, 256, None, None),
     _native.QIM_ERR_ARG),
    ("qim_mxfp8_gemm_ex", (16, 16, 16, 16, 4, 256, 128, 0, 4, None, None, None, 0, 16, 256, None, None),
     _native.QIM_ERR_ARG),
    ("qim_mx_quantize_tiled", (16, 128, 1, 100, 16, 16, None), _native.QIM_ERR_SHAPE),
    ("qim_qk_norm_rope_pack", (16, 16, None, None, None, 16, 16, 16, 16, 16, None, 1, 4, 3, 2, 128,
                               256, 1e-6, 1e-6, None), _native.QIM_ERR_ARG),
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
