"""ctypes binding of libqim.so (the HIP kernels behind include/qim.h).

torch is imported before the library is opened so that libqim.so binds to the
HIP runtime torch already loaded (both name libamdhip64.so.7); device pointers
and streams are then shared.  There is no CPU fallback here: if the library is
missing every call raises NativeUnavailable.
"""
import ctypes
import os
import threading

import torch

LIB_PATH = os.environ.get("QIM_LIBRARY", os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                       "libqim.so"))

QIM_OK, QIM_ERR_ARG, QIM_ERR_SHAPE, QIM_ERR_LAYOUT, QIM_ERR_LAUNCH = range(5)
ADALN_ADD_ONE, ADALN_TILED = 1, 2
GEMM_A_TILED, GEMM_B_TILED, GEMM_OUT_TILED, GEMM_OUT_F32, GEMM_OUT_F16 = 1, 2, 4, 8, 16
EPI_NONE, EPI_BIAS, EPI_GATED_RESIDUAL, EPI_SWIGLU, EPI_SWIGLU_QUANT, EPI_QK_NORM_ROPE = range(6)
SWIGLU_GROUP = 32


class QimError(RuntimeError):
    """A libqim entry point returned a nonzero status."""

    def __init__(self, name, code, message):
        super().__init__(f"{name} failed (status {code}): {message}")
        self.code = code


class Unsupported(QimError):
    """The kernels do not support this shape, stride or alignment."""


class NativeUnavailable(RuntimeError):
    """libqim.so is not built or cannot be loaded."""


_P = ctypes.c_void_p
_I = ctypes.c_int64
_F = ctypes.c_float
_C = ctypes.c_int
_U = ctypes.c_uint32

SIGNATURES = {
    "qim_last_error": (ctypes.c_char_p, []),
    "qim_abi_version": (_C, []),
    "qim_mx_quantize": (_C, [_P, _I, _I, _I, _P, _P, _P]),
    "qim_mx_quantize_tiled": (_C, [_P, _I, _I, _I, _P, _P, _P]),
    "qim_adaln": (_C, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _C, _P]),
    "qim_adaln_quantize": (_C, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _C, _P]),
    "qim_gated_residual": (_C, [_P, _P, _P, _P, _I, _I, _I, _P]),
    "qim_modulation_values": (_C, [_P, _I, _I, _U, _C, _P, _P]),
    "qim_swiglu": (_C, [_P, _I, _P, _I, _P, _I, _I, _I, _P]),
    "qim_swiglu_quantize": (_C, [_P, _I, _P, _I, _P, _P, _I, _I, _P]),
    "qim_swiglu_quantize_tiled": (_C, [_P, _I, _P, _I, _P, _P, _I, _I, _P]),
    "qim_rms_norm": (_C, [_P, _P, _P, _I, _I, _F, _P]),
    "qim_rope_qk": (_C, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "qim_qk_norm_rope_pack": (_C, [_P] * 11 + [_I] * 6 + [_F, _F, _P]),
    "qim_mxfp8_gemm": (_C, [_P, _P, _P, _P, _I, _I, _I, _C, _P, _P, _P, _I, _P, _I, _P, _P]),
    "qim_mxfp8_gemm_ex": (_C, [_P, _P, _P, _P, _I, _I, _I, _C, _C, _P, _P, _P, _I, _P, _I, _P, _P]),
    "qim_mxfp8_gemm_ws": (_C, [_P, _P, _P, _P, _I, _I, _I, _C, _C, _P, _P, _P, _I, _P, _I, _P, _P, _I, _P]),
    "qim_mxfp8_gemm_ws_bytes": (_I, [_I, _I, _I, _C]),
    "qim_mxfp8_gemm_qk_norm_rope": (_C, [_P, _P, _P, _P, _I, _I, _I, _C, _P, _P, _P, _I, _F, _F, _P, _I, _P]),
    "qim_mxfp8_gemm_qk_norm_rope_vt": (_C, [_P, _P, _P, _P, _I, _I, _I, _C, _P, _P, _P, _I, _F, _F, _P, _I, _P,
                                           _P]),
    "qim_attention": (_C, [_P, _I, _P, _I, _P, _I, _P, _I, _P, _I, _I, _I, _I, _I, _I, _F, _P]),
    "qim_attention_workspace_bytes": (_I, [_I, _I, _I, _I, _I]),
    "qim_attention_mxfp8": (_C, [_P, _I, _P, _I, _P, _I, _P, _P, _C, _P, _I, _I, _I, _I, _I, _I, _F, _P]),
    "qim_attention_noalloc": (_C, [_P, _I, _P, _I, _P, _I, _P, _I, _I, _I, _I, _I, _I, _F, _P]),
    "qim_debug_e4m3_encode": (_C, [_P, _P, _I, _P]),
    "qim_debug_e4m3_encode_scaled": (_C, [_P, _C, _P, _I, _P]),
    "qim_debug_bf16_round": (_C, [_P, _P, _I, _P]),
    "qim_debug_mfma_tile": (_C, [_P, _P, _P, _P, _P, _P]),
    "qim_debug_mfma_probe": (_C, [_C, _P, _P]),
    "qim_debug_copy": (_C, [_P, _P, _I, _P]),
    "qim_debug_copy_ex": (_C, [_P, _P, _I, _C, _C, _P]),
    "qim_debug_silu": (_C, [_P, _P, _I, _P]),
    "qim_debug_rstd_sweep": (_C, [_U, _U, _F, _P, _P]),
}

_lib = None
_lock = threading.Lock()
calls = {}  # entry point name -> number of successful launches (tests use it)


def available():
    return os.path.exists(LIB_PATH)


def lib():
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise NativeUnavailable(
                        f"{LIB_PATH} is not built; run qwen-image-2.1-accel_amd/build_native.py")
                handle = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_LOCAL)
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


def call(name, *args):
    """Call an entry point; raise Unsupported / QimError on a nonzero status."""
    rc = getattr(lib(), name)(*args)
    if rc != QIM_OK:
        msg = lib().qim_last_error().decode(errors="replace")
        if rc in (QIM_ERR_SHAPE, QIM_ERR_LAYOUT):
            raise Unsupported(name, rc, msg)
        raise QimError(name, rc, msg)
    calls[name] = calls.get(name, 0) + 1


def ptr(t):
    """Device address of a tensor (None stays NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream(device=None):
    """The current torch stream of `device` as a hipStream_t."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def loaded_hip_runtimes():
    """Paths of every libamdhip64 mapped into this process (must be exactly one)."""
    paths = set()
    with open("/proc/self/maps") as f:
        for line in f:
            if "libamdhip64" in line:
                paths.add(line.split()[-1])
    return sorted(paths)
