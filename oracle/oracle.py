"""numpy front-end of the CPU oracle (oracle/qim_oracle.c).

TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels.  Only tests/,
``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg import this
module; the product path (the ``qwen_image_accel`` package) never does.

bf16 tensors cross this boundary as ``np.uint16`` bit patterns, E4M3 codes and
E8M0 exponents as ``np.uint8``, complex64 RoPE tables as interleaved float32.
Each function cites the reference code it restates (paths under the reference
tree ``src/qwen_image_accel/``; ``WHL!`` = a file of the vendored diffusers
wheel).  How each function is pinned is stated in its docstring; the checks
themselves live in tests/test_oracle.py.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libqim_oracle.so")
_lib = None

ADD_ONE = 1


def build():
    """Compile oracle/libqim_oracle.so from qim_oracle.c (gcc, see Makefile)."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "libqim_oracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I = ctypes.c_int64


def _declare(L):
    sig = {
        "oracle_f32_to_bf16": (None, [_P, _P, _I]),
        "oracle_set_threads": (None, [ctypes.c_int]),
        "oracle_get_threads": (ctypes.c_int, []),
        "oracle_e4m3_encode": (ctypes.c_uint8, [ctypes.c_float]),
        "oracle_e4m3_decode": (ctypes.c_float, [ctypes.c_uint8]),
        "oracle_mx_exponent": (ctypes.c_int, [ctypes.c_float]),
        "oracle_mx_scale_index": (_I, [_I, _I, _I]),
        "oracle_mx_quantize": (None, [_P, _I, _I, _I, _P, _P]),
        "oracle_mx_dequantize": (None, [_P, _P, _I, _I, _P]),
        "oracle_adaln": (None, [_P, _P, _P, _P, _P, _P, _I, _I, _I, ctypes.c_float, ctypes.c_int]),
        "oracle_adaln_quantize": (None, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, ctypes.c_float,
                                         ctypes.c_int]),
        "oracle_residual": (None, [_P, _P, _P, _P, _I, _I, _I]),
        "oracle_swiglu": (None, [_P, _I, _P, _I, _P, _I, _I, _I]),
        "oracle_swiglu_quantize": (None, [_P, _I, _P, _I, _P, _P, _I, _I]),
        "oracle_rms_norm": (None, [_P, _P, _P, _I, _I, ctypes.c_float]),
        "oracle_rope": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I]),
        "oracle_norm_rope_pack": (None, [_P] * 11 + [_I] * 5 + [ctypes.c_float] * 2),
        "oracle_rope_freqs": (None, [_P, _I, _P, ctypes.c_float, _P]),
        "oracle_mx_gemm": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


def set_threads(n):
    lib().oracle_set_threads(int(n))


def get_threads():
    return int(lib().oracle_get_threads())


# ------------------------------------------------------------------ bf16 --

def bf16_to_f32(bits):
    """bf16 bit patterns -> float32 values (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x):
    """float32 -> bf16 bit patterns, round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_bf16(_p(x), _p(out), x.size)
    return out


def round_bf16(x):
    return bf16_to_f32(f32_to_bf16(x))


# ----------------------------------------------------------- E4M3 / E8M0 --

def e4m3_encode(x):
    """fp32 -> OCP E4M3 code, round to nearest even (NaN code for |x| >= 464).
    Pinned exhaustively against torch's float8_e4m3fn cast."""
    L = lib()
    flat = np.asarray(x, dtype=np.float32).ravel()
    return np.array([L.oracle_e4m3_encode(float(v)) for v in flat], dtype=np.uint8).reshape(
        np.shape(x))


def e4m3_decode(codes):
    L = lib()
    flat = np.asarray(codes, dtype=np.uint8).ravel()
    return np.array([L.oracle_e4m3_decode(int(c)) for c in flat], dtype=np.float32).reshape(
        np.shape(codes))


E4M3_TABLE = None


def e4m3_values():
    """Decoded value of every code 0..255 (float32)."""
    global E4M3_TABLE
    if E4M3_TABLE is None:
        E4M3_TABLE = e4m3_decode(np.arange(256, dtype=np.uint8))
    return E4M3_TABLE


def mx_exponent(amax):
    """E8M0 exponent of a block with maximum |x| = amax (kernels/mxfp8.py:42-48).
    Pinned by KATs and by the brute-force 'smallest power of two' definition."""
    return int(lib().oracle_mx_exponent(float(amax)))


def mx_scale_index(r, kb, K):
    return int(lib().oracle_mx_scale_index(int(r), int(kb), int(K)))


def padded_rows(rows):
    return (rows + 127) // 128 * 128


def mx_quantize(x_bits, ldx=None):
    """quantize(x) (kernels/mxfp8.py:59-67): bf16 (M, K) -> codes (Mp, K),
    flat swizzled scales (Mp*K/32,)."""
    x_bits = np.asarray(x_bits, dtype=np.uint16)
    M, K = x_bits.shape if ldx is None else (x_bits.shape[0], x_bits.shape[1])
    if ldx is None:
        x_bits = np.ascontiguousarray(x_bits)
        ldx = K
    Mp = padded_rows(M)
    q = np.empty((Mp, K), dtype=np.uint8)
    s = np.empty(Mp * K // 32, dtype=np.uint8)
    lib().oracle_mx_quantize(_p(x_bits), ldx, M, K, _p(q), _p(s))
    return q, s


def mx_dequantize(q, s, rows=None):
    q = np.ascontiguousarray(q, dtype=np.uint8)
    s = np.ascontiguousarray(s, dtype=np.uint8)
    M, K = q.shape
    out = np.empty((M, K), dtype=np.float32)
    lib().oracle_mx_dequantize(_p(q), _p(s), M, K, _p(out))
    return out if rows is None else out[:rows]


# -------------------------------------------------------------- LayerNorm --

def adaln(x, scale, shift=None, gate=None, res=None, eps=1e-6, add_one=False):
    """Modulated LayerNorm chain (kernels/layernorm.py:49-55 extended with the
    MMDiT shift/gate/residual; rounding points in qim_oracle.c adaln_row).
    x: (B, S, D) bf16 bits; scale/shift/gate: (B, D) or (B, 1, D); res like x."""
    x = _c(x, np.uint16)
    B, S, D = x.shape
    out = np.empty_like(x)
    args = [_c(a, np.uint16) for a in (scale, shift, gate, res)]
    lib().oracle_adaln(_p(x), *[_p(a) for a in args], _p(out), B * S, D, S, float(eps),
                       ADD_ONE if add_one else 0)
    return out


def adaln_quantize(x, scale, shift=None, gate=None, res=None, eps=1e-6, add_one=False):
    """quantize(adaln(...).reshape(-1, D)) byte-identically (kernels/epilogue.py:23-92)."""
    x = _c(x, np.uint16)
    B, S, D = x.shape
    Mp = padded_rows(B * S)
    q = np.empty((Mp, D), dtype=np.uint8)
    s = np.empty(Mp * D // 32, dtype=np.uint8)
    args = [_c(a, np.uint16) for a in (scale, shift, gate, res)]
    lib().oracle_adaln_quantize(_p(x), *[_p(a) for a in args], _p(q), _p(s), B * S, D, S,
                                float(eps), ADD_ONE if add_one else 0)
    return q, s


def residual(h, x, gate):
    """bf16(h + bf16(gate * x)) (kernels/elementwise.py:10-34). h, x: (B, S, D)."""
    h = _c(h, np.uint16)
    x = _c(x, np.uint16)
    B, S, D = h.shape
    out = np.empty_like(h)
    lib().oracle_residual(_p(h), _p(x), _p(_c(gate, np.uint16)), _p(out), B * S, D, S)
    return out


def swiglu(g, v):
    """bf16(bf16(silu(g)) * v) (kernels/bf16.py:12-36). g, v: (M, F) bf16 bits."""
    g = _c(g, np.uint16)
    v = _c(v, np.uint16)
    M, F = g.shape
    out = np.empty((M, F), dtype=np.uint16)
    lib().oracle_swiglu(_p(g), F, _p(v), F, _p(out), F, M, F)
    return out


def swiglu_quantize(g, v):
    """quantize(swiglu(g, v)) byte-identically (kernels/epilogue.py:95-136)."""
    g = _c(g, np.uint16)
    v = _c(v, np.uint16)
    M, F = g.shape
    Mp = padded_rows(M)
    q = np.empty((Mp, F), dtype=np.uint8)
    s = np.empty(Mp * F // 32, dtype=np.uint8)
    lib().oracle_swiglu_quantize(_p(g), F, _p(v), F, _p(q), _p(s), M, F)
    return q, s


def rms_norm(x, w, eps=1e-6):
    """Diffusers RMSNorm with bf16 weight (kernels/bf16.py:46-63)."""
    x = _c(x, np.uint16)
    D = x.shape[-1]
    out = np.empty_like(x)
    lib().oracle_rms_norm(_p(x), _p(_c(w, np.uint16)), _p(out), x.size // D, D, float(eps))
    return out


def rope(q, k, freqs):
    """rope_qk (kernels/elementwise.py:37-69). q, k: (B, S, H, D) bf16 bits;
    freqs: (S, D/2, 2) float32 (cos, sin)."""
    q = _c(q, np.uint16)
    k = _c(k, np.uint16)
    B, S, H, D = q.shape
    oq, ok = np.empty_like(q), np.empty_like(k)
    lib().oracle_rope(_p(q), _p(k), _p(_c(freqs, np.float32)), _p(oq), _p(ok), B, S, H, D)
    return oq, ok


def norm_rope_pack(q, k, v, wq, wk, freqs, ck=None, cv=None, epsq=1e-6, epsk=1e-6):
    """prepare_attention_inputs (kernels/attention.py:16-159): returns
    (oq (B,S,H,D), ok (B,P+S,H,D), ov (B,P+S,H,D))."""
    q, k, v = (_c(t, np.uint16) for t in (q, k, v))
    B, S, H, D = q.shape
    P = 0 if ck is None else ck.shape[1]
    ck = _c(ck, np.uint16)
    cv = _c(cv, np.uint16)
    oq = np.empty_like(q)
    ok = np.empty((B, P + S, H, D), dtype=np.uint16)
    ov = np.empty_like(ok)
    lib().oracle_norm_rope_pack(_p(q), _p(k), _p(v), _p(ck), _p(cv), _p(_c(wq, np.uint16)),
                                _p(_c(wk, np.uint16)), _p(_c(freqs, np.float32)), _p(oq), _p(ok),
                                _p(ov), B, S, P, H, D, float(epsq), float(epsk))
    return oq, ok, ov


def rope_positions(text_tokens, frames, height, width):
    """(frame, h, w) positions of `text_tokens` text tokens followed by one
    frames x height x width image block, per QwenImage21Rope.forward
    (WHL!transformer_qwenimage21.py:677-710): text advances one shared position
    on all three axes; the image freezes the frame axis at the position after
    the text and centres h, w on zero."""
    pos = []
    for t in range(text_tokens):
        pos.append((t, t, t))
    for _f in range(frames):
        for h in range(-(height - height // 2), height // 2):
            for w in range(-(width - width // 2), width // 2):
                pos.append((text_tokens, h, w))
    return np.array(pos, dtype=np.int64)


def rope_freqs(pos, dims=(16, 56, 56), theta=10000.0):
    """3-axis complex RoPE table (S, sum(dims)/2, 2) float32 (cos, sin)
    (WHL!transformer_qwenimage21.py:652-675)."""
    pos = _c(pos, np.int64)
    S = pos.shape[0]
    d = np.array(dims, dtype=np.int64)
    out = np.empty((S, int(d.sum()) // 2, 2), dtype=np.float32)
    lib().oracle_rope_freqs(_p(pos), S, _p(d), float(theta), _p(out))
    return out


def mx_gemm(aq, as_, bq, bs, rows=None):
    """Dequantize-then-matmul in float64, rounded to fp32: (len(rows) or Mp, N)
    (optimizations/mxfp8.py:32-36 checked against this)."""
    aq = _c(aq, np.uint8)
    bq = _c(bq, np.uint8)
    K = aq.shape[1]
    N = bq.shape[0]
    if rows is None:
        r = None
        n_rows = aq.shape[0]
    else:
        r = _c(rows, np.int64)
        n_rows = r.size
    out = np.empty((n_rows, N), dtype=np.float32)
    lib().oracle_mx_gemm(_p(aq), _p(_c(as_, np.uint8)), _p(bq), _p(_c(bs, np.uint8)), _p(r),
                         n_rows, N, K, _p(out))
    return out
