"""INT4 group quantizer restatement (TEST INFRASTRUCTURE ONLY, see oracle/__init__.py).

Thin numpy/ctypes front end of hkv_oracle.c, which follows
src/quantization/kv_compressor.py:66-132 of the reference line by line.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libhkv_oracle.so")
_lib = None

F16, BF16, F32 = 0, 1, 2


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        from . import build as _b  # noqa: F401  (local import keeps the module light)
        _b.build(verbose=False)
    lib = ctypes.CDLL(_LIB_PATH)
    vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
    lib.hkvo_compress.argtypes = [vp, ctypes.c_int, i64, i32, vp, vp, vp]
    lib.hkvo_compress.restype = i64
    lib.hkvo_decompress.argtypes = [vp, vp, vp, i64, i32, vp, ctypes.c_int]
    lib.hkvo_decompress.restype = None
    for name in ("hkvo_f2h_array", "hkvo_h2f_array", "hkvo_f2bf_array"):
        getattr(lib, name).argtypes = [vp, i64, vp]
        getattr(lib, name).restype = None
    lib.hkvo_group_params.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.POINTER(ctypes.c_float),
                                      ctypes.POINTER(ctypes.c_uint8)]
    lib.hkvo_group_params.restype = None
    _lib = lib
    return lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _dtype_code(x):
    if x.dtype == np.float16:
        return F16
    if x.dtype == np.float32:
        return F32
    if x.dtype == np.uint16:  # raw bfloat16 bits
        return BF16
    raise TypeError("oracle compress: unsupported dtype %s" % x.dtype)


def compress(x, group_size=128):
    """kv_compressor.py:50-98.  x: float16/float32 array, or uint16 holding bfloat16 bits.

    Returns (codes uint8 same shape as x, scales float32 [ngroups], zps uint8 [ngroups]).
    """
    lib = _load()
    x = np.ascontiguousarray(x)
    n = x.size
    ng = (n + group_size - 1) // group_size
    codes = np.empty(x.shape, dtype=np.uint8)
    scales = np.empty(ng, dtype=np.float32)
    zps = np.empty(ng, dtype=np.uint8)
    if n:
        lib.hkvo_compress(_ptr(x), _dtype_code(x), n, group_size, _ptr(codes), _ptr(scales), _ptr(zps))
    return codes, scales, zps


def decompress(codes, scales, zps, group_size=128, out_dtype=np.float16):
    """kv_compressor.py:100-132.  out_dtype: np.float16, np.float32 or 'bf16' (uint16 bits)."""
    lib = _load()
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    zps = np.ascontiguousarray(zps, dtype=np.uint8)
    if out_dtype == "bf16":
        out = np.empty(codes.shape, dtype=np.uint16)
        code = BF16
    else:
        out = np.empty(codes.shape, dtype=out_dtype)
        code = F16 if out.dtype == np.float16 else F32
    if codes.size:
        lib.hkvo_decompress(_ptr(codes), _ptr(scales), _ptr(zps), codes.size, group_size, _ptr(out), code)
    return out


def relative_error(original, codes, scales, zps, group_size=128):
    """kv_compressor.py:146-154: mean|deq - x| / (mean|x| + 1e-8) * 100, deq in x's dtype."""
    restored = decompress(codes, scales, zps, group_size,
                          out_dtype=np.float16 if original.dtype == np.float16 else np.float32)
    o = original.astype(np.float64)
    r = restored.astype(np.float64)
    return float(np.abs(r - o).mean() / (np.abs(o).mean() + 1e-8) * 100.0)


def group_params(mn, mx):
    """kv_compressor.py:76-84 for one group: returns (scale, zp)."""
    lib = _load()
    s = ctypes.c_float()
    z = ctypes.c_uint8()
    lib.hkvo_group_params(ctypes.c_float(mn), ctypes.c_float(mx), ctypes.byref(s), ctypes.byref(z))
    return np.float32(s.value), int(z.value)


def f32_to_f16_bits(a):
    lib = _load()
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib.hkvo_f2h_array(_ptr(a), a.size, _ptr(out))
    return out


def f16_bits_to_f32(a):
    lib = _load()
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    lib.hkvo_h2f_array(_ptr(a), a.size, _ptr(out))
    return out


def f32_to_bf16_bits(a):
    lib = _load()
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib.hkvo_f2bf_array(_ptr(a), a.size, _ptr(out))
    return out


def bf16_bits_to_f32(a):
    return (np.ascontiguousarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
