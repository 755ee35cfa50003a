"""ctypes binding of the CPU oracle (oracle/_build/liboracle.so).

Test infrastructure: the oracle that the HIP path is compared against.
"""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(ROOT, "oracle", "_build", "liboracle.so")

E4M3FN, E5M2, BF16, F16, F32 = 0, 1, 2, 3, 4
SCALE_NONE, SCALE_TENSOR, SCALE_ROW = 0, 1, 2
DTYPE_CODES = {"F8_E4M3": E4M3FN, "F8_E5M2": E5M2, "BF16": BF16, "F16": F16, "F32": F32}


class OrcLora(ctypes.Structure):
    _fields_ = [
        ("b", ctypes.c_void_p),
        ("a", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("rank", ctypes.c_int32),
        ("coeff", ctypes.c_float),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        L.orc_e4m3fn_to_f32.restype = ctypes.c_float
        L.orc_e4m3fn_to_f32.argtypes = [ctypes.c_uint8]
        L.orc_e5m2_to_f32.restype = ctypes.c_float
        L.orc_e5m2_to_f32.argtypes = [ctypes.c_uint8]
        L.orc_bf16_from_f32.restype = ctypes.c_uint16
        L.orc_bf16_from_f32.argtypes = [ctypes.c_float]
        L.orc_lora_coeff.restype = ctypes.c_float
        L.orc_lora_coeff.argtypes = [ctypes.c_float, ctypes.c_int, ctypes.c_float, ctypes.c_int32]
        L.orc_decode_to_f32.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p]
        common = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        L.orc_read_f32_mt.argtypes = common + [ctypes.c_void_p, ctypes.c_int]
        L.orc_read_bf16_mt.argtypes = common + [ctypes.c_void_p, ctypes.c_int]
        L.orc_read_f64_rows.argtypes = common + [ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
        L.orc_abs_bound_rows.argtypes = common + [ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
        L.orc_set_mutation.argtypes = [ctypes.c_int]
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


class _Args:
    """Keeps numpy buffers alive for the duration of one oracle call."""

    def __init__(self, base, base_dtype, scale_mode, scales, loras):
        self.base = np.ascontiguousarray(base)
        self.rows, self.cols = self.base.shape[0], self.base.shape[1]
        self.base_dtype = base_dtype
        self.scale_mode = scale_mode
        self.scales = None if scales is None else np.ascontiguousarray(scales, dtype=np.float32)
        self.keep = []
        arr = (OrcLora * max(1, len(loras)))()
        for k, (b, a, dtype, coeff) in enumerate(loras):
            b = np.ascontiguousarray(b)
            a = np.ascontiguousarray(a)
            self.keep += [b, a]
            arr[k] = OrcLora(_ptr(b).value, _ptr(a).value, dtype, a.shape[0], coeff)
        self.loras = arr
        self.n = len(loras)

    def common(self):
        return [_ptr(self.base), self.base_dtype, self.rows, self.cols, self.scale_mode,
                _ptr(self.scales), ctypes.cast(self.loras, ctypes.c_void_p), self.n]


def read_f32(base, base_dtype, scale_mode=SCALE_NONE, scales=None, loras=(), threads=1):
    """Reference read path to f32. loras: list of (B, A, dtype_code, coeff)."""
    a = _Args(base, base_dtype, scale_mode, scales, list(loras))
    out = np.empty((a.rows, a.cols), dtype=np.float32)
    lib().orc_read_f32_mt(*a.common(), _ptr(out), threads)
    return out


def read_bf16(base, base_dtype, scale_mode=SCALE_NONE, scales=None, loras=(), threads=1):
    a = _Args(base, base_dtype, scale_mode, scales, list(loras))
    out = np.empty((a.rows, a.cols), dtype=np.uint16)
    lib().orc_read_bf16_mt(*a.common(), _ptr(out), threads)
    return out


def read_f64_rows(base, base_dtype, scale_mode=SCALE_NONE, scales=None, loras=(), row0=0, nrows=None):
    a = _Args(base, base_dtype, scale_mode, scales, list(loras))
    nrows = a.rows - row0 if nrows is None else nrows
    out = np.empty((nrows, a.cols), dtype=np.float64)
    lib().orc_read_f64_rows(*a.common(), row0, nrows, _ptr(out))
    return out


def abs_bound_rows(base, base_dtype, scale_mode=SCALE_NONE, scales=None, loras=(), row0=0, nrows=None):
    a = _Args(base, base_dtype, scale_mode, scales, list(loras))
    nrows = a.rows - row0 if nrows is None else nrows
    out = np.empty((nrows, a.cols), dtype=np.float64)
    lib().orc_abs_bound_rows(*a.common(), row0, nrows, _ptr(out))
    return out


def decode(raw, dtype):
    raw = np.ascontiguousarray(raw)
    n = raw.size
    out = np.empty(n, dtype=np.float32)
    lib().orc_decode_to_f32(_ptr(raw), dtype, n, _ptr(out))
    return out


def bf16_from_f32(x):
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    f = lib().orc_bf16_from_f32
    return np.array([f(float(v)) for v in x], dtype=np.uint16)


def lora_coeff(strength, alpha, rank):
    """alpha None = no `prefix.alpha` tensor."""
    return lib().orc_lora_coeff(strength, 0 if alpha is None else 1, 0.0 if alpha is None else alpha, rank)


class mutation:
    """Context manager that plants oracle mistake `m` (see oracle.c)."""

    def __init__(self, m):
        self.m = m

    def __enter__(self):
        lib().orc_set_mutation(self.m)

    def __exit__(self, *exc):
        lib().orc_set_mutation(0)
