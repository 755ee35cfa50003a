"""ctypes binding of libltxw.so (include/ltxw.h).

This is the Python counterpart of the FFI crate a Rust caller would use:
a mechanical mirror of the C ABI. It loads the in-tree library and fails
loudly when it is missing; there is no fallback path.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "_build", "libltxw.so")

# include/ltxw.h enums
OK = 0
FMT_E4M3FN, FMT_E5M2, FMT_BF16, FMT_F16, FMT_F32 = 0, 1, 2, 3, 4
SCALE_NONE, SCALE_TENSOR, SCALE_ROW = 0, 1, 2
OUT_BF16, OUT_F32 = 0, 1
MAX_LORAS = 4
NOALLOC_MAX_DESCS = 128  # LTXW_NOALLOC_MAX_DESCS


class WeightError(Exception):
    """Base of every ltxw error (the reference's `WeightError`, src/error.rs:7)."""

    code = -1


class InvalidArgument(WeightError):
    code = 1


class UnsupportedDtype(WeightError):
    code = 2


class OutOfMemory(WeightError):
    code = 3


class DeviceError(WeightError):
    code = 4


class IoError(WeightError):
    code = 5


class InvalidTensorData(WeightError):
    code = 6


class MissingKey(WeightError):
    code = 7


class DuplicateKey(WeightError):
    code = 8


class LoraShapeMismatch(WeightError):
    code = 9


class LoraRankMismatch(WeightError):
    code = 10


class NoLoraMatches(WeightError):
    code = 11


class QkvSplitDim(WeightError):
    code = 12


class GateNotScalar(WeightError):
    code = 13


_ERRORS = {c.code: c for c in (InvalidArgument, UnsupportedDtype, OutOfMemory, DeviceError, IoError,
                               InvalidTensorData, MissingKey, DuplicateKey, LoraShapeMismatch,
                               LoraRankMismatch, NoLoraMatches, QkvSplitDim, GateNotScalar)}


FACTOR_BF16, FACTOR_F32, FACTOR_F16, FACTOR_E4M3FN, FACTOR_E5M2 = 0, 1, 2, 3, 4


class Lora(ctypes.Structure):
    _fields_ = [
        ("b", ctypes.c_void_p),
        ("a", ctypes.c_void_p),
        ("rank", ctypes.c_int32),
        ("coeff", ctypes.c_float),
        ("dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class TensorDesc(ctypes.Structure):
    _fields_ = [
        ("w", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
        ("fmt", ctypes.c_int32),
        ("scale_mode", ctypes.c_int32),
        ("out_dtype", ctypes.c_int32),
        ("n_loras", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("loras", Lora * MAX_LORAS),
    ]


DESC_EXACT = 1


class KeyRule(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("n", ctypes.c_int32),
        ("strs", ctypes.POINTER(ctypes.c_char_p)),
    ]


EXPORTS = [
    "ltxw_ctx_create", "ltxw_ctx_destroy", "ltxw_last_error", "ltxw_alloc", "ltxw_free",
    "ltxw_memset", "ltxw_upload", "ltxw_download", "ltxw_synchronize", "ltxw_dequant",
    "ltxw_dequant_lora", "ltxw_dequant_lora_grouped", "ltxw_dequant_lora_grouped_noalloc", "ltxw_ctx_stream",
    "ltxw_ctx_set_host_threads",
    # include/ltxw_store.h
    "ltxw_store_last_error", "ltxw_store_open", "ltxw_store_close", "ltxw_store_n_keys",
    "ltxw_store_key", "ltxw_store_contains", "ltxw_store_tensor_info", "ltxw_store_metadata",
    "ltxw_lora_open", "ltxw_lora_close", "ltxw_lora_n_tensors", "ltxw_lora_tensor_name",
    "ltxw_lora_tensor_info", "ltxw_lora_metadata", "ltxw_lora_ic_layout", "ltxw_lora_read_f32",
    "ltxw_store_merge_lora", "ltxw_report_n_matched", "ltxw_report_matched", "ltxw_report_n_unmatched",
    "ltxw_report_unmatched", "ltxw_report_free", "ltxw_store_n_deltas", "ltxw_store_delta",
    "ltxw_store_materialize", "ltxw_store_read",
]

_lib = None


def lib():
    """Load libltxw.so (no GPU call is made by loading it)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"libltxw.so is not built: {LIB_PATH} (run __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    vp, i32, i64, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
    L.ltxw_ctx_create.argtypes = [i32, sz, i32, ctypes.POINTER(vp)]
    L.ltxw_ctx_destroy.argtypes = [vp]
    L.ltxw_ctx_destroy.restype = None
    L.ltxw_last_error.argtypes = [vp]
    L.ltxw_last_error.restype = ctypes.c_char_p
    L.ltxw_alloc.argtypes = [vp, sz, ctypes.POINTER(vp)]
    L.ltxw_free.argtypes = [vp, vp]
    L.ltxw_memset.argtypes = [vp, vp, i32, sz]
    L.ltxw_upload.argtypes = [vp, vp, sz, vp]
    L.ltxw_download.argtypes = [vp, vp, sz, vp]
    L.ltxw_synchronize.argtypes = [vp]
    L.ltxw_dequant.argtypes = [vp, vp, i64, i64, i32, i32, vp, vp, i32]
    L.ltxw_dequant_lora.argtypes = [vp, vp, i64, i64, i32, i32, vp, ctypes.POINTER(Lora), i32, vp, i32]
    L.ltxw_dequant_lora_grouped.argtypes = [vp, ctypes.POINTER(TensorDesc), i32]
    L.ltxw_dequant_lora_grouped_noalloc.argtypes = [vp, ctypes.POINTER(TensorDesc), i32]
    L.ltxw_ctx_stream.argtypes = [vp]
    L.ltxw_ctx_stream.restype = vp
    L.ltxw_ctx_set_host_threads.argtypes = [vp, i32]
    # include/ltxw_store.h
    cp, u32, f32 = ctypes.c_char_p, ctypes.c_uint32, ctypes.c_float
    pi32, pi64 = ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int64)
    L.ltxw_store_last_error.argtypes = []
    L.ltxw_store_last_error.restype = cp
    L.ltxw_store_open.argtypes = [ctypes.POINTER(cp), i32, ctypes.POINTER(KeyRule), i32, ctypes.POINTER(vp)]
    L.ltxw_store_close.argtypes = [vp]
    L.ltxw_store_close.restype = None
    L.ltxw_store_n_keys.argtypes = [vp]
    L.ltxw_store_n_keys.restype = i64
    L.ltxw_store_key.argtypes = [vp, i64]
    L.ltxw_store_key.restype = cp
    L.ltxw_store_contains.argtypes = [vp, cp]
    L.ltxw_store_tensor_info.argtypes = [vp, cp, pi32, pi32, pi64, i32]
    L.ltxw_store_metadata.argtypes = [vp, cp]
    L.ltxw_store_metadata.restype = cp
    L.ltxw_lora_open.argtypes = [cp, ctypes.POINTER(vp)]
    L.ltxw_lora_close.argtypes = [vp]
    L.ltxw_lora_close.restype = None
    L.ltxw_lora_n_tensors.argtypes = [vp]
    L.ltxw_lora_n_tensors.restype = i64
    L.ltxw_lora_tensor_name.argtypes = [vp, i64]
    L.ltxw_lora_tensor_name.restype = cp
    L.ltxw_lora_tensor_info.argtypes = [vp, cp, pi32, pi32, pi64, i32]
    L.ltxw_lora_metadata.argtypes = [vp, cp]
    L.ltxw_lora_metadata.restype = cp
    L.ltxw_lora_ic_layout.argtypes = [vp, ctypes.POINTER(u32), ctypes.POINTER(u32)]
    L.ltxw_lora_read_f32.argtypes = [vp, cp, vp, i64]
    L.ltxw_store_merge_lora.argtypes = [vp, vp, f32, ctypes.POINTER(vp)]
    L.ltxw_report_n_matched.argtypes = [vp]
    L.ltxw_report_n_matched.restype = i64
    L.ltxw_report_matched.argtypes = [vp, i64]
    L.ltxw_report_matched.restype = cp
    L.ltxw_report_n_unmatched.argtypes = [vp]
    L.ltxw_report_n_unmatched.restype = i64
    L.ltxw_report_unmatched.argtypes = [vp, i64]
    L.ltxw_report_unmatched.restype = cp
    L.ltxw_report_free.argtypes = [vp]
    L.ltxw_report_free.restype = None
    L.ltxw_store_n_deltas.argtypes = [vp, cp]
    L.ltxw_store_delta.argtypes = [vp, cp, i32, pi32, ctypes.POINTER(f32)]
    L.ltxw_store_materialize.argtypes = [vp, vp, ctypes.POINTER(cp), i64, i32, u32, ctypes.POINTER(vp)]
    L.ltxw_store_read.argtypes = [vp, vp, cp, u32, vp, i64]
    _lib = L
    return L


def check_store(rc):
    """Raise the WeightError subclass of a failed store / LoRA-file call."""
    if rc == OK:
        return
    msg = lib().ltxw_store_last_error()
    msg = msg.decode("utf-8", "replace") if msg else ""
    raise _ERRORS.get(rc, WeightError)(msg)


def check(rc, ctx_handle=None):
    if rc == OK:
        return
    msg = lib().ltxw_last_error(ctx_handle)
    msg = msg.decode("utf-8", "replace") if msg else ""
    raise _ERRORS.get(rc, WeightError)(msg)


class Context:
    """One ltxw context (device, compute + copy streams, pinned staging ring)."""

    def __init__(self, device=0, staging_bytes=0, n_staging=0):
        h = ctypes.c_void_p()
        check(lib().ltxw_ctx_create(device, staging_bytes, n_staging, ctypes.byref(h)), None)
        self.h = h
        self.device = device

    def close(self):
        if self.h:
            lib().ltxw_ctx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _chk(self, rc):
        check(rc, self.h)

    def alloc(self, nbytes):
        p = ctypes.c_void_p()
        self._chk(lib().ltxw_alloc(self.h, nbytes, ctypes.byref(p)))
        return p.value

    def free(self, ptr):
        self._chk(lib().ltxw_free(self.h, ptr))

    def memset(self, ptr, value, nbytes):
        self._chk(lib().ltxw_memset(self.h, ptr, value, nbytes))

    def upload(self, array, dptr):
        """Host numpy array -> device pointer (staged, ordered before later work)."""
        a = np.ascontiguousarray(array)
        self._chk(lib().ltxw_upload(self.h, a.ctypes.data, a.nbytes, dptr))

    def download(self, dptr, out):
        """Device pointer -> C-contiguous numpy array `out` (waits for prior work)."""
        if not out.flags.c_contiguous:
            raise InvalidArgument("download target must be C-contiguous")
        self._chk(lib().ltxw_download(self.h, dptr, out.nbytes, out.ctypes.data))

    def synchronize(self):
        self._chk(lib().ltxw_synchronize(self.h))

    def stream(self):
        return lib().ltxw_ctx_stream(self.h)

    def set_host_threads(self, n):
        self._chk(lib().ltxw_ctx_set_host_threads(self.h, n))

    def dequant(self, w, rows, cols, fmt, scale_mode, scales, out, out_dtype=OUT_BF16):
        self._chk(lib().ltxw_dequant(self.h, w, rows, cols, fmt, scale_mode, scales, out, out_dtype))

    def dequant_lora(self, w, rows, cols, fmt, scale_mode, scales, loras, out, out_dtype=OUT_BF16):
        """loras: list of (b_ptr, a_ptr, rank, coeff[, factor_dtype])."""
        arr = (Lora * max(1, len(loras)))(*[Lora(*x) for x in loras])
        self._chk(lib().ltxw_dequant_lora(self.h, w, rows, cols, fmt, scale_mode, scales, arr,
                                          len(loras), out, out_dtype))

    def grouped(self, descs):
        """descs: list of dicts with the TensorDesc fields, loras as (b, a, rank,
        coeff[, dtype]); or an array from make_descs (marshalled once, reusable)."""
        if not isinstance(descs, ctypes.Array):
            if not descs:
                self._chk(lib().ltxw_dequant_lora_grouped(self.h, None, 0))
                return
            descs = self.make_descs(descs)
        self._chk(lib().ltxw_dequant_lora_grouped(self.h, descs, len(descs)))

    def grouped_noalloc(self, descs):
        """As grouped, through ltxw_dequant_lora_grouped_noalloc: no device or
        pinned allocation (job tables in the library's static device scratch),
        at most NOALLOC_MAX_DESCS descriptors."""
        if not isinstance(descs, ctypes.Array):
            if not descs:
                self._chk(lib().ltxw_dequant_lora_grouped_noalloc(self.h, None, 0))
                return
            descs = self.make_descs(descs)
        self._chk(lib().ltxw_dequant_lora_grouped_noalloc(self.h, descs, len(descs)))

    @staticmethod
    def make_descs(descs):
        """The ctypes TensorDesc array of a non-empty list of descriptor dicts."""
        arr = (TensorDesc * len(descs))()
        for k, d in enumerate(descs):
            t = arr[k]
            t.w, t.out, t.scales = d["w"], d["out"], d.get("scales")
            t.rows, t.cols = d["rows"], d["cols"]
            t.fmt, t.scale_mode = d.get("fmt", FMT_E4M3FN), d.get("scale_mode", SCALE_NONE)
            t.out_dtype = d.get("out_dtype", OUT_BF16)
            t.flags = d.get("flags", 0)
            loras = d.get("loras", [])
            t.n_loras = len(loras)
            for l, x in enumerate(loras[:MAX_LORAS]):
                t.loras[l] = Lora(*x)
        return arr
