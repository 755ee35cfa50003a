"""DLPack capsules over ltxw device memory (DLPack 0.x ABI: DLManagedTensor
in a PyCapsule named "dltensor"), so materialised weights can be handed to
another framework without a copy."""
import ctypes

KDL_ROCM = 10
KDL_FLOAT, KDL_BFLOAT = 2, 4


class DLDevice(ctypes.Structure):
    _fields_ = [("device_type", ctypes.c_int32), ("device_id", ctypes.c_int32)]


class DLDataType(ctypes.Structure):
    _fields_ = [("code", ctypes.c_uint8), ("bits", ctypes.c_uint8), ("lanes", ctypes.c_uint16)]


class DLTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("device", DLDevice),
        ("ndim", ctypes.c_int32),
        ("dtype", DLDataType),
        ("shape", ctypes.POINTER(ctypes.c_int64)),
        ("strides", ctypes.POINTER(ctypes.c_int64)),
        ("byte_offset", ctypes.c_uint64),
    ]


class DLManagedTensor(ctypes.Structure):
    pass


_DELETER = ctypes.CFUNCTYPE(None, ctypes.POINTER(DLManagedTensor))
DLManagedTensor._fields_ = [("dl_tensor", DLTensor), ("manager_ctx", ctypes.c_void_p), ("deleter", _DELETER)]

_py = ctypes.pythonapi
_py.PyCapsule_New.restype = ctypes.py_object
_py.PyCapsule_New.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p]
_py.PyCapsule_GetPointer.restype = ctypes.c_void_p
_py.PyCapsule_GetPointer.argtypes = [ctypes.py_object, ctypes.c_char_p]
# The capsule destructor receives the capsule as a raw pointer.
_IsValid = ctypes.PYFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_char_p)(("PyCapsule_IsValid", _py))
_GetPointerRaw = ctypes.PYFUNCTYPE(ctypes.c_void_p, ctypes.c_void_p, ctypes.c_char_p)(("PyCapsule_GetPointer", _py))

# Managed tensors handed out and not yet released by their consumer.
_live = {}


@_DELETER
def _release(mt):
    _live.pop(ctypes.addressof(mt.contents), None)


@ctypes.CFUNCTYPE(None, ctypes.c_void_p)
def _capsule_destructor(cap):
    """DLPack producer rule: a capsule dropped without being consumed (its
    name is still "dltensor"; a consumer renames it "used_dltensor" and calls
    the deleter itself) releases its managed tensor here."""
    if _IsValid(cap, b"dltensor"):
        addr = _GetPointerRaw(cap, b"dltensor")
        if addr:
            _release(ctypes.cast(addr, ctypes.POINTER(DLManagedTensor)))


def capsule(ptr, shape, bf16, device, owner):
    """A "dltensor" capsule describing `ptr` (row-major `shape`, bf16 or f32)."""
    n = len(shape)
    shp = (ctypes.c_int64 * max(1, n))(*shape)
    strides = [1] * n
    for k in range(n - 2, -1, -1):
        strides[k] = strides[k + 1] * shape[k + 1]
    strd = (ctypes.c_int64 * max(1, n))(*strides)
    mt = DLManagedTensor()
    mt.dl_tensor.data = ptr
    mt.dl_tensor.device = DLDevice(KDL_ROCM, device)
    mt.dl_tensor.ndim = n
    mt.dl_tensor.dtype = DLDataType(KDL_BFLOAT if bf16 else KDL_FLOAT, 16 if bf16 else 32, 1)
    mt.dl_tensor.shape = shp
    mt.dl_tensor.strides = strd
    mt.dl_tensor.byte_offset = 0
    mt.manager_ctx = None
    mt.deleter = _release
    _live[ctypes.addressof(mt)] = (mt, shp, strd, owner)
    return _py.PyCapsule_New(ctypes.addressof(mt), b"dltensor", ctypes.cast(_capsule_destructor, ctypes.c_void_p))


def view(cap):
    """The DLManagedTensor behind a capsule (for inspection)."""
    addr = _py.PyCapsule_GetPointer(cap, b"dltensor")
    return DLManagedTensor.from_address(addr)
