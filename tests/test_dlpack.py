"""DLPack producer rules of the materialised-tensor export (CPU only: the
capsule describes device memory but building and dropping it touches none)."""
import ctypes
import gc

from ltx_weights import _dlpack as D


def test_unconsumed_capsule_releases_its_tensor():
    cap = D.capsule(0x1000, (2, 3), True, 0, owner=object())
    assert len(D._live) == 1
    del cap
    gc.collect()
    assert len(D._live) == 0


def test_consumed_capsule_is_released_by_the_consumer_only():
    cap = D.capsule(0x2000, (4,), False, 0, owner=object())
    mt = D.view(cap)
    assert (mt.dl_tensor.ndim, mt.dl_tensor.shape[0], mt.dl_tensor.strides[0]) == (1, 4, 1)
    # What a consumer does: rename the capsule, keep the tensor, call the deleter when done.
    set_name = ctypes.pythonapi.PyCapsule_SetName
    set_name.argtypes = [ctypes.py_object, ctypes.c_char_p]
    assert set_name(cap, b"used_dltensor") == 0
    del cap
    gc.collect()
    assert len(D._live) == 1
    mt.deleter(ctypes.pointer(mt))
    assert len(D._live) == 0
