"""CPU checks of the C ABI boundary: the library loads, exports every entry
point the headers in include/ declare, and reports a missing device as an error."""
import ctypes
import os
import re

import pytest

import ltx_weights as lw

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_entry_points():
    names = set()
    inc = os.path.join(ROOT, "include")
    for h in sorted(os.listdir(inc)):
        if not h.endswith(".h"):
            continue
        with open(os.path.join(inc, h)) as f:
            text = f.read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(ltxw_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_declares_the_entry_points():
    names = declared_entry_points()
    assert "ltxw_dequant" in names and "ltxw_dequant_lora" in names and "ltxw_dequant_lora_grouped" in names
    assert "ltxw_store_open" in names and "ltxw_store_materialize" in names and "ltxw_store_merge_lora" in names


def test_library_exports_every_declared_symbol():
    L = lw.lib()
    missing = [n for n in declared_entry_points() if not hasattr(L, n)]
    assert not missing, missing


def test_python_binding_covers_every_declared_symbol():
    from ltx_weights import _native
    assert sorted(_native.EXPORTS) == declared_entry_points()


def test_context_without_device_reports_error():
    hip = ctypes.CDLL("libamdhip64.so")
    n = ctypes.c_int(0)
    if hip.hipGetDeviceCount(ctypes.byref(n)) == 0 and n.value > 0:
        pytest.skip("a GPU is visible")
    with pytest.raises(lw.WeightError) as e:
        lw.Context(0)
    assert isinstance(e.value, (lw.DeviceError, lw.InvalidArgument))
    assert str(e.value)


def test_null_context_calls_fail_cleanly():
    L = lw.lib()
    assert L.ltxw_synchronize(None) == lw.InvalidArgument.code
    assert L.ltxw_dequant(None, None, 1, 1, 0, 0, None, None, 0) == lw.InvalidArgument.code
    assert L.ltxw_ctx_stream(None) is None
    L.ltxw_ctx_destroy(None)


def test_null_store_calls_fail_cleanly():
    L = lw.lib()
    assert L.ltxw_store_n_keys(None) == 0 and L.ltxw_store_key(None, 0) is None
    assert L.ltxw_store_contains(None, b"x") == 0 and L.ltxw_store_metadata(None, b"x") is None
    assert L.ltxw_store_materialize(None, None, None, 0, 0, 0, None) == lw.InvalidArgument.code
    assert L.ltxw_store_read(None, None, b"x", 0, None, 0) == lw.InvalidArgument.code
    assert L.ltxw_store_merge_lora(None, None, ctypes.c_float(1.0), None) == lw.InvalidArgument.code
    assert L.ltxw_lora_open(None, None) == lw.InvalidArgument.code
    assert L.ltxw_store_last_error()
    L.ltxw_store_close(None)
    L.ltxw_lora_close(None)
    L.ltxw_report_free(None)
