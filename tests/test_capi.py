"""C-ABI library (libvkwr_amd.so): loads, exports every symbol include/vkwr_amd.h
declares, and rejects bad arguments on the host before any GPU work."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vkwr_amd.h")
LIBPATH = os.path.join(ROOT, "vkwr_amd", "libvkwr_amd.so")


def declared_symbols():
    text = open(HEADER).read()
    return re.findall(r"^VKWR_EXPORT\s+[\w\s\*]+?\b(vkwr_\w+)\s*\(", text, flags=re.M)


@pytest.fixture(scope="module")
def capi():
    import torch  # noqa: F401  (bind to torch's HIP runtime first)

    assert os.path.exists(LIBPATH), "libvkwr_amd.so not built (run __graft_entry__.build())"
    L = ctypes.CDLL(LIBPATH)
    L.vkwr_status_string.restype = ctypes.c_char_p
    L.vkwr_last_error.restype = ctypes.c_char_p
    return L


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert len(syms) >= 7
    assert len(set(syms)) == len(syms)


def test_every_declared_symbol_is_exported(capi):
    missing = [s for s in declared_symbols() if not hasattr(capi, s)]
    assert not missing, missing


def test_status_strings(capi):
    assert capi.vkwr_status_string(0) == b"ok"
    assert capi.vkwr_status_string(1) == b"invalid argument"
    assert capi.vkwr_status_string(2) == b"launch failure"


def _fake():
    # non-null pointers that are never dereferenced: validation fails first
    return ctypes.c_void_p(0x1000)


def test_rejects_bad_head_size(capi):
    p = _fake()
    st = capi.vkwr_wkv7_fp32_forward(1, 1, 100, 2, 0, p, p, p, p, p, p, p, p, None)
    assert st == 1
    assert b"head size 64" in capi.vkwr_last_error()


def test_rejects_bad_mode(capi):
    p = _fake()
    assert capi.vkwr_wkv7_fp32_forward(1, 1, 64, 1, 7, p, p, p, p, p, p, p, p, None) == 1
    assert b"mode" in capi.vkwr_last_error()


def test_rejects_null_pointers(capi):
    p = _fake()
    assert capi.vkwr_wkv7_fp32_forward_slots(1, 1, 64, 1, None, 4, p, p, p, p, p, p, p, p, None) == 1
    assert b"null" in capi.vkwr_last_error()
    assert capi.vkwr_wkv7_fp16_forward(1, 1, 64, 1, p, p, p, None, p, p, p, p, p, None, None) == 1
    assert capi.vkwr_advance_i32(None, ctypes.c_int64(4), 1, None) == 1


def test_empty_work_is_a_noop(capi):
    # B = 0 or T = 0: nothing to launch, success, pointers untouched
    assert capi.vkwr_wkv7_fp32_forward(0, 1, 64, 1, 0, None, None, None, None, None, None, None, None, None) == 0
    assert capi.vkwr_wkv7_fp32_forward(1, 0, 64, 1, 0, None, None, None, None, None, None, None, None, None) == 0
    assert capi.vkwr_advance_i32(None, ctypes.c_int64(0), 1, None) == 0
