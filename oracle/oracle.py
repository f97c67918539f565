"""ctypes binding of the C oracle (``wkv_oracle.c``) -- test infrastructure only.

Arrays are numpy: fp16 tensors travel as ``np.float16`` (bit-identical uint16
views are passed to C), fp32 states as ``np.float32``.  Every function mutates
``state`` in place and returns ``y``, mirroring the reference ops'
``Tensor(a!) state`` contract (csrc/v1/wkv/torch_bindings.cpp:231-258).
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library not built: run `make -C {_HERE}`")
        L = ctypes.CDLL(path)
        p = ctypes.c_void_p
        i = ctypes.c_int
        L.oracle_wkv_fp32.argtypes = [i, i, i, i, p, p, p, p, p, p, p, p]
        L.oracle_wkv_fp32_rows.argtypes = [i, i, i, i, p, p, p, p, p, p, p, p]
        L.oracle_wkv_fp16.argtypes = [i, i, i, i, p, p, p, p, p, p, p, p, p, p, i]
        L.oracle_advance_i32.argtypes = [p, ctypes.c_int64, ctypes.c_int32]
        L.oracle_decay.argtypes = [ctypes.c_float]
        L.oracle_decay.restype = ctypes.c_float
        L.oracle_exp2.argtypes = [ctypes.c_float]
        L.oracle_exp2.restype = ctypes.c_float
        L.oracle_rotator.argtypes = [ctypes.c_int32]
        L.oracle_rotator.restype = ctypes.c_float
        L.oracle_w_delta.argtypes = [ctypes.c_float, ctypes.c_int32]
        L.oracle_w_delta.restype = ctypes.c_uint16
        L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        for fn in ("oracle_fma16", "oracle_add16", "oracle_mul16"):
            getattr(L, fn).restype = ctypes.c_uint16
        L.oracle_fma16.argtypes = [ctypes.c_uint16] * 3
        L.oracle_add16.argtypes = [ctypes.c_uint16] * 2
        L.oracle_mul16.argtypes = [ctypes.c_uint16] * 2
        L.oracle_set_threads.argtypes = [i]
        L.oracle_get_threads.restype = i
        _LIB = L
    return _LIB


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c16(x):
    x = np.ascontiguousarray(x)
    assert x.dtype == np.float16, x.dtype
    return x


def set_threads(n):
    lib().oracle_set_threads(int(n))


def get_threads():
    return lib().oracle_get_threads()


def wkv_fp32(B, T, C, H, state, r, w, k, v, a, b, order="seq"):
    """fp32-state WKV-7 (wkv_fp32_v2.cu:59-125). state [B,H,64,64] f32 (in place).

    order "seq": each dot product one FMA chain over j (the reference's row-per-thread
    kernel); "rows": the row-split order of the prefill kernel (wkv_oracle.c row_dot)."""
    assert state.dtype == np.float32 and state.flags.c_contiguous
    assert state.shape == (B, H, 64, 64) and C == H * 64
    assert order in ("seq", "rows"), order
    ins = [_c16(x).reshape(B, T, C) for x in (r, w, k, v, a, b)]
    y = np.empty((B, T, C), dtype=np.float16)
    fn = lib().oracle_wkv_fp32 if order == "seq" else lib().oracle_wkv_fp32_rows
    fn(B, T, C, H, _ptr(state), *[_ptr(x) for x in ins], _ptr(y))
    return y


def wkv_fp16(B, T, C, H, state, r, w, k, v, a, b, elapsed_t, w0=None, legacy=False):
    """fp16-state WKV-7 (wkv_fp16_v2.cu) or, with legacy=True, vkwr_rwkv7 (state_fwd_fp16.cu)."""
    assert state.dtype == np.float16 and state.flags.c_contiguous
    assert state.size == B * H * 64 * 64 and C == H * 64
    ins = [_c16(x).reshape(B, T, C) for x in (r, w, k, v, a, b)]
    el = np.ascontiguousarray(elapsed_t, dtype=np.int32)
    w0p = None if w0 is None else _c16(w0).reshape(-1)
    y = np.empty((B, T, C), dtype=np.float16)
    lib().oracle_wkv_fp16(B, T, C, H, _ptr(state), _ptr(ins[0]), _ptr(ins[1]),
                          None if w0p is None else _ptr(w0p),
                          *[_ptr(x) for x in ins[2:]], _ptr(y), _ptr(el), 1 if legacy else 0)
    return y


def wkv_fp32_slots(B, T, C, H, pool, slots, r, w, k, v, a, b, order="seq"):
    """Slot-indexed reference semantics: pool[slots] -> wkv_fp32 -> pool[slots] = result."""
    st = np.ascontiguousarray(pool[slots])
    y = wkv_fp32(B, T, C, H, st, r, w, k, v, a, b, order=order)
    pool[slots] = st
    return y


def advance_i32(x, amount):
    assert x.dtype == np.int32 and x.flags.c_contiguous
    lib().oracle_advance_i32(_ptr(x), x.size, int(amount))


def decay(w):
    return lib().oracle_decay(float(w))


def exp2(x):
    return lib().oracle_exp2(float(x))


def rotator(phase):
    return lib().oracle_rotator(int(phase))


def w_delta(w, phase):
    return lib().oracle_w_delta(float(w), int(phase))


def f32_to_f16_bits(f):
    return lib().oracle_f32_to_f16(float(f))


def fma16_bits(a, b, c):
    return lib().oracle_fma16(int(a), int(b), int(c))


def add16_bits(a, b):
    return lib().oracle_add16(int(a), int(b))


def mul16_bits(a, b):
    return lib().oracle_mul16(int(a), int(b))
