"""ctypes access to the C restatement (oracle/cref.c). Test infrastructure only."""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "liboracle_c.so")
_LIB = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _SO


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        f32p = ctypes.POINTER(ctypes.c_float)
        L.cref_round.restype = ctypes.c_double
        L.cref_round.argtypes = [ctypes.c_double, ctypes.c_int]
        L.cref_bf16_bits.restype = ctypes.c_uint16
        L.cref_bf16_bits.argtypes = [ctypes.c_float]
        L.cref_dequant.restype = None
        L.cref_dequant.argtypes = [ctypes.c_void_p, ctypes.c_long, f32p, ctypes.c_int,
                                   ctypes.c_int, ctypes.c_int, f32p]
        L.cref_expert.restype = None
        L.cref_expert.argtypes = [f32p, f32p, f32p, f32p, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_int, f32p, f32p]
        L.cref_e4m3.restype = ctypes.c_float
        L.cref_e4m3.argtypes = [ctypes.c_uint8]
        L.cref_e2m1.restype = ctypes.c_float
        L.cref_e2m1.argtypes = [ctypes.c_uint8]
        _LIB = L
    return _LIB


def _fp(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


ACT = {"bf16": 0, "fp16": 1, "fp32": 2}


def round_act(values, act: str) -> np.ndarray:
    L = lib()
    v = np.asarray(values, dtype=np.float64).reshape(-1)
    return np.array([L.cref_round(float(x), ACT[act]) for x in v], dtype=np.float32)


def dequant(packed_words, scale_values, bits: int, gs: int, act: str) -> np.ndarray:
    p = np.ascontiguousarray(np.asarray(packed_words).astype(np.int32))
    s = np.ascontiguousarray(np.asarray(scale_values, dtype=np.float32))
    out = np.empty(p.size * 32 // bits, dtype=np.float32)
    lib().cref_dequant(p.ctypes.data, p.size, _fp(s), bits, gs, ACT[act], _fp(out))
    return out


def expert(x, wg, wd, wu, act: str):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    wg, wd, wu = (np.ascontiguousarray(w, dtype=np.float32) for w in (wg, wd, wu))
    inter, hidden = wg.shape
    h = np.empty(inter, np.float32)
    y = np.empty(hidden, np.float32)
    lib().cref_expert(_fp(x), _fp(wg), _fp(wd), _fp(wu), hidden, inter, ACT[act], _fp(h), _fp(y))
    return h, y


def e4m3(byte: int) -> float:
    return lib().cref_e4m3(byte)


def e2m1(nibble: int) -> float:
    return lib().cref_e2m1(nibble)
