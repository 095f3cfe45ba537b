"""ctypes view of the oracle's C++ OpenMP restatement of the decode composition (cpu_moe.cpp; test infrastructure
only: the CPU baseline's second leg and a cross-check of oracle.moe.decode_apply)."""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libcpu_moe.so")
_L = None


def build():
    """Compile libcpu_moe.so with the Makefile beside this file."""
    subprocess.run(["make", "-s", "-C", HERE, "-B", "libcpu_moe.so"], check=True)
    return LIB


def lib():
    global _L
    if _L is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        P, I, F = ctypes.c_void_p, ctypes.c_int32, ctypes.c_float
        L.cpu_moe_decode_cb3.restype = I
        L.cpu_moe_decode_cb3.argtypes = [I, I, I, P, P, P, P, P, P, P, I, I, P, P, I, F, P, I]
        L.cpu_moe_threads.restype = I
        _L = L
    return _L


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def decode_cb3(gate, up, down, x, idx, w, limit, shared=-1, threads=0):
    """gate/up/down: (words u32 [E, R, ceil(K/10)], codebook u16 [E, R, K/128, 8]) in the canonical CB3 packing;
    x [N, D]; idx int32 [N, k]; w f32 [N, k] -> f64 [N, D] (routed slots + the shared expert, weight 1)."""
    (gw, gc), (uw, uc), (dw, dc) = [(np.ascontiguousarray(a, np.uint32), np.ascontiguousarray(b, np.uint16))
                                    for a, b in (gate, up, down)]
    E, I = gw.shape[0], gw.shape[1]
    D = dw.shape[1]
    x = np.ascontiguousarray(x, np.float32)
    idx = np.ascontiguousarray(idx, np.int32)
    w = np.ascontiguousarray(w, np.float32)
    N, k = idx.shape
    out = np.empty((N, D), np.float64)
    rc = lib().cpu_moe_decode_cb3(E, D, I, _p(gw), _p(gc), _p(uw), _p(uc), _p(dw), _p(dc), _p(x), N, k, _p(idx),
                                  _p(w), int(shared), float(limit), _p(out), int(threads))
    if rc != 0:
        raise ValueError("cpu_moe_decode_cb3: invalid arguments")
    return out


def threads():
    return lib().cpu_moe_threads()
