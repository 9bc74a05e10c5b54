"""ctypes loader of the oracle's C restatement (oracle/topk_radix.c) -- test infrastructure only."""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "liboracle.so")
_lib = None


def build():
    """Compiles oracle/topk_radix.c with gcc into oracle/_build/liboracle.so."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        lib = ctypes.CDLL(LIB)
        P = ctypes.c_void_p
        lib.topk_radix.argtypes = [P, ctypes.c_int64, ctypes.c_int, P, ctypes.c_int64, P, ctypes.c_int, P,
                                   ctypes.c_int64, ctypes.c_int, P, ctypes.c_int, P]
        lib.topk_radix.restype = None
        _lib = lib
    return _lib


def topk_radix(score, mask, lengths, page_table, width, cu_seqlens_q=None):
    """int32 [rows, 2048] in the reference single kernel's output order."""
    score = np.ascontiguousarray(score, dtype=np.float32)
    rows = score.shape[0]
    lengths = np.ascontiguousarray(lengths, dtype=np.int32)
    pt = np.ascontiguousarray(page_table, dtype=np.int32)
    out = np.empty((rows, 2048), dtype=np.int32)
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.int16)
    cu = None if cu_seqlens_q is None else np.ascontiguousarray(cu_seqlens_q, dtype=np.int32)
    ptr = lambda a: None if a is None else a.ctypes.data_as(ctypes.c_void_p)
    _load().topk_radix(ptr(score), score.shape[1], int(width), ptr(m), 0 if m is None else m.shape[1], ptr(lengths),
                       rows, ptr(pt), pt.shape[1], pt.shape[1], ptr(cu), 0 if cu is None else cu.shape[0] - 1, ptr(out))
    return out
