"""TEST INFRASTRUCTURE ONLY -- ctypes front-end of assign.c, the C restatement
of the reference's assignment solver (src/cpu/matching.cpp:71-571, 690-719)."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "liboracle_assign.so")
_lib = None

STRATEGIES = {"global": 0, "round": 1, "greedy": 2, "pseudo_greedy": 3}


def build() -> str:
    """Compile assign.c into liboracle_assign.so (gcc, OpenMP)."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle_assign.so"], check=True)
    return _LIB


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            build()
        lib = ctypes.CDLL(_LIB)
        i64p = ctypes.POINTER(ctypes.c_int64)
        dp = ctypes.POINTER(ctypes.c_double)
        lib.ml_oracle_assign_batch.argtypes = [dp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                               ctypes.c_double, ctypes.c_int64, ctypes.c_int,
                                               i64p, i64p, ctypes.c_int, i64p]
        lib.ml_oracle_assign_batch.restype = ctypes.c_int
        _lib = lib
    return _lib


def assign_batch(costs, inf_thresh=1e30, topk=1, strategy=0, nthreads=1, return_iters=False):
    """costs: (N, Q, GT_out) float64.  Returns (pred_to_gt, pred_round) int64
    (N, Q) [, iterations of the solver's inner loop per slice]."""
    lib = _load()
    c = np.ascontiguousarray(costs, dtype=np.float64)
    N, Q, G = c.shape
    p2g = np.empty((N, Q), dtype=np.int64)
    pr = np.empty((N, Q), dtype=np.int64)
    it = np.zeros((N,), dtype=np.int64)
    i64p = ctypes.POINTER(ctypes.c_int64)
    rc = lib.ml_oracle_assign_batch(c.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), N, Q, G,
                                    float(inf_thresh), int(topk), int(strategy),
                                    p2g.ctypes.data_as(i64p), pr.ctypes.data_as(i64p),
                                    int(nthreads), it.ctypes.data_as(i64p))
    if rc == 1:
        raise RuntimeError("Hungarian: no augmenting path found; check costs/inf_thresh.")
    if rc != 0:
        raise RuntimeError(f"oracle assign failed rc={rc}")
    if return_iters:
        return p2g, pr, it
    return p2g, pr
