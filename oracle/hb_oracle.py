"""ctypes loader of the CPU oracle (oracle/hb_oracle.c).  TEST INFRASTRUCTURE:
only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker (or the timed CPU baseline), never as a
product path.  Builds liboracle.so with `make` when it is missing and gcc is
there.

Parity pinning of each function is listed in hb_oracle.c's header.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

OUT_BF16, OUT_F32, OUT_RESIDUAL = 0, 1, 2


def build():
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)


def _load():
    src = os.path.join(HERE, "hb_oracle.c")
    if not os.path.exists(LIB_PATH) or os.path.getmtime(LIB_PATH) < os.path.getmtime(src):
        build()
    return ctypes.CDLL(LIB_PATH)


lib = _load()
_P = ctypes.c_void_p
lib.hbo_bf16_to_f32.argtypes = [ctypes.c_uint16]
lib.hbo_bf16_to_f32.restype = ctypes.c_float
lib.hbo_f32_to_bf16.argtypes = [ctypes.c_float]
lib.hbo_f32_to_bf16.restype = ctypes.c_uint16
lib.hbo_f32_to_bf16_range.argtypes = [ctypes.c_uint32, ctypes.c_uint32, _P]
lib.hbo_gemm.argtypes = [_P, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                         ctypes.c_int]
lib.hbo_experts_gemm.argtypes = [_P, _P, _P, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_int, ctypes.c_int, ctypes.c_int]
lib.hbo_expf.argtypes = [ctypes.c_float]
lib.hbo_expf.restype = ctypes.c_float
lib.hbo_route.argtypes = [_P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P]
lib.hbo_moe_sort.argtypes = [_P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P, _P]
lib.hbo_moe_sort.restype = ctypes.c_uint32
lib.hbo_moe_tiles.argtypes = [ctypes.c_int] * 4
lib.hbo_moe_tiles.restype = ctypes.c_uint32
lib.hbo_gather_rows.argtypes = [_P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P]
lib.hbo_swiglu.argtypes = [_P, ctypes.c_int, ctypes.c_int, _P]
lib.hbo_gemm_swiglu.argtypes = [_P, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
lib.hbo_combine.argtypes = [_P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P]


def _p(a):
    return a.ctypes.data_as(_P)


def _c(a, dtype):
    a = np.ascontiguousarray(a)
    assert a.dtype == dtype, (a.dtype, dtype)
    return a


def threads_default():
    return min(16, os.cpu_count() or 1)


def rne_range(first, n):
    """hbo_f32_to_bf16_range: the bf16 RNE of the f32 patterns first..first+n-1."""
    out = np.empty(n, np.uint16)
    lib.hbo_f32_to_bf16_range(first, n, _p(out))
    return out


def gemm(x, w, out=OUT_BF16, y=None, threads=None):
    """Y[m][n] = X[m][k] . W[n][k]^T under the contract; y: Residual's input."""
    x = _c(x, np.uint16)
    w = _c(w, np.uint16)
    m, k = x.shape
    n = w.shape[0]
    assert w.shape[1] == k
    if out == OUT_F32:
        res = np.zeros((m, n), np.float32)
    elif out == OUT_RESIDUAL:
        res = np.array(y, dtype=np.uint16, order="C", copy=True).reshape(m, n)
    else:
        res = np.zeros((m, n), np.uint16)
    lib.hbo_gemm(_p(x), _p(w), _p(res), m, k, n, out, threads or threads_default())
    return res


def experts_gemm(x, w, list_, tiles, k, n, mode, top_k, pairs, out=OUT_BF16, threads=None):
    """The grouped expert GEMM (mode 1 Gather, 2 Scatter); rows not covered stay 0."""
    x = _c(x, np.uint16)
    w = _c(w, np.uint16)
    list_ = _c(list_, np.uint32)
    tiles = _c(tiles, np.uint32)
    res = np.zeros((pairs, n), np.float32 if out == OUT_F32 else np.uint16)
    lib.hbo_experts_gemm(_p(x), _p(w), _p(res), _p(list_), _p(tiles), k, n, mode, top_k, out,
                         threads or threads_default())
    return res


def expf(x):
    return lib.hbo_expf(float(x))


def route(scores, top_k):
    scores = _c(scores, np.uint16)
    rows, experts = scores.shape
    out = np.zeros((rows, 2 * top_k), np.uint32)
    lib.hbo_route(_p(scores), rows, experts, top_k, _p(out))
    return out


def moe_sort(route_, top_k, experts, bm):
    route_ = _c(route_, np.uint32)
    rows = route_.shape[0]
    lst = np.zeros(rows * top_k, np.uint32)
    tiles = np.zeros(1 + 3 * int(lib.hbo_moe_tiles(rows, top_k, experts, bm)), np.uint32)
    lib.hbo_moe_sort(_p(route_), rows, top_k, experts, bm, _p(lst), _p(tiles))
    return lst, tiles


def gather_rows(x, list_, top_k):
    x = _c(x, np.uint16)
    list_ = _c(list_, np.uint32)
    xs = np.zeros((len(list_), x.shape[1]), np.uint16)
    lib.hbo_gather_rows(_p(x), _p(list_), len(list_), top_k, x.shape[1], _p(xs))
    return xs


def swiglu(gu, n):
    gu = _c(gu, np.uint16)
    slots = gu.size // (2 * n)
    h = np.zeros((slots, n), np.uint16)
    lib.hbo_swiglu(_p(gu), slots, n, _p(h))
    return h


def gemm_swiglu(x, w, inter, threads=None):
    x = _c(x, np.uint16)
    w = _c(w, np.uint16)
    m, k = x.shape
    h = np.zeros((m, inter), np.uint16)
    lib.hbo_gemm_swiglu(_p(x), _p(w), _p(h), m, k, inter, threads or threads_default())
    return h


lib.hbo_rmsnorm_rows.argtypes = [_P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int,
                                 ctypes.c_int, _P]


def rmsnorm_rows(x, w, eps, plus_one=False, order=0):
    """XSrc::Norm's normed rows (hb_oracle.c hbo_rmsnorm_rows): order 0 the
    HIP kernel's summation order, 1 increasing index."""
    x = _c(x, np.uint16)
    w = _c(w, np.uint16)
    m, k = x.shape
    out = np.zeros((m, k), np.uint16)
    lib.hbo_rmsnorm_rows(_p(x), _p(w), m, k, float(eps), 1 if plus_one else 0, order, _p(out))
    return out


lib.hbo_moe_out.argtypes = [_P, _P, _P, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int]


def moe_out(xn, gate, ex, sh, x, order=0):
    """moe_out (hb_oracle.c hbo_moe_out): the updated x (a copy)."""
    xn, gate, ex, sh = (_c(a, np.uint16) for a in (xn, gate, ex, sh))
    out = np.array(x, dtype=np.uint16, order="C", copy=True)
    rows, d = out.shape
    lib.hbo_moe_out(_p(xn), _p(gate), _p(ex), _p(sh), _p(out), rows, d, order)
    return out


def combine(y, route_, top_k, d):
    y = _c(y, np.uint16)
    route_ = _c(route_, np.uint32)
    rows = route_.shape[0]
    out = np.zeros((rows, d), np.uint16)
    lib.hbo_combine(_p(y), _p(route_), rows, top_k, d, _p(out))
    return out
