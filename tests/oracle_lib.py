"""ctypes bindings of the CPU oracle (oracle/liboracle.so) and, where it was
built, of the reference's own code (oracle/_ref/libref.so).  Test
infrastructure only: the checker, never the thing measured or shipped."""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "liboracle.so")
REF_SO = os.path.join(ORACLE_DIR, "_ref", "libref.so")
REF_KAT = os.path.join(ORACLE_DIR, "_ref", "q4_down_exec148_synthetic")

Q4_K, Q6_K = 12, 14
BLOCK_BYTES = {Q4_K: 144, Q6_K: 210}

_P = C.c_void_p
_U32 = C.c_uint32
_o = None
_r = None


class Top2(C.Structure):
    _fields_ = [("top1", C.c_uint32), ("top2", C.c_uint32), ("logit1", C.c_float), ("logit2", C.c_float),
                ("finite", C.c_int)]


def oracle() -> C.CDLL:
    global _o
    if _o is None:
        if not os.path.exists(ORACLE_SO):
            subprocess.run(["make", "-s", "-C", ORACLE_DIR, "liboracle.so"], check=True)
        L = C.CDLL(ORACLE_SO)
        sig = {
            "orc_half_to_float": ([C.c_uint16], C.c_float),
            "orc_float_to_half_rne": ([C.c_float], C.c_uint16),
            "orc_q4k_weight": ([_P, _U32], C.c_float),
            "orc_q6k_weight": ([_P, _U32], C.c_float),
            "orc_q4k_code": ([_P, _U32], C.c_uint32),
            "orc_q6k_code": ([_P, _U32, C.POINTER(C.c_int)], C.c_int),
            "orc_q4k_scale_min": ([_P, _U32, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)], None),
            "orc_dequant": ([C.c_int, _P, _U32, _U32, _P], C.c_int),
            "orc_gemv_r0": ([C.c_int, _P, _U32, _U32, _P, _P, _P], C.c_int),
            "orc_gemv_r0_mt": ([C.c_int, _P, _U32, _U32, _P, _P, _P, C.c_int], C.c_int),
            "orc_gemv_r64": ([C.c_int, _P, _U32, _U32, _P, _P, _P], C.c_int),
            "orc_gemv_splitk_r64": ([C.c_int, _P, _U32, _U32, _U32, _P, _P], C.c_int),
            "orc_gemv_r64_xd": ([C.c_int, _P, _U32, _U32, _P, _P], C.c_int),
            "orc_rmsnorm_f32": ([_P, _P, _U32, C.c_float, _P], None),
            "orc_rmsnorm_f64": ([_P, _P, _U32, C.c_double, _P], None),
            "orc_swiglu_f32": ([_P, _P, _U32, _P], None),
            "orc_swiglu_f64": ([_P, _P, _U32, _P], None),
            "orc_rope_f32": ([_P, _U32, _U32, _U32, C.c_float], None),
            "orc_rope_f64": ([_P, _U32, _U32, _U32, C.c_double], None),
            "orc_top2": ([_P, _U32, C.POINTER(Top2)], None),
            "orc_attention_decode_f64": ([_P, _P, _P, _U32, _U32, _U32, _U32, _P], None),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _o = L
    return _o


def have_ref() -> bool:
    return os.path.exists(REF_SO)


def ref() -> C.CDLL:
    global _r
    if _r is None:
        L = C.CDLL(REF_SO)
        sig = {
            "ref_half_to_float": ([C.c_uint16], C.c_float),
            "ref_q6_decode_block": ([_P, _P, _P, _P], None),
            "ref_q6_fixture": ([_U32, _U32, C.c_uint64, C.c_int, _P, _P, _P, _P], C.c_int),
            "ref_q6_arms": ([_P, C.c_size_t, _U32, _U32, _P, _P, _P, _P], C.c_int),
            "ref_q4_source_tuple": ([_P, _P], None),
            "ref_exec148_materialize_block": ([_P, _P], None),
            "ref_sha256": ([_P, C.c_size_t, _P], None),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _r = L
    return _r


def _p(a: np.ndarray):
    return a.ctypes.data


# ----------------------------------------------------------- conveniences
def dequant(qtype: int, w: np.ndarray, rows: int, K: int) -> np.ndarray:
    out = np.empty(rows * K, dtype=np.float32)
    assert oracle().orc_dequant(qtype, _p(w), rows, K, _p(out)) == 0
    return out.reshape(rows, K)


def gemv_r64(qtype: int, w: np.ndarray, rows: int, K: int, x: np.ndarray, bias=None) -> np.ndarray:
    y = np.empty(rows, dtype=np.float64)
    assert oracle().orc_gemv_r64(qtype, _p(w), rows, K, _p(x), None if bias is None else _p(bias), _p(y)) == 0
    return y


def gemv_r64_xd(qtype: int, w: np.ndarray, rows: int, K: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float64)
    y = np.empty(rows, dtype=np.float64)
    assert oracle().orc_gemv_r64_xd(qtype, _p(w), rows, K, _p(x), _p(y)) == 0
    return y


def gemv_r0(qtype: int, w: np.ndarray, rows: int, K: int, x: np.ndarray, bias=None, threads: int = 0) -> np.ndarray:
    y = np.empty(rows, dtype=np.float32)
    b = None if bias is None else _p(bias)
    if threads > 0:
        assert oracle().orc_gemv_r0_mt(qtype, _p(w), rows, K, _p(x), b, _p(y), threads) == 0
    else:
        assert oracle().orc_gemv_r0(qtype, _p(w), rows, K, _p(x), b, _p(y)) == 0
    return y


def splitk_r64(qtype: int, w: np.ndarray, rows: int, K: int, splits: int, x: np.ndarray) -> np.ndarray:
    part = np.empty(splits * rows, dtype=np.float64)
    assert oracle().orc_gemv_splitk_r64(qtype, _p(w), rows, K, splits, _p(x), _p(part)) == 0
    return part.reshape(splits, rows)


def rmsnorm_f64(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x64 = np.ascontiguousarray(x, dtype=np.float64)
    y = np.empty_like(x64)
    oracle().orc_rmsnorm_f64(_p(x64), _p(w), len(x64), eps, _p(y))
    return y


def rmsnorm_f32(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    y = np.empty_like(x)
    oracle().orc_rmsnorm_f32(_p(x), _p(w), len(x), eps, _p(y))
    return y


def swiglu_f64(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, dtype=np.float64)
    u = np.ascontiguousarray(u, dtype=np.float64)
    s = np.empty_like(g)
    oracle().orc_swiglu_f64(_p(g), _p(u), len(g), _p(s))
    return s


def top2(logits: np.ndarray) -> Top2:
    t = Top2()
    oracle().orc_top2(_p(logits), len(logits), C.byref(t))
    return t


def rel_err(y: np.ndarray, r: np.ndarray) -> float:
    """max_i |y_i - r_i| / max(|r_i|, tau), tau = 1e-3 * max|r| (documented floor)."""
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    tau = 1e-3 * float(np.max(np.abs(r))) if r.size else 0.0
    den = np.maximum(np.abs(r), tau)
    den[den == 0] = 1.0
    return float(np.max(np.abs(y - r) / den)) if r.size else 0.0
