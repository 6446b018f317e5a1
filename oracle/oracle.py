"""numpy front end of the CPU oracle (liboracle.so) and of oracle/_ref.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  Product code never imports it.

Attention functions take float32 arrays holding fp16-rounded values and return
float32, like the reference CPU ops (src/cpu/ops.h); KV-movement functions
take uint16 arrays (raw binary16 patterns) so comparisons are bit-exact.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(_HERE, "liboracle.so")
REF_LIB = os.path.join(_HERE, "_ref", "libref_ops.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64
_int = ctypes.c_int
_flt = ctypes.c_float

_ORACLE_SIGS = {
    "kvo_f32_to_f16": (ctypes.c_uint16, [_flt]),
    "kvo_f16_to_f32": (_flt, [ctypes.c_uint16]),
    "kvo_f32_to_f16_array": (None, [_f32p, _u16p, _i64]),
    "kvo_f16_to_f32_array": (None, [_u16p, _f32p, _i64]),
    "kvo_causal_gqa": (None, [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, _i64]),
    "kvo_causal_gqa_rows": (None, [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _i64,
                                   _i64, _int]),
    "kvo_causal_gqa_rowlist": (None, [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, _i64,
                                      _i64p, _i64, _int]),
    "kvo_decode_attention": (None, [_f32p, _f32p, _f32p, _i32p, _f32p, _i64, _i64, _i64, _i64,
                                    _i64, _int]),
    "kvo_decode_split_partial": (None, [_f32p, _f32p, _f32p, _i64, _i64, _i64,
                                        ctypes.POINTER(_flt), ctypes.POINTER(ctypes.c_double),
                                        _f64p]),
    "kvo_lse_merge": (None, [_f32p, _f64p, _f64p, _i64, _i64, _f32p]),
    "kvo_decode_attention_splitk": (None, [_f32p, _f32p, _f32p, _i32p, _f32p, _i64, _i64, _i64,
                                           _i64, _i64, _i64, _int]),
    "kvo_append_kv": (None, [_u16p, _u16p, _u16p, _u16p, _i64, _i64, _i64, _i64, _i64]),
    "kvo_paged_append": (None, [_u16p, _u16p, _u16p, _u16p, _i32p, _i64, _i32p, _i64, _i64,
                                _i64, _i64, _i64, _i64]),
    "kvo_paged_gather": (None, [_u16p, _u16p, _i32p, _i64, _i32p, _i64, _i64, _i64, _i64, _i64,
                                _i64, _u16p, _u16p]),
    "kvo_rmsnorm": (None, [_f32p, _f32p, _f32p, _i64, _i64, _flt]),
    "kvo_matmul_transB": (None, [_f32p, _f32p, _f32p, _i64, _i64, _i64, _int]),
    "kvo_matmul_transB_scalar": (None, [_f32p, _f32p, _f32p, _i64, _i64, _i64, _int]),
    "kvo_apply_rope": (None, [_f32p, _f32p, _i64, _i64, _i64, _i64, _i64, _flt]),
    "kvo_swiglu": (None, [_f32p, _f32p, _f32p, _i64]),
}

_REF_SIGS = {
    "ref_causal_gqa": (None, [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, _i64]),
    "ref_rmsnorm": (None, [_f32p, _f32p, _f32p, _i64, _i64, _flt]),
    "ref_matmul_transB_blocked": (None, [_f32p, _f32p, _f32p, _i64, _i64, _i64]),
    "ref_apply_rope": (None, [_f32p, _f32p, _i64, _i64, _i64, _i64, _i64, _flt]),
    "ref_swiglu": (None, [_f32p, _f32p, _f32p, _i64]),
}

_lib = None
_ref = None


def _bind(path, sigs):
    lib = ctypes.CDLL(path)
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_LIB):
            raise FileNotFoundError(f"{ORACLE_LIB} missing: run `make -C oracle`")
        _lib = _bind(ORACLE_LIB, _ORACLE_SIGS)
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_LIB)


def ref():
    """The reference's own src/cpu/ops.cpp, compiled by `make -C oracle ref`."""
    global _ref
    if _ref is None:
        _ref = _bind(REF_LIB, _REF_SIGS)
    return _ref


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# ------------------------------------------------------------------ fp16 --
def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32).ravel()
    out = np.empty(x.shape, np.uint16)
    lib().kvo_f32_to_f16_array(x, out, x.size)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = _c(h, np.uint16).ravel()
    out = np.empty(h.shape, np.float32)
    lib().kvo_f16_to_f32_array(h, out, h.size)
    return out


# ------------------------------------------------------------- attention --
def causal_gqa(q, k, v, hq, hkv, d, rows: Optional[tuple] = None, nthreads: int = 1):
    """q [S][Hq][D], k/v [S][Hkv][D] (float32) -> out [S][Hq][D] float32.
    rows=(begin, end) computes only those rows (others left zero)."""
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    s = q.size // (hq * d)
    out = np.zeros(q.shape, np.float32)
    rb, re = (0, s) if rows is None else rows
    lib().kvo_causal_gqa_rows(q, k, v, out, s, hq, hkv, d, rb, re, nthreads)
    return out


def causal_gqa_rowlist(q, k, v, hq, hkv, d, rows, nthreads: int = 1):
    """Rows `rows` (a list of indices) of causal_gqa -> out [len(rows)][Hq][D]."""
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    s = q.size // (hq * d)
    r = _c(rows, np.int64).ravel()
    if r.size and (r.min() < 0 or r.max() >= s):
        raise ValueError("causal_gqa_rowlist: row outside [0, S)")
    out = np.zeros((r.size, hq, d), np.float32)
    lib().kvo_causal_gqa_rowlist(q, k, v, out, s, hq, hkv, d, r, r.size, nthreads)
    return out


def ref_causal_gqa(q, k, v, hq, hkv, d):
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    s = q.size // (hq * d)
    out = np.zeros(q.shape, np.float32)
    ref().ref_causal_gqa(q, k, v, out, s, hq, hkv, d)
    return out


def decode_attention(q, k, v, seq_lens, hq, hkv, d, nthreads: int = 1):
    """q [B][Hq][D]; k/v contiguous [B][Hkv][cap][D] float32 -> [B][Hq][D]."""
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    sl = _c(seq_lens, np.int32)
    b = sl.size
    cap = k.size // (b * hkv * d)
    out = np.zeros((b, hq, d), np.float32)
    lib().kvo_decode_attention(q, k, v, sl, out, b, hq, hkv, d, cap, nthreads)
    return out


def decode_attention_splitk(q, k, v, seq_lens, hq, hkv, d, chunk, nthreads: int = 1):
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    sl = _c(seq_lens, np.int32)
    b = sl.size
    cap = k.size // (b * hkv * d)
    out = np.zeros((b, hq, d), np.float32)
    lib().kvo_decode_attention_splitk(q, k, v, sl, out, b, hq, hkv, d, cap, chunk, nthreads)
    return out


def split_partial(q_vec, k_head, v_head, t0, t1):
    d = q_vec.size
    m = ctypes.c_float()
    l = ctypes.c_double()
    o = np.zeros(d, np.float64)
    lib().kvo_decode_split_partial(_c(q_vec, np.float32), _c(k_head, np.float32),
                                   _c(v_head, np.float32), d, t0, t1, ctypes.byref(m),
                                   ctypes.byref(l), o)
    return m.value, l.value, o


def lse_merge(ms, ls, os_):
    ms = _c(ms, np.float32)
    ls = _c(ls, np.float64)
    os_ = _c(os_, np.float64)
    n, d = os_.shape
    out = np.zeros(d, np.float32)
    lib().kvo_lse_merge(ms, ls, os_, n, d, out)
    return out


# ----------------------------------------------------------- KV movement --
def append_kv(src_k, src_v, dst_k, dst_v, num_tokens, start_pos, hkv, max_seq, d):
    """In place on uint16 dst arrays [Hkv][max_seq][D]."""
    lib().kvo_append_kv(_c(src_k, np.uint16), _c(src_v, np.uint16), dst_k, dst_v,
                        num_tokens, start_pos, hkv, max_seq, d)


def paged_append(src_k, src_v, pool_k, pool_v, block_tables, start_pos, b, t, hkv, d):
    """In place on uint16 pools [Hkv][P][16][D]."""
    bt = _c(block_tables, np.int32)
    p, page = pool_k.shape[1], pool_k.shape[2]
    lib().kvo_paged_append(_c(src_k, np.uint16), _c(src_v, np.uint16), pool_k, pool_v, bt,
                           bt.shape[1], _c(start_pos, np.int32), b, t, hkv, d, p, page)


def paged_gather(pool_k, pool_v, block_tables, seq_lens, max_len):
    bt = _c(block_tables, np.int32)
    sl = _c(seq_lens, np.int32)
    hkv, p, page, d = pool_k.shape
    b = sl.size
    ok = np.zeros((b, hkv, max_len, d), np.uint16)
    ov = np.zeros((b, hkv, max_len, d), np.uint16)
    lib().kvo_paged_gather(_c(pool_k, np.uint16), _c(pool_v, np.uint16), bt, bt.shape[1], sl,
                           b, hkv, d, p, page, max_len, ok, ov)
    return ok, ov


# ------------------------------------------------------- supporting ops --
def rmsnorm(x, w, eps, use_ref=False):
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    dim = w.size
    out = np.empty_like(x)
    (ref().ref_rmsnorm if use_ref else lib().kvo_rmsnorm)(x, w, out, x.size // dim, dim, eps)
    return out


def matmul_transB(a, b, nthreads=1, use_ref=False, scalar=False):
    a = _c(a, np.float32)
    b = _c(b, np.float32)
    m, k = a.shape
    n = b.shape[0]
    out = np.empty((m, n), np.float32)
    if use_ref:
        ref().ref_matmul_transB_blocked(a, b, out, m, k, n)
    elif scalar:
        lib().kvo_matmul_transB_scalar(a, b, out, m, k, n, nthreads)
    else:
        lib().kvo_matmul_transB(a, b, out, m, k, n, nthreads)
    return out


def apply_rope(q, k, hq, hkv, d, start_pos, theta, use_ref=False):
    q = _c(q, np.float32).copy()
    k = _c(k, np.float32).copy()
    s = q.size // (hq * d)
    (ref().ref_apply_rope if use_ref else lib().kvo_apply_rope)(q, k, s, hq, hkv, d, start_pos,
                                                                 theta)
    return q, k


def swiglu(gate, up, use_ref=False):
    gate = _c(gate, np.float32)
    up = _c(up, np.float32)
    out = np.empty_like(gate)
    (ref().ref_swiglu if use_ref else lib().kvo_swiglu)(gate, up, out, gate.size)
    return out


# ---------------------------------------------------------------- inputs --
def normal_f16(rng: np.random.Generator, shape, scale: float = 1.0) -> np.ndarray:
    """N(0, scale^2) samples rounded to fp16 (numpy's cast is IEEE RNE)."""
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float16)
