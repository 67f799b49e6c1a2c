"""TEST INFRASTRUCTURE ONLY -- ctypes front end of the fp64 CPU oracle (oracle.c).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may
import this module, and only as the checker; the product path never does.

Every function restates an operator of the reference's GEMM family
(champloo2878/cuPilot-Kernels, kernels/1..18 except 5); the file:line of the
wrapper whose shape logic it follows is given per function.  Results are fp64.
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

DENSE, LOWER, UPPER = 0, 1, 2

_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i64p = ctypes.POINTER(ctypes.c_int64)


def build() -> str:
    """Compile oracle.c (gcc) into liboracle.so next to this file."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_splitmix64.restype = _u64
        L.orc_splitmix64.argtypes = [_u64]
        L.orc_fill_uniform_f32.argtypes = [_f32p, _i64, _u64, _i64]
        L.orc_fill_int_f32.argtypes = [_f32p, _i64, _u64, _i64, ctypes.c_int32, ctypes.c_int32]
        L.orc_gemm_f64.argtypes = [_f32p, _f32p, _f64p, _i64, _i64, _i64, _i64,
                                   _i64, _i64, _i64, _i64, _i64, _i64,
                                   ctypes.c_int32, _i64p, _i64]
        L.orc_gemm_entries_f64.argtypes = [_f32p, _f32p, _f64p, _i64p, _i64, _i64,
                                           _i64, _i64, _i64, _i64, _i64, _i64]
        L.orc_gemv_f64.argtypes = [_f32p, _f32p, _f64p, _i64, _i64, _i64, _i64p, _i64]
        L.orc_gemv_generated_f64.argtypes = [_u64, _f32p, _f64p, _i64, _i64p, _i64]
        L.orc_diag_f32.argtypes = [_f32p, _f32p, _f32p, _i64, _i64]
        L.orc_scale_f32.argtypes = [_f32p, _f32p, _i64, ctypes.c_float]
        L.orc_pointwise_conv_f64.argtypes = [_f32p, _f32p, _f32p, _f64p, _i64, _i64, _i64, _i64]
        L.orc_half_to_double.argtypes = [ctypes.c_uint16]
        L.orc_half_to_double.restype = ctypes.c_double
        _u16p = ctypes.POINTER(ctypes.c_uint16)
        L.orc_sdpa_f64.argtypes = [_u16p, _u16p, _u16p, _f64p, _i64, _i64, _i64, ctypes.c_double]
        L.orc_matvec_f64.argtypes = [_f32p, _i64, _i64, _i64, _i64, _f64p, _f64p]
        L.orc_checksums_f32.argtypes = [_f32p, _i64, _i64, _i64, _f64p, _f64p, _f64p, _f64p]
        L.orc_max_abs_diff.restype = ctypes.c_double
        L.orc_max_abs_diff.argtypes = [_f32p, _f64p, _i64]
        L.orc_num_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def _fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_f32p)


def _dp(a: np.ndarray):
    return a.ctypes.data_as(_f64p)


# ---- generator ------------------------------------------------------------

def splitmix64(x: int) -> int:
    return int(lib().orc_splitmix64(x))


def uniform(shape, seed: int, offset: int = 0) -> np.ndarray:
    """Counter-based uniform[-1, 1) fp32 tensor, identical to the device fill."""
    n = int(np.prod(shape)) if len(shape) else 1
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_uniform_f32(out.ctypes.data_as(_f32p), n, seed, offset)
    return out.reshape(shape)


def integers(shape, seed: int, lo: int = -2, hi: int = 2, offset: int = 0) -> np.ndarray:
    """Counter-based integer-valued fp32 tensor in [lo, hi] (exact products)."""
    n = int(np.prod(shape)) if len(shape) else 1
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_int_f32(out.ctypes.data_as(_f32p), n, seed, offset, lo, hi)
    return out.reshape(shape)


# ---- contractions -----------------------------------------------------------

def _strides2(x: np.ndarray):
    """(row, col) element strides of the last two dims."""
    it = x.itemsize
    return x.strides[-2] // it, x.strides[-1] // it


def gemm(a: np.ndarray, b: np.ndarray, structure: int = DENSE,
         rows: Optional[Sequence[int]] = None) -> np.ndarray:
    """fp64-accumulated ``a @ b`` of fp32 operands (any strides; batched if 3-D).

    ``a`` is the *logical* left operand (..., M, K) and ``b`` the logical right
    operand (..., K, N); pass ``x.T`` views to express the reference's
    transposed layouts without copying (kernels/16_...:127-132,
    17_...:268-272, 18_...:156-160).  ``structure`` LOWER / UPPER computes
    tril(tril(a)@tril(b)) / triu(triu(a)@triu(b)) (kernels/15_...:155-206,
    14_...:57-130).  ``rows`` restricts the output to those rows of every batch.
    """
    assert a.dtype == np.float32 and b.dtype == np.float32
    batched = a.ndim == 3
    if not batched:
        a, b = a[None], b[None]
    B_, M, K = a.shape
    Kb, N = b.shape[-2:]
    assert K == Kb, (a.shape, b.shape)
    if b.shape[0] == 1 and B_ > 1:
        sb = 0
    else:
        assert b.shape[0] == B_
        sb = b.strides[0] // 4
    sa = a.strides[0] // 4 if B_ > 1 else 0
    a_rs, a_cs = _strides2(a)
    b_rs, b_cs = _strides2(b)
    # The C side indexes from the first element with the given strides; numpy
    # views with negative strides are not used here.
    assert min(a.strides) >= 0 and min(b.strides) >= 0
    R = M if rows is None else len(rows)
    out = np.empty((B_, R, N), dtype=np.float64)
    rows_arr = None if rows is None else np.ascontiguousarray(rows, dtype=np.int64)
    lib().orc_gemm_f64(
        ctypes.cast(a.ctypes.data, _f32p), ctypes.cast(b.ctypes.data, _f32p), _dp(out),
        B_, M, N, K, sa, a_rs, a_cs, sb, b_rs, b_cs, structure,
        None if rows_arr is None else rows_arr.ctypes.data_as(_i64p),
        0 if rows_arr is None else len(rows_arr))
    return out if batched else out[0]


def gemm_entries(a: np.ndarray, b: np.ndarray, bij: np.ndarray) -> np.ndarray:
    """fp64 values of selected output entries (b, i, j) of ``a @ b``."""
    if a.ndim == 2:
        a = a[None]
    if b.ndim == 2:
        b = b[None]
    B_, M, K = a.shape
    sa = a.strides[0] // 4 if a.shape[0] > 1 else 0
    sb = b.strides[0] // 4 if b.shape[0] > 1 else 0
    a_rs, a_cs = _strides2(a)
    b_rs, b_cs = _strides2(b)
    bij = np.ascontiguousarray(bij, dtype=np.int64).reshape(-1, 3)
    out = np.empty(len(bij), dtype=np.float64)
    lib().orc_gemm_entries_f64(
        ctypes.cast(a.ctypes.data, _f32p), ctypes.cast(b.ctypes.data, _f32p), _dp(out),
        bij.ctypes.data_as(_i64p), len(bij), K, sa, a_rs, a_cs, sb, b_rs, b_cs)
    return out


def gemv(a: np.ndarray, x: np.ndarray, rows: Optional[Sequence[int]] = None) -> np.ndarray:
    """fp64 ``a @ x`` for a row-major MxK ``a`` and a length-K ``x``
    (kernels/4_...:84-92: B is Kx1, output Mx1)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    M, K = a.shape
    assert x.shape[0] == K
    rows_arr = None if rows is None else np.ascontiguousarray(rows, dtype=np.int64)
    R = M if rows is None else len(rows_arr)
    out = np.empty(R, dtype=np.float64)
    lib().orc_gemv_f64(_fp(a), _fp(x), _dp(out), M, K, K,
                       None if rows_arr is None else rows_arr.ctypes.data_as(_i64p), R)
    return out


def gemv_generated(seed_a: int, x: np.ndarray, rows: Sequence[int]) -> np.ndarray:
    """fp64 rows of ``A @ x`` where A is the generated stream ``seed_a`` with
    row length len(x); A is regenerated row by row on the host."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    rows_arr = np.ascontiguousarray(rows, dtype=np.int64)
    out = np.empty(len(rows_arr), dtype=np.float64)
    lib().orc_gemv_generated_f64(seed_a, _fp(x), _dp(out), x.shape[0],
                                 rows_arr.ctypes.data_as(_i64p), len(rows_arr))
    return out


def matvec(a: np.ndarray, v: np.ndarray) -> np.ndarray:
    """fp64 ``a @ v`` for a 2-D fp32 array or view (any non-negative strides,
    so ``x.T`` needs no copy) and a length-cols vector."""
    assert a.dtype == np.float32 and a.ndim == 2 and min(a.strides) >= 0
    v = np.ascontiguousarray(v, dtype=np.float64).reshape(-1)
    rows, cols = a.shape
    assert v.shape[0] == cols
    rs, cs = _strides2(a)
    out = np.empty(rows, dtype=np.float64)
    lib().orc_matvec_f64(ctypes.cast(a.ctypes.data, _f32p), rows, cols, rs, cs, _dp(v), _dp(out))
    return out


def checksums(c: np.ndarray, v: np.ndarray, u: np.ndarray, utc: Optional[np.ndarray] = None):
    """fp64 row checksums ``c @ v`` and column checksums ``u @ c`` of an fp32
    block with unit column stride.  ``utc`` (float64, length cols) is
    accumulated into when given, so a large output can be reduced in row
    blocks; returns (c @ v, utc)."""
    assert c.dtype == np.float32 and c.ndim == 2 and c.strides[1] == 4
    rows, cols = c.shape
    v = np.ascontiguousarray(v, dtype=np.float64).reshape(-1)
    u = np.ascontiguousarray(u, dtype=np.float64).reshape(-1)
    assert v.shape[0] == cols and u.shape[0] == rows
    if utc is None:
        utc = np.zeros(cols, dtype=np.float64)
    assert utc.dtype == np.float64 and utc.shape == (cols,) and utc.flags["C_CONTIGUOUS"]
    cv = np.empty(rows, dtype=np.float64)
    lib().orc_checksums_f32(ctypes.cast(c.ctypes.data, _f32p), rows, cols, c.strides[0] // 4,
                            _dp(v), _dp(u), _dp(cv), _dp(utc))
    return cv, utc


def diag_mult(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """fp32 ``diag(a) @ b`` = ``a[:, None] * b`` (kernels/12_...:43-62)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    N, M = b.shape
    assert a.shape == (N,)
    out = np.empty_like(b)
    lib().orc_diag_f32(_fp(a), _fp(b), _fp(out), N, M)
    return out


def scale(a: np.ndarray, s: float) -> np.ndarray:
    """fp32 ``a * s`` elementwise (kernels/5_...:10-42, :47-71), same shape as ``a``."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty_like(a)
    lib().orc_scale_f32(_fp(a), _fp(out), a.size, float(s))
    return out


def pointwise_conv(x: np.ndarray, w: np.ndarray, bias: Optional[np.ndarray] = None) -> np.ndarray:
    """fp64-accumulated 1x1 convolution (kernels/87_...:451-492): x is
    N x Cin x H x W, w is Cout x Cin (or Cout x Cin x 1 x 1), bias Cout or
    None; returns N x Cout x H x W float64."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, cin, h, wd = x.shape
    w2 = np.ascontiguousarray(w, dtype=np.float32).reshape(w.shape[0], -1)
    cout = w2.shape[0]
    assert w2.shape[1] == cin
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32).reshape(cout)
    out = np.empty((n, cout, h, wd), dtype=np.float64)
    lib().orc_pointwise_conv_f64(_fp(x), _fp(w2), None if b is None else _fp(b), _dp(out),
                                 n, cin, cout, h * wd)
    return out


def sdpa(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: Optional[float] = None) -> np.ndarray:
    """fp64 scaled dot-product attention (kernels/97_...:136-296) of float16
    arrays (..., seq, embed); returns float64 of the same shape.  scale
    defaults to 1/sqrt(embed) (kernels/97_...:275)."""
    q, k, v = (np.ascontiguousarray(x, dtype=np.float16) for x in (q, k, v))
    assert q.shape == k.shape == v.shape
    seq, embed = q.shape[-2:]
    heads = int(np.prod(q.shape[:-2])) if q.ndim > 2 else 1
    out = np.empty(q.shape, dtype=np.float64)
    u16 = ctypes.POINTER(ctypes.c_uint16)
    lib().orc_sdpa_f64(q.ctypes.data_as(u16), k.ctypes.data_as(u16), v.ctypes.data_as(u16), _dp(out),
                       heads, seq, embed, (1.0 / math.sqrt(embed)) if scale is None else scale)
    return out


def half_ulp(x: np.ndarray) -> np.ndarray:
    """Spacing of IEEE binary16 values at |x| (subnormal spacing 2^-24 below 2^-14)."""
    ax = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(ax, 2.0 ** -14)))
    return np.exp2(e - 10)


# ---- tolerance ----------------------------------------------------------------

TOL = 1e-4  # north-star bound on the normalised error below


def norm_err(got: np.ndarray, ref: np.ndarray, K: int, max_a: float, max_b: float) -> float:
    """max|got - ref| / (sqrt(K) * max|A| * max|B|); NaN/Inf count as failure."""
    got = np.asarray(got, dtype=np.float32)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    if got.size == 0:
        return 0.0
    d = float(lib().orc_max_abs_diff(np.ascontiguousarray(got).ctypes.data_as(_f32p),
                                     np.ascontiguousarray(ref).ctypes.data_as(_f64p), got.size))
    scale = math.sqrt(max(K, 1)) * max(float(max_a), 1e-30) * max(float(max_b), 1e-30)
    return d / scale
