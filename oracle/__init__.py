"""CPU oracle for the MI355X matmul / attention dispatch path.

TEST INFRASTRUCTURE ONLY: tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker (or the timed CPU baseline). The product path never calls it.

Thin numpy wrappers over ``liboracle.so`` (oracle.c). Half-precision arrays are
numpy float16; they are handed to C as raw binary16 bits. See oracle.h for the
reference file:line each routine restates and for how each is pinned.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

B_TRANSPOSED = 1
ACCUMULATE = 2
OUT_F32 = 4
A_TRANSPOSED = 8


def build() -> None:
    """Compile liboracle.so with gcc (make)."""
    subprocess.check_call(["make", "-s", "-C", _HERE])


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    p = ctypes.c_void_p
    i64 = ctypes.c_int64
    lib.oracle_f16_to_f32.restype = ctypes.c_float
    lib.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.oracle_f32_to_f16.restype = ctypes.c_uint16
    lib.oracle_f32_to_f16.argtypes = [ctypes.c_float]
    lib.oracle_f16_to_f32_array.argtypes = [p, p, i64]
    lib.oracle_f32_to_f16_array.argtypes = [p, p, i64]
    lib.oracle_matmul_f16.argtypes = [p, p, p, i64, i64, i64, i64, i64, i64,
                                      ctypes.c_uint32, ctypes.c_int]
    lib.oracle_matmul_i8.argtypes = [p, p, p, i64, i64, i64, i64, i64, i64,
                                     ctypes.c_uint32, ctypes.c_int]
    lib.oracle_batch_matmul_f16.argtypes = [
        p, p, p, i64, i64, i64, i64, i64, i64, i64, i64, i64, i64,
        ctypes.c_uint32, p, p, i64, i64, ctypes.c_uint32, ctypes.c_int]
    lib.oracle_activation.argtypes = [ctypes.c_float, ctypes.c_uint32]
    lib.oracle_activation.restype = ctypes.c_float
    lib.oracle_geglu_f16_ops.argtypes = [ctypes.c_float, ctypes.c_uint16]
    lib.oracle_geglu_f16_ops.restype = ctypes.c_uint16
    lib.oracle_w8a16.argtypes = [p, p, p, p, i64, i64, i64, i64, i64, i64,
                                 ctypes.c_uint32, ctypes.c_int]
    lib.oracle_attention_f16.argtypes = [p, p, p, p, i64, i64, i64, i64, i64,
                                         ctypes.c_float, ctypes.c_int,
                                         ctypes.c_int]
    lib.oracle_attention_f16_strided.argtypes = [
        p, p, p, p, i64, i64, i64, i64, i64, i64, ctypes.POINTER(i64),
        ctypes.c_float, ctypes.c_int, ctypes.c_int]
    lib.oracle_attention.argtypes = [
        p, p, p, p, p, i64, i64, i64, i64, i64, i64, i64, ctypes.POINTER(i64),
        ctypes.POINTER(i64), ctypes.c_float, ctypes.c_int, ctypes.c_int,
        ctypes.c_int]
    lib.oracle_choose_static_tiling_factor.restype = i64
    lib.oracle_choose_static_tiling_factor.argtypes = [i64, i64, i64]
    lib.oracle_select_hmx_tile_sizes.argtypes = [p, p, ctypes.c_int, i64,
                                                 ctypes.c_int, i64, i64, p]
    for name in ("oracle_matmul_f16", "oracle_matmul_i8", "oracle_w8a16",
                 "oracle_batch_matmul_f16",
                 "oracle_attention_f16", "oracle_attention_f16_strided",
                 "oracle_attention",
                 "oracle_select_hmx_tile_sizes"):
        getattr(lib, name).restype = ctypes.c_int
    _lib = lib
    return lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def default_threads() -> int:
    return max(1, min(os.cpu_count() or 1, 16))


def f16_to_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float16)
    out = np.empty(x.shape, np.float32)
    _load().oracle_f16_to_f32_array(_ptr(x), _ptr(out), x.size)
    return out


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.float16)
    _load().oracle_f32_to_f16_array(_ptr(x), _ptr(out), x.size)
    return out


def matmul_f16(a, b, c_init=None, *, b_transposed=False, out_f32=False,
               a_transposed=False, threads=None) -> np.ndarray:
    """C = [C_init +] A.B with f16 inputs, f32 accumulation, f16/f32 output.
    a is [M, K], or [K, M] with ``a_transposed``; b is [K, N], or [N, K] with
    ``b_transposed``."""
    a = np.ascontiguousarray(a, np.float16)
    b = np.ascontiguousarray(b, np.float16)
    k, m = a.shape if a_transposed else a.shape[::-1]
    n = b.shape[0] if b_transposed else b.shape[1]
    assert (b.shape[1] if b_transposed else b.shape[0]) == k
    dt = np.float32 if out_f32 else np.float16
    flags = ((B_TRANSPOSED if b_transposed else 0) |
             (OUT_F32 if out_f32 else 0) |
             (A_TRANSPOSED if a_transposed else 0))
    if c_init is not None:
        c = np.array(c_init, dtype=dt, copy=True, order="C")
        flags |= ACCUMULATE
    else:
        c = np.empty((m, n), dt)
    rc = _load().oracle_matmul_f16(_ptr(a), _ptr(b), _ptr(c), m, n, k,
                                   a.shape[1], b.shape[1], n, flags,
                                   threads or default_threads())
    assert rc == 0, rc
    return c



ACT_NONE, ACT_RELU, ACT_GELU_TANH, ACT_SILU = 0, 1, 2, 3


def batch_matmul_f16(a, b, c_init=None, *, b_transposed=False, out_f32=False,
                     bias=None, activation=ACT_NONE, multiplier=None,
                     threads=None) -> np.ndarray:
    """Per batch z: out = [C_init +] multiplier * act(A_z.B_z + bias).

    a: [Z, M, K] f16; b: [Z, K, N] (or [Z, N, K] transposed) f16, or 2-D to
    share one B across the batch; bias [N] f16; multiplier [Z, M, N] or
    [M, N] f16. f32 accumulation and epilogue, one rounding."""
    a = np.ascontiguousarray(a, np.float16)
    b = np.ascontiguousarray(b, np.float16)
    z, m, k = a.shape
    shared_b = b.ndim == 2
    n = (b.shape[-2] if b_transposed else b.shape[-1])
    ldb = b.shape[-1]
    sb = 0 if shared_b else b.shape[1] * b.shape[2]
    flags = (B_TRANSPOSED if b_transposed else 0) | (OUT_F32 if out_f32 else 0)
    dt = np.float32 if out_f32 else np.float16
    if c_init is not None:
        c = np.ascontiguousarray(c_init, dt).copy()
        flags |= ACCUMULATE
    else:
        c = np.zeros((z, m, n), dt)
    bias_a = None if bias is None else np.ascontiguousarray(bias, np.float16)
    mul_a, s_mul = None, 0
    if multiplier is not None:
        mul_a = np.ascontiguousarray(multiplier, np.float16)
        s_mul = 0 if mul_a.ndim == 2 else m * n
    rc = _load().oracle_batch_matmul_f16(
        _ptr(a), _ptr(b), _ptr(c), z, m, n, k, k, ldb, n, m * k, sb, m * n,
        flags, None if bias_a is None else _ptr(bias_a),
        None if mul_a is None else _ptr(mul_a), n, s_mul, activation,
        threads or default_threads())
    assert rc == 0, rc
    return c


def activation(v: float, act: int) -> float:
    """The oracle's f32 activation of one value."""
    return float(_load().oracle_activation(v, act))


def geglu_f16_ops(acc, up) -> np.ndarray:
    """The reference IR's GeGLU epilogue with every op rounded to f16."""
    acc = np.asarray(acc, np.float32).ravel()
    up = np.asarray(up, np.float16).ravel()
    lib = _load()
    out = np.array([lib.oracle_geglu_f16_ops(float(x), int(u.view(np.uint16)))
                    for x, u in zip(acc, up)], np.uint16)
    return out.view(np.float16)

def matmul_i8(a, b, c_init=None, *, b_transposed=False, threads=None):
    """C = [C_init +] A.B, int8 inputs, exact int32 accumulation/output."""
    a = np.ascontiguousarray(a, np.int8)
    b = np.ascontiguousarray(b, np.int8)
    m, k = a.shape
    n = b.shape[0] if b_transposed else b.shape[1]
    flags = B_TRANSPOSED if b_transposed else 0
    if c_init is not None:
        c = np.array(c_init, dtype=np.int32, copy=True, order="C")
        flags |= ACCUMULATE
    else:
        c = np.empty((m, n), np.int32)
    rc = _load().oracle_matmul_i8(_ptr(a), _ptr(b), _ptr(c), m, n, k, k,
                                  b.shape[1], n, flags,
                                  threads or default_threads())
    assert rc == 0, rc
    return c


def matmul_i8_rows(a, b, rows, *, b_transposed=False, threads=None):
    """The first ``rows`` output rows of matmul_i8 (bounded CPU baseline)."""
    return matmul_i8(np.ascontiguousarray(a[:rows]), b,
                     b_transposed=b_transposed, threads=threads)


def w8a16(x, w, scale, *, w_transposed=False, threads=None) -> np.ndarray:
    """y = f16((x.w_int8) * scale[n]) with f32 accumulation, zero point 0."""
    x = np.ascontiguousarray(x, np.float16)
    w = np.ascontiguousarray(w, np.int8)
    scale = np.ascontiguousarray(scale, np.float16)
    m, k = x.shape
    n = w.shape[0] if w_transposed else w.shape[1]
    y = np.empty((m, n), np.float16)
    rc = _load().oracle_w8a16(_ptr(x), _ptr(w), _ptr(scale), _ptr(y), m, n, k,
                              k, w.shape[1], n,
                              B_TRANSPOSED if w_transposed else 0,
                              threads or default_threads())
    assert rc == 0, rc
    return y


def _rows_view(a):
    """An f16 array whose last dimension is contiguous (a strided view is
    kept as it is) and its first three element strides."""
    if a.dtype != np.float16 or a.strides[-1] != 2:
        a = np.ascontiguousarray(a, np.float16)
    return a, [st // 2 for st in a.strides[:3]]


def attention_f16(q, k, v, *, scale=None, causal=True, out=None, threads=None):
    """softmax(QK^T*scale + causal mask) V for q [B,Hq,Sq,D] and k, v
    [B,Hkv,Skv,D] f16 arrays (strided views allowed: the last dimension
    contiguous). Hq is a multiple of Hkv and query head h reads KV head
    h // (Hq // Hkv). The result goes into `out` ([B,Hq,Sq,D], possibly a
    strided view) or a new contiguous array."""
    q, qs = _rows_view(q)
    k, ks = _rows_view(k)
    v, vs = _rows_view(v)
    b, h, sq, d = q.shape
    hkv, skv = k.shape[1], k.shape[2]
    if scale is None:
        scale = 1.0 / float(np.sqrt(d))
    o = np.empty_like(q, order="C") if out is None else out
    assert o.dtype == np.float16 and o.shape == q.shape and o.strides[-1] == 2
    os_ = [st // 2 for st in o.strides[:3]]
    strides = (ctypes.c_int64 * 12)(*(qs + ks + vs + os_))
    rc = _load().oracle_attention_f16_strided(
        _ptr(q), _ptr(k), _ptr(v), _ptr(o), b, h, hkv, sq, skv, d, strides,
        float(scale), int(causal), threads or default_threads())
    assert rc == 0, rc
    return o


def attention(q, k, v, *, scale=None, causal=False, mask=None,
              out_f32=False, out=None, threads=None):
    """The general form: softmax(QK^T*scale + mask [+ causal]) V for q
    [B,Hq,Sq,Dqk], k [B,Hkv,Skv,Dqk], v [B,Hkv,Skv,Dv] f16 arrays (strided
    views allowed, the last dimension contiguous); mask an f16 array that
    broadcasts to [B,Hq,Sq,Skv] (numpy broadcasting; its strides are read,
    0 for a broadcast dimension). Masked (-inf) keys weigh 0 and a row with
    no other key is 0. The result is f16, or f32 with `out_f32`, in `out`
    or a new contiguous [B,Hq,Sq,Dv] array."""
    q, qs = _rows_view(q)
    k, ks = _rows_view(k)
    v, vs = _rows_view(v)
    b, h, sq, d = q.shape
    hkv, skv, dv = k.shape[1], k.shape[2], v.shape[3]
    if scale is None:
        scale = 1.0 / float(np.sqrt(d))
    dt = np.float32 if out_f32 else np.float16
    o = np.empty((b, h, sq, dv), dt) if out is None else out
    assert o.dtype == dt and o.shape == (b, h, sq, dv)
    assert o.strides[-1] == o.itemsize
    os_ = [st // o.itemsize for st in o.strides[:3]]
    strides = (ctypes.c_int64 * 12)(*(qs + ks + vs + os_))
    mptr, mst = None, (ctypes.c_int64 * 4)(0, 0, 0, 0)
    if mask is not None:
        mask = np.asarray(mask)
        assert mask.dtype == np.float16
        mask = np.broadcast_to(mask, (b, h, sq, skv))
        mst = (ctypes.c_int64 * 4)(*[st // 2 for st in mask.strides])
        mptr = mask.ctypes.data
    rc = _load().oracle_attention(
        _ptr(q), _ptr(k), _ptr(v), o.ctypes.data, mptr, b, h, hkv, sq, skv, d,
        dv, strides, mst, float(scale), int(causal), int(out_f32),
        threads or default_threads())
    assert rc == 0, rc
    return o


DYNAMIC = -(2 ** 63)


def choose_static_tiling_factor(bound: int, preferred: int,
                                multiple_of: int = 1) -> int:
    return int(_load().oracle_choose_static_tiling_factor(bound, preferred,
                                                          multiple_of))


def select_hmx_tile_sizes(m, n, k, *, elem_bytes=(2, 2, 4), b_transposed=False,
                          budget_bytes=2 * 1024 * 1024, double_buffering=True,
                          hmx_m=32, hmx_n=32):
    """Restated selectHmxTileSizes; returns [m, n, k] tiles or None."""
    ranges = np.array([m, n, k], np.int64)
    eb = np.array(elem_bytes, np.int64)
    out = np.zeros(3, np.int64)
    ok = _load().oracle_select_hmx_tile_sizes(
        _ptr(ranges), _ptr(eb), int(b_transposed), budget_bytes,
        int(double_buffering), hmx_m, hmx_n, _ptr(out))
    return [int(t) for t in out] if ok else None


def fp16_parity(y, ref) -> float:
    """max|y - ref| / max|ref|: the fp16 parity metric (bound 2e-3)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    denom = float(np.abs(ref).max()) if ref.size else 0.0
    if denom == 0.0:
        return float(np.abs(y - ref).max()) if y.size else 0.0
    return float(np.abs(y - ref).max() / denom)


def compare_arrays(reference, actual, atol, rtol):
    """IT/stages/checking.py:46-83 recipe: (relative L2 %, max abs, allclose)."""
    ref = np.asarray(reference, np.float64)
    act = np.asarray(actual, np.float64)
    ref_norm = float(np.linalg.norm(ref))
    err = float(np.linalg.norm(act - ref))
    rel = err / ref_norm * 100.0 if ref_norm > 0 else 100.0
    max_abs = float(np.abs(act - ref).max()) if ref.size else 0.0
    close = bool(np.allclose(act, ref, atol=atol, rtol=rtol, equal_nan=False))
    return rel, max_abs, close
