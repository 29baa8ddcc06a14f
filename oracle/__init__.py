"""CPU oracle for the conv / GEMM / AdamW path -- test infrastructure only.

Python face of oracle/oracle.c (a plain-C restatement of the reference's
arithmetic; see that file's header for what pins it).  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may use it, and only
as the checker: the product (libmx.so, torch_vulkan) never calls it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "liboracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    if force or not os.path.exists(_LIB) or os.path.getmtime(_LIB) < os.path.getmtime(os.path.join(_HERE, "oracle.c")):
        subprocess.run(["make", "-s", "-B" if force else "-s", "-C", _HERE, "liboracle.so"], check=True)
    return _LIB


def lib():
    global _lib
    if _lib is None:
        build()
        L = C.CDLL(_LIB)
        P = np.ctypeslib.ndpointer
        f32 = P(np.float32, flags="C_CONTIGUOUS")
        f64 = P(np.float64, flags="C_CONTIGUOUS")
        i64 = C.c_int64
        vp = C.c_void_p
        L.oracle_conv2d_shape.argtypes = [i64] * 15 + [C.POINTER(i64), C.POINTER(i64)]
        L.oracle_conv2d_shape.restype = C.c_int
        for name in ("oracle_conv2d_forward",):
            getattr(L, name).argtypes = [P(np.int64), f32, f32, vp, f64, vp]
        L.oracle_conv2d_backward_input.argtypes = [P(np.int64), f32, f32, f64, vp]
        L.oracle_conv2d_backward_weight.argtypes = [P(np.int64), f32, f32, f64, vp]
        L.oracle_conv2d_backward_bias.argtypes = [P(np.int64), f32, f64, vp]
        L.oracle_conv2d_winograd_forward.argtypes = [P(np.int64), f32, f32, vp, f64]
        L.oracle_conv2d_winograd_forward.restype = C.c_int
        L.oracle_gemm.argtypes = [i64] * 4 + [f32, i64, i64, i64, i64, f32, i64, i64, i64, i64, vp, C.c_int, i64,
                                              i64, i64, C.c_double, C.c_double, f64, vp]
        L.oracle_adamw_step.argtypes = [f32, f32, f32, f32, vp, i64] + [C.c_double] * 6 + [C.c_int]
        L.oracle_partition.argtypes = [P(np.uint8), i64, i64, P(np.int64)]
        L.oracle_partition.restype = i64
        _lib = L
    return _lib


def _f32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class ConvError(ValueError):
    pass


def conv2d_shape(x_shape, w_shape, stride=(1, 1), padding=(0, 0), dilation=(1, 1), groups=1):
    """(oh, ow) or ConvError (convolution_params validation)."""
    oh, ow = C.c_int64(), C.c_int64()
    rc = lib().oracle_conv2d_shape(x_shape[0], x_shape[1], x_shape[2], x_shape[3], w_shape[0], w_shape[1],
                                   w_shape[2], w_shape[3], stride[0], stride[1], padding[0], padding[1], dilation[0],
                                   dilation[1], groups, C.byref(oh), C.byref(ow))
    if rc != 0:
        raise ConvError(f"invalid convolution geometry (code {rc})")
    return oh.value, ow.value


def _desc(x_shape, w_shape, stride, padding, dilation, groups):
    oh, ow = conv2d_shape(x_shape, w_shape, stride, padding, dilation, groups)
    d = np.array([x_shape[0], x_shape[1], x_shape[2], x_shape[3], w_shape[0], w_shape[2], w_shape[3], oh, ow,
                  stride[0], stride[1], padding[0], padding[1], dilation[0], dilation[1], groups], dtype=np.int64)
    return d, oh, ow


def conv2d_forward(x, w, b=None, stride=(1, 1), padding=(0, 0), dilation=(1, 1), groups=1, winograd=False):
    """(y, magnitude) in float64; magnitude = sum of |terms| per output."""
    x, w = _f32(x), _f32(w)
    b = None if b is None else _f32(b)
    d, oh, ow = _desc(x.shape, w.shape, stride, padding, dilation, groups)
    y = np.zeros((x.shape[0], w.shape[0], oh, ow))
    mag = np.zeros_like(y)
    lib().oracle_conv2d_forward(d, x, w, _ptr(b), y, _ptr(mag))
    if winograd:
        yw = np.zeros_like(y)
        if lib().oracle_conv2d_winograd_forward(d, x, w, _ptr(b), yw) != 0:
            raise ConvError("winograd needs 3x3, stride 1, dilation 1")
        return yw, mag
    return y, mag


def conv2d_backward(x, w, dy, stride=(1, 1), padding=(0, 0), dilation=(1, 1), groups=1):
    """dict name -> (value, magnitude) for dx, dw, db (float64)."""
    x, w, dy = _f32(x), _f32(w), _f32(dy)
    d, oh, ow = _desc(x.shape, w.shape, stride, padding, dilation, groups)
    assert dy.shape == (x.shape[0], w.shape[0], oh, ow)
    dx, mdx = np.zeros(x.shape), np.zeros(x.shape)
    dw, mdw = np.zeros(w.shape), np.zeros(w.shape)
    db, mdb = np.zeros(w.shape[0]), np.zeros(w.shape[0])
    lib().oracle_conv2d_backward_input(d, dy, w, dx, _ptr(mdx))
    lib().oracle_conv2d_backward_weight(d, x, dy, dw, _ptr(mdw))
    lib().oracle_conv2d_backward_bias(d, dy, db, _ptr(mdb))
    return {"dx": (dx, mdx), "dw": (dw, mdw), "db": (db, mdb)}


def gemm(a, b, bias=None, alpha=1.0, beta=0.0):
    """(alpha * a @ b + beta * bias, magnitude) in float64 for 2-D or 3-D inputs.

    Any numpy view is accepted: its element strides and offset are passed to
    the strided C restatement as they are (no copy), like the reference's
    matmul_strided shaders read transposed views.
    """
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    batched = a.ndim == 3
    A, aoff, ast = _strided(a)
    B, boff, bst = _strided(b)
    if not batched:
        ast, bst = [0] + ast, [0] + bst
    batch = a.shape[0] if batched else 1
    M, K, N = a.shape[-2], a.shape[-1], b.shape[-1]
    kind, bsm, bsn, bias_base, bias_off = 0, 0, 0, None, 0
    if bias is not None:
        bias = np.asarray(bias, dtype=np.float32)
        if bias.ndim == 1 and bias.shape[0] == N:
            kind = 1
            bias_base, bias_off, (bsn,) = _strided(bias)
        else:
            kind = 2
            bias_base, bias_off, (bsm, bsn) = _strided(np.broadcast_to(bias, (M, N)))
    c = np.zeros((batch, M, N))
    mag = np.zeros_like(c)
    lib().oracle_gemm(batch, M, N, K, A, aoff, ast[0], ast[1], ast[2], B, boff, bst[0], bst[1], bst[2],
                      _ptr(bias_base), kind, bias_off, bsm, bsn, alpha, beta, c, _ptr(mag))
    return (c, mag) if batched else (c[0], mag[0])


def _strided(arr):
    """(contiguous base buffer, element offset, element strides) describing a view."""
    base = arr
    while isinstance(base.base, np.ndarray):
        base = base.base
    if base.dtype != np.float32 or not base.flags["C_CONTIGUOUS"] or any(s % 4 for s in arr.strides) or \
            any(s < 0 for s in arr.strides):
        arr = np.ascontiguousarray(arr)
        base = arr
    off = (arr.__array_interface__["data"][0] - base.__array_interface__["data"][0]) // 4
    flat = base.reshape(-1)
    return flat, int(off), [s // 4 for s in arr.strides]


def adamw_step(p, g, m, v, *, lr, beta1, beta2, eps, weight_decay, step, vmax=None, maximize=False):
    """In-place AdamW step on float32 numpy arrays (torch single-tensor order)."""
    for arr in (p, g, m, v) + ((vmax,) if vmax is not None else ()):
        assert arr.dtype == np.float32 and arr.flags["C_CONTIGUOUS"]
    lib().oracle_adamw_step(p, g, m, v, _ptr(vmax), p.size, lr, beta1, beta2, eps, weight_decay, float(step),
                            1 if maximize else 0)


def partition(conflict, slots=0):
    """Launch-group start indices for a count x count 0/1 conflict matrix."""
    conflict = np.ascontiguousarray(np.asarray(conflict, dtype=np.uint8))
    n = conflict.shape[0]
    starts = np.zeros(max(n, 1), dtype=np.int64)
    k = lib().oracle_partition(conflict, n, slots, starts)
    return starts[:k].tolist()
