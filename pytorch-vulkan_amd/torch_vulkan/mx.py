"""ctypes binding of the C ABI in include/mx.h (libmx.so).

This is the binding a Python caller of the reference's path would add: plain
pointers and sizes in, an int status out (MXError raised with mx_last_error()
on failure).  Device buffers can come from anywhere in the process that uses
the same HIP runtime (torch's ROCm tensors included); ``stream`` is a
hipStream_t as an int, 0/None for the library's default stream.

Load order matters: torch must be imported before libmx.so so that both bind
the same HIP runtime (torch/lib/libamdhip64.so).
"""
from __future__ import annotations

import ctypes as C
import math
import os

import torch  # noqa: F401  (HIP runtime first, see module docstring)

# MX_LIBRARY names another build of the same C ABI (the sanitizer build of
# pytorch-vulkan_amd/sanitize.py); by default the in-tree libmx.so.
_LIB_PATH = os.environ.get("MX_LIBRARY") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmx.so")

MX_OK, MX_ERR_INVALID, MX_ERR_UNSUPPORTED, MX_ERR_OOM, MX_ERR_HIP, MX_ERR_WORKSPACE = range(6)
MX_COPY_H2D, MX_COPY_D2H, MX_COPY_D2D = 1, 2, 3
MX_CONV_FORWARD, MX_CONV_DINPUT, MX_CONV_DWEIGHT, MX_CONV_DBIAS = range(4)
ALGO_AUTO, ALGO_DIRECT, ALGO_IMPLICIT_GEMM, ALGO_WINOGRAD, ALGO_REDUCE, ALGO_DEPTHWISE = range(6)
BIAS_NONE, BIAS_COL, BIAS_MATRIX = range(3)
ABI_VERSION = 3  # struct layouts of include/mx.h

# Every entry point declared in include/mx.h (checked by the CPU test suite).
EXPORTS = [
    "mx_last_error", "mx_abi_version", "mx_init", "mx_device_count", "mx_get_device", "mx_set_device",
    "mx_device_name", "mx_device_synchronize", "mx_default_stream", "mx_stream_create", "mx_stream_destroy",
    "mx_stream_synchronize", "mx_stream_query", "mx_stream_wait_event", "mx_event_create", "mx_event_destroy",
    "mx_event_record", "mx_event_query", "mx_event_synchronize", "mx_event_elapsed_ms", "mx_malloc", "mx_free",
    "mx_record_stream", "mx_empty_cache", "mx_memory_stats_get", "mx_memcpy", "mx_host_is_pinned",
    "mx_memcpy_async", "mx_host_malloc", "mx_host_free", "mx_fill", "mx_copy_strided",
    "mx_add_f32", "mx_scale_f32", "mx_mul_f32", "mx_sum_f32", "mx_foreach_add_scalar_f32", "mx_conv2d_check",
    "mx_conv2d_select", "mx_conv2d_forward", "mx_conv2d_backward_input", "mx_conv2d_backward_weight", "mx_conv2d_backward",
    "mx_conv2d_backward_bias", "mx_conv2d_dweight_plan", "mx_conv2d_kernel_name", "mx_gemm_f32", "mx_adamw_step",
    "mx_group_norm_forward", "mx_group_norm_backward", "mx_batch_norm_forward", "mx_batch_norm_backward",
    "mx_unary_f32", "mx_unary_backward_f32", "mx_upsample_nearest2d", "mx_upsample_nearest2d_backward",
    "mx_softmax_f32", "mx_softmax_backward_f32", "mx_mse_loss_f32", "mx_mse_loss_backward_f32", "mx_copy_rows",
    "mx_foreach_f32", "mx_conv2d_plan", "mx_gemm_variant", "mx_conv2d_backward_weight_noalloc",
    "mx_conv2d_backward_one_launch",
]


class MXError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"mx status {status}: {message}")
        self.status = status


class ConvDesc(C.Structure):
    _fields_ = [(n, C.c_int64) for n in
                ("n", "cin", "h", "w", "cout", "kh", "kw", "sh", "sw", "ph", "pw", "dh", "dw", "groups", "oh", "ow")]


class ConvPlanInfo(C.Structure):
    _fields_ = [("algo", C.c_int), ("tile", C.c_int), ("splits", C.c_int64), ("span", C.c_int64),
                ("workspace_bytes", C.c_int64), ("variant", C.c_char * 256)]


class GemmDesc(C.Structure):
    _fields_ = [(n, C.c_int64) for n in
                ("batch", "m", "n", "k", "a_offset", "a_stride_b", "a_stride_m", "a_stride_k",
                 "b_offset", "b_stride_b", "b_stride_k", "b_stride_n", "c_offset", "c_stride_b", "ldc",
                 "bias_offset", "bias_stride_m", "bias_stride_n")] + [
                ("alpha", C.c_float), ("beta", C.c_float), ("bias_kind", C.c_int), ("bias_stride_b", C.c_int64),
                ("kernel", C.c_int)]


class AdamWTensor(C.Structure):
    _fields_ = [("param", C.c_void_p), ("grad", C.c_void_p), ("exp_avg", C.c_void_p), ("exp_avg_sq", C.c_void_p),
                ("max_exp_avg_sq", C.c_void_p), ("numel", C.c_int64), ("step", C.c_int64),
                ("step_dev", C.c_void_p)]


class AdamWHParams(C.Structure):
    _fields_ = [("lr", C.c_double), ("beta1", C.c_double), ("beta2", C.c_double), ("eps", C.c_double),
                ("weight_decay", C.c_double), ("amsgrad", C.c_int), ("maximize", C.c_int),
                ("lr_dev", C.c_void_p), ("grad_scale", C.c_void_p), ("found_inf", C.c_void_p)]


class ForeachTensor(C.Structure):
    _fields_ = [("out", C.c_void_p), ("a", C.c_void_p), ("b", C.c_void_p), ("c", C.c_void_p),
                ("numel", C.c_int64), ("scalar", C.c_double)]


class MemoryStats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in
                ("allocated_bytes", "reserved_bytes", "cached_blocks", "device_mallocs", "cache_hits")]


_lib = None


def lib() -> C.CDLL:
    """The loaded libmx.so with argument types declared."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise ImportError(f"{_LIB_PATH} is not built; run `python pytorch-vulkan_amd/build.py`")
        L = C.CDLL(_LIB_PATH)
        vp, i64, i32 = C.c_void_p, C.c_int64, C.c_int
        sig = {
            "mx_last_error": ([], C.c_char_p),
            "mx_abi_version": ([], i32),
            "mx_init": ([i32], i32),
            "mx_device_count": ([C.POINTER(i32)], i32),
            "mx_get_device": ([C.POINTER(i32)], i32),
            "mx_set_device": ([i32], i32),
            "mx_device_name": ([i32, C.c_char_p, C.c_size_t], i32),
            "mx_device_synchronize": ([], i32),
            "mx_default_stream": ([C.POINTER(vp)], i32),
            "mx_stream_create": ([C.POINTER(vp)], i32),
            "mx_stream_destroy": ([vp], i32),
            "mx_stream_synchronize": ([vp], i32),
            "mx_stream_query": ([vp, C.POINTER(i32)], i32),
            "mx_stream_wait_event": ([vp, vp], i32),
            "mx_event_create": ([C.POINTER(vp), i32], i32),
            "mx_event_destroy": ([vp], i32),
            "mx_event_record": ([vp, vp], i32),
            "mx_event_query": ([vp, C.POINTER(i32)], i32),
            "mx_event_synchronize": ([vp], i32),
            "mx_event_elapsed_ms": ([vp, vp, C.POINTER(C.c_float)], i32),
            "mx_malloc": ([C.POINTER(vp), C.c_size_t, vp], i32),
            "mx_free": ([vp], i32),
            "mx_record_stream": ([vp, vp], i32),
            "mx_empty_cache": ([], i32),
            "mx_memory_stats_get": ([C.POINTER(MemoryStats)], i32),
            "mx_memcpy": ([vp, vp, C.c_size_t, i32, vp], i32),
            "mx_host_is_pinned": ([vp, C.POINTER(i32)], i32),
            "mx_memcpy_async": ([vp, vp, C.c_size_t, i32, vp], i32),
            "mx_host_malloc": ([C.POINTER(vp), C.c_size_t], i32),
            "mx_host_free": ([vp], i32),
            "mx_fill": ([vp, i64, i32, C.c_uint64, vp], i32),
            "mx_copy_strided": ([vp, vp, i32, C.POINTER(i64), C.POINTER(i64), C.POINTER(i64), i64, i64, i32, vp], i32),
            "mx_add_f32": ([vp, vp, vp, C.c_float, i64, vp], i32),
            "mx_scale_f32": ([vp, vp, C.c_float, i64, vp], i32),
            "mx_mul_f32": ([vp, vp, vp, i64, vp], i32),
            "mx_sum_f32": ([vp, vp, i64, i64, i64, vp], i32),
            "mx_foreach_add_scalar_f32": ([C.POINTER(vp), C.POINTER(i64), i64, C.c_float, vp], i32),
            "mx_conv2d_check": ([C.POINTER(ConvDesc)], i32),
            "mx_conv2d_select": ([C.POINTER(ConvDesc), i32, i32, C.POINTER(i32)], i32),
            "mx_conv2d_forward": ([C.POINTER(ConvDesc), vp, vp, vp, vp, i32, vp], i32),
            "mx_conv2d_backward_input": ([C.POINTER(ConvDesc), vp, vp, vp, i32, vp], i32),
            "mx_conv2d_backward_weight": ([C.POINTER(ConvDesc), vp, vp, vp, vp, i32, vp], i32),
            "mx_conv2d_backward": ([C.POINTER(ConvDesc), vp, vp, vp, vp, vp, vp, i32, i32, vp], i32),
            "mx_conv2d_backward_weight_noalloc": ([C.POINTER(ConvDesc), vp, vp, vp, vp, i32, vp], i32),
            "mx_conv2d_backward_bias": ([C.POINTER(ConvDesc), vp, vp, vp], i32),
            "mx_conv2d_dweight_plan": ([C.POINTER(ConvDesc), C.POINTER(i64), C.POINTER(i64), C.POINTER(i64)], i32),
            "mx_conv2d_kernel_name": ([C.POINTER(ConvDesc), i32, i32, C.c_char_p, C.c_size_t], i32),
            "mx_conv2d_backward_one_launch": ([C.POINTER(ConvDesc), i32, i32, i32, C.POINTER(i32)], i32),
            "mx_gemm_f32": ([C.POINTER(GemmDesc), vp, vp, vp, vp, vp], i32),
            "mx_gemm_variant": ([C.POINTER(GemmDesc), vp, vp, C.c_char_p, C.c_size_t], i32),
            "mx_conv2d_plan": ([C.POINTER(ConvDesc), i32, i32, i32, C.POINTER(ConvPlanInfo)], i32),
            "mx_adamw_step": ([C.POINTER(AdamWTensor), i64, C.POINTER(AdamWHParams), C.POINTER(i64), vp], i32),
            "mx_group_norm_forward": ([vp, vp, vp, i64, i64, i64, i64, C.c_float, vp, vp, vp, vp], i32),
            "mx_group_norm_backward": ([vp, vp, vp, vp, vp, i64, i64, i64, i64, vp, vp, vp, vp], i32),
            "mx_batch_norm_forward": ([vp, vp, vp, vp, i64, vp, i64, i64, i64, i64, i32, C.c_float, C.c_float,
                                       vp, vp, vp, vp], i32),
            "mx_batch_norm_backward": ([vp, vp, vp, vp, vp, i64, i64, i64, i32, C.c_float, vp, vp, vp, vp], i32),
            "mx_unary_f32": ([i32, vp, vp, i64, vp], i32),
            "mx_unary_backward_f32": ([i32, vp, vp, C.c_float, vp, i64, vp], i32),
            "mx_upsample_nearest2d": ([vp, i64, i64, i64, i64, i64, C.c_double, C.c_double, vp, vp], i32),
            "mx_upsample_nearest2d_backward": ([vp, i64, i64, i64, i64, i64, C.c_double, C.c_double, vp, vp], i32),
            "mx_softmax_f32": ([vp, i64, i64, i64, vp, vp], i32),
            "mx_softmax_backward_f32": ([vp, vp, i64, i64, i64, vp, vp], i32),
            "mx_mse_loss_f32": ([vp, vp, i64, i32, vp, vp], i32),
            "mx_mse_loss_backward_f32": ([vp, vp, vp, i64, i32, vp, vp], i32),
            "mx_copy_rows": ([vp, i64, vp, i64, i64, i64, vp], i32),
            "mx_foreach_f32": ([i32, C.POINTER(ForeachTensor), i64, C.POINTER(i64), vp], i32),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        if L.mx_abi_version() != ABI_VERSION:
            raise ImportError(f"{_LIB_PATH} has ABI {L.mx_abi_version()}, this binding expects {ABI_VERSION}; rebuild")
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != MX_OK:
        raise MXError(status, lib().mx_last_error().decode())


def ptr(t) -> int | None:
    """Device pointer of a tensor (or None)."""
    return None if t is None else t.data_ptr()


def conv_desc(x_shape, w_shape, stride=(1, 1), padding=(0, 0), dilation=(1, 1), groups=1) -> ConvDesc:
    d = ConvDesc(n=x_shape[0], cin=x_shape[1], h=x_shape[2], w=x_shape[3], cout=w_shape[0], kh=w_shape[2],
                 kw=w_shape[3], sh=stride[0], sw=stride[1], ph=padding[0], pw=padding[1], dh=dilation[0],
                 dw=dilation[1], groups=groups)
    check(lib().mx_conv2d_check(C.byref(d)))
    return d


def conv2d_forward(d: ConvDesc, x, w, b, y, algo=ALGO_AUTO, stream=None) -> None:
    check(lib().mx_conv2d_forward(C.byref(d), ptr(x), ptr(w), ptr(b), ptr(y), algo, stream))


def conv2d_backward_input(d: ConvDesc, dy, w, dx, algo=ALGO_AUTO, stream=None) -> None:
    check(lib().mx_conv2d_backward_input(C.byref(d), ptr(dy), ptr(w), ptr(dx), algo, stream))


def conv2d_backward(d: ConvDesc, x, w, dy, dx, dw, db, algo_dx=ALGO_AUTO, algo_dw=ALGO_AUTO, stream=None) -> None:
    check(lib().mx_conv2d_backward(C.byref(d), ptr(x), ptr(w), ptr(dy), ptr(dx), ptr(dw), ptr(db), algo_dx, algo_dw,
                                   stream))


def conv2d_backward_weight(d: ConvDesc, x, dy, dw, db, algo=ALGO_AUTO, stream=None) -> None:
    check(lib().mx_conv2d_backward_weight(C.byref(d), ptr(x), ptr(dy), ptr(dw), ptr(db), algo, stream))


NOALLOC_SCRATCH_BYTES = 16 * 1024 * 1024  # MX_NOALLOC_SCRATCH_BYTES


def conv2d_backward_weight_noalloc(d: ConvDesc, x, dy, dw, db, algo=ALGO_AUTO, stream=None) -> None:
    """mx_conv2d_backward_weight without any device allocation (library-owned
    scratch; overlapping calls on one GPU race)."""
    check(lib().mx_conv2d_backward_weight_noalloc(C.byref(d), ptr(x), ptr(dy), ptr(dw), ptr(db), algo, stream))


def conv2d_backward_bias(d: ConvDesc, dy, db, stream=None) -> None:
    check(lib().mx_conv2d_backward_bias(C.byref(d), ptr(dy), ptr(db), stream))


def conv2d_select(d: ConvDesc, phase: int, requested: int = ALGO_AUTO) -> int:
    out = C.c_int(-1)
    check(lib().mx_conv2d_select(C.byref(d), phase, requested, C.byref(out)))
    return out.value


def gemm_desc(a, b, c, *, bias=None, alpha=1.0, beta=0.0, bias_kind=None) -> GemmDesc:
    """Descriptor of c[b] = alpha * a[b] @ b[b] + beta * bias for 2-D or 3-D strided tensors
    (any object with torch's shape / stride / storage_offset / dim accessors)."""
    batched = a.dim() == 3
    m, k = a.shape[-2], a.shape[-1]
    n = b.shape[-1]
    d = GemmDesc(batch=a.shape[0] if batched else 1, m=m, n=n, k=k,
                 a_offset=a.storage_offset(), a_stride_b=a.stride(0) if batched else 0,
                 a_stride_m=a.stride(-2), a_stride_k=a.stride(-1),
                 b_offset=b.storage_offset(), b_stride_b=b.stride(0) if batched else 0,
                 b_stride_k=b.stride(-2), b_stride_n=b.stride(-1),
                 c_offset=c.storage_offset(), c_stride_b=c.stride(0) if batched else 0, ldc=c.stride(-2),
                 alpha=alpha, beta=beta, bias_kind=BIAS_NONE)
    if bias is not None:
        if bias_kind is None:
            bias_kind = BIAS_COL if bias.dim() == 1 else BIAS_MATRIX
        d.bias_kind = bias_kind
        d.bias_offset = bias.storage_offset()
        if bias_kind == BIAS_COL:
            d.bias_stride_n = bias.stride(-1)
            if batched and bias.dim() == 3:
                d.bias_stride_b = bias.stride(0)
        else:
            e = bias.expand(a.shape[0], m, n) if batched else bias.expand(m, n)
            d.bias_stride_m, d.bias_stride_n = e.stride(-2), e.stride(-1)
            if batched:
                d.bias_stride_b = e.stride(0)
    assert c.stride(-1) == 1, "output rows must be contiguous"
    return d


def gemm(a, b, c, *, bias=None, alpha=1.0, beta=0.0, bias_kind=None, stream=None) -> None:
    """c[b] = alpha * a[b] @ b[b] + beta * bias for 2-D or 3-D strided torch tensors (any device layout)."""
    d = gemm_desc(a, b, c, bias=bias, alpha=alpha, beta=beta, bias_kind=bias_kind)
    bias_base = bias.untyped_storage().data_ptr() if bias is not None else None
    check(lib().mx_gemm_f32(C.byref(d), a.untyped_storage().data_ptr(), b.untyped_storage().data_ptr(), bias_base,
                            c.untyped_storage().data_ptr(), stream))


def gemm_variant(d: GemmDesc, a_base: int = 256, b_base: int = 256) -> str:
    """Kernel instantiation mx_gemm_f32 launches for descriptor d with operand
    storages at these addresses (only their alignment matters)."""
    buf = C.create_string_buffer(128)
    check(lib().mx_gemm_variant(C.byref(d), a_base, b_base, buf, 128))
    return buf.value.decode()


def adamw_step(params, grads, exp_avgs, exp_avg_sqs, *, lr, beta1, beta2, eps, weight_decay, steps=None,
               step_tensors=None, max_exp_avg_sqs=None, maximize=False, stream=None) -> int:
    """One fused AdamW step over tensor lists; returns the number of launches."""
    n = len(params)
    arr = (AdamWTensor * max(n, 1))()
    for i in range(n):
        e = arr[i]
        e.param, e.grad = params[i].data_ptr(), grads[i].data_ptr()
        e.exp_avg, e.exp_avg_sq = exp_avgs[i].data_ptr(), exp_avg_sqs[i].data_ptr()
        e.max_exp_avg_sq = max_exp_avg_sqs[i].data_ptr() if max_exp_avg_sqs is not None else None
        e.numel = params[i].numel()
        if step_tensors is not None:
            e.step_dev = step_tensors[i].data_ptr()
        else:
            e.step = int(steps[i])
    hp = AdamWHParams(lr=lr, beta1=beta1, beta2=beta2, eps=eps, weight_decay=weight_decay,
                      amsgrad=1 if max_exp_avg_sqs is not None else 0, maximize=1 if maximize else 0)
    launches = C.c_int64(0)
    check(lib().mx_adamw_step(arr, n, C.byref(hp), C.byref(launches), stream))
    return launches.value


def sum_mid(out, src, outer, reduce, inner, stream=None) -> None:
    check(lib().mx_sum_f32(ptr(out), ptr(src), outer, reduce, inner, stream))


UNARY_SILU, UNARY_RELU = 0, 1
UNARY_SILU_GRAD, UNARY_THRESHOLD_GRAD = 0, 1
REDUCE_NONE, REDUCE_MEAN, REDUCE_SUM = 0, 1, 2


def group_norm_forward(x, gamma, beta, groups, eps, y, mean, rstd, stream=None) -> None:
    """x [N, C, *] contiguous FP32; mean / rstd [N, groups]."""
    n, c = x.shape[0], x.shape[1]
    hw = math.prod(x.shape[2:])
    check(lib().mx_group_norm_forward(ptr(x), ptr(gamma), ptr(beta), n, c, hw, groups, eps, ptr(y), ptr(mean),
                                      ptr(rstd), stream))


def group_norm_backward(dy, x, mean, rstd, gamma, groups, dx, dgamma, dbeta, stream=None) -> None:
    n, c = x.shape[0], x.shape[1]
    hw = math.prod(x.shape[2:])
    check(lib().mx_group_norm_backward(ptr(dy), ptr(x), ptr(mean), ptr(rstd), ptr(gamma), n, c, hw, groups,
                                       ptr(dx), ptr(dgamma), ptr(dbeta), stream))


def batch_norm_forward(x, gamma, beta, running_mean, running_var, training, momentum, eps, y, save_mean,
                       save_invstd, stream=None) -> None:
    n, c = x.shape[0], x.shape[1]
    hw = math.prod(x.shape[2:])
    rms = running_mean.stride(0) if running_mean is not None else 0
    rvs = running_var.stride(0) if running_var is not None else 0
    check(lib().mx_batch_norm_forward(ptr(x), ptr(gamma), ptr(beta), ptr(running_mean), rms, ptr(running_var), rvs,
                                      n, c, hw, 1 if training else 0, momentum, eps, ptr(y), ptr(save_mean),
                                      ptr(save_invstd), stream))


def batch_norm_backward(dy, x, gamma, mean, invstd_or_var, training, eps, dx, dgamma, dbeta, stream=None) -> None:
    n, c = x.shape[0], x.shape[1]
    hw = math.prod(x.shape[2:])
    check(lib().mx_batch_norm_backward(ptr(dy), ptr(x), ptr(gamma), ptr(mean), ptr(invstd_or_var), n, c, hw,
                                       1 if training else 0, eps, ptr(dx), ptr(dgamma), ptr(dbeta), stream))


def unary(op, x, y, stream=None) -> None:
    check(lib().mx_unary_f32(op, ptr(x), ptr(y), x.numel(), stream))


def unary_backward(op, dy, x, dx, threshold=0.0, stream=None) -> None:
    check(lib().mx_unary_backward_f32(op, ptr(dy), ptr(x), threshold, ptr(dx), x.numel(), stream))


def upsample_nearest2d(x, y, scale_h=0.0, scale_w=0.0, stream=None) -> None:
    n, c, ih, iw = x.shape
    check(lib().mx_upsample_nearest2d(ptr(x), n * c, ih, iw, y.shape[2], y.shape[3], scale_h or 0.0, scale_w or 0.0,
                                      ptr(y), stream))


def upsample_nearest2d_backward(dy, dx, scale_h=0.0, scale_w=0.0, stream=None) -> None:
    n, c, ih, iw = dx.shape
    check(lib().mx_upsample_nearest2d_backward(ptr(dy), n * c, ih, iw, dy.shape[2], dy.shape[3], scale_h or 0.0,
                                               scale_w or 0.0, ptr(dx), stream))


def _axis_split(shape, dim):
    outer = inner = 1
    for i, s in enumerate(shape):
        if i < dim:
            outer *= s
        elif i > dim:
            inner *= s
    return outer, (shape[dim] if shape else 1), inner


def softmax(x, dim, y, stream=None) -> None:
    o, a, i = _axis_split(tuple(x.shape), dim % max(1, x.dim()))
    check(lib().mx_softmax_f32(ptr(x), o, a, i, ptr(y), stream))


def softmax_backward(dy, y, dim, dx, stream=None) -> None:
    o, a, i = _axis_split(tuple(y.shape), dim % max(1, y.dim()))
    check(lib().mx_softmax_backward_f32(ptr(dy), ptr(y), o, a, i, ptr(dx), stream))


def mse_loss(x, t, reduction, out, stream=None) -> None:
    check(lib().mx_mse_loss_f32(ptr(x), ptr(t), x.numel(), reduction, ptr(out), stream))


def mse_loss_backward(dy, x, t, reduction, dx, stream=None) -> None:
    check(lib().mx_mse_loss_backward_f32(ptr(dy), ptr(x), ptr(t), x.numel(), reduction, ptr(dx), stream))


def copy_rows(dst, dst_pitch, src, src_pitch, row_bytes, rows, stream=None) -> None:
    """Pitches and row length in bytes; dst / src are raw device addresses."""
    check(lib().mx_copy_rows(dst, dst_pitch, src, src_pitch, row_bytes, rows, stream))


(FE_MUL_SCALAR, FE_ADD_SCALAR, FE_DIV_SCALAR, FE_LERP_SCALAR, FE_LERP_TENSOR, FE_ADDCMUL, FE_ADDCDIV,
 FE_MAXIMUM, FE_MINIMUM, FE_SQRT, FE_ADD_LIST) = range(11)


def foreach(op, outs, a, b=None, c=None, scalars=0.0, stream=None) -> int:
    """One multi-tensor pointwise call; scalars is one number or one per tensor.
    Returns the number of launches."""
    n = len(outs)
    arr = (ForeachTensor * max(1, n))()
    for i in range(n):
        s = scalars[i] if isinstance(scalars, (list, tuple)) else scalars
        arr[i] = ForeachTensor(ptr(outs[i]), ptr(a[i]), ptr(b[i]) if b is not None else None,
                               ptr(c[i]) if c is not None else None, outs[i].numel(), float(s))
    launches = C.c_int64(0)
    check(lib().mx_foreach_f32(op, arr, n, C.byref(launches), stream))
    return launches.value


def conv2d_kernel_name(d: ConvDesc, phase: int, algo: int = ALGO_AUTO) -> str:
    buf = C.create_string_buffer(128)
    check(lib().mx_conv2d_kernel_name(C.byref(d), phase, algo, buf, 128))
    return buf.value.decode()


def conv2d_backward_one_launch(d: ConvDesc, algo_dx: int = ALGO_AUTO, algo_dw: int = ALGO_AUTO,
                               with_bias: bool = True) -> bool:
    """Whether conv2d_backward with these algorithms runs both gradients as
    one Winograd launch (mx_conv2d_backward_one_launch)."""
    one = C.c_int(0)
    check(lib().mx_conv2d_backward_one_launch(C.byref(d), algo_dx, algo_dw, 1 if with_bias else 0, C.byref(one)))
    return bool(one.value)


def conv2d_plan(d: ConvDesc, phase: int, algo: int = ALGO_AUTO, with_bias: bool = True) -> dict:
    """Plan of one conv call (mx_conv2d_plan): algorithm, tile, K splits and
    span, workspace bytes, and the kernel instantiations it launches."""
    info = ConvPlanInfo()
    check(lib().mx_conv2d_plan(C.byref(d), phase, algo, 1 if with_bias else 0, C.byref(info)))
    return {"algo": info.algo, "tile": info.tile, "splits": info.splits, "span": info.span,
            "workspace_bytes": info.workspace_bytes, "variant": info.variant.decode()}


def dweight_plan(d: ConvDesc):
    s, sp, ws = C.c_int64(), C.c_int64(), C.c_int64()
    check(lib().mx_conv2d_dweight_plan(C.byref(d), C.byref(s), C.byref(sp), C.byref(ws)))
    return s.value, sp.value, ws.value


class Event:
    """HIP event through the C ABI (timing enabled)."""

    def __init__(self):
        h = C.c_void_p()
        check(lib().mx_event_create(C.byref(h), 1))
        self.h = h

    def record(self, stream=None):
        check(lib().mx_event_record(self.h, stream))

    def synchronize(self):
        check(lib().mx_event_synchronize(self.h))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        check(lib().mx_event_elapsed_ms(self.h, end.h, C.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            lib().mx_event_destroy(self.h)
        except Exception:
            pass
