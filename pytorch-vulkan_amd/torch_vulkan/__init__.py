"""torch_vulkan: MI355X (gfx950) FP32 conv / GEMM / fused-AdamW backend for PyTorch.

A drop-in for the operator surface of the mistrjirka/Pytorch-vulkan backend
(torch_vulkan/__init__.py there): importing this package registers the
PrivateUse1 device under the same name, ``"vulkan"``, so code written for the
reference runs unchanged::

    import torch, torch_vulkan
    x = torch.randn(8, 64, 56, 56).to("vulkan")
    w = torch.randn(64, 64, 3, 3).to("vulkan")
    y = torch.nn.functional.conv2d(x, w, padding=1)   # gfx950 MFMA kernels

Device work runs in ``libmx.so`` (C ABI, ``include/mx.h``) on HIP streams;
``_C.so`` maps the ATen operators onto it.  Both must be built
(``python pytorch-vulkan_amd/build.py``); importing without them raises, there
is no CPU substitute for the conv / GEMM / AdamW path.
"""
from __future__ import annotations

import contextlib
import os
import sys

import torch  # loads torch's HIP runtime first; libmx.so binds to the same one

_here = os.path.dirname(os.path.abspath(__file__))
for _lib in ("libmx.so", "_C.so"):
    if not os.path.exists(os.path.join(_here, _lib)):
        raise ImportError(
            f"torch_vulkan: {_lib} is not built; run `python pytorch-vulkan_amd/build.py` "
            "(the gfx950 kernels have no CPU substitute)")

from . import _C  # noqa: E402  (registers PrivateUse1 as "vulkan", hooks, allocator, kernels)

__all__ = [
    "is_available", "device_count", "current_device", "set_device", "synchronize", "device_name",
    "execution_stats", "reset_execution_stats", "conv_dispatch_stats", "clear_conv_dispatch_cache",
    "gpu_timing_stats", "reset_gpu_timing_stats",
    "memory_stats", "empty_cache", "queue_stats", "performance_options", "Stream", "Event",
    "current_stream", "default_stream", "set_stream", "stream", "manual_seed", "manual_seed_all",
    "device", "is_hardware_accelerated", "runtime_hotpath_stats", "cache_stats", "clear_algorithm_cache",
    "get_rng_state", "set_rng_state",
]


def _tensor_vulkan(self, *args, **kwargs):
    # torch already defines Tensor.is_vulkan for its legacy Vulkan tensors, so
    # the generated PrivateUse1 methods cannot be used; define .vulkan() only.
    if args:
        raise TypeError("tensor.vulkan() takes no positional arguments")
    return self.to(device="vulkan", **kwargs)


torch.Tensor.vulkan = _tensor_vulkan


def is_available() -> bool:
    """True when at least one gfx950 device is visible."""
    return _C._is_available()


def is_hardware_accelerated() -> bool:
    """True when the device is a physical GPU (reference:
    torch_vulkan/__init__.py:61-63, False there for a software rasteriser).
    Every device this backend opens is a gfx950 GPU, so this is
    ``is_available()``."""
    return is_available()


def runtime_hotpath_stats() -> dict:
    """Cumulative host-side timers of the hot path, recorded when
    ``TORCH_VULKAN_PROFILE_HOST_HOTPATH=1`` is set at start-up (the
    reference's knob and keys): ``enqueue_ns`` / ``enqueue_count`` (host time
    of each conv / GEMM / AdamW op's library calls), ``allocator_*`` (device
    allocations, ``fresh`` = new device memory, ``reused`` = served from the
    cache) and ``algo_hit_*`` / ``algo_miss_*`` (lookups in the convolution
    autotune plan cache)."""
    return dict(_C._runtime_hotpath_stats())


def cache_stats() -> dict:
    """The reference's cache counters (torch_vulkan/__init__.py:114-123).
    HIP code objects are loaded once per process, so there is no pipeline or
    command-sequence cache: ``pipeline_*`` and ``seq_*`` stay 0.  ``algo_*``
    count the convolution autotune plan cache (hits, misses, evictions;
    ``bound_algorithms`` is its size); the device allocator's cache is reported
    as ``bound_cached_buffer_bytes`` (reserved but free bytes) and
    ``allocator_cache_hits`` / ``allocator_device_mallocs``."""
    conv = dict(_C._conv_dispatch_stats())
    mem = dict(_C._memory_stats())
    reserved = int(mem.get("reserved_bytes", 0))
    allocated = int(mem.get("allocated_bytes", 0))
    return {"algo_hits": int(conv.get("hits", 0)), "algo_misses": int(conv.get("misses", 0)),
            "seq_reuses": 0, "seq_creates": 0, "algo_evictions": int(conv.get("evictions", 0)),
            "bound_algorithms": int(conv.get("entries", 0)),
            "bound_cached_buffer_bytes": max(0, reserved - allocated),
            "pipeline_hits": 0, "pipeline_misses": 0, "pipeline_evictions": 0, "pipeline_entries": 0,
            "allocator_cache_hits": int(mem.get("cache_hits", 0)),
            "allocator_device_mallocs": int(mem.get("device_mallocs", 0))}


def clear_algorithm_cache() -> None:
    """Forget the convolution algorithms chosen by autotuning (the plan cache;
    its counters stay).  The reference drops its compiled-pipeline cache here
    (torch_vulkan/__init__.py:126-132); cached device memory is released by
    ``empty_cache()``."""
    _C._clear_conv_plan_cache()


def device_count() -> int:
    return _C._device_count()


def current_device() -> int:
    return _C._current_device()


def _validate_device(value=None) -> int:
    if value is None:
        return current_device()
    d = torch.device("vulkan", value) if isinstance(value, int) else torch.device(value)
    if d.type != "vulkan":
        raise RuntimeError(f"expected a vulkan device, got {d}")
    idx = current_device() if d.index is None else d.index
    if not 0 <= idx < max(1, device_count()):
        raise RuntimeError(f"vulkan device index {idx} out of range")
    return idx


def set_device(value) -> None:
    _C._set_device(_validate_device(value))


def device(index: int = 0) -> torch.device:
    return torch.device("vulkan", index)


def synchronize(device=None) -> None:
    """Wait for all queued work on the device."""
    if device is not None:
        _validate_device(device)
    _C._synchronize()


def device_name(index: int = 0) -> str:
    return _C._device_name(index)


def execution_stats() -> dict:
    """Counters: CPU fallbacks, host reads, kernel launches, AdamW launches."""
    return dict(_C._execution_stats())


def reset_execution_stats() -> None:
    synchronize()
    _C._reset_execution_stats()


def queue_stats() -> dict:
    """Launch counter under the reference's key name (``recorded_ops``)."""
    s = _C._execution_stats()
    return {"recorded_ops": s["kernel_launches"], "adamw_launches": s["adamw_launches"]}


def gpu_timing_stats() -> dict:
    """Per-kernel GPU time of the conv / GEMM / AdamW ops since the last reset,
    recorded when ``TORCH_VULKAN_PROFILE_TIMESTAMPS=1`` (the reference's
    opt-in knob): ``{kernel: {"samples", "shader_ms", "host_eval_ms",
    "upload_ms", "download_ms", "flops"}}``.  Waits for the timed work to
    finish.  ``shader_ms`` is the time between HIP events recorded around each
    op on its stream; ``flops`` the ops' algorithmic work (2 per multiply-add
    of the direct convolution / GEMM); buffers never leave the device, so
    upload / download are 0."""
    return dict(_C._gpu_timing_stats())


def reset_gpu_timing_stats() -> None:
    _C._reset_gpu_timing_stats()


def conv_dispatch_stats() -> dict:
    """``selected_<phase>_<algorithm>`` counters of the convolution planner."""
    return dict(_C._conv_dispatch_stats())


def clear_conv_dispatch_cache() -> None:
    _C._clear_conv_dispatch_cache()


def memory_stats() -> dict:
    return dict(_C._memory_stats())


def empty_cache() -> None:
    _C._empty_cache()


def performance_options() -> dict:
    return {
        "device_resident": True,
        "streams": "hip",
        "adamw_multitensor": True,
        "conv_algo": os.environ.get("TORCH_VULKAN_CONV_ALGO", "auto"),
        "conv_backward_algo": os.environ.get("TORCH_VULKAN_CONV_BACKWARD_ALGO", "auto"),
    }


# ----------------------------------------------------------------- RNG API
def manual_seed(seed: int) -> None:
    _C._manual_seed(int(seed))


def manual_seed_all(seed: int) -> None:
    _C._manual_seed(int(seed))


def initial_seed() -> int:
    return _C._initial_seed()


def seed() -> None:
    import random
    _C._manual_seed(random.getrandbits(63))


def seed_all() -> None:
    seed()


def get_rng_state(device="vulkan") -> torch.Tensor:
    """The device generator's state (seed and offset, 16 bytes), as the
    reference's get_rng_state (torch_vulkan/__init__.py:190-193)."""
    return _C._get_rng_state(_rng_device(device))


def set_rng_state(state: torch.Tensor, device="vulkan") -> None:
    _C._set_rng_state(_rng_device(device), state)


def _rng_device(device) -> int:
    return _validate_device(device)


def _is_in_bad_fork() -> bool:
    return False


# ---------------------------------------------------------------- streams
def current_stream(device=None):
    return _C._current_stream(-1 if device is None else _validate_device(device))


def default_stream(device=None):
    return _C._default_stream(-1 if device is None else _validate_device(device))


def set_stream(value) -> None:
    if value is not None:
        _C._set_stream(value.stream_id, value.device_index)


@contextlib.contextmanager
def stream(value):
    if value is None:
        yield
        return
    prev = current_stream(value.device_index)
    set_stream(value)
    try:
        yield
    finally:
        set_stream(prev)


class Stream(torch.Stream):
    def __new__(cls, device="vulkan", priority=0):
        if priority != 0:
            raise RuntimeError("vulkan streams support the default priority only")
        return super().__new__(cls, device=device, priority=0)


def Event(enable_timing: bool = False, blocking: bool = False, interprocess: bool = False):
    if interprocess:
        raise RuntimeError("interprocess vulkan events are unsupported")
    return torch.Event(device="vulkan", enable_timing=enable_timing, blocking=blocking)


torch._register_device_module("vulkan", sys.modules[__name__])

from . import optim  # noqa: E402,F401
