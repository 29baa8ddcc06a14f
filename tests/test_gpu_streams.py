"""GPU tests of stream, event and allocator semantics on the "vulkan" device.

The reference serialises every logical stream on one Vulkan queue
(csrc/torch_vulkan.cpp:34-37) and has no pinned memory; here every logical
stream is its own HIP stream, so the tests check what that adds: the
reference's own stream / event / lifetime test (tests/test_complete_runtime.py:6-31),
ordering across streams through wait_stream / wait_event, deferred reuse of
memory handed to another stream with record_stream, work on two streams
running at the same time, and non_blocking copies from and to page-locked
host memory (queued on the stream, host storage held until they complete).
"""
import gc
import time

import pytest
import torch

pytestmark = pytest.mark.gpu

# One 64x64 output tile with a long K: a single workgroup for several
# milliseconds, so two of them on two streams can only finish early together
# if the streams really run at the same time.
LONG_K = 1 << 19


@pytest.fixture(scope="module")
def vk():
    import torch_vulkan
    assert torch_vulkan.is_available(), "no gfx950 device visible"
    return torch_vulkan


@pytest.fixture(scope="module")
def long_operands(vk):
    g = torch.Generator().manual_seed(5)
    a = torch.randn(64, LONG_K, generator=g) / 256
    b = torch.randn(LONG_K, 64, generator=g) / 256
    return a, b, a.to("vulkan"), b.to("vulkan")


def test_reference_stream_context_events_and_lifetimes(vk):
    default = vk.current_stream()
    s = torch.Stream(device="vulkan")
    other = vk.Stream()
    assert s != default and other != s
    begin, end = vk.Event(enable_timing=True), vk.Event(enable_timing=True)
    with s:
        assert vk.current_stream() == s
        begin.record(s)
        x = torch.arange(64.0).to("vulkan")
        y = x.sin().mul(3)  # sin runs through the counted CPU fallback, on stream s
        del x
        end.record(s)
    assert vk.current_stream() == default
    with other:
        other.wait_event(end)
        z = y.cos()
    end.synchronize()
    assert end.query()
    assert begin.elapsed_time(end) >= 0
    torch.testing.assert_close(z.cpu(), (torch.arange(64.0).sin() * 3).cos(), rtol=1e-4, atol=3e-5)
    other.synchronize()
    assert other.query()
    for _ in range(5):
        with s:
            y = torch.ones(1000, device="vulkan").sin()
            end.record(s)
        del y
    gc.collect()
    vk.synchronize()
    assert end.query()


def test_wait_stream_orders_dependent_work(vk, long_operands):
    a, b, da, db = long_operands
    s1, s2 = vk.Stream(), vk.Stream()
    s1.wait_stream(vk.current_stream())
    with vk.stream(s1):
        c = da @ db                     # milliseconds of work on s1
    s2.wait_stream(s1)
    with vk.stream(s2):
        d = c * 2.0                     # must see the finished product
    c.record_stream(s2)
    s2.synchronize()
    want = (a.double() @ b.double()) * 2
    terms = (a.double().abs() @ b.double().abs()) * 2   # error model: rel 1e-4 + 1e-5 of the summed magnitudes
    assert torch.all((d.cpu().double() - want).abs() <= 1e-4 * want.abs() + 1e-5 * terms)


def test_record_stream_defers_reuse(vk, long_operands):
    _, _, da, db = long_operands
    s2 = vk.Stream()
    n = 1 << 22
    x = torch.full((n,), 3.0, device="vulkan")
    s2.wait_stream(vk.current_stream())
    with vk.stream(s2):
        busy = da @ db                  # keeps s2 busy before it reads x
        y = x * 2.0
    x.record_stream(s2)
    ptr = x.data_ptr()
    del x
    still_busy = not s2.query()
    z = torch.empty(n, device="vulkan")
    z.fill_(-1.0)                       # default stream: may not reuse x's block while s2 needs it
    if still_busy:
        assert z.data_ptr() != ptr
    s2.synchronize()
    assert torch.all(y.cpu() == 6.0)
    del busy


def _timed(vk, fn):
    """Host wall time of fn() between two device synchronisations, in ms."""
    vk.synchronize()
    t0 = time.perf_counter()
    fn()
    vk.synchronize()
    return 1e3 * (time.perf_counter() - t0)


def test_two_streams_run_concurrently(vk, long_operands):
    _, _, da, db = long_operands
    s1, s2 = vk.Stream(), vk.Stream()
    for s in (s1, s2):
        s.wait_stream(vk.current_stream())

    def serial():
        with vk.stream(s1):
            da @ db
            da @ db

    def parallel():
        with vk.stream(s1):
            da @ db
        with vk.stream(s2):
            da @ db

    serial(), parallel()
    t_serial = min(_timed(vk, serial) for _ in range(3))
    t_parallel = min(_timed(vk, parallel) for _ in range(3))
    assert t_serial > 2.0, f"the probe GEMM is too short to time ({t_serial:.2f} ms)"
    assert t_parallel < 0.75 * t_serial, f"serial {t_serial:.2f} ms, two streams {t_parallel:.2f} ms"


def test_non_blocking_pinned_copies(vk):
    ref = torch.randn(1 << 20)
    h = ref.clone().pin_memory()
    assert h.is_pinned()
    before = vk.execution_stats()["async_copies"]
    d = h.to("vulkan", non_blocking=True)
    del h                               # the backend holds the pages until the copy is done
    gc.collect()
    back = torch.empty(1 << 20).pin_memory()
    back.copy_(d, non_blocking=True)
    vk.synchronize()
    assert torch.equal(back, ref)
    stats = vk.execution_stats()
    assert stats["async_copies"] - before == 2
    assert stats["pending_host_copies"] == 0
    # pageable memory: the same call is a blocking copy, still correct
    p = torch.randn(1000)
    dp = p.to("vulkan", non_blocking=True)
    assert vk.execution_stats()["async_copies"] - before == 2
    assert torch.equal(dp.cpu(), p)


def test_memcpy_async_rejects_pageable_memory(vk):
    import ctypes as C
    from torch_vulkan import mx
    lib = mx.lib()
    host = torch.randn(256)
    dev = torch.empty(256, device="vulkan")
    flag = C.c_int(-1)
    assert lib.mx_host_is_pinned(C.c_void_p(host.data_ptr()), C.byref(flag)) == 0 and flag.value == 0
    rc = lib.mx_memcpy_async(C.c_void_p(dev.data_ptr()), C.c_void_p(host.data_ptr()), host.nbytes, mx.MX_COPY_H2D,
                             C.c_void_p(vk._C._current_stream_ptr()))
    assert rc != 0 and b"page-locked" in lib.mx_last_error()
    pinned = torch.randn(256).pin_memory()
    assert lib.mx_host_is_pinned(C.c_void_p(pinned.data_ptr()), C.byref(flag)) == 0 and flag.value == 1


def test_copy_overlaps_compute(vk, long_operands):
    """A page-locked upload on one stream while a GEMM runs on another."""
    _, _, da, db = long_operands
    compute, copy = vk.Stream(), vk.Stream()
    for s in (compute, copy):
        s.wait_stream(vk.current_stream())
    h = torch.randn(64 << 20).pin_memory()          # 256 MiB
    dst = torch.empty(64 << 20, device="vulkan")

    def upload():
        with vk.stream(copy):
            dst.copy_(h, non_blocking=True)

    def gemm():
        with vk.stream(compute):
            da @ db
            da @ db

    def both():
        upload()
        gemm()

    both()
    t_copy = min(_timed(vk, upload) for _ in range(3))
    t_gemm = min(_timed(vk, gemm) for _ in range(3))
    t_both = min(_timed(vk, both) for _ in range(3))
    assert torch.equal(dst.cpu(), h)
    assert t_both < 0.9 * (t_copy + t_gemm), f"copy {t_copy:.2f}, gemm {t_gemm:.2f}, both {t_both:.2f} ms"


def test_new_streams_come_from_a_fixed_pool(vk):
    """Stream() hands out the device's pooled HIP streams round-robin: a
    thousand requests create at most the pool's 32 streams, and each stream
    still orders its own work."""
    from torch_vulkan import _C
    streams = [vk.Stream() for _ in range(1000)]
    assert _C._stream_pool_size(0) <= 32
    assert len({s.stream_id for s in streams}) <= 32
    x = torch.arange(1 << 16, dtype=torch.float32).to("vulkan")
    for s in streams[:40]:
        s.wait_stream(vk.current_stream())
        with vk.stream(s):
            y = x * 2
        s.synchronize()
        assert torch.equal(y.cpu(), torch.arange(1 << 16, dtype=torch.float32) * 2)
    assert _C._stream_pool_size(0) <= 32
