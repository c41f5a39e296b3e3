"""Host <-> device copies through the C ABI on the GPU: device-to-host reads
return the exact bytes from any source offset, for any length (sizes from one
byte to past 4 MiB), and a stream's pending work lands before a read on that
stream."""
import ctypes

import numpy as np
import pytest

import oracle
import wxo_q8

pytestmark = pytest.mark.gpu

LIMIT = 4 << 20


@pytest.fixture(scope="module")
def source():
    wxo_q8.init()
    data = np.random.default_rng(11).integers(0, 256, LIMIT + 4096, dtype=np.uint8)
    buf = wxo_q8.DeviceBuffer.from_array(data)
    yield data, buf
    buf.free()


@pytest.mark.parametrize("offset", [0, 1, 3, 4, 12, 16, 4095])
@pytest.mark.parametrize("length", [1, 3, 4, 15, 16, 17, 44032, 65536, 65537, 600000])
def test_read_any_offset_and_length(source, offset, length):
    data, buf = source
    print(f"read offset={offset} length={length}", flush=True)
    got = buf.download(np.uint8, length, offset=offset)
    assert np.array_equal(got, data[offset:offset + length])


@pytest.mark.parametrize("length", [LIMIT - 16, LIMIT, LIMIT + 1, LIMIT + 4096])
def test_read_around_4_mib(source, length):
    data, buf = source
    print(f"read length={length}", flush=True)
    got = buf.download(np.uint8, length)
    assert np.array_equal(got, data[:length])


def test_small_reads_after_a_large_one(source):
    data, buf = source
    for length in (100, LIMIT, 7, 300000, 64):
        print(f"read length={length}", flush=True)
        assert np.array_equal(buf.download(np.uint8, length, offset=5), data[5:5 + length])


def test_read_waits_for_the_stream():
    # A matvec enqueued on a stream, then read back on that stream: the read
    # sees the finished output, every call.
    wxo_q8.init()
    stream = wxo_q8.Stream()
    N, K = 4096, 1024
    W = K // 4
    rng = np.random.default_rng(5)
    weight = wxo_q8.DeviceBuffer.from_array(rng.integers(0, 2**32, N * W, dtype=np.uint64).astype(np.uint32))
    scale = wxo_q8.DeviceBuffer.from_array(np.full(N, 0.5, np.float32))
    out = wxo_q8.DeviceBuffer(N * 4)
    L = wxo_q8.lib()
    first = None
    for i in range(20):
        x = wxo_q8.DeviceBuffer.from_array(np.full(K, float(i), np.float32))
        assert L.wxo_matvec_q8(weight.ptr, scale.ptr, x.ptr, out.ptr, N, K, 1, stream.handle) == 0
        y = out.download(np.float32, N, stream)
        if i == 1:
            first = y.copy()
        if i >= 1:
            # y is linear in the constant vector value i
            np.testing.assert_allclose(y, first * i, rtol=1e-5, atol=1e-3)
        else:
            assert np.all(y == 0)
        x.free()
    for b in (weight, scale, out):
        b.free()
    stream.destroy()


def test_async_read_into_page_locked_memory():
    """wxo_memcpy_dtoh_async into wxo_host_malloc memory returns while the
    work ahead of it on its stream still runs, and the bytes are there once an
    event recorded after it completes; a later write on the stream does not
    reach the bytes already read."""
    import time
    wxo_q8.init()
    L = wxo_q8.lib()
    n = 1 << 16
    src = np.arange(n, dtype=np.uint32) * np.uint32(2654435761)
    dev = wxo_q8.DeviceBuffer.from_array(src)
    host = ctypes.c_void_p(0)
    assert L.wxo_host_malloc(ctypes.byref(host), n * 4) == 0 and host.value
    pinned = np.ctypeslib.as_array((ctypes.c_uint32 * n).from_address(host.value))
    pinned[:] = 0
    stream = wxo_q8.Stream()
    done = wxo_q8.Event()
    try:
        assert L.wxo_spin(30000, stream.handle) == 0  # 30 ms of work ahead of the copy
        t0 = time.perf_counter()
        assert L.wxo_memcpy_dtoh_async(host.value, dev.ptr, n * 4, stream.handle) == 0
        issued = time.perf_counter() - t0
        assert L.wxo_memset(dev.ptr, 0, n * 4, stream.handle) == 0  # after the copy, in stream order
        done.record(stream)
        done.synchronize()
        assert issued < 0.02, f"the async copy held the host {issued * 1e3:.1f} ms"
        np.testing.assert_array_equal(pinned, src)
        assert np.all(dev.download(np.uint32, n) == 0)
        assert L.wxo_host_free(None) == 0
        assert L.wxo_memcpy_dtoh_async(None, dev.ptr, 4, stream.handle) == wxo_q8.WXO_ERR_INVALID
    finally:
        wxo_q8.synchronize()
        done.destroy()
        stream.destroy()
        assert L.wxo_host_free(host.value) == 0
        dev.free()


def test_gate_holds_the_stream_until_released():
    """wxo_gate_hold: work enqueued behind a held gate waits for the host's
    release (the host sleeps 30 ms before it); releasing a later gate opens
    an earlier one too; a gate nobody releases opens by itself after its time
    limit, and gates still work afterwards."""
    import time
    wxo_q8.init()
    L = wxo_q8.lib()
    n = 4096
    buf = wxo_q8.DeviceBuffer.from_array(np.arange(n, dtype=np.uint32))
    stream = wxo_q8.Stream()
    ev = [wxo_q8.Event(timer=True) for _ in range(3)]
    g1, g2 = ctypes.c_uint32(0), ctypes.c_uint32(0)
    try:
        ev[0].record(stream)
        assert L.wxo_gate_hold(500000, stream.handle, ctypes.byref(g1)) == 0
        assert L.wxo_memset(buf.ptr, 0x11, n * 4, stream.handle) == 0
        assert L.wxo_gate_hold(500000, stream.handle, ctypes.byref(g2)) == 0
        assert g2.value == g1.value + 1
        assert L.wxo_memset(buf.ptr, 0x22, n * 4, stream.handle) == 0
        ev[1].record(stream)
        time.sleep(0.03)
        assert L.wxo_gate_release(g2.value) == 0  # opens g1 as well
        ev[1].synchronize()
        held = ev[0].elapsed_ms(ev[1])
        assert 25.0 < held < 400.0, f"the stream ran {held:.1f} ms after it was held"
        assert np.all(buf.download(np.uint32, n) == 0x22222222)
        assert L.wxo_gate_release(g1.value) == 0  # a late release of an opened gate is harmless
        # nobody releases: the gate opens after its 5 ms
        ev[0].record(stream)
        assert L.wxo_gate_hold(5000, stream.handle, ctypes.byref(g1)) == 0
        ev[2].record(stream)
        ev[2].synchronize()
        alone = ev[0].elapsed_ms(ev[2])
        assert 4.0 < alone < 200.0, f"an unreleased 5 ms gate held the stream {alone:.2f} ms"
        # and later gates still hold and release
        ev[0].record(stream)
        assert L.wxo_gate_hold(500000, stream.handle, ctypes.byref(g2)) == 0
        ev[1].record(stream)
        time.sleep(0.01)
        assert L.wxo_gate_release(g2.value) == 0
        ev[1].synchronize()
        assert 8.0 < ev[0].elapsed_ms(ev[1]) < 400.0
        # numbers never handed out are refused
        assert L.wxo_gate_release(0) == wxo_q8.WXO_ERR_INVALID
        assert L.wxo_gate_release(g2.value + 1) == wxo_q8.WXO_ERR_INVALID
        assert L.wxo_gate_hold(1000, stream.handle, None) == wxo_q8.WXO_ERR_INVALID
    finally:
        wxo_q8.synchronize()
        for e in ev:
            e.destroy()
        stream.destroy()
        buf.free()


@pytest.mark.parametrize("offset", [0, 1, 3, 16, 17])
@pytest.mark.parametrize("length", [0, 1, 15, 16, 17, 1000, 65536 + 5])
def test_memset_any_offset_and_length(offset, length):
    """wxo_memset sets exactly [offset, offset + length) and no byte around it."""
    wxo_q8.init()
    size = 70000
    before = np.random.default_rng(offset * 7 + length).integers(0, 256, size, dtype=np.uint8)
    buf = wxo_q8.DeviceBuffer.from_array(before)
    wxo_q8._check(wxo_q8.lib().wxo_memset(buf.ptr + offset, 0x15a, length, None))  # value & 0xff = 0x5a
    wxo_q8.synchronize()
    got = buf.download(np.uint8, size)
    want = before.copy()
    want[offset:offset + length] = 0x5a
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"offset={offset} length={length}: {bad.size} bytes differ, first at {bad[0]}"
    buf.free()


def test_failed_allocation_leaves_later_calls_working():
    """An allocation the device cannot hold fails with WXO_ERR_OOM and
    allocates nothing; the next allocation and launch on the same thread
    succeed (the failure is not reported a second time)."""
    with pytest.raises(wxo_q8.WxoError) as e:
        wxo_q8.DeviceBuffer(1 << 50)
    assert e.value.status == wxo_q8.WXO_ERR_OOM, e.value
    rng = np.random.default_rng(5)
    N, K = 300, 1030
    w = rng.integers(0, 2 ** 32, N * ((K + 3) // 4), dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(1e-3, 1e-2, N).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    y = wxo_q8.matvecQ8(weight=w, scale=s, vector=x, N=N, K=K)
    ok, msg = oracle.check_matvec(y, oracle.matvec_q8(w, s, x, N, K), oracle.absterm(w, s, x, N, K))
    assert ok, msg


def test_roofline_ceilings():
    """wxo_roofline: the calibrated HBM read ceiling and one-wide f32 FMA rate
    fall inside what the hardware allows, either part can be asked for alone,
    and neither part is an error; the matvec at cfg2 does not stream faster
    than the ceiling (beyond timing noise)."""
    print("wxo_roofline", flush=True)
    r = wxo_q8.roofline()
    assert 3e12 < r["bandwidth"] < 8.2e12, r
    # one-wide v_fma_f32 (packed FP32 is disabled in this build) under MI355X's
    # published 157.3 TFLOP/s FP32 vector peak
    assert 2e13 < r["compute"] < 1.6e14, r
    only_bw = wxo_q8.roofline(compute=False)
    assert only_bw["compute"] is None and 3e12 < only_bw["bandwidth"] < 8.2e12
    with pytest.raises(wxo_q8.WxoError, match="roofline"):
        wxo_q8.roofline(bandwidth=False, compute=False)


def test_roofline_matrix_ceiling():
    """wxo_roofline_matrix: the sustained bf16 matrix-core rate with
    matmulQ8-like operands is positive and under MI355X's published dense
    2.5 PFLOP/s (with margin for timing), and a second measurement agrees
    with the first within a quarter."""
    print("wxo_roofline_matrix", flush=True)
    a = wxo_q8.roofline_matrix()
    assert 5e14 < a < 2.6e15, a
    b = wxo_q8.roofline_matrix()
    assert 0.75 < b / a < 1.33, (a, b)
