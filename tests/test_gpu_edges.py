"""Edges the other GPU suites do not reach, through the C ABI:

  * quantize / quantize+pack into device buffers with sentinel tails after the
    codes, the packed words and the scales (the kernels store a row's last
    partial word as a full 16-byte store clamped by the row's buffer
    resource: a store past the row or the buffer would change a sentinel);
  * rows whose absmax is normal but tiny (the f32 fast path's inverse stays
    finite) with subnormal elements, so the fast path meets subnormal operands;
  * the batched LM head (cfg5) checked against the oracle on every row;
  * which kernel instance ran (wxo_last_variant), per thread.
  * rows far longer than the other suites' (K = 65539 and 131075) on every
    kernel family.
  * the batched k-split kernel at its store wave's limit (1023 tiles of 16
    rows per workgroup) and one row past it.
  * a weight past 4 GiB (64-bit row addressing), one and five vectors;
    packInt8Rows and quantize+pack with inputs and outputs past 4 GiB.
  * eight host threads on their own streams at once.

Bars as everywhere: codes, packed words and scales bit-exact;
matvecQ8 |y - y_ref| <= 1e-5 * sum_k |s q x| + 1e-7 per row.
"""
import re
import threading

import numpy as np
import pytest

import oracle
import wxo_q8
import wxo_workloads as wl
from test_gpu_parity import assert_bits_equal, assert_ffn, assert_matvec, assert_residual, random_weights

pytestmark = pytest.mark.gpu

SENT_I32 = np.int32(0x5A5A5A5A)
SENT_U32 = np.uint32(0xA5A5A5A5)
SENT_F32 = np.float32(-12345.5)
TAIL = 80  # elements of slack after each output


@pytest.fixture(scope="module", autouse=True)
def device():
    wxo_q8.init()


def edge_matrix(rng, N, D):
    x = (rng.standard_normal((N, D)) * 0.02).astype(np.float32)
    x[1 % N, D - 1] = 3.0  # absmax in the row's last element (the partial word)
    if N > 2:
        x[2, :] = 0.0
    if N > 3:
        x[3, D // 2] = np.nan
    return x


@pytest.mark.parametrize("D", [5, 1027, 4099])
def test_quantize_and_pack_device_sentinel_tails(D):
    rng = np.random.default_rng(D)
    N = 7
    W = (D + 3) // 4
    x = edge_matrix(rng, N, D)
    want_codes, want_scales = oracle.quantize(x, N, D)
    want_packed = oracle.pack_q8(want_codes, N, D)
    # input followed by huge values: reading past the last row would change its scale
    src = wxo_q8.DeviceBuffer.from_array(np.concatenate([x.reshape(-1), np.full(TAIL, 1e30, np.float32)]))
    codes = wxo_q8.DeviceBuffer.from_array(np.full(N * D + TAIL, SENT_I32, np.int32))
    scales = wxo_q8.DeviceBuffer.from_array(np.full(N + TAIL, SENT_F32, np.float32))
    packed = wxo_q8.DeviceBuffer.from_array(np.full(N * W + TAIL, SENT_U32, np.uint32))
    scales2 = wxo_q8.DeviceBuffer.from_array(np.full(N + TAIL, SENT_F32, np.float32))
    print(f"quantize D={D}: {wxo_q8.last_variant()}", flush=True)
    wxo_q8.quantize_device(src, N, D, codes, scales)
    print(f"  {wxo_q8.last_variant()}", flush=True)
    wxo_q8.quantize_pack_q8_device(src, N, D, packed, scales2)
    print(f"  {wxo_q8.last_variant()}", flush=True)
    wxo_q8.synchronize()
    c = codes.download(np.int32, N * D + TAIL)
    s = scales.download(np.float32, N + TAIL)
    p = packed.download(np.uint32, N * W + TAIL)
    s2 = scales2.download(np.float32, N + TAIL)
    assert_bits_equal(c[:N * D], want_codes, f"codes D={D}")
    assert_bits_equal(s[:N], want_scales, f"scales D={D}")
    assert_bits_equal(p[:N * W], want_packed, f"packed D={D}")
    assert_bits_equal(s2[:N], want_scales, f"fused scales D={D}")
    assert np.all(c[N * D:] == SENT_I32), "codes: wrote past the output"
    assert np.all(s[N:].view(np.uint32) == SENT_F32.view(np.uint32)), "scales: wrote past the output"
    assert np.all(p[N * W:] == SENT_U32), "packed: wrote past the output"
    assert np.all(s2[N:].view(np.uint32) == SENT_F32.view(np.uint32)), "fused scales: wrote past the output"
    for b in (src, codes, scales, packed, scales2):
        b.free()


@pytest.mark.parametrize("D", [5, 1027, 4099])
def test_quantize_pack_multi_device_sentinel_gaps(D):
    """Several matrices of one K in one launch, their outputs laid out in one
    allocation with sentinel gaps between them."""
    rng = np.random.default_rng(100 + D)
    W = (D + 3) // 4
    Ns = [3, 9, 5]
    xs = [edge_matrix(rng, n, D) for n in Ns]
    gap = 32
    words = sum(n * W + gap for n in Ns)
    pk = wxo_q8.DeviceBuffer.from_array(np.full(words, SENT_U32, np.uint32))
    sc = wxo_q8.DeviceBuffer.from_array(np.full(sum(n + gap for n in Ns), SENT_F32, np.float32))
    srcs = [wxo_q8.DeviceBuffer.from_array(x) for x in xs]
    mats, po, so = [], 0, 0
    offsets = []
    for n, src in zip(Ns, srcs):
        mats.append((src.ptr, n, pk.ptr + 4 * po, sc.ptr + 4 * so))
        offsets.append((po, so))
        po += n * W + gap
        so += n + gap
    wxo_q8.quantize_pack_q8_multi_device(mats, D)
    print(f"quantize_pack_multi D={D}: {wxo_q8.last_variant()}", flush=True)
    wxo_q8.synchronize()
    p = pk.download(np.uint32, words)
    s = sc.download(np.float32, so)
    for (n, x), (po, so) in zip(zip(Ns, xs), offsets):
        wc, ws = oracle.quantize(x, n, D)
        assert_bits_equal(p[po:po + n * W], oracle.pack_q8(wc, n, D), f"packed n={n}")
        assert_bits_equal(s[so:so + n], ws, f"scales n={n}")
        assert np.all(p[po + n * W:po + n * W + gap] == SENT_U32), "packed gap overwritten"
        assert np.all(s[so + n:so + n + gap].view(np.uint32) == SENT_F32.view(np.uint32)), "scales gap overwritten"
    for b in (pk, sc, *srcs):
        b.free()


def tiny_absmax_rows(rng, N, D):
    """Rows with a normal absmax in [4e-37, 1e-35] (127/absmax finite in f32)
    and subnormal elements: random subnormals, exact multiples of the smallest
    subnormal, values near absmax * (k + 1/2) / 127 (near-ties) and signs mixed."""
    x = np.zeros((N, D), np.float32)
    tiny = np.float32(1.4e-45)
    for r in range(N):
        amax = np.float32(np.exp(rng.uniform(np.log(4e-37), np.log(1e-35))))
        sub = (rng.integers(-(2 ** 23) + 1, 2 ** 23, D).astype(np.float64) * float(tiny)).astype(np.float32)
        x[r] = sub
        k = rng.integers(0, 127, D // 4 + 1)
        near = (amax.astype(np.float64) * (k + 0.5) / 127.0).astype(np.float32)
        near = np.where(np.abs(near) < np.float32(1.17549435e-38), near, sub[: near.size])
        x[r, : near.size] = near * np.where(rng.random(near.size) < 0.5, -1, 1).astype(np.float32)
        x[r, rng.integers(0, D)] = amax * (1 if r % 2 else -1)
    return x


@pytest.mark.parametrize("D", [7, 256, 1031, 4096])
def test_quantize_fast_path_meets_subnormal_elements(D):
    rng = np.random.default_rng(7 * D)
    N = 16
    x = tiny_absmax_rows(rng, N, D)
    absmax = np.abs(x).max(axis=1)
    assert np.all(absmax >= 3.9e-37) and np.all(absmax <= 1e-35)
    assert np.all(np.isfinite(np.float32(127.0) / absmax))
    assert np.mean((np.abs(x) < 1.17549435e-38) & (x != 0)) > 0.5, "mostly subnormal elements"
    want_codes, want_scales = oracle.quantize(x, N, D)
    assert np.any(want_codes != 0), "the subnormal elements must reach non-zero codes"
    codes, scales = wxo_q8.quantize(input=x, N=N, D=D)
    assert_bits_equal(codes, want_codes, f"codes D={D}")
    assert_bits_equal(scales, want_scales, f"scales D={D}")
    packed, s2 = wxo_q8.quantizePackQ8(input=x, N=N, K=D)
    assert_bits_equal(packed, oracle.pack_q8(want_codes, N, D), f"packed D={D}")
    assert_bits_equal(s2, want_scales, f"fused scales D={D}")


@pytest.mark.parametrize("M", [1, 4, 8, 16])
def test_batched_lm_head_every_row(M):
    """cfg5 (N=151936, K=1024) at every M the configuration names, every row
    against the oracle; M = 1 is the single-vector kernel's own instance
    (9,496 blocks of 16 rows, one chunk per wave)."""
    c = wl.make_config("cfg5", M=M)
    N, K = c["N"], c["K"]
    codes, scales = oracle.quantize(c["w"], N, K)
    w = oracle.pack_q8(codes, N, K)
    xs = c["x"].reshape(M, K)
    print(f"cfg5 M={M}: every row", flush=True)
    ys = wxo_q8.matvecQ8Batched(weight=w, scale=scales, vectors=xs, N=N, K=K, M=M)
    print(f"  {wxo_q8.last_variant()}", flush=True)
    if M == 1:
        assert wxo_q8.last_variant().startswith("matvec_q8_m1 "), wxo_q8.last_variant()
    for m in range(M):
        assert_matvec(ys[m], w, scales, xs[m], N, K)


def parse_variant(v):
    head, *rest = v.split(" ")
    kv = {}
    form = None
    for t in rest:
        if "=" in t:
            k, val = t.split("=", 1)
            kv[k] = val
        else:
            form = t
    return head, form, kv


@pytest.mark.parametrize("N,K,form,extra", [
    (4096, 4099, "xreg.tailwave", 1),   # 256 blocks: one per CU, the tail words on a wave of their own
    (2048, 4099, "xreg.tailwave", 1),   # 256 blocks of 8 rows
    (100, 8200, "xreg.tailwave", 1),
    (4097, 4099, "xreg.tail", 0),       # 257 blocks: the tail words ride with wave 0
    (11008, 8200, "xreg.tail", 0),      # 688 blocks of 9 waves would share CUs
])
def test_tail_form_choice(N, K, form, extra):
    """Rows of whole chunks plus 1-4 words: the extra tail wave runs only while
    the grid is at most one workgroup per CU; either form matches the oracle."""
    W = (K + 3) // 4
    rng = np.random.default_rng(N + K)
    w = rng.integers(0, 2 ** 32, N * W, dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(0.001, 0.05, N).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    got = wxo_q8.matvecQ8(weight=w, scale=s, vector=x, N=N, K=K)
    head, got_form, kv = parse_variant(wxo_q8.last_variant())
    assert head == "matvec_q8_m1" and got_form == form and int(kv["waves"]) == W // 256 + extra
    assert_matvec(got, w, s, x, N, K)


@pytest.mark.parametrize("cfg,M", [("cfg1", 1), ("cfg2", 1), ("cfg3", 1), ("cfg5", 16)])
def test_variant_names_the_instance_that_ran(cfg, M):
    c = wl.CONFIGS[cfg]
    N, K = c["N"], c["K"]
    W = (K + 3) // 4
    rng = np.random.default_rng(1)
    w = wxo_q8.DeviceBuffer.from_array(rng.integers(0, 2 ** 32, N * W, dtype=np.uint64).astype(np.uint32))
    s = wxo_q8.DeviceBuffer.from_array(np.full(N, 0.01, np.float32))
    x = wxo_q8.DeviceBuffer.from_array(rng.standard_normal(M * K).astype(np.float32))
    y = wxo_q8.DeviceBuffer(4 * M * N)
    wxo_q8.matvec_q8_device(w, s, x, y, N, K, M)
    wxo_q8.synchronize()
    v = wxo_q8.last_variant()
    print(f"{cfg} M={M}: {v}", flush=True)
    head, form, kv = parse_variant(v)
    grid = [int(t) for t in kv["grid"].split("x")]
    if M == 1:
        full, tail = divmod(W, 256)
        assert head == "matvec_q8_m1"
        rows = int(kv["rows"])
        assert grid[0] * rows >= N > (grid[0] - 1) * rows
        if 1 <= tail <= 4 and 1 <= full <= 8:
            # cfg3 (K = 4099, 256 blocks of 16 rows, one per CU): one wave per
            # whole 1 KiB chunk and one more for the rows' last words
            assert form == "xreg.tailwave" and int(kv["waves"]) == full + 1 and grid[0] <= 256
        else:
            assert int(kv["waves"]) == (W + 255) // 256  # one wave per 1 KiB chunk of a row
            assert form == ("xreg.masked" if tail else "xreg")
    else:
        # cfg5 (K = 1024): the k-split kernel, 128 codes per wave, 16 vectors per
        # tile, 8 streaming waves and the store wave
        assert head == "matvec_q8_ksplit" and form == "x16"
        assert int(kv["vectors"]) == M and grid[1] == 1 and int(kv["slots"]) == 1 and int(kv["waves"]) == 9
    # describe() carries the same variant
    assert f'last="{v}"' in wxo_q8.describe()
    # thread-local: another thread's calls do not change this thread's variant
    seen = {}

    def other():
        seen["before"] = wxo_q8.last_variant()
        wxo_q8.matvec_q8_device(w, s, x, y, 16, 64, 1)
        seen["after"] = wxo_q8.last_variant()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["before"] == "" and seen["after"].startswith("matvec_q8_m1 ")
    assert wxo_q8.last_variant() == v
    # a refused call leaves the last variant as it was
    with pytest.raises(wxo_q8.WxoError):
        wxo_q8.matvec_q8_device(w, s, x, y, N, K, 0)
    assert wxo_q8.last_variant() == v
    wxo_q8.synchronize()
    for b in (w, s, x, y):
        b.free()


@pytest.mark.parametrize("K", list(range(1, 20)) + [31, 63, 64, 65, 255, 256, 257, 1023, 1025, 2049, 4096, 4099, 5001])
@pytest.mark.parametrize("N", [1, 3, 50])
@pytest.mark.parametrize("offset", [0, 3])
def test_pack_int8_rows_any_alignment_sentinel_tail(K, N, offset):
    """packInt8Rows (llm/weights-q8.ts:137-139) bit-exact for row lengths on both
    sides of the streaming kernel's 4W >= 16 switch, codes starting at any byte
    (a row slice of a larger buffer) and a sentinel tail after the output."""
    rng = np.random.default_rng(K * 131 + N * 7 + offset)
    W = (K + 3) // 4
    codes = rng.integers(-128, 128, N * K).astype(np.int8)
    src = wxo_q8.DeviceBuffer.from_array(np.concatenate([rng.integers(-128, 128, offset).astype(np.int8), codes,
                                                         np.full(8, 0x55, np.int8)]))
    dst = wxo_q8.DeviceBuffer.from_array(np.full(N * W + TAIL, SENT_U32, np.uint32))
    wxo_q8.pack_int8_rows_device(src.ptr + offset, N, K, dst)
    wxo_q8.synchronize()
    got = dst.download(np.uint32, N * W + TAIL)
    assert_bits_equal(got[:N * W], oracle.pack_int8_rows(codes, N, K), f"packInt8Rows N={N} K={K} +{offset}")
    assert np.all(got[N * W:] == SENT_U32), "wrote past the output"
    for b in (src, dst):
        b.free()


def test_pack_int8_rows_exact_size_input_ends_the_buffer():
    """The input is an exactly sized allocation whose byte count is not a
    multiple of 4: the last row's last codes come from a partial dword."""
    for N, K in ((3, 4099), (1, 13), (5, 1021), (4096, 4099)):
        rng = np.random.default_rng(N + K)
        codes = rng.integers(-128, 128, N * K).astype(np.int8)
        src = wxo_q8.DeviceBuffer.from_array(codes)
        W = (K + 3) // 4
        dst = wxo_q8.DeviceBuffer(N * W * 4)
        wxo_q8.pack_int8_rows_device(src, N, K, dst)
        wxo_q8.synchronize()
        assert_bits_equal(dst.download(np.uint32, N * W), oracle.pack_int8_rows(codes, N, K), f"N={N} K={K}")
        src.free()
        dst.free()


def test_spin_holds_the_stream():
    """wxo_spin: the stream's next work starts after the requested time of the
    100 MHz clock, and launches queued behind it run back to back."""
    L = wxo_q8.lib()
    st = wxo_q8.Stream()
    w = wxo_q8.DeviceBuffer.from_array(np.zeros(64 * 4, np.uint32))
    s = wxo_q8.DeviceBuffer.from_array(np.ones(64, np.float32))
    x = wxo_q8.DeviceBuffer.from_array(np.ones(16, np.float32))
    y = wxo_q8.DeviceBuffer(64 * 4)
    wxo_q8.matvec_q8_device(w, s, x, y, 64, 16, 1, st)  # the kernel's first launch (code object load) untimed
    st.synchronize()
    e0, e1, e2 = (wxo_q8.Event(timer=True) for _ in range(3))
    e0.record(st)
    assert L.wxo_spin(300, st.handle) == wxo_q8.WXO_OK
    e1.record(st)
    for _ in range(20):
        wxo_q8.matvec_q8_device(w, s, x, y, 64, 16, 1, st)
    e2.record(st)
    e2.synchronize()
    spun = e0.elapsed_ms(e1) * 1e3
    assert 290.0 <= spun < 5000.0, spun
    assert e1.elapsed_ms(e2) * 1e3 < 20 * 50.0  # 20 small launches, queued: well under 50 us each
    assert np.all(y.download(np.float32, 64) == 0.0)
    st.destroy()


def test_graph_replays_match_eager_issue():
    """A captured sequence (three same-vector projections in one launch, a
    residual projection into the residual stream, a device copy) replayed
    several times, with eager uploads, eager launches and synchronisations
    between the replays: every replay equals the same ops issued directly."""
    rng = np.random.default_rng(21)
    N, K = 2048, 2048
    W = (K + 3) // 4
    ws = [wxo_q8.DeviceBuffer.from_array(rng.integers(0, 2 ** 32, N * W, dtype=np.uint64).astype(np.uint32))
          for _ in range(4)]
    sc = wxo_q8.DeviceBuffer.from_array(rng.uniform(0.001, 0.01, N).astype(np.float32))
    x = wxo_q8.DeviceBuffer(4 * K)
    qkv = wxo_q8.DeviceBuffer(3 * 4 * N)
    resid = wxo_q8.DeviceBuffer(4 * N)
    copy = wxo_q8.DeviceBuffer(4 * N)
    st = wxo_q8.Stream()

    def ops(stream):
        wxo_q8.matvec_q8_multi_device([(ws[i].ptr, sc.ptr, qkv.ptr + 4 * N * i, N) for i in range(3)], x.ptr, K,
                                      stream)
        wxo_q8.matvec_q8_residual_device(ws[3], sc, qkv, resid, resid, N, K, stream)
        wxo_q8._check(wxo_q8.lib().wxo_memcpy_dtod(copy.ptr, resid.ptr, 4 * N, stream.handle))

    g = wxo_q8.Graph.capture(st, lambda: ops(st))
    try:
        for step in range(4):
            xv = rng.standard_normal(K).astype(np.float32)
            r0 = rng.standard_normal(N).astype(np.float32)
            x.upload(xv)
            resid.upload(r0)
            wxo_q8.synchronize()
            g.launch(st)
            st.synchronize()
            got = (qkv.download(np.float32, 3 * N), resid.download(np.float32, N), copy.download(np.float32, N))
            # the same ops issued directly on the same inputs
            resid.upload(r0)
            wxo_q8.synchronize()
            ops(st)
            st.synchronize()
            want = (qkv.download(np.float32, 3 * N), resid.download(np.float32, N), copy.download(np.float32, N))
            for a, b, what in zip(got, want, ("qkv", "residual", "copy")):
                assert_bits_equal(a, b, f"step {step} {what}")
            # eager work of another shape between replays
            wxo_q8.matvec_q8_device(ws[0], sc, x, copy, 1000, K, 1, st)
            st.synchronize()
    finally:
        g.destroy()
        st.destroy()



# ---------------------------------------------------------------- long rows

def test_long_rows_single_vector_and_fused_forms():
    """K = 131075 (128 whole 1 KiB chunks and one word): the single-vector
    kernel's chunk-slot loop far past the sweeps' 20000, with the fused
    residual and FFN epilogues on the same rows."""
    rng = np.random.default_rng(131075)
    N, K = 37, 131075
    w = random_weights(rng, N, K, full_range=True)
    wu = random_weights(rng, N, K, full_range=True)
    s = rng.uniform(1e-4, 1e-2, N).astype(np.float32)
    su = rng.uniform(1e-4, 1e-2, N).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    r = rng.standard_normal(N).astype(np.float32)
    assert_matvec(wxo_q8.matvecQ8(weight=w, scale=s, vector=x, N=N, K=K), w, s, x, N, K)
    assert_residual(wxo_q8.matvecQ8Residual(weight=w, scale=s, vector=x, residual=r, N=N, K=K), w, s, x, r, N, K)
    assert_ffn(wxo_q8.matvecQ8Ffn(weightGate=w, scaleGate=s, weightUp=wu, scaleUp=su, vector=x, N=N, K=K),
               w, s, wu, su, x, N, K)


@pytest.mark.parametrize("M", [3, 8, 16])
def test_long_rows_batched(M):
    """K = 65539 with several vectors: past every matrix-core kernel's LDS
    budget for the vectors' parts, so the VALU kernel's chunk loop runs."""
    rng = np.random.default_rng(65539 + M)
    N, K = 19, 65539
    w = random_weights(rng, N, K, full_range=True)
    s = rng.uniform(1e-4, 1e-2, N).astype(np.float32)
    xs = rng.standard_normal((M, K)).astype(np.float32)
    y = wxo_q8.matvecQ8Batched(weight=w, scale=s, vectors=xs.reshape(-1), N=N, K=K, M=M).reshape(M, N)
    for m in range(M):
        assert_matvec(y[m], w, s, xs[m], N, K)


def test_long_rows_matmul_with_and_without_workspace():
    """matmulQ8 over K = 65539 (1025 steps of 64 codes, 65 accumulator folds):
    the plain plan and the workspace's K split, each within the bar."""
    from test_gpu_prefill import assert_matmul
    rng = np.random.default_rng(40 * 65539)
    N, M, K = 40, 300, 65539
    w = random_weights(rng, M, K, full_range=True)
    s = rng.uniform(1e-4, 1e-2, M).astype(np.float32)
    a = rng.standard_normal(N * K).astype(np.float32)
    ba, bw, bs = (wxo_q8.DeviceBuffer.from_array(v) for v in (a, w, s))
    ws_bytes = wxo_q8.matmul_q8_workspace_bytes()
    ws = wxo_q8.DeviceBuffer(ws_bytes)
    for workspace, nbytes in ((None, 0), (ws, ws_bytes)):
        out = wxo_q8.DeviceBuffer(4 * N * M)
        wxo_q8.matmul_q8_multi_device(ba, [(bw, bs, out, M)], N, K, workspace=workspace, workspace_bytes=nbytes)
        wxo_q8.synchronize()
        assert ("wgsplit" in wxo_q8.last_variant()) == (workspace is not None), wxo_q8.last_variant()
        assert_matmul(out.download(np.float32, N * M), a, w, s, N, M, K)


def test_long_rows_quantize_and_pack():
    """Rows of D = 131075 through the two-pass quantize+pack: codes, scales
    and packed words bit-exact, the absmax in the row's last element."""
    rng = np.random.default_rng(7)
    N, D = 3, 131075
    x = (rng.standard_normal((N, D)) * 0.05).astype(np.float32)
    x[0, D - 1] = 2.5
    want_codes, want_scales = oracle.quantize(x, N, D)
    codes, scales = wxo_q8.quantize(input=x.reshape(-1), N=N, D=D)
    assert_bits_equal(codes, want_codes, "codes")
    assert_bits_equal(scales, want_scales, "scales")
    packed, scales2 = wxo_q8.quantizePackQ8(input=x.reshape(-1), N=N, K=D)
    assert_bits_equal(packed, oracle.pack_q8(want_codes, N, D), "packed words")
    assert_bits_equal(scales2, want_scales, "scales (fused)")


@pytest.mark.parametrize("M", [1, 4])
def test_two_million_short_rows(M):
    """N = 2,000,003 rows of K = 7 (two words, one partial): grids of more than
    100,000 workgroups, the row tail in the last block."""
    rng = np.random.default_rng(2_000_003 + M)
    N, K = 2_000_003, 7
    w = random_weights(rng, N, K, full_range=True)
    s = rng.uniform(1e-3, 1e-1, N).astype(np.float32)
    xs = rng.standard_normal((M, K)).astype(np.float32)
    y = wxo_q8.matvecQ8Batched(weight=w, scale=s, vectors=xs.reshape(-1), N=N, K=K, M=M).reshape(M, N)
    for m in range(M):
        assert_matvec(y[m], w, s, xs[m], N, K)
    x = rng.standard_normal((N, K)).astype(np.float32)
    want_codes, want_scales = oracle.quantize(x, N, K)
    packed, scales = wxo_q8.quantizePackQ8(input=x.reshape(-1), N=N, K=K)
    assert_bits_equal(packed, oracle.pack_q8(want_codes, N, K), "packed words")
    assert_bits_equal(scales, want_scales, "scales")


@pytest.mark.parametrize("M", [5, 16])
def test_ksplit_store_wave_limit(M):
    """The batched k-split kernel's store wave (K <= 1024) keeps its
    workgroup's scales in LDS, up to 1023 tiles of 16 rows per workgroup; one
    more row runs the eight-wave form.  Rows are independent and both forms
    add the same partials in the same order, so the shared rows are
    bit-equal; rows at both ends and a random sample are checked against the
    oracle.  The weight is one random 4096-row block repeated (3.4 GB)."""
    cus = int(re.search(r" cus=(\d+)", wxo_q8.describe()).group(1))
    K, W = 800, 200
    N1 = 1023 * 16 * cus
    N2 = N1 + 20
    rng = np.random.default_rng(N1 + M)
    w = np.tile(random_weights(rng, 4096, K, full_range=True).reshape(4096, W), ((N2 + 4095) // 4096, 1))[:N2]
    w = np.ascontiguousarray(w).reshape(-1)
    s = rng.uniform(1e-3, 1e-1, N2).astype(np.float32)
    xs = rng.standard_normal((M, K)).astype(np.float32)
    y1 = wxo_q8.matvecQ8Batched(weight=w[: N1 * W], scale=s[:N1], vectors=xs.reshape(-1), N=N1, K=K, M=M)
    v1 = wxo_q8.last_variant()
    y2 = wxo_q8.matvecQ8Batched(weight=w, scale=s, vectors=xs.reshape(-1), N=N2, K=K, M=M)
    v2 = wxo_q8.last_variant()
    print(v1, v2, flush=True)
    assert parse_variant(v1)[0] == parse_variant(v2)[0] == "matvec_q8_ksplit"
    assert int(parse_variant(v1)[2]["waves"]) == 9 and int(parse_variant(v2)[2]["waves"]) == 8
    y1 = y1.reshape(M, N1)
    y2 = y2.reshape(M, N2)
    assert_bits_equal(y2[:, :N1], y1, "store-wave form against the eight-wave form")
    rows = np.unique(np.concatenate([np.arange(64), np.arange(N1 - 64, N2), rng.integers(0, N2, 512)]))
    ws = w.reshape(N2, W)[rows].reshape(-1)
    for m in range(M):
        assert_matvec(y2[m][rows], ws, s[rows], xs[m], len(rows), K)


@pytest.mark.parametrize("M", [1, 5])
def test_weight_past_4_gib(M):
    """A 4.6 GB weight (4.5M rows of K = 1024): every kernel addresses its
    block of rows from a 64-bit base, so rows past the first 4 GiB read
    their own words.  The last rows' outputs are bit-equal to a call on those
    rows alone; rows at both ends and a random sample are checked against the
    oracle.  The weight is one random 4096-row block repeated."""
    K, W = 1024, 256
    N = 4_500_000
    rng = np.random.default_rng(4500 + M)
    w = np.tile(random_weights(rng, 4096, K, full_range=True).reshape(4096, W), ((N + 4095) // 4096, 1))[:N]
    w = np.ascontiguousarray(w).reshape(-1)
    s = rng.uniform(1e-3, 1e-1, N).astype(np.float32)
    xs = rng.standard_normal((M, K)).astype(np.float32)
    y = wxo_q8.matvecQ8Batched(weight=w, scale=s, vectors=xs.reshape(-1), N=N, K=K, M=M).reshape(M, N)
    print(wxo_q8.last_variant(), flush=True)
    tail = 100
    yt = wxo_q8.matvecQ8Batched(weight=w[(N - tail) * W:], scale=s[N - tail:], vectors=xs.reshape(-1), N=tail, K=K,
                                M=M).reshape(M, tail)
    if M == 1:  # the same kernel on both calls: the same bits
        assert_bits_equal(y[:, N - tail:], yt, "rows past 4 GiB against a call on them alone")
    rows = np.unique(np.concatenate([np.arange(64), np.arange(N - tail, N), rng.integers(0, N, 512)]))
    ws = w.reshape(N, W)[rows].reshape(-1)
    for m in range(M):
        assert_matvec(y[m][rows], ws, s[rows], xs[m], len(rows), K)


def test_pack_and_quantize_past_4_gib():
    """packInt8Rows with 4.5 GB of codes in and out (1.1M rows of K = 4099:
    the streaming kernel's 64-bit output offsets, rows ending mid-word), and
    quantize+pack of a 4.5 GB f32 matrix (1.1M rows of K = 1024).  Rows at
    both ends and a random sample checked bit for bit against the oracle; the
    inputs are one random 4096-row block repeated."""
    rng = np.random.default_rng(1100)
    N, K = 1_100_000, 4099
    W = (K + 3) // 4
    block = rng.integers(-128, 128, (4096, K)).astype(np.int8)
    codes = np.ascontiguousarray(np.tile(block, ((N + 4095) // 4096, 1))[:N]).reshape(-1)
    assert N * W * 4 > 1 << 32
    packed = wxo_q8.packInt8Rows(codes, N, K).reshape(N, W)
    rows = np.unique(np.concatenate([np.arange(32), np.arange(N - 64, N), rng.integers(0, N, 256)]))
    sub = codes.reshape(N, K)[rows].reshape(-1)
    assert_bits_equal(packed[rows].reshape(-1), oracle.pack_int8_rows(sub, len(rows), K), "packInt8Rows past 4 GiB")
    del codes, packed
    N, K = 1_100_000, 1024
    fblock = (rng.standard_normal((4096, K)) * 0.02).astype(np.float32)
    x = np.ascontiguousarray(np.tile(fblock, ((N + 4095) // 4096, 1))[:N]).reshape(-1)
    assert N * K * 4 > 1 << 32
    pk, sc = wxo_q8.quantizePackQ8(input=x, N=N, K=K)
    rows = np.unique(np.concatenate([np.arange(32), np.arange(N - 64, N), rng.integers(0, N, 256)]))
    want_codes, want_scales = oracle.quantize(x.reshape(N, K)[rows], len(rows), K)
    assert_bits_equal(pk.reshape(N, K // 4)[rows].reshape(-1), oracle.pack_q8(want_codes, len(rows), K),
                      "quantize+pack past 4 GiB")
    assert_bits_equal(sc[rows], want_scales, "scales past 4 GiB")


# ---------------------------------------------------------------- threads

def test_threads_on_their_own_streams():
    """Eight host threads, each on its own stream and buffers, issue the
    library's kernels at the same time (ctypes drops the GIL for every call):
    every result within its bar, every repeat bit-equal to the first, and each
    thread's wxo_last_variant its own kernel's."""
    jobs = []
    for t in range(8):
        rng = np.random.default_rng(900 + t)
        kind = t % 4
        if kind == 0:    # single vector, ragged rows
            N, K, M = 4096, 4099, 1
        elif kind == 1:  # 8 vectors on the k-split kernel
            N, K, M = 20000, 1024, 8
        elif kind == 2:  # prefill GEMM with its own workspace
            N, K, M = 128, 2048, 1000
        else:            # quantize + pack
            N, K, M = 512, 5000, 0
        job = {"kind": kind, "N": N, "K": K, "M": M, "outs": [], "error": None}
        if kind == 3:
            job["x"] = (rng.standard_normal(N * K) * 0.05).astype(np.float32)
        else:
            rows = M if kind == 2 else N
            job["w"] = random_weights(rng, rows, K, full_range=True)
            job["s"] = rng.uniform(1e-3, 5e-2, rows).astype(np.float32)
            job["x"] = rng.standard_normal((N if kind == 2 else M) * K).astype(np.float32)
        jobs.append(job)

    def run(job):
        try:
            st = wxo_q8.Stream()
            kind, N, K, M = job["kind"], job["N"], job["K"], job["M"]
            bx = wxo_q8.DeviceBuffer.from_array(job["x"])
            if kind == 3:
                W = (K + 3) // 4
                bp, bsc = wxo_q8.DeviceBuffer(4 * N * W), wxo_q8.DeviceBuffer(4 * N)
            else:
                bw, bs = wxo_q8.DeviceBuffer.from_array(job["w"]), wxo_q8.DeviceBuffer.from_array(job["s"])
                by = wxo_q8.DeviceBuffer(4 * N * M)
            if kind == 2:
                ws_bytes = wxo_q8.matmul_q8_workspace_bytes()
                ws = wxo_q8.DeviceBuffer(ws_bytes)
            for _ in range(10):
                if kind in (0, 1):
                    wxo_q8.matvec_q8_device(bw, bs, bx, by, N, K, M, stream=st)
                elif kind == 2:
                    wxo_q8.matmul_q8_multi_device(bx, [(bw, bs, by, M)], N, K, stream=st, workspace=ws,
                                                  workspace_bytes=ws_bytes)
                else:
                    wxo_q8.quantize_pack_q8_device(bx, N, K, bp, bsc, stream=st)
                st.synchronize()
                if kind == 3:
                    job["outs"].append((bp.download(np.uint32, N * W), bsc.download(np.float32, N)))
                else:
                    job["outs"].append(by.download(np.float32, N * M))
            job["variant"] = wxo_q8.last_variant()
            st.destroy()
        except Exception as e:  # reported by the main thread
            job["error"] = e

    threads = [threading.Thread(target=run, args=(job,)) for job in jobs]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    heads = {0: "matvec_q8_m1 ", 1: "matvec_q8_ksplit ", 2: "matmul_q8 ", 3: "quantize_row_wg "}
    for job in jobs:
        assert job["error"] is None, job["error"]
        kind, N, K, M = job["kind"], job["N"], job["K"], job["M"]
        assert job["variant"].startswith(heads[kind]), job["variant"]
        first = job["outs"][0]
        for again in job["outs"][1:]:
            if kind == 3:
                assert_bits_equal(again[0], first[0], "packed words on a repeat")
                assert_bits_equal(again[1], first[1], "scales on a repeat")
            else:
                assert_bits_equal(again, first, "output on a repeat")
        if kind == 0:
            assert_matvec(first, job["w"], job["s"], job["x"], N, K)
        elif kind == 1:
            y = first.reshape(M, N)
            xs = job["x"].reshape(M, K)
            for m in range(M):
                assert_matvec(y[m], job["w"], job["s"], xs[m], N, K)
        elif kind == 2:
            from test_gpu_prefill import assert_matmul
            assert_matmul(first, job["x"], job["w"], job["s"], N, M, K)
        else:
            codes, scales = oracle.quantize(job["x"], N, K)
            assert_bits_equal(first[0], oracle.pack_q8(codes, N, K), "packed words")
            assert_bits_equal(first[1], scales, "scales")
