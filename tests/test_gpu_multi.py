"""wxo_matvec_q8_multi: several projections of one vector in one launch, the
form the resident decode takes for wq/wk/wv (llm/engine-q8-resident.ts:1843-1845)
and the lm_head chunks (:1869).  Every output must meet the matvecQ8 bar
against the oracle (|y - y_ref| <= 1e-5 * sum_k |s q x| + 1e-7), the same
as separate wxo_matvec_q8 calls, and nothing outside the outputs is written.
"""
import numpy as np
import pytest

import oracle
import wxo_q8
import wxo_workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    wxo_q8.init()


def random_weights(rng, N, K):
    return oracle.pack_q8(rng.integers(-127, 128, N * K, dtype=np.int32), N, K)


def assert_matvec(got, w, s, x, N, K, what):
    ok, msg = oracle.check_matvec(got, oracle.matvec_q8(w, s, x, N, K), oracle.absterm(w, s, x, N, K))
    assert ok, f"{what} N={N} K={K}: {msg}"


def run_multi(rng, Ns, K, guard=64):
    """Projections Ns of one vector; outputs packed into one buffer with
    `guard` sentinel floats around each, to catch writes past a projection."""
    x = rng.standard_normal(K).astype(np.float32)
    mats = [(random_weights(rng, N, K), rng.uniform(0.001, 0.05, N).astype(np.float32)) for N in Ns]
    bx = wxo_q8.DeviceBuffer.from_array(x)
    bufs = [(wxo_q8.DeviceBuffer.from_array(w) if w.size else None,
             wxo_q8.DeviceBuffer.from_array(s) if s.size else None) for w, s in mats]
    offsets, total = [], guard
    for N in Ns:
        offsets.append(total)
        total += N + guard
    sentinel = np.float32(-7.25e30)
    by = wxo_q8.DeviceBuffer.from_array(np.full(total, sentinel, np.float32))
    projs = [(bw.ptr if bw else 0, bs.ptr if bs else 0, by.ptr + 4 * off, N)
             for (bw, bs), off, N in zip(bufs, offsets, Ns)]
    wxo_q8.matvec_q8_multi_device(projs, bx, K)
    wxo_q8.synchronize()
    y = by.download(np.float32, total)
    outside = np.ones(total, bool)
    for (w, s), off, N in zip(mats, offsets, Ns):
        assert_matvec(y[off:off + N], w, s, x, N, K, f"projection of {N} rows")
        outside[off:off + N] = False
    assert np.all(y[outside] == sentinel), "a launch wrote outside its outputs"
    for bw, bs in bufs:
        for b in (bw, bs):
            if b:
                b.free()
    bx.free()
    by.free()
    return mats, x, y, offsets


# K over every vector-slice class of the single-vector kernel (1, 2, 3, 4,
# <= 8, <= 16 and > 16 chunks of 1024 codes), ragged ends included.
@pytest.mark.parametrize("K", [3, 1000, 2048, 3000, 4096, 4099, 8000, 11008, 20000])
def test_multi_matches_oracle(K):
    rng = np.random.default_rng(K)
    run_multi(rng, (300, 17, 1, 64), K)


@pytest.mark.parametrize("Ns", [(5,), (16, 16), (2048, 512, 512), (0, 33, 0, 7), (9, 1, 130, 0, 77, 3, 40)])
def test_multi_projection_counts(Ns):
    # one projection, the engine's GQA shape, empty projections, and more than
    # the four a launch takes (run four at a time)
    rng = np.random.default_rng(len(Ns))
    run_multi(rng, Ns, 2048 if max(Ns) >= 512 else 1030)


def test_multi_cfg4_qkv_and_lm_head_chunks():
    # cfg4's wq/wk/wv (2048 x 2048 each) on one normalised vector
    mats, xh, _ = wl.make_decoder_layer()
    qkv = []
    for name, N, K, wf in mats:
        if name in ("wq", "wk", "wv"):
            codes, scales = oracle.quantize(wf, N, K)
            qkv.append((oracle.pack_q8(codes, N, K), scales, N))
    K = 2048
    bx = wxo_q8.DeviceBuffer.from_array(xh)
    bufs = [(wxo_q8.DeviceBuffer.from_array(w), wxo_q8.DeviceBuffer.from_array(s), wxo_q8.DeviceBuffer(4 * N))
            for w, s, N in qkv]
    wxo_q8.matvec_q8_multi_device([(bw, bs, by, N) for (bw, bs, by), (_, _, N) in zip(bufs, qkv)], bx, K)
    for (bw, bs, by), (w, s, N) in zip(bufs, qkv):
        assert_matvec(by.download(np.float32, N), w, s, xh, N, K, "cfg4 qkv")
        for b in (bw, bs, by):
            b.free()
    bx.free()
    # an lm_head of 151936 rows at K = 1024 in the engine's 65535-row chunks
    # (llm/engine-q8-resident.ts:1214-1230): chunks are sub-ranges of one weight
    rng = np.random.default_rng(11)
    N, K = 151936, 1024
    W = K // 4
    w = random_weights(rng, N, K)
    s = rng.uniform(0.001, 0.02, N).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    bw, bs, bx = (wxo_q8.DeviceBuffer.from_array(a) for a in (w, s, x))
    by = wxo_q8.DeviceBuffer(4 * N)
    chunks = [(0, 65535), (65535, 65535), (131070, N - 131070)]
    wxo_q8.matvec_q8_multi_device([(bw.ptr + 4 * W * r0, bs.ptr + 4 * r0, by.ptr + 4 * r0, n) for r0, n in chunks],
                                  bx, K)
    assert_matvec(by.download(np.float32, N), w, s, x, N, K, "lm_head chunks")
    for b in (bw, bs, bx, by):
        b.free()


def test_multi_k_zero_and_nonfinite():
    # K = 0: y = 0 * s for each projection (NaN for a non-finite scale)
    s0 = np.array([1.0, np.inf, 2.0], np.float32)
    s1 = np.array([np.nan, 0.5], np.float32)
    b0, b1 = wxo_q8.DeviceBuffer.from_array(s0), wxo_q8.DeviceBuffer.from_array(s1)
    y0, y1 = wxo_q8.DeviceBuffer(12), wxo_q8.DeviceBuffer(8)
    dummy = wxo_q8.DeviceBuffer(16)
    wxo_q8.matvec_q8_multi_device([(dummy, b0, y0, 3), (dummy, b1, y1, 2)], dummy, 0)
    wxo_q8.synchronize()
    np.testing.assert_array_equal(y0.download(np.float32, 3), np.float32(0) * s0)
    np.testing.assert_array_equal(y1.download(np.float32, 2), np.float32(0) * s1)
    # Inf / NaN in the vector reach every projection as in separate calls
    rng = np.random.default_rng(3)
    K = 2050
    x = rng.standard_normal(K).astype(np.float32)
    x[7], x[2049] = np.inf, np.nan
    ws = [random_weights(rng, N, K) for N in (40, 9)]
    ss = [rng.uniform(0.01, 0.02, N).astype(np.float32) for N in (40, 9)]
    bx = wxo_q8.DeviceBuffer.from_array(x)
    bufs = [(wxo_q8.DeviceBuffer.from_array(w), wxo_q8.DeviceBuffer.from_array(s), wxo_q8.DeviceBuffer(4 * len(s)))
            for w, s in zip(ws, ss)]
    wxo_q8.matvec_q8_multi_device([(bw, bs, by, len(s)) for (bw, bs, by), s in zip(bufs, ss)], bx, K)
    for (bw, bs, by), w, s in zip(bufs, ws, ss):
        N = len(s)
        got = by.download(np.float32, N)
        one = wxo_q8.DeviceBuffer(4 * N)
        wxo_q8.matvec_q8_device(bw, bs, bx, one, N, K)
        want = one.download(np.float32, N)
        np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
        np.testing.assert_array_equal(got[~np.isnan(got)], want[~np.isnan(want)])
        for b in (bw, bs, by, one):
            b.free()
    for b in (b0, b1, y0, y1, dummy, bx):
        b.free()


def test_multi_rejects_overlapping_outputs():
    bw = wxo_q8.DeviceBuffer(4 * 64 * 16)
    bs = wxo_q8.DeviceBuffer(4 * 64)
    bx = wxo_q8.DeviceBuffer(4 * 64)
    by = wxo_q8.DeviceBuffer(4 * 128)
    with pytest.raises(wxo_q8.WxoError, match="overlap"):
        wxo_q8.matvec_q8_multi_device([(bw, bs, by, 64), (bw, bs, by.ptr + 4 * 63, 64)], bx, 64)
    with pytest.raises(wxo_q8.WxoError, match="overlaps the vector"):
        wxo_q8.matvec_q8_multi_device([(bw, bs, bx, 64)], bx, 64)
    for b in (bw, bs, bx, by):
        b.free()
