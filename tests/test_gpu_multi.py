"""Several operations in one launch.

wxo_matvec_q8_multi: several projections of one vector, the form the resident
decode takes for wq/wk/wv (llm/engine-q8-resident.ts:1843-1845) and the
lm_head chunks (:1869).  Every output must meet the matvecQ8 bar against the
oracle (|y - y_ref| <= 1e-5 * sum_k |s q x| + 1e-7), the same as separate
wxo_matvec_q8 calls, and nothing outside the outputs is written.

wxo_quantize_pack_q8_multi: quantize + packQ8 of several matrices with one K;
every matrix bit-exact to the oracle's quantize + packQ8 of it alone.
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
@pytest.mark.parametrize("K", [3, 1000, 2048, 3000, 4096, 4099, 5632, 7000, 8000, 11008, 20000])
def test_multi_matches_oracle(K):
    rng = np.random.default_rng(K)
    run_multi(rng, (300, 17, 1, 64), K)


@pytest.mark.parametrize("Ns,K", [((5,), 1030), ((16, 16), 1030), ((2048, 512, 512), 2048), ((0, 33, 0, 7), 1030),
                                  ((9, 1, 130, 0, 77, 3, 40), 1030), ((4096, 1024, 1024), 5632),
                                  ((2048, 2048, 2048), 8192), ((4096, 1024, 1024), 11008)])
def test_multi_projection_counts(Ns, K):
    # one projection, the engine's GQA shape, empty projections, more than
    # the four a launch takes (run four at a time), and 5 to 8 chunks per row
    # (one wave per chunk) at sizes that pick 16 and 8 rows per block
    rng = np.random.default_rng(len(Ns))
    run_multi(rng, Ns, K)


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
    with np.errstate(invalid="ignore"):  # 0 * inf is the NaN expected here
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


# ------------------------------------------------ quantize + packQ8 of several matrices

def quantize_multi(mats, K):
    """mats: list of f32 arrays [N, K]; returns [(packed, scales)] from one multi call."""
    bufs = []
    for a in mats:
        N = a.shape[0]
        bufs.append((wxo_q8.DeviceBuffer.from_array(a.reshape(-1)) if a.size else None, N,
                     wxo_q8.DeviceBuffer(max(4, N * ((K + 3) // 4) * 4)), wxo_q8.DeviceBuffer(max(4, 4 * N))))
    wxo_q8.quantize_pack_q8_multi_device([(b[0].ptr if b[0] else 0, b[1], b[2], b[3]) for b in bufs], K)
    wxo_q8.synchronize()
    out = []
    for (bi, N, bp, bs) in bufs:
        out.append((bp.download(np.uint32, N * ((K + 3) // 4)), bs.download(np.float32, N)))
        for b in (bi, bp, bs):
            if b:
                b.free()
    return out


@pytest.mark.parametrize("K,Ns", [(2048, (2048, 2048, 2048, 2048, 5632, 5632)), (5632, (2048, 1)),
                                  (4099, (7, 0, 300, 1)), (300, (5, 9)), (1030, (3,) * 11), (40000, (2, 3))])
def test_quantize_pack_multi_bit_exact(K, Ns):
    # every matrix equals the oracle's quantize + packQ8 of it alone, bit for
    # bit: cfg4's six K = 2048 matrices, ragged K, an empty matrix, short rows
    # (one launch per matrix), more than 8 matrices, rows read twice (K > 8192)
    rng = np.random.default_rng(K + len(Ns))
    mats = []
    for i, N in enumerate(Ns):
        a = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        if N > 2:
            a[1, :] = 0.0                      # all-zero row: scale 1, codes 0
            a[2, K // 2] = np.float32(3.5)    # outlier row
        mats.append(a)
    got = quantize_multi(mats, K)
    for a, (packed, scales) in zip(mats, got):
        N = a.shape[0]
        codes, want_scales = oracle.quantize(a.reshape(-1), N, K)
        want_packed = oracle.pack_q8(codes, N, K)
        np.testing.assert_array_equal(packed, want_packed)
        np.testing.assert_array_equal(scales.view(np.uint32), want_scales.view(np.uint32))


def test_quantize_pack_multi_rejects_overlap():
    a = wxo_q8.DeviceBuffer(4 * 4 * 512)
    p = wxo_q8.DeviceBuffer(4 * 512 * 2)
    s = wxo_q8.DeviceBuffer(64)
    with pytest.raises(wxo_q8.WxoError, match="overlap the input"):
        wxo_q8.quantize_pack_q8_multi_device([(a, 4, a, s)], 512)
    with pytest.raises(wxo_q8.WxoError, match="outputs of matrices 0 and 1 overlap"):
        wxo_q8.quantize_pack_q8_multi_device([(a, 2, p, s), (a.ptr + 2 * 512 * 4, 2, p.ptr + 4, s.ptr + 32)], 512)
    for b in (a, p, s):
        b.free()
