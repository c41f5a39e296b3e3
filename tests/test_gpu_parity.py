"""Parity of the gfx950 path with the oracle, through the C ABI (wxo_q8 / ctypes).

Bars (from the reference's definitions):
  * quantize codes, scales and packed words: bit-exact;
  * matvecQ8 outputs: |y - y_ref| <= 1e-5 * sum_k |s*q*x| + 1e-7 per row
    (oracle.REL, oracle.ABS), y_ref the f64 reference sum.
Shapes follow the reference's own tests (ops/matvec/q8.wgsl.test.ts:48-149,
ops/quantize/wgsl.test.ts, ops/matvec/reference.test.ts) plus every BASELINE
configuration at full size.
"""
import json
import os

import numpy as np
import pytest

import oracle
import wxo_q8
import wxo_workloads as wl

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module", autouse=True)
def device():
    wxo_q8.init()
    print(wxo_q8.describe(), flush=True)


def kat():
    with open(os.path.join(GOLDEN, "kat.json")) as f:
        return json.load(f)


def assert_matvec(got, w, s, x, N, K):
    want = oracle.matvec_q8(w, s, x, N, K)
    bound = oracle.absterm(w, s, x, N, K)
    ok, msg = oracle.check_matvec(got, want, bound)
    assert ok, f"N={N} K={K}: {msg}"


def assert_bits_equal(got, want, what):
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, what
    if got.dtype.kind == "f":
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan), f"{what}: NaN positions differ"
        g, w = got[~nan].view(np.uint32), want[~nan].view(np.uint32)
    else:
        g, w = got, want
    bad = np.flatnonzero(g != w)
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[0]}: got {got.reshape(-1)[bad[0]]!r} want {want.reshape(-1)[bad[0]]!r}"


def random_weights(rng, N, K, full_range=False):
    W = (K + 3) // 4
    if full_range:  # any byte, 0x80 (-128) included
        return rng.integers(0, 2 ** 32, N * W, dtype=np.uint64).astype(np.uint32)
    codes = rng.integers(-127, 128, N * K, dtype=np.int32)
    return oracle.pack_q8(codes, N, K)


# ---------------------------------------------------------------- matvecQ8

@pytest.mark.parametrize("case", kat()["matvec_q8"], ids=lambda c: c["source"].split(" ")[0])
def test_matvec_kat(case):
    N, K = case["N"], case["K"]
    w = oracle.pack_q8(np.array(case["codes"], np.int32), N, K)
    if "pad_patch" in case:
        w[case["pad_patch"]["word"]] |= np.uint32(int(case["pad_patch"]["or"], 16))
    x = np.array(case["vector"], np.float32)
    y = wxo_q8.matvecQ8(weight=w, scale=np.array(case["scale"], np.float32), vector=x[:K], N=N, K=K)
    assert y.tolist() == case["want"]


def code_wave(n, k, phase=0.0):
    return np.round(np.sin(np.arange(n) * k + phase) * 100).astype(np.int32)


def wave(n, k, phase=0.0):
    return (np.sin(np.arange(n) * k + phase) * 1.5).astype(np.float32)


def scale_wave(n):
    return (0.02 * (np.arange(n) + 1) + 0.007).astype(np.float32)


@pytest.mark.parametrize("N,K", [(1, 3), (1, 8), (5, 1024), (3, 1030), (7, 1027), (2, 2600)])
def test_matvec_reference_shapes(N, K):
    # ops/matvec/q8.wgsl.test.ts:48-71 inputs (codeWave / scaleWave / wave).
    w = oracle.pack_q8(code_wave(N * K, 0.37), N, K)
    s = scale_wave(N)
    x = wave(K, 0.11, 0.8)
    assert_matvec(wxo_q8.matvecQ8(weight=w, scale=s, vector=x, N=N, K=K), w, s, x, N, K)


def test_matvec_reads_past_first_pass():
    # ops/matvec/q8.wgsl.test.ts:73-106
    N, K = 3, 1030
    codes = np.zeros((N, K), np.int32)
    x = np.zeros(K, np.float32)
    x[1027], x[K - 1] = 2, -3
    for r in range(N):
        codes[r, 1027] = 1 + r
        codes[r, K - 1] = 2 * (r + 1)
    w = oracle.pack_q8(codes, N, K)
    s = scale_wave(N)
    y = wxo_q8.matvecQ8(weight=w, scale=s, vector=x, N=N, K=K)
    assert_matvec(y, w, s, x, N, K)
    assert np.all(y != 0)


def test_matvec_sentinel_padded_device_buffers():
    # ops/matvec/q8.wgsl.test.ts:108-149: buffers longer than N*W words and K
    # floats, slack filled with sentinels; over-reads would change the answer.
    N, K = 4, 1023
    W = (K + 3) // 4
    codes = np.array([(i // K) % 5 + 1 for i in range(N * K)], np.int32)
    packed = oracle.pack_q8(codes, N, K)
    w = np.concatenate([packed, np.full(256, 0x7F7F7F7F, np.uint32)])
    x = np.concatenate([np.ones(K, np.float32), np.full(256, 1000, np.float32)])
    s = scale_wave(N)
    bw, bs, bx = (wxo_q8.DeviceBuffer.from_array(a) for a in (w, s, x))
    by = wxo_q8.DeviceBuffer(4 * (N + 64))
    by.upload(np.full(N + 64, -7.0, np.float32))
    wxo_q8.matvec_q8_device(bw, bs, bx, by, N, K)
    out = by.download(np.float32, N + 64)
    assert_matvec(out[:N], packed, s, x[:K], N, K)
    assert np.all(out[N:] == -7.0), "wrote past the output"
    for b in (bw, bs, bx, by):
        b.free()
    assert W == 256


@pytest.mark.parametrize("K", [1, 2, 3, 4, 5, 63, 64, 65, 255, 1023, 1024, 1025, 2048, 3072, 4095, 4096, 4099,
                               5632, 8192, 12288, 16384, 16385, 20000])
@pytest.mark.parametrize("N", [1, 17, 33])
def test_matvec_k_sweep(N, K):
    rng = np.random.default_rng(N * 100003 + K)
    w = random_weights(rng, N, K, full_range=(K % 2 == 1))
    s = rng.uniform(0.001, 0.05, N).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    assert_matvec(wxo_q8.matvecQ8(weight=w, scale=s, vector=x, N=N, K=K), w, s, x, N, K)


@pytest.mark.parametrize("K", [1025, 1028, 1040, 2049, 3076, 4097, 4099, 4100, 4112, 4113, 5121, 6150, 7180, 8193,
                               8200, 8208, 8209])
@pytest.mark.parametrize("N", [1, 15, 100, 4097])
def test_matvec_tail_words(N, K):
    # Rows of 1 to 8 whole 1024-code chunks plus 1 to 4 words run without a
    # wave streaming the partial chunk: one extra wave's lanes take the tail
    # words (their 16-byte loads run into the next row, whose codes meet x
    # entries past K).
    # K = 4113 and 8209 (5 tail words) keep the masked partial-chunk wave.
    # Every byte value, pad codes included; row tails at N = 15 and 4097.
    rng = np.random.default_rng(N * 7919 + K)
    w = random_weights(rng, N, K, full_range=True)
    s = rng.uniform(0.001, 0.05, N).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    assert_matvec(wxo_q8.matvecQ8(weight=w, scale=s, vector=x, N=N, K=K), w, s, x, N, K)


@pytest.mark.parametrize("K", [4100, 5000, 5632, 7000, 8192, 9000, 11008, 12288, 16384])
@pytest.mark.parametrize("N", [100, 1000, 4097, 11008])
def test_matvec_one_wave_per_chunk(N, K):
    # 5 to 16 chunks of 1024 codes run one wave per chunk; N spans every
    # rows-per-block choice (16, 8, 4, 2), ragged K and row tails included
    rng = np.random.default_rng(N * 7 + K)
    w = random_weights(rng, N, K, full_range=(K % 2 == 0))
    s = rng.uniform(0.001, 0.05, N).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    assert_matvec(wxo_q8.matvecQ8(weight=w, scale=s, vector=x, N=N, K=K), w, s, x, N, K)


@pytest.mark.parametrize("N", [2, 15, 16, 31, 32, 1000, 4097])
def test_matvec_row_tails(N):
    rng = np.random.default_rng(N)
    K = 4096
    w = random_weights(rng, N, K)
    s = rng.uniform(0.001, 0.05, N).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    assert_matvec(wxo_q8.matvecQ8(weight=w, scale=s, vector=x, N=N, K=K), w, s, x, N, K)


def test_matvec_degenerate():
    # N = 0: nothing; K = 0: y = 0 * s (NaN for non-finite scale), as the reference.
    assert wxo_q8.matvecQ8(weight=np.zeros(0, np.uint32), scale=np.zeros(0, np.float32),
                           vector=np.ones(4, np.float32), N=0, K=4).size == 0
    s = np.array([2.0, -3.0, np.inf, np.nan], np.float32)
    y = wxo_q8.matvecQ8(weight=np.zeros(0, np.uint32), scale=s, vector=np.zeros(0, np.float32), N=4, K=0)
    want = oracle.matvec_q8(np.zeros(0, np.uint32), s, np.zeros(0, np.float32), 4, 0)
    assert_bits_equal(y, want, "K=0")


def test_matvec_nonfinite_scale_and_vector():
    rng = np.random.default_rng(5)
    N, K = 8, 100
    w = random_weights(rng, N, K)
    s = rng.uniform(0.01, 0.02, N).astype(np.float32)
    s[2] = np.inf
    s[3] = np.nan
    x = rng.standard_normal(K).astype(np.float32)
    y = wxo_q8.matvecQ8(weight=w, scale=s, vector=x, N=N, K=K)
    assert_matvec(y, w, s, x, N, K)
    assert np.isnan(y[3])


@pytest.mark.parametrize("N,K,chunks", [
    (1000, 1030, ((0, 333), (333, 1), (334, 666))),  # tail words: extra wave (333, 1) and wave 0 (1000, 666)
    (4096, 4099, ((0, 2500), (2500, 1596))),         # whole: extra wave; chunks: tail words on wave 0
    (5632, 2048, ((0, 2048), (2048, 3584))),         # whole chunks: rows per block 2 (whole), 8 and 2
    (11008, 4096, ((0, 4096), (4096, 6912))),        # rows per block 16, 16 and 16 on different grids
])
def test_matvec_row_chunks_equal_whole(N, K, chunks):
    # llm/engine-q8-resident.ts:1214-1230 / llm/kernels.ts:140-151: a caller may
    # run a projection as row chunks on sub-buffers; each chunk must give the
    # same rows as one whole call, whatever grid and form each call picks.
    rng = np.random.default_rng(9)
    W = (K + 3) // 4
    w = random_weights(rng, N, K)
    s = rng.uniform(0.01, 0.02, N).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    bw, bs, bx = (wxo_q8.DeviceBuffer.from_array(a) for a in (w, s, x))
    whole = wxo_q8.DeviceBuffer(4 * N)
    wxo_q8.matvec_q8_device(bw, bs, bx, whole, N, K)
    parts = wxo_q8.DeviceBuffer(4 * N)
    for start, count in chunks:
        wxo_q8.matvec_q8_device(bw.ptr + 4 * W * start, bs.ptr + 4 * start, bx, parts.ptr + 4 * start, count, K)
    a = whole.download(np.float32, N)
    b = parts.download(np.float32, N)
    assert_matvec(a, w, s, x, N, K)
    assert_bits_equal(b, a, "chunked vs whole")


@pytest.mark.parametrize("N,K,chunks", [(5632, 2048, ((0, 2048), (2048, 3584))),
                                        (4096, 4100, ((0, 1000), (1000, 3096)))])
def test_ffn_row_chunks_equal_whole(N, K, chunks):
    """The fused FFN form, chunked over rows, gives the whole call's bits."""
    rng = np.random.default_rng(11)
    W = (K + 3) // 4
    wg, wu = random_weights(rng, N, K), random_weights(rng, N, K)
    sg, su = (rng.uniform(0.01, 0.02, N).astype(np.float32) for _ in range(2))
    x = rng.standard_normal(K).astype(np.float32)
    b_wg, b_sg, b_wu, b_su, bx = (wxo_q8.DeviceBuffer.from_array(a) for a in (wg, sg, wu, su, x))
    whole = wxo_q8.DeviceBuffer(4 * N)
    wxo_q8.matvec_q8_ffn_device(b_wg, b_sg, b_wu, b_su, bx, whole, N, K)
    parts = wxo_q8.DeviceBuffer(4 * N)
    for start, count in chunks:
        wxo_q8.matvec_q8_ffn_device(b_wg.ptr + 4 * W * start, b_sg.ptr + 4 * start, b_wu.ptr + 4 * W * start,
                                    b_su.ptr + 4 * start, bx, parts.ptr + 4 * start, count, K)
    assert_bits_equal(parts.download(np.float32, N), whole.download(np.float32, N), "FFN chunked vs whole")


@pytest.mark.parametrize("cfg", ["cfg1", "cfg2", "cfg3"])
def test_matvec_baseline_configs(cfg):
    c = wl.make_config(cfg)
    N, K = c["N"], c["K"]
    codes, scales = oracle.quantize(c["w"], N, K)
    w = oracle.pack_q8(codes, N, K)
    y = wxo_q8.matvecQ8(weight=w, scale=scales, vector=c["x"], N=N, K=K)
    assert_matvec(y, w, scales, c["x"], N, K)
    if cfg == "cfg3":
        # outlier rows: absmax set by the x50 element, which alone codes to +-127
        cr = codes.reshape(N, K)
        assert np.all(np.max(np.abs(cr[c["outliers"]]), axis=1) == 127)


def test_matvec_decoder_layer():
    mats, xh, xf = wl.make_decoder_layer()
    for name, N, K, wf in mats:
        codes, scales = oracle.quantize(wf, N, K)
        w = oracle.pack_q8(codes, N, K)
        x = xf if K == 5632 else xh
        assert_matvec(wxo_q8.matvecQ8(weight=w, scale=scales, vector=x, N=N, K=K), w, scales, x, N, K)


# ---------------------------------------------------------------- batched

@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 13, 16, 17, 32])
@pytest.mark.parametrize("N,K", [(37, 64), (100, 1024), (9, 1030), (70, 2048), (21, 4099), (5, 8200), (3, 20000)])
def test_batched_equals_m_calls(M, N, K):
    rng = np.random.default_rng(M * 7919 + N * 31 + K)
    w = random_weights(rng, N, K, full_range=(M % 2 == 1))
    s = rng.uniform(0.001, 0.05, N).astype(np.float32)
    xs = rng.standard_normal((M, K)).astype(np.float32)
    ys = wxo_q8.matvecQ8Batched(weight=w, scale=s, vectors=xs, N=N, K=K, M=M)
    for m in range(M):
        assert_matvec(ys[m], w, s, xs[m], N, K)


@pytest.mark.parametrize("M,K", [(2, 8200), (3, 8200), (2, 13000), (16, 1024), (6, 4096)])
def test_batched_same_sign_long_k(M, K):
    # No cancellation: every term is positive, so y equals sum |s q x| and the
    # bar is relative to y itself; the largest K at which the tile's x parts
    # still fit in LDS gives the longest matrix-core accumulation chain.
    rng = np.random.default_rng(K + M)
    N = 40
    codes = rng.integers(64, 128, size=(N, K)).astype(np.int32)
    w = oracle.pack_q8(codes.reshape(-1), N, K)
    s = rng.uniform(0.5, 1.0, N).astype(np.float32)
    xs = rng.uniform(1.0, 2.0, (M, K)).astype(np.float32)
    ys = wxo_q8.matvecQ8Batched(weight=w, scale=s, vectors=xs, N=N, K=K, M=M)
    for m in range(M):
        assert_matvec(ys[m], w, s, xs[m], N, K)


@pytest.mark.parametrize("N,K,M,kernel", [
    (11008, 2048, 5, "matvec_q8_ksplit"), (11003, 2048, 16, "matvec_q8_ksplit"), (5632, 2048, 12, "matvec_q8_ksplit"),
    (8191, 1900, 24, "matvec_q8_ksplit"), (2048, 2048, 32, "matvec_q8_ksplit"), (2047, 1500, 32, "matvec_q8_ksplit"),
    (8192, 1024, 5, "matvec_q8_ksplit"), (5632, 1000, 8, "matvec_q8_ksplit"), (4096, 1024, 16, "matvec_q8_ksplit"),
    (4100, 800, 12, "matvec_q8_ksplit"),
    # fewer tiles than CUs (one per workgroup, its barrier group half empty), ragged rows
    (1000, 900, 32, "matvec_q8_ksplit"), (33, 1024, 48, "matvec_q8_ksplit"), (17, 1000, 35, "matvec_q8_ksplit"),
    (4096, 2048, 16, "matvec_q8_mv"), (11008, 2048, 4, "matvec_q8_mv"), (2048, 2048, 16, "matvec_q8_mv"),
    (4096, 2048, 32, "matvec_q8_mv"), (4096, 1024, 24, "matvec_q8_mv"), (5632, 768, 16, "matvec_q8_mv"),
])
def test_batched_decoder_sized_weights(N, K, M, kernel):
    # Below 16384 rows the k-split kernel runs where it beats the VALU path
    # (enough rows times vectors for its fixed pass, or 32 vectors in one
    # round of workgroups); ragged rows and K, full-range codes.
    rng = np.random.default_rng(N * 31 + K + M)
    w = random_weights(rng, N, K, full_range=True)
    s = rng.uniform(0.001, 0.05, N).astype(np.float32)
    xs = rng.standard_normal((M, K)).astype(np.float32)
    ys = wxo_q8.matvecQ8Batched(weight=w, scale=s, vectors=xs, N=N, K=K, M=M)
    assert wxo_q8.last_variant().split(" ")[0] == kernel, wxo_q8.last_variant()
    for m in range(M):
        assert_matvec(ys[m], w, s, xs[m], N, K)


@pytest.mark.parametrize("M,K", [(5, 1030), (8, 64), (12, 2048), (13, 4099), (16, 1024), (17, 1500), (32, 520),
                                 (6, 3000), (14, 1000), (16, 768), (13, 1536), (20, 1024), (33, 1000),
                                 (5, 769), (5, 2047), (6, 897), (7, 1024), (8, 1025), (8, 2048), (9, 1100),
                                 (16, 2048), (16, 2047), (18, 900), (21, 1999)])
def test_batched_matrix_core_shapes(M, K):
    # From 16384 rows and 5 vectors the batched call runs on the matrix cores;
    # smaller shapes take the VALU path, which the other batched tests cover.
    # Ragged row tail (N % 16 != 0), ragged K, vector tiles past 16,
    # full-range codes (-128 included).  768 < K <= 2048 runs the k-split
    # kernel: 128 codes per wave (K <= 1024) or 256, vectors packed 5 (h|m|l
    # in one operand), 8 (h|m, l) or 16 per tile (groups on grid y, the last
    # one partial at 18, 21 and 33); K = 769 and 897 leave waves with no codes
    # or a partial slice.  Other K run the x-parts-in-LDS kernels.
    rng = np.random.default_rng(M * 1009 + K)
    N = 16397
    w = random_weights(rng, N, K, full_range=True)
    s = rng.uniform(0.001, 0.05, N).astype(np.float32)
    xs = rng.standard_normal((M, K)).astype(np.float32)
    ys = wxo_q8.matvecQ8Batched(weight=w, scale=s, vectors=xs, N=N, K=K, M=M)
    for m in range(M):
        assert_matvec(ys[m], w, s, xs[m], N, K)


@pytest.mark.parametrize("M,K", [(5, 5376), (16, 1536), (16, 1024), (13, 1536), (16, 2048), (8, 2048), (5, 2048)])
def test_batched_matrix_core_same_sign_long_k(M, K):
    # The longest K whose x parts still fit in LDS for the tile, all terms
    # positive: the matrix cores' longest accumulation chains.
    rng = np.random.default_rng(K + M)
    N = 16400
    codes = rng.integers(64, 128, size=(N, K)).astype(np.int32)
    w = oracle.pack_q8(codes.reshape(-1), N, K)
    s = rng.uniform(0.5, 1.0, N).astype(np.float32)
    xs = rng.uniform(1.0, 2.0, (M, K)).astype(np.float32)
    ys = wxo_q8.matvecQ8Batched(weight=w, scale=s, vectors=xs, N=N, K=K, M=M)
    for m in range(M):
        assert_matvec(ys[m], w, s, xs[m], N, K)


@pytest.mark.parametrize("M,K,N", [(M, K, 37) for M in (2, 4, 8, 12, 16) for K in (1030, 4096)]
                         + [(M, 1030, 16397) for M in (5, 8, 12, 16)] + [(6, 4096, 16397), (16, 1000, 16397),
                                                                         (13, 1500, 16397), (5, 1000, 16397),
                                                                         (8, 1000, 16397), (4, 1000, 32771)])
def test_batched_nonfinite_vectors(M, K, N):
    # Inf and NaN entries reach every row as the reference's f64 sum has them
    # (q * Inf = +-Inf, 0 * Inf = NaN), including NaNs whose payload sits only
    # in the low 16 bits, which a bf16 truncation would turn into infinities
    # (N = 16397 with 5 or more vectors runs on the matrix cores, which split
    # x into bf16 parts).
    rng = np.random.default_rng(M * 13 + K)
    codes = rng.integers(-127, 128, N * K, dtype=np.int32)
    codes[::5] = 0
    w = oracle.pack_q8(codes, N, K)
    s = rng.uniform(0.001, 0.05, N).astype(np.float32)
    xs = rng.standard_normal((M, K)).astype(np.float32)
    bits = xs.view(np.uint32)
    specials = [(0, 5, 0x7F800001), (1, 100, 0xFF800000), (0, K - 1, 0xFF800001), (1, 7, 0x7FC00000),
                (M - 1, 64, 0x7F800000), (M - 1, 65, 0x7FBFFFFF)]
    for m, k, b in specials:
        bits[m, k] = b
    ys = wxo_q8.matvecQ8Batched(weight=w, scale=s, vectors=xs, N=N, K=K, M=M)
    for m in range(M):
        assert_matvec(ys[m], w, s, xs[m], N, K)
    assert np.isnan(ys[0]).all()  # every row meets a NaN in vector 0


@pytest.mark.parametrize("M,K", [(4, 1024), (4, 1500), (3, 1024), (4, 512)])
def test_batched_four_vectors_large_n(M, K):
    # 4 vectors from 32768 rows run on the k-split kernel (5 vectors per tile,
    # one filled with zeros); 3 vectors and K = 512 stay on the VALU path.
    rng = np.random.default_rng(M * 31 + K)
    N = 32771
    w = random_weights(rng, N, K, full_range=True)
    s = rng.uniform(0.001, 0.05, N).astype(np.float32)
    xs = rng.standard_normal((M, K)).astype(np.float32)
    ys = wxo_q8.matvecQ8Batched(weight=w, scale=s, vectors=xs, N=N, K=K, M=M)
    for m in range(M):
        assert_matvec(ys[m], w, s, xs[m], N, K)


@pytest.mark.parametrize("M", [1, 4, 8, 16])
def test_batched_lm_head(M):
    c = wl.make_config("cfg5", M=M)
    N, K = c["N"], c["K"]
    codes, scales = oracle.quantize(c["w"], N, K)
    w = oracle.pack_q8(codes, N, K)
    xs = c["x"].reshape(M, K)
    ys = wxo_q8.matvecQ8Batched(weight=w, scale=scales, vectors=xs, N=N, K=K, M=M)
    rows = np.arange(0, N, 97)  # oracle on a row sample; all M vectors
    W = (K + 3) // 4
    wsub = w.reshape(N, W)[rows].reshape(-1)
    for m in range(M):
        assert_matvec(ys[m][rows], wsub, scales[rows], xs[m], rows.size, K)
    assert np.all(np.isfinite(ys))


# ---------------------------------------------------------------- fused decode forms

def assert_ffn(got, wg, sg, wu, su, x, N, K):
    g, u = oracle.matvec_q8(wg, sg, x, N, K), oracle.matvec_q8(wu, su, x, N, K)
    ok, msg = oracle.check_ffn(got, g, u, oracle.absterm(wg, sg, x, N, K), oracle.absterm(wu, su, x, N, K))
    assert ok, f"N={N} K={K}: {msg}"


def assert_residual(got, w, s, x, r, N, K):
    want = oracle.matvec_q8_residual(w, s, x, r, N, K)
    ok, msg = oracle.check_residual(got, want, oracle.absterm(w, s, x, N, K))
    assert ok, f"N={N} K={K}: {msg}"


@pytest.mark.parametrize("case", kat()["matvec_q8_ffn"], ids=lambda c: c["source"].split(" ")[0])
def test_ffn_kat(case):
    N, K = case["N"], case["K"]
    wg = oracle.pack_q8(np.array(case["gate_codes"], np.int32), N, K)
    wu = oracle.pack_q8(np.array(case["up_codes"], np.int32), N, K)
    y = wxo_q8.matvecQ8Ffn(weightGate=wg, scaleGate=np.array(case["scale_gate"], np.float32), weightUp=wu,
                           scaleUp=np.array(case["scale_up"], np.float32), vector=np.array(case["vector"], np.float32),
                           N=N, K=K)
    assert np.all(np.abs(y.astype(np.float64) - np.array(case["want"])) < case["abs_tol"])


@pytest.mark.parametrize("case", kat()["matvec_q8_residual"], ids=lambda c: c["source"].split(" ")[0])
def test_residual_kat(case):
    N, K = case["N"], case["K"]
    w = oracle.pack_q8(np.array(case["codes"], np.int32), N, K)
    y = wxo_q8.matvecQ8Residual(weight=w, scale=np.array(case["scale"], np.float32),
                                vector=np.array(case["vector"], np.float32),
                                residual=np.array(case["residual"], np.float32), N=N, K=K)
    assert np.all(np.abs(y.astype(np.float64) - np.array(case["want"])) < case["abs_tol"])


FUSED_SHAPES = [(1, 1), (1, 4), (3, 7), (37, 64), (100, 1024), (9, 1030), (70, 2048), (21, 4099), (513, 4096),
                (5, 8200), (3, 20000), (2000, 300), (4097, 1000), (2048, 5632), (700, 7000), (4097, 8192), (4096, 11008),
                (300, 16384), (100, 1028), (4097, 4100), (33, 8208)]


@pytest.mark.parametrize("N,K", FUSED_SHAPES)
def test_ffn_matches_oracle(N, K):
    rng = np.random.default_rng(N * 31 + K + 1)
    wg, wu = random_weights(rng, N, K, full_range=True), random_weights(rng, N, K)
    sg = rng.uniform(0.001, 0.05, N).astype(np.float32)
    su = rng.uniform(0.001, 0.05, N).astype(np.float32)
    x = (3 * rng.standard_normal(K)).astype(np.float32)
    y = wxo_q8.matvecQ8Ffn(weightGate=wg, scaleGate=sg, weightUp=wu, scaleUp=su, vector=x, N=N, K=K)
    assert_ffn(y, wg, sg, wu, su, x, N, K)


@pytest.mark.parametrize("N,K", FUSED_SHAPES)
def test_residual_matches_oracle(N, K):
    rng = np.random.default_rng(N * 37 + K + 2)
    w = random_weights(rng, N, K, full_range=(K % 2 == 1))
    s = rng.uniform(0.001, 0.05, N).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    r = (10 * rng.standard_normal(N)).astype(np.float32)
    y = wxo_q8.matvecQ8Residual(weight=w, scale=s, vector=x, residual=r, N=N, K=K)
    assert_residual(y, w, s, x, r, N, K)


def test_fused_decoder_layer():
    # cfg4 shapes: gate/up [5632, 2048] through the fused FFN; wo [2048, 2048]
    # and down [2048, 5632] through the fused residual add.
    mats, xh, xf = wl.make_decoder_layer()
    packed = {}
    for name, N, K, wf in mats:
        codes, scales = oracle.quantize(wf, N, K)
        packed[name] = (oracle.pack_q8(codes, N, K), scales, N, K)
    wg, sg, N, K = packed["wGate"]
    wu, su, _, _ = packed["wUp"]
    assert_ffn(wxo_q8.matvecQ8Ffn(weightGate=wg, scaleGate=sg, weightUp=wu, scaleUp=su, vector=xh, N=N, K=K),
               wg, sg, wu, su, xh, N, K)
    rng = np.random.default_rng(4)
    for name, x in (("wo", xh), ("wDown", xf)):
        w, s, N, K = packed[name]
        r = rng.standard_normal(N).astype(np.float32)
        assert_residual(wxo_q8.matvecQ8Residual(weight=w, scale=s, vector=x, residual=r, N=N, K=K), w, s, x, r, N, K)


def test_residual_in_place_on_device():
    # the resident engine adds into the residual stream: output == residual
    rng = np.random.default_rng(5)
    N, K = 2048, 2048
    w = random_weights(rng, N, K)
    s = rng.uniform(0.001, 0.05, N).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    r = rng.standard_normal(N).astype(np.float32)
    bw, bs, bx = (wxo_q8.DeviceBuffer.from_array(a) for a in (w, s, x))
    br = wxo_q8.DeviceBuffer.from_array(r)
    wxo_q8.matvec_q8_residual_device(bw, bs, bx, br, br, N, K)
    wxo_q8.synchronize()
    assert_residual(br.download(np.float32, N), w, s, x, r, N, K)
    for b in (bw, bs, bx, br):
        b.free()


def test_fused_k_zero_and_nonfinite():
    N = 5
    w = np.zeros(0, np.uint32)
    sg = np.array([1, 2, np.inf, 0.5, 3], np.float32)
    su = np.array([1, 1, 1, np.nan, 2], np.float32)
    r = np.array([1, -2, 3, 4, np.inf], np.float32)
    y = wxo_q8.matvecQ8Ffn(weightGate=w, scaleGate=sg, weightUp=w, scaleUp=su, vector=np.zeros(0, np.float32), N=N, K=0)
    want = oracle.matvec_q8_ffn(w, sg, w, su, np.zeros(0, np.float32), N, 0)
    assert_bits_equal(y, want, "ffn K=0")
    y = wxo_q8.matvecQ8Residual(weight=w, scale=sg, vector=np.zeros(0, np.float32), residual=r, N=N, K=0)
    assert_bits_equal(y, oracle.matvec_q8_residual(w, sg, np.zeros(0, np.float32), r, N, 0), "residual K=0")
    # non-finite vector entries and scales propagate as in the reference
    rng = np.random.default_rng(6)
    N, K = 40, 300
    wg, wu = random_weights(rng, N, K), random_weights(rng, N, K)
    sg = rng.uniform(0.01, 0.05, N).astype(np.float32)
    su = rng.uniform(0.01, 0.05, N).astype(np.float32)
    sg[3], su[4] = np.inf, np.nan
    x = rng.standard_normal(K).astype(np.float32)
    y = wxo_q8.matvecQ8Ffn(weightGate=wg, scaleGate=sg, weightUp=wu, scaleUp=su, vector=x, N=N, K=K)
    assert_ffn(y, wg, sg, wu, su, x, N, K)
    x[7] = np.inf
    r = rng.standard_normal(N).astype(np.float32)
    y = wxo_q8.matvecQ8Residual(weight=wg, scale=sg, vector=x, residual=r, N=N, K=K)
    assert_residual(y, wg, sg, x, r, N, K)


# ---------------------------------------------------------------- quantize / packQ8

@pytest.mark.parametrize("case", kat()["quantize"], ids=lambda c: c["source"].split(" ")[0])
def test_quantize_kat(case):
    x = np.array(case["input"], np.float32)
    codes, scales = wxo_q8.quantize(input=x, N=1, D=x.size)
    assert codes.tolist() == case["codes"]
    assert int(scales.view(np.uint32)[0]) == int(case["scale_bits"], 16)
    packed, s2 = wxo_q8.quantizePackQ8(input=x, N=1, K=x.size)
    assert_bits_equal(packed, oracle.pack_q8(np.array(case["codes"], np.int32), 1, x.size), "fused words")
    assert_bits_equal(s2, scales, "fused scale")


def test_quantize_reference_fixture():
    from test_oracle import _tiny_q8_pairs
    for name, N, K, w, want_codes, want_scales in _tiny_q8_pairs():
        codes, scales = wxo_q8.quantize(input=w, N=N, D=K)
        assert_bits_equal(codes, want_codes.astype(np.int32), name + " codes")
        assert_bits_equal(scales, want_scales, name + " scales")
        packed, s2 = wxo_q8.quantizePackQ8(input=w, N=N, K=K)
        assert_bits_equal(packed, oracle.pack_int8_rows(want_codes, N, K), name + " packed")
        assert_bits_equal(s2, want_scales, name + " fused scales")
        assert_bits_equal(wxo_q8.packInt8Rows(want_codes, N, K), packed, name + " packInt8Rows")


def edge_rows(rng, N, D):
    from test_oracle import tie_heavy_rows
    x = tie_heavy_rows(rng, N, D)
    x[3] = 0.0
    x[4] = -0.0
    x[5, 7 % D] = np.nan
    x[6, 9 % D] = np.inf
    x[7] = 1e-42
    x[8, 11 % D] = -np.inf
    x[9, 0] = 1.3530999422073364
    if D > 1:
        x[9, 1] = 0.005327165126800537
    x[10] = np.float32(3.4e38)
    x[11, :] = np.float32(1e-45) * np.arange(D)
    return x


def test_quantize_exact_half_ties_after_rounded_product():
    # x = -absmax/2 and +absmax/2: x * (127/absmax) rounds (in f64) to exactly
    # -63.5 / +63.5 while the exact product is not a tie.  Math.round on the
    # rounded product gives -63 and 64; a fused multiply-subtract that skips
    # the product's rounding gets -64 / 63.  (Regression: hipcc contracted
    # x * inverse - floor(...) into one v_fma_f64.)
    rows = np.array([[2.1543185710906982, -1.0771592855453491],
                     [2.5792481899261475, 1.2896240949630737],
                     [1.9307280778884888, 0.9653640389442444]], np.float32)
    codes, _ = wxo_q8.quantize(input=rows, N=3, D=2)
    assert codes.tolist() == [127, -63, 127, 64, 127, 64]
    assert oracle.quantize(rows, 3, 2)[0].tolist() == [127, -63, 127, 64, 127, 64]
    packed, _ = wxo_q8.quantizePackQ8(input=rows, N=3, K=2)
    assert packed.tolist() == [0x0000C17F, 0x0000407F, 0x0000407F]


@pytest.mark.parametrize("D", [1, 3, 4, 5, 64, 300, 517, 1023, 2048, 4096, 4099, 5632, 6144, 8000, 8192, 9000, 20001])
def test_quantize_edges_bit_exact(D):
    rng = np.random.default_rng(D)
    N = 24
    x = edge_rows(rng, N, D)
    want_codes, want_scales = oracle.quantize(x, N, D)
    codes, scales = wxo_q8.quantize(input=x, N=N, D=D)
    assert_bits_equal(codes, want_codes, f"codes D={D}")
    assert_bits_equal(scales, want_scales, f"scales D={D}")
    packed, s2 = wxo_q8.quantizePackQ8(input=x, N=N, K=D)
    assert_bits_equal(packed, oracle.pack_q8(want_codes, N, D), f"packed D={D}")
    assert_bits_equal(s2, want_scales, f"fused scales D={D}")


def test_quantize_decoder_layer_bit_exact():
    mats, _, _ = wl.make_decoder_layer()
    for name, N, K, wf in mats:
        want_codes, want_scales = oracle.quantize(wf, N, K)
        packed, scales = wxo_q8.quantizePackQ8(input=wf, N=N, K=K)
        assert_bits_equal(packed, oracle.pack_q8(want_codes, N, K), name + " packed")
        assert_bits_equal(scales, want_scales, name + " scales")
    name, N, K, wf = mats[-1]
    codes, scales = wxo_q8.quantize(input=wf, N=N, D=K)
    assert_bits_equal(codes, oracle.quantize(wf, N, K)[0], "wDown codes")


@pytest.mark.parametrize("N,K", [(1, 1), (3, 4), (5, 7), (7, 1027), (64, 4099), (2, 2), (300, 64)])
def test_pack_bit_exact(N, K):
    rng = np.random.default_rng(N * 17 + K)
    codes = rng.integers(-300, 300, N * K, dtype=np.int32)
    assert_bits_equal(wxo_q8.packQ8(codes=codes, N=N, K=K), oracle.pack_q8(codes, N, K), "packQ8")
    i8 = rng.integers(-128, 128, N * K).astype(np.int8)
    assert_bits_equal(wxo_q8.packInt8Rows(i8, N, K), oracle.pack_int8_rows(i8, N, K), "packInt8Rows")


@pytest.mark.parametrize("case", kat()["pack_q8"], ids=lambda c: c["source"].split(" ")[0])
def test_pack_kat(case):
    words = wxo_q8.packQ8(codes=np.array(case["codes"], np.int32), N=case["N"], K=case["K"])
    assert [f"0x{w:08x}" for w in words.tolist()] == case["words"]


def test_round_trip_full_size():
    # quantize -> packQ8 -> matvecQ8 on the GPU equals the oracle pipeline
    # (cfg2 shape): codes/scales bit-exact, outputs within tolerance.
    c = wl.make_config("cfg2")
    N, K = c["N"], c["K"]
    packed, scales = wxo_q8.quantizePackQ8(input=c["w"], N=N, K=K)
    codes, want_scales = oracle.quantize(c["w"], N, K)
    assert_bits_equal(packed, oracle.pack_q8(codes, N, K), "cfg2 packed")
    assert_bits_equal(scales, want_scales, "cfg2 scales")
    y = wxo_q8.matvecQ8(weight=packed, scale=scales, vector=c["x"], N=N, K=K)
    assert_matvec(y, packed, scales, c["x"], N, K)
