"""Parity of the gfx950 prefill-side ops with the oracle, through the C ABI.

  * matmulQ8 (ops/matmul/reference.ts:124-137): |y - y_ref| <= 1e-5 * sum_k
    |a * fround(q * s)| + 1e-7 per output element, y_ref the reference's f64
    sum of per-term dequantized products.  That bar is tighter than the
    reference's own GPU test tolerance (rel 1e-4 or abs 6e-4,
    ops/matmul/q8.wgsl.test.ts:33); shapes follow that file and
    q8-edges.wgsl.test.ts, plus tile-boundary sweeps and the decoder layer's
    projections at a 512-token prompt.
  * dequantizePackedQ8, dequantTranspose, gatherDequantRows: bit-exact
    (ops/dequant_transpose/wgsl.test.ts:37 holds its kernel to rel 0, abs 0).
"""
import json
import math
import os

import numpy as np
import pytest

import oracle
import wxo_q8

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module", autouse=True)
def device():
    wxo_q8.init()


def kat():
    with open(os.path.join(GOLDEN, "kat.json")) as f:
        return json.load(f)


def assert_bits_equal(got, want, what):
    got = np.asarray(got).reshape(-1)
    want = np.asarray(want).reshape(-1)
    assert got.shape == want.shape, what
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[0]}: got {got[bad[0]]!r} want {want[bad[0]]!r}"


def assert_matmul(got, a, w, s, N, M, K, rows=None):
    """Checks output rows `rows` (all by default) against the oracle."""
    got = np.asarray(got).reshape(N, M)
    rows = np.arange(N) if rows is None else np.asarray(rows)
    asub = np.ascontiguousarray(np.asarray(a, np.float32).reshape(N, K)[rows])
    want = oracle.matmul_q8(asub, w, s, len(rows), M, K)
    bound = oracle.matmul_absterm(asub, w, s, len(rows), M, K)
    ok, msg = oracle.check_matvec(got[rows].reshape(-1), want.reshape(-1), bound.reshape(-1))
    assert ok, f"N={N} M={M} K={K}: {msg}"


def sin_wave(n, k, mul):
    return np.array([math.sin(i * k) * mul for i in range(n)], dtype=np.float32)


def code_wave(n, k):
    return np.array([int(oracle.js_round(math.sin(i * k) * 100)) for i in range(n)], dtype=np.int32)


def scale_wave(n):
    return np.array([0.02 * (i + 1) + 0.007 for i in range(n)], dtype=np.float32)


# ---------------------------------------------------------------- matmulQ8

def test_matmul_hand_kat():
    c = kat()["matmul_q8"][1]
    w = oracle.pack_q8(np.array(c["codes"], np.int32), c["M"], c["K"])
    y = wxo_q8.matmulQ8(a=np.array(c["a"], np.float32), weight=w, scale=np.array(c["scale"], np.float32),
                        N=c["N"], M=c["M"], K=c["K"])
    assert y.reshape(-1).tolist() == c["want"]


@pytest.mark.parametrize("shape", kat()["matmul_q8"][0]["shapes"], ids=lambda s: "x".join(map(str, s)))
def test_matmul_reference_shapes(shape):
    N, M, K = shape
    a = sin_wave(N * K, 0.37, 1.5)
    w = oracle.pack_q8(code_wave(M * K, 0.19), M, K)
    s = scale_wave(M)
    y = wxo_q8.matmulQ8(a=a, weight=w, scale=s, N=N, M=M, K=K)
    if K == 0:
        assert np.array_equal(y, np.zeros((N, M), np.float32))
    assert_matmul(y, a, w, s, N, M, K)


def test_matmul_does_not_read_past_a_ragged_row():
    # q8-edges.wgsl.test.ts:29-74: K = 19, sentinel words after the weight
    N, M, K = 5, 7, 19
    a = sin_wave(N * K, 0.41, 1.5)
    w = oracle.pack_q8(code_wave(M * K, 0.23), M, K)
    padded = np.concatenate([w, np.full(64, 0x7F7F7F7F, np.uint32)])
    s = scale_wave(M)
    y = wxo_q8.matmulQ8(a=a, weight=padded, scale=s, N=N, M=M, K=K)
    assert_matmul(y, a, w, s, N, M, K)


def test_matmul_own_scale_per_feature():
    # q8-edges.wgsl.test.ts:110-139: identical code rows, scales 0.03 and 0.11
    N, M, K = 2, 2, 12
    shared = code_wave(K, 0.27)
    w = oracle.pack_q8(np.concatenate([shared, shared]), M, K)
    a = sin_wave(N * K, 0.5, 1.5)
    s = np.array([0.03, 0.11], np.float32)
    y = wxo_q8.matmulQ8(a=a, weight=w, scale=s, N=N, M=M, K=K)
    assert_matmul(y, a, w, s, N, M, K)
    assert not np.allclose(y[:, 0], y[:, 1])


def test_matmul_writes_nothing_past_the_output():
    # q8-edges.wgsl.test.ts:76-108 (M = TILE + 1), on device buffers with a
    # sentinel after the output and in the pad lanes of the weight
    rng = np.random.default_rng(1)
    for N, M, K in [(4, 17, 8), (65, 129, 70), (1, 3, 5)]:
        a = rng.standard_normal(N * K).astype(np.float32)
        w = oracle.pack_q8(rng.integers(-128, 128, M * K).astype(np.int32), M, K)
        s = rng.uniform(0.01, 0.1, M).astype(np.float32)
        da = wxo_q8.DeviceBuffer.from_array(a)
        dw = wxo_q8.DeviceBuffer.from_array(w)
        ds = wxo_q8.DeviceBuffer.from_array(s)
        sentinel = np.full(N * M + 256, 12345.0, np.float32)
        dy = wxo_q8.DeviceBuffer.from_array(sentinel)
        wxo_q8.matmul_q8_device(da, dw, ds, dy, N, M, K)
        out = dy.download(np.float32, N * M + 256)
        assert np.all(out[N * M:] == 12345.0), (N, M, K)
        assert_matmul(out[:N * M], a, w, s, N, M, K)


@pytest.mark.parametrize("K", [1, 3, 4, 5, 63, 64, 65, 127, 255, 256, 257, 1030])
@pytest.mark.parametrize("N,M", [(1, 1), (63, 31), (64, 64), (65, 127), (130, 129), (7, 300)])
def test_matmul_tile_boundaries(N, M, K):
    rng = np.random.default_rng(N * 7919 + M * 31 + K)
    a = rng.standard_normal(N * K).astype(np.float32)
    w = rng.integers(0, 2 ** 32, M * ((K + 3) // 4), dtype=np.uint64).astype(np.uint32)  # any byte, -128 included
    s = rng.uniform(-0.05, 0.05, M).astype(np.float32)
    y = wxo_q8.matmulQ8(a=a, weight=w, scale=s, N=N, M=M, K=K)
    assert_matmul(y, a, w, s, N, M, K)


@pytest.mark.parametrize("N,M,K", [(3, 5, 4097), (65, 70, 4100), (64, 129, 5000), (7, 33, 8191), (130, 64, 6000)])
def test_matmul_long_ragged_k(N, M, K):
    # K > 4096 with 64-row tiles runs 128-code steps: their ragged last step
    rng = np.random.default_rng(N + M + K)
    a = rng.standard_normal(N * K).astype(np.float32)
    w = rng.integers(0, 2 ** 32, M * ((K + 3) // 4), dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(-0.05, 0.05, M).astype(np.float32)
    y = wxo_q8.matmulQ8(a=a, weight=w, scale=s, N=N, M=M, K=K)
    assert_matmul(y, a, w, s, N, M, K)


@pytest.mark.parametrize("N,M,K", [(N, M, K) for N in (1, 2, 5, 8, 16, 17, 31, 32, 33) for M, K in ((300, 1030), (20000, 520))])
def test_matmul_small_token_counts(N, M, K):
    # up to 32 tokens run on the batched single-vector kernels (VALU, or the
    # matrix cores from 5 tokens on 16384+ rows), from 33 on the GEMM
    rng = np.random.default_rng(N * 131 + M + K)
    a = rng.standard_normal(N * K).astype(np.float32)
    w = rng.integers(0, 2 ** 32, M * ((K + 3) // 4), dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(-0.05, 0.05, M).astype(np.float32)
    y = wxo_q8.matmulQ8(a=a, weight=w, scale=s, N=N, M=M, K=K)
    assert_matmul(y, a, w, s, N, M, K)


@pytest.mark.parametrize("N,M,K", [(400, 3000, 300), (450, 4096, 1030), (200, 700, 2061), (40, 64, 64)])
def test_matmul_kernel_variants(N, M, K):
    # every GEMM form: 64-row tiles with one K group (more tiles than CUs) and
    # with two (the K steps split in halves, an odd count included), 128-row
    # tiles with two K groups (exactly one tile per CU), one K step
    rng = np.random.default_rng(N + M + K)
    a = rng.standard_normal(N * K).astype(np.float32)
    w = rng.integers(0, 2 ** 32, M * ((K + 3) // 4), dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(-0.05, 0.05, M).astype(np.float32)
    y = wxo_q8.matmulQ8(a=a, weight=w, scale=s, N=N, M=M, K=K)
    assert_matmul(y, a, w, s, N, M, K)


@pytest.mark.parametrize("N", [70, 8])
def test_matmul_nonfinite_activations(N):
    rng = np.random.default_rng(2)
    M, K = 40, 200
    a = rng.standard_normal(N * K).astype(np.float32)
    a[3] = np.inf                     # token 0
    a[K + 5] = -np.inf                # token 1
    a[2 * K + 7] = np.nan             # token 2
    a[3 * K + 1] = np.uint32(0x7F800001).view(np.float32)  # token 3: a NaN whose top bits read as Inf
    a[4 * K + 2], a[4 * K + 9] = np.inf, -np.inf  # token 4: Inf - Inf
    a[5 * K:6 * K] = 1e-40            # token 5: subnormal row
    codes = rng.integers(1, 128, M * K).astype(np.int32)  # no zero code: Inf * q stays infinite
    codes[::3] *= -1
    w = oracle.pack_q8(codes, M, K)
    s = rng.uniform(0.01, 0.1, M).astype(np.float32)
    y = wxo_q8.matmulQ8(a=a, weight=w, scale=s, N=N, M=M, K=K)
    assert_matmul(y, a, w, s, N, M, K)
    assert np.isnan(y[3]).all() and np.isnan(y[2]).all() and np.isinf(y[0]).all()


@pytest.mark.parametrize("K", [4096, 11008])
def test_matmul_same_sign_long_k(K):
    # all terms positive: no cancellation hides accumulated rounding
    rng = np.random.default_rng(K)
    N, M = 64, 128
    a = rng.uniform(0.0, 2.0, N * K).astype(np.float32)
    w = oracle.pack_q8(rng.integers(0, 128, M * K).astype(np.int32), M, K)
    s = rng.uniform(0.001, 0.01, M).astype(np.float32)
    y = wxo_q8.matmulQ8(a=a, weight=w, scale=s, N=N, M=M, K=K)
    assert_matmul(y, a, w, s, N, M, K, rows=np.arange(0, N, 9))


def test_matmul_k_zero_gives_zeros():
    s = np.array([np.inf, np.nan, 1.0], np.float32)
    y = wxo_q8.matmulQ8(a=np.zeros(0, np.float32), weight=np.zeros(0, np.uint32), scale=s, N=4, M=3, K=0)
    assert np.array_equal(y, np.zeros((4, 3), np.float32)) and not np.signbit(y).any()


@pytest.mark.parametrize("M,K", [(2048, 2048), (5632, 2048), (2048, 5632)])
def test_matmul_prefill_layer_projection(M, K):
    # one decoder layer's projections (hidden 2048, FFN 5632) on a 512-token
    # prompt, W ~ N(0, 0.02) quantized by the product; a sample of tokens is
    # checked against the oracle (each output row depends on its token only)
    N = 512
    rng = np.random.default_rng(M + K)
    wf = (rng.standard_normal(M * K, dtype=np.float32) * np.float32(0.02))
    w, s = wxo_q8.quantizePackQ8(input=wf, N=M, K=K)
    a = rng.standard_normal(N * K, dtype=np.float32)
    y = wxo_q8.matmulQ8(a=a, weight=w, scale=s, N=N, M=M, K=K)
    assert_matmul(y, a, w, s, N, M, K, rows=[0, 1, 63, 64, 200, 511])


@pytest.mark.parametrize("N,K,Ms", [
    (512, 2048, (2048, 2048, 2048)),       # a prompt's q, k, v: one launch
    (512, 2048, (5632, 5632)),             # gate and up
    (100, 2048, (2048, 256, 256)),         # grouped-query k and v
    (33, 1000, (1000, 37, 3000)),          # ragged rows per projection, ragged K
    (70, 4099, (130, 64, 1, 200, 65)),     # five projections: two launches
    (64, 64, (64, 0, 16)),                 # an empty projection is skipped
    (8, 520, (300, 20000)),                # up to 32 tokens: the batched path per projection
])
def test_matmul_multi_projection(N, K, Ms):
    """Several weights on the same activations in one launch: every output
    within the matmulQ8 bound of the oracle, nothing written outside them."""
    rng = np.random.default_rng(N + K + len(Ms))
    a = rng.standard_normal(N * K).astype(np.float32)
    ba = wxo_q8.DeviceBuffer.from_array(a)
    W = (K + 3) // 4
    host, bufs = [], []
    for M in Ms:
        codes = rng.integers(-128, 128, (M, K)).astype(np.int32)
        w = oracle.pack_q8(codes.reshape(-1), M, K) if M else np.zeros(1, np.uint32)
        s = rng.uniform(0.001, 0.05, max(M, 1)).astype(np.float32)
        out = wxo_q8.DeviceBuffer(4 * (N * M + 64))
        out.upload(np.full(N * M + 64, 7.5, np.float32))
        host.append((w, s, M))
        bufs.append((wxo_q8.DeviceBuffer.from_array(w), wxo_q8.DeviceBuffer.from_array(s), out, M))
    wxo_q8.matmul_q8_multi_device(ba, bufs, N, K)
    wxo_q8.synchronize()
    if N > 32 and 1 < sum(1 for M in Ms if M) <= 4:  # one launch over all of them
        assert wxo_q8.last_variant().startswith("matmul_q8.multi "), wxo_q8.last_variant()
    for (w, s, M), (_, _, out, _) in zip(host, bufs):
        got = out.download(np.float32, N * M + 64)
        assert np.all(got[N * M:] == np.float32(7.5)), f"M={M}: written past the output"
        if M:
            assert_matmul(got[:N * M], a, w, s[:M], N, M, K)


@pytest.mark.parametrize("N,M,K", [(64, 2048, 5632), (100, 2048, 2048), (33, 300, 1030), (200, 1000, 4099)])
def test_matmul_short_prompt_is_deterministic(N, M, K):
    """Short prompts run one workgroup per tile with the tile's K steps split
    between two groups of waves, whose sums meet in LDS in a fixed order: every
    run gives the same bits, within the bar of the oracle."""
    rng = np.random.default_rng(N * M + K)
    codes = rng.integers(-128, 128, (M, K)).astype(np.int32)
    w = oracle.pack_q8(codes.reshape(-1), M, K)
    s = rng.uniform(0.001, 0.05, M).astype(np.float32)
    a = rng.standard_normal(N * K).astype(np.float32)
    a[5] = np.nan
    a[K + 7] = np.inf
    first = wxo_q8.matmulQ8(a=a, weight=w, scale=s, N=N, M=M, K=K)
    assert "ksplit2" in wxo_q8.last_variant(), wxo_q8.last_variant()
    for _ in range(3):
        assert_bits_equal(wxo_q8.matmulQ8(a=a, weight=w, scale=s, N=N, M=M, K=K), first, "repeat")
    assert_matmul(first, a, w, s, N, M, K)


SPLIT_CASES = [
    # (N, Ms, K, form): tokens, the projections' rows, columns, the expected split
    (64, [2048], 2048, "wgsplit4"),     # 64 tiles of 32 rows: four workgroups per tile
    (33, [300], 4099, "wgsplit4"),      # ragged rows and K, a one-token second tile row
    (200, [256], 2048, "wgsplit4"),
    (100, [1000], 1030, "wgsplit2"),    # 17 steps: two runs of at least 4 per K group
    (128, [2048], 5632, "wgsplit2"),    # 128 tiles: two workgroups per tile
    (64, [512, 256, 256], 2048, "wgsplit4"),  # three projections (q, k, v of a small model)
    (64, [2048, 2048, 2048], 2048, "ksplit2"),  # 192 tiles: no room to split
    (40, [96, 32, 32], 520, "ksplit2"),  # 9 steps: too few to split
]


@pytest.mark.parametrize("N,Ms,K,form", SPLIT_CASES)
def test_matmul_workspace_split(N, Ms, K, form):
    """wxo_matmul_q8_multi_ws: short prompts split each tile's K steps between
    workgroups whose parts meet in a second launch, in part order.  Every
    output within the matmulQ8 bar of the oracle (Inf and NaN activations
    included), the same bits on every run, nothing written outside the
    outputs, and the workspace left as scratch."""
    rng = np.random.default_rng(N * 7 + K + len(Ms))
    a = rng.standard_normal(N * K).astype(np.float32)
    a[3] = np.inf
    a[K + 11] = np.nan
    ba = wxo_q8.DeviceBuffer.from_array(a)
    ws_bytes = wxo_q8.matmul_q8_workspace_bytes()
    ws = wxo_q8.DeviceBuffer(ws_bytes)
    host, bufs = [], []
    for M in Ms:
        codes = rng.integers(-128, 128, (M, K)).astype(np.int32)
        w = oracle.pack_q8(codes.reshape(-1), M, K)
        s = rng.uniform(0.001, 0.05, M).astype(np.float32)
        out = wxo_q8.DeviceBuffer(4 * (N * M + 64))
        out.upload(np.full(N * M + 64, 7.5, np.float32))
        host.append((w, s, M))
        bufs.append((wxo_q8.DeviceBuffer.from_array(w), wxo_q8.DeviceBuffer.from_array(s), out, M))
    runs = []
    for _ in range(3):
        wxo_q8.matmul_q8_multi_device(ba, bufs, N, K, workspace=ws, workspace_bytes=ws_bytes)
        wxo_q8.synchronize()
        assert wxo_q8.last_variant().split()[1].endswith(form), wxo_q8.last_variant()
        runs.append([b[2].download(np.float32, N * b[3] + 64) for b in bufs])
    for r in runs[1:]:
        for got, first in zip(r, runs[0]):
            assert_bits_equal(got, first, "repeat")
    for (w, s, M), got in zip(host, runs[0]):
        assert np.all(got[N * M:] == np.float32(7.5)), f"M={M}: written past the output"
        assert_matmul(got[:N * M], a, w, s, N, M, K)


BALANCE_CASES = [
    # (N, Ms, K, form with a workspace, form without): between cus and 2 x cus
    # 128-row tiles
    (512, [2048, 2048, 2048], 2048, "D256.PD2", "D256.PD2"),  # 512-token q, k, v: 192 256-row tiles
    (256, [5632, 5632], 2048, "D256.PD2", "D256.PD2"),        # 256-token gate, up: 176 256-row tiles
    (500, [3000, 2800], 1030, "D256.PD2", "D256.PD2"),        # ragged tokens, rows and K: 184 256-row tiles
    (700, [2048, 1500], 1030, "FB4.balance2", "D128"),        # 154 256-row tiles: 308 128-row tiles, 204 split
]


@pytest.mark.parametrize("N,Ms,K,form_ws,form_plain", BALANCE_CASES)
def test_matmul_workspace_balance(N, Ms, K, form_ws, form_plain):
    """Prompts whose 128-row tiles fill one round of two workgroups per CU
    unevenly.  Where 256-row tiles fill two thirds of the CUs or more they run
    on the direct kernel, workspace or not; otherwise with a workspace the
    last 128-row tiles split their K steps in two, so every CU holds the same
    work, and without one the direct kernel runs the 128-row tiles.  Outputs
    within the matmulQ8 bar of the oracle (every 5th token, split and whole
    tiles among them), Inf and NaN activations included; the same bits on
    every run; nothing written past the outputs."""
    rng = np.random.default_rng(N + K + sum(Ms))
    a = rng.standard_normal(N * K).astype(np.float32)
    a[(N - 1) * K + 2] = np.inf   # the last token row is a split tile's
    a[3 * K + 9] = np.nan
    ba = wxo_q8.DeviceBuffer.from_array(a)
    ws_bytes = wxo_q8.matmul_q8_workspace_bytes()
    ws = wxo_q8.DeviceBuffer(ws_bytes)
    host, bufs = [], []
    for M in Ms:
        codes = rng.integers(-128, 128, (M, K)).astype(np.int32)
        w = oracle.pack_q8(codes.reshape(-1), M, K)
        s = rng.uniform(0.001, 0.05, M).astype(np.float32)
        out = wxo_q8.DeviceBuffer(4 * (N * M + 64))
        out.upload(np.full(N * M + 64, 7.5, np.float32))
        host.append((w, s, M))
        bufs.append((wxo_q8.DeviceBuffer.from_array(w), wxo_q8.DeviceBuffer.from_array(s), out, M))
    runs = []
    for _ in range(2):
        wxo_q8.matmul_q8_multi_device(ba, bufs, N, K, workspace=ws, workspace_bytes=ws_bytes)
        wxo_q8.synchronize()
        assert wxo_q8.last_variant().split()[1] == form_ws, wxo_q8.last_variant()
        runs.append([b[2].download(np.float32, N * b[3] + 64) for b in bufs])
    rows = np.unique(np.concatenate([np.arange(0, N, 5), [3, N - 1]]))
    for (w, s, M), got, again in zip(host, runs[0], runs[1]):
        assert_bits_equal(again, got, "repeat")
        assert np.all(got[N * M:] == np.float32(7.5)), f"M={M}: written past the output"
        assert_matmul(got[:N * M], a, w, s, N, M, K, rows=rows)
    # without the workspace: the unsplit kernel, the same bound
    for (_, _, out, _) in bufs:
        out.upload(np.zeros(out.nbytes // 4, np.float32))
    wxo_q8.matmul_q8_multi_device(ba, bufs, N, K)
    wxo_q8.synchronize()
    assert wxo_q8.last_variant().split()[1] == form_plain, wxo_q8.last_variant()
    for (w, s, M), b in zip(host, bufs):
        assert_matmul(b[2].download(np.float32, N * M), a, w, s, N, M, K, rows=rows)


MIB = 1 << 20
FB4_CASES = [
    # (N, Ms, K, workspace bytes (True: the full size), form): tiles that fill
    # the CUs once, with two K groups or split between workgroups
    (128, [5632, 5632], 2048, False, "FB4.ksplit2"),          # 176 tiles: most of the CUs
    (256, [2048, 2048, 2048], 2048, True, "FB4.ksplit2"),     # 192 tiles, with a workspace too
    (512, [2048], 4096, True, "D256.split4"),                  # 64 256-row tiles x 4 parts
    (512, [2048], 2048, True, "FB2.PD4.ksplit2"),              # too few steps for 4 parts: 64-row tiles
    (256, [2048], 5632, True, "D256.split8"),                  # 32 256-row tiles x 8 parts
    (500, [1900], 3000, True, "D256.split4"),                  # ragged tokens, rows and K: 64 tiles x 4
    (512, [2048], 4096, 4 * MIB, "FB4.ksplit2.wgsplit2"),      # no room for 4 parts of 256 rows: 128 x 2
    (256, [2048], 5632, 12 * MIB, "FB4.ksplit2.wgsplit4"),     # no room for 8 parts: 64 tiles x 4
    (500, [1900], 3000, 4 * MIB, "FB4.ksplit2.wgsplit2"),      # ragged: 120 tiles x 2
]


@pytest.mark.parametrize("N,Ms,K,use_ws,form", FB4_CASES)
def test_matmul_128_row_tiles(N, Ms, K, use_ws, form):
    """Tiles filling most of the CUs once (128 rows, two K groups), or all of
    them with their K steps split between workgroups through the workspace:
    256-row direct tiles in 4 or 8 parts, or, with less workspace, the 128-row
    two-group tiles in 2 or 4.  Within the matmulQ8 bar of the oracle (every
    3rd token), Inf and NaN activations included, the same bits on a second
    run, nothing written past the outputs."""
    rng = np.random.default_rng(N * 3 + K + len(Ms))
    a = rng.standard_normal(N * K).astype(np.float32)
    a[(N - 1) * K + 5] = np.inf
    a[6 * K + 1] = np.nan
    ba = wxo_q8.DeviceBuffer.from_array(a)
    ws_bytes = (wxo_q8.matmul_q8_workspace_bytes() if use_ws is True else use_ws) if use_ws else 0
    ws = wxo_q8.DeviceBuffer(wxo_q8.matmul_q8_workspace_bytes()) if use_ws else None
    host, bufs = [], []
    for M in Ms:
        codes = rng.integers(-128, 128, (M, K)).astype(np.int32)
        w = oracle.pack_q8(codes.reshape(-1), M, K)
        s = rng.uniform(0.001, 0.05, M).astype(np.float32)
        out = wxo_q8.DeviceBuffer(4 * (N * M + 64))
        out.upload(np.full(N * M + 64, 7.5, np.float32))
        host.append((w, s, M))
        bufs.append((wxo_q8.DeviceBuffer.from_array(w), wxo_q8.DeviceBuffer.from_array(s), out, M))
    runs = []
    for _ in range(2):
        wxo_q8.matmul_q8_multi_device(ba, bufs, N, K, workspace=ws, workspace_bytes=ws_bytes)
        wxo_q8.synchronize()
        assert wxo_q8.last_variant().split()[1] == form, wxo_q8.last_variant()
        runs.append([b[2].download(np.float32, N * b[3] + 64) for b in bufs])
    rows = np.unique(np.concatenate([np.arange(0, N, 3), [6, N - 1]]))
    for (w, s, M), got, again in zip(host, runs[0], runs[1]):
        assert_bits_equal(again, got, "repeat")
        assert np.all(got[N * M:] == np.float32(7.5)), f"M={M}: written past the output"
        assert_matmul(got[:N * M], a, w, s, N, M, K, rows=rows)


def random_packed(rng, M, K):
    """Packed weight words with any bytes and zero pad codes past K (the wire format)."""
    W = (K + 3) // 4
    w = rng.integers(0, 2 ** 32, (M, W), dtype=np.uint64).astype(np.uint32)
    if K % 4:
        w[:, -1] &= np.uint32((1 << (8 * (K % 4))) - 1)
    return w.reshape(-1)


def test_matmul_random_shapes_every_plan():
    """Seeded random shapes across the dispatch's plans (32-, 64- and 128-row
    tiles, one or two K groups, splits in 2 or 4 parts, the balanced round,
    several projections), with and without a workspace: every output row
    sampled is within the matmulQ8 bar of the oracle, and nothing is written
    past the outputs."""
    rng = np.random.default_rng(20261202)
    forms = set()
    for case in range(24):
        N = int(rng.integers(33, 700))
        Ms = [int(rng.integers(1, 2600)) for _ in range(int(rng.integers(1, 4)))]
        K = int(rng.integers(64, 5200))
        a = rng.standard_normal(N * K).astype(np.float32)
        ba = wxo_q8.DeviceBuffer.from_array(a)
        host, bufs = [], []
        for M in Ms:
            w = random_packed(rng, M, K)
            s = rng.uniform(0.001, 0.05, M).astype(np.float32)
            out = wxo_q8.DeviceBuffer(4 * (N * M + 64))
            host.append((w, s, M))
            bufs.append((wxo_q8.DeviceBuffer.from_array(w), wxo_q8.DeviceBuffer.from_array(s), out, M))
        rows = np.unique(np.r_[rng.integers(0, N, 5), N - 1])
        ws_bytes = wxo_q8.matmul_q8_workspace_bytes()
        ws = wxo_q8.DeviceBuffer(ws_bytes)
        for use_ws in (False, True):
            for (_, _, out, M) in bufs:
                out.upload(np.full(N * M + 64, 7.5, np.float32))
            if use_ws:
                wxo_q8.matmul_q8_multi_device(ba, bufs, N, K, workspace=ws, workspace_bytes=ws_bytes)
            else:
                wxo_q8.matmul_q8_multi_device(ba, bufs, N, K)
            wxo_q8.synchronize()
            form = wxo_q8.last_variant().split()[1]
            forms.add(form)
            for (w, s, M), (_, _, out, _) in zip(host, bufs):
                got = out.download(np.float32, N * M + 64)
                where = f"case {case} N={N} Ms={Ms} K={K} workspace={use_ws} {form}"
                assert np.all(got[N * M:] == np.float32(7.5)), f"{where}: written past the output"
                asub = np.ascontiguousarray(a.reshape(N, K)[rows])
                want = oracle.matmul_q8(asub, w, s, len(rows), M, K)
                bound = oracle.matmul_absterm(asub, w, s, len(rows), M, K)
                ok, msg = oracle.check_matvec(got[:N * M].reshape(N, M)[rows].reshape(-1), want.reshape(-1),
                                              bound.reshape(-1))
                assert ok, f"{where}: {msg}"
        ws.free()
    assert len(forms) >= 5, forms


def test_matmul_workspace_leaves_several_rounds_unsplit():
    """704 tiles (a 512-token gate and up) take several rounds of two
    workgroups per CU: the dispatch evens the CUs out itself and the split
    does not pay, so a workspace changes nothing there."""
    N, M, K = 512, 5632, 2048
    rng = np.random.default_rng(11)
    ba = wxo_q8.DeviceBuffer.from_array(rng.standard_normal(N * K).astype(np.float32))
    bw = wxo_q8.DeviceBuffer.from_array(rng.integers(0, 2 ** 32, M * K // 4, dtype=np.uint64).astype(np.uint32))
    bs = wxo_q8.DeviceBuffer.from_array(np.full(M, 0.01, np.float32))
    outs = [wxo_q8.DeviceBuffer(4 * N * M) for _ in range(2)]
    ws_bytes = wxo_q8.matmul_q8_workspace_bytes()
    ws = wxo_q8.DeviceBuffer(ws_bytes)
    wxo_q8.matmul_q8_multi_device(ba, [(bw, bs, outs[0], M), (bw, bs, outs[1], M)], N, K, workspace=ws,
                                  workspace_bytes=ws_bytes)
    wxo_q8.synchronize()
    assert wxo_q8.last_variant().split()[1] == "D128", wxo_q8.last_variant()
    assert_bits_equal(outs[1].download(np.float32, N * M), outs[0].download(np.float32, N * M), "same weight")


def test_matmul_workspace_size_sets_the_split():
    """A workspace too small for four parts splits in two; one too small for
    that (or none) does not split; the results agree within the bar either
    way."""
    N, M, K = 64, 2048, 2048
    rng = np.random.default_rng(5)
    a = rng.standard_normal(N * K).astype(np.float32)
    codes = rng.integers(-128, 128, (M, K)).astype(np.int32)
    w = oracle.pack_q8(codes.reshape(-1), M, K)
    s = rng.uniform(0.001, 0.05, M).astype(np.float32)
    ba, bw, bs = (wxo_q8.DeviceBuffer.from_array(x) for x in (a, w, s))
    out = wxo_q8.DeviceBuffer(4 * N * M)
    ws = wxo_q8.DeviceBuffer(3 * 4 * N * M)
    for nbytes, form in [(3 * 4 * N * M, "wgsplit4"), (3 * 4 * N * M - 16, "wgsplit2"), (4 * N * M, "wgsplit2"),
                         (4 * N * M - 16, "ksplit2"), (0, "ksplit2")]:
        wxo_q8.matmul_q8_multi_device(ba, [(bw, bs, out, M)], N, K, workspace=ws, workspace_bytes=nbytes)
        wxo_q8.synchronize()
        assert wxo_q8.last_variant().split()[1].endswith(form), (nbytes, wxo_q8.last_variant())
        assert_matmul(out.download(np.float32, N * M), a, w, s, N, M, K)


def test_matmul_invalid_sizes_raise():
    with pytest.raises(wxo_q8.WxoError):
        wxo_q8.matmulQ8(a=np.zeros(4, np.float32), weight=np.zeros(1, np.uint32), scale=np.zeros(1, np.float32),
                        N=2, M=1, K=4)  # a too short
    # a K beyond 2^22 is refused before any launch
    assert wxo_q8.lib().wxo_matmul_q8(None, None, None, None, 1, 1, (1 << 22) + 1, None) == wxo_q8.WXO_ERR_INVALID
    assert "2^22" in wxo_q8.lib().wxo_last_error().decode()


# ---------------------------------------------------------------- dequant / gather

@pytest.mark.parametrize("N,K", [(1, 1), (3, 5), (4, 9), (7, 64), (5, 1027), (300, 4099), (2048, 2048)])
def test_dequantize_packed_bit_exact(N, K):
    rng = np.random.default_rng(N + K)
    w = rng.integers(0, 2 ** 32, N * ((K + 3) // 4), dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(-1, 1, N).astype(np.float32)
    s[0] = np.inf
    got = wxo_q8.dequantizePackedQ8(w, s, N, K)
    want = oracle.dequantize_packed_q8(w, s, N, K)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    got[nan] = 0
    want[nan] = 0
    assert_bits_equal(got, want, f"dequantizePackedQ8 N={N} K={K}")


@pytest.mark.parametrize("N,K", [(1, 1), (2, 2), (3, 3), (5, 1), (7, 2), (9, 5), (11, 6), (13, 7), (31, 1027),
                                 (4096, 4099)])
def test_dequantize_packed_ragged_sentinels(N, K):
    """Rows that end mid-word (K % 4 != 0): a thread writes four consecutive
    outputs, which cross one row end or, for K < 4, several, and the last
    thread writes the 1-3 outputs left.  Bit-exact against the oracle on
    device buffers with sentinels after the output, none overwritten."""
    rng = np.random.default_rng(N * 31 + K)
    W = (K + 3) // 4
    w = rng.integers(0, 2 ** 32, N * W, dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(-1, 1, N).astype(np.float32)
    bw, bs = wxo_q8.DeviceBuffer.from_array(w), wxo_q8.DeviceBuffer.from_array(s)
    out = wxo_q8.DeviceBuffer(4 * (N * K + 64))
    out.upload(np.full(N * K + 64, 7.5, np.float32))
    wxo_q8.dequantize_packed_q8_device(bw, bs, N, K, out)
    wxo_q8.synchronize()
    got = out.download(np.float32, N * K + 64)
    assert np.all(got[N * K:] == np.float32(7.5)), "written past the output"
    assert_bits_equal(got[:N * K], oracle.dequantize_packed_q8(w, s, N, K), f"dequantizePackedQ8 N={N} K={K}")


def test_dequantize_packed_kats():
    c = kat()["dequantize_packed_q8"][1]
    w = oracle.pack_int8_rows(np.array(c["codes"], np.int8), c["N"], c["K"])
    assert wxo_q8.dequantizePackedQ8(w, np.array(c["scale"], np.float32), c["N"], c["K"]).tolist() == c["want"]


@pytest.mark.parametrize("outF,inF", [(1, 1), (5, 3), (3, 8), (16, 112), (512, 1792), (67, 1027), (2048, 5632)])
def test_dequant_transpose_bit_exact(outF, inF):
    codes = np.array([((i * 37) % 200) - 100 for i in range(outF * inF)], dtype=np.int8) if outF * inF < 10 ** 6 \
        else np.random.default_rng(0).integers(-128, 128, outF * inF).astype(np.int8)
    s = np.array([0.01 + i * 1e-4 for i in range(outF)], dtype=np.float32)
    w = oracle.pack_int8_rows(codes, outF, inF)
    got = wxo_q8.dequantTranspose(weight=w, scale=s, outFeatures=outF, inFeatures=inF)
    assert_bits_equal(got, oracle.dequant_transpose(w, s, outF, inF), f"dequantTranspose {outF}x{inF}")


def test_dequant_transpose_size_errors():
    c = kat()["dequant_transpose"][1]
    w = oracle.pack_int8_rows(np.zeros(15, np.int8), 3, 5)
    wxo_q8.dequantTranspose(weight=w, scale=np.zeros(3, np.float32), outFeatures=3, inFeatures=5)
    with pytest.raises(wxo_q8.WxoError, match=c["errors"][0]):
        wxo_q8.dequantTranspose(weight=w, scale=np.zeros(3, np.float32), outFeatures=4, inFeatures=5)
    with pytest.raises(wxo_q8.WxoError, match=c["errors"][1]):
        wxo_q8.dequantTranspose(weight=w, scale=np.zeros(2, np.float32), outFeatures=3, inFeatures=5)


@pytest.mark.parametrize("case", kat()["gather_dequant_rows"], ids=lambda c: c["source"].split(" ")[0])
def test_gather_kat(case):
    got = wxo_q8.gatherDequantRows((np.array(case["codes"], np.int8), np.array(case["scale"], np.float32)),
                                   case["indices"], case["D"])
    assert got.tolist() == case["want"]


@pytest.mark.parametrize("rows,D", [(37, 70), (1000, 2048), (300, 4099), (5, 16)])
def test_gather_bit_exact(rows, D):
    rng = np.random.default_rng(rows + D)
    codes = rng.integers(-128, 128, rows * D).astype(np.int8)
    s = rng.uniform(0.001, 0.1, rows).astype(np.float32)
    idx = np.concatenate([rng.integers(0, rows, 50), [-1, rows, 2 ** 40, -(2 ** 40), 0, rows - 1, 0]]).astype(np.int64)
    got = wxo_q8.gatherDequantRows((codes, s), idx, D)
    assert_bits_equal(got, oracle.gather_dequant_rows(codes, s, rows, D, idx), f"gather rows={rows} D={D}")


@pytest.mark.parametrize("N,Ms,K", [(2048, [2176, 1920], 4100), (1024, [4224, 3968], 4096)])
def test_matmul_tile_pairs(N, Ms, K):
    """Long rows whose 128-row tiles make two whole rounds of two per CU: one
    workgroup of 16 waves per two tiles, one per K group (in the second case
    a pair of tiles straddles the two projections).  Every 37th token
    against the oracle, nothing past the outputs."""
    rng = np.random.default_rng(N + sum(Ms) + K)
    a = rng.standard_normal(N * K).astype(np.float32)
    a[3 * K + 5] = np.inf
    ba = wxo_q8.DeviceBuffer.from_array(a)
    host, bufs = [], []
    for M in Ms:
        w = oracle.pack_q8(rng.integers(-128, 128, (M, K)).astype(np.int32).reshape(-1), M, K)
        s = rng.uniform(0.001, 0.05, M).astype(np.float32)
        out = wxo_q8.DeviceBuffer(4 * (N * M + 64))
        out.upload(np.full(N * M + 64, 7.5, np.float32))
        host.append((w, s, M))
        bufs.append((wxo_q8.DeviceBuffer.from_array(w), wxo_q8.DeviceBuffer.from_array(s), out, M))
    wxo_q8.matmul_q8_multi_device(ba, bufs, N, K)
    wxo_q8.synchronize()
    assert " FB4.pairs " in wxo_q8.last_variant(), wxo_q8.last_variant()
    rows = np.unique(np.r_[np.arange(0, N, 37), 3, N - 1])
    for (w, s, M), (_, _, out, _) in zip(host, bufs):
        got = out.download(np.float32, N * M + 64)
        assert np.all(got[N * M:] == np.float32(7.5)), f"M={M}: written past the output"
        assert_matmul(got[:N * M], a, w, s, N, M, K, rows=rows)


def test_matmul_tile_pairs_ragged_tokens_match_one_group():
    """Tile pairs with a partial last token tile (N = 2040: 31 whole 64-token
    tiles and one of 56) over two projections (2176 and 1920 rows: 17 + 15
    tiles of 128 rows, 1024 tiles in all, whose 256-row tiles would not make
    whole rounds): every 29th token against the oracle, nothing past the
    outputs, and the bits of both halves of the tokens equal to runs of those
    halves alone, whose 512 tiles take the one-group form on the direct
    kernel (D128: the same sums in the same order; token tile boundaries line
    up at token 1024)."""
    N, K = 2040, 4096
    Ms = [2176, 1920]
    rng = np.random.default_rng(2040)
    a = rng.standard_normal(N * K).astype(np.float32)
    ba = wxo_q8.DeviceBuffer.from_array(a)
    host, dev, outs = [], [], []
    for M in Ms:
        w = oracle.pack_q8(rng.integers(-128, 128, (M, K)).astype(np.int32).reshape(-1), M, K)
        s = rng.uniform(0.001, 0.05, M).astype(np.float32)
        o = wxo_q8.DeviceBuffer(4 * (N * M + 64))
        o.upload(np.full(N * M + 64, 7.5, np.float32))
        host.append((w, s, M))
        dev.append((wxo_q8.DeviceBuffer.from_array(w), wxo_q8.DeviceBuffer.from_array(s)))
        outs.append(o)
    wxo_q8.matmul_q8_multi_device(ba, [(bw, bs, o, M) for (bw, bs), o, M in zip(dev, outs, Ms)], N, K)
    wxo_q8.synchronize()
    assert " FB4.pairs " in wxo_q8.last_variant(), wxo_q8.last_variant()
    got = []
    for (w, s, M), o in zip(host, outs):
        g = o.download(np.float32, N * M + 64)
        assert np.all(g[N * M:] == np.float32(7.5)), f"M={M}: written past the output"
        assert_matmul(g[:N * M], a, w, s, N, M, K, rows=np.unique(np.r_[np.arange(0, N, 29), N - 1]))
        got.append(g)
    for t0, t1 in ((0, 1024), (1024, N)):
        n = t1 - t0
        bh = wxo_q8.DeviceBuffer.from_array(a[t0 * K:t1 * K])
        ohs = [wxo_q8.DeviceBuffer(4 * n * M) for M in Ms]
        wxo_q8.matmul_q8_multi_device(bh, [(bw, bs, oh, M) for (bw, bs), oh, M in zip(dev, ohs, Ms)], n, K)
        wxo_q8.synchronize()
        variant = wxo_q8.last_variant()
        assert " D128 " in variant, variant
        for oh, g, M in zip(ohs, got, Ms):
            assert_bits_equal(oh.download(np.float32, n * M), g[t0 * M:t1 * M], f"M={M} tokens {t0}..{t1}: pairs vs one group")


def test_matmul_256_row_tiles_match_the_one_group_form():
    """Launches whose 256-row tiles make whole rounds of the CUs take them on
    the direct kernel (8 waves of 32 rows): 2048 tokens x 2048 x 2048 is 256
    such tiles.  The bits of its first 1280 tokens equal a launch of those
    tokens alone, whose 320 tiles of 128 rows (160 of 256 rows: under two
    thirds of the CUs) take the 128-row direct form; every 41st token against
    the oracle."""
    N, M, K = 2048, 2048, 2048
    rng = np.random.default_rng(256)
    a = rng.standard_normal(N * K).astype(np.float32)
    w = oracle.pack_q8(rng.integers(-128, 128, (M, K)).astype(np.int32).reshape(-1), M, K)
    s = rng.uniform(0.001, 0.05, M).astype(np.float32)
    bw, bs = wxo_q8.DeviceBuffer.from_array(w), wxo_q8.DeviceBuffer.from_array(s)
    out = wxo_q8.DeviceBuffer(4 * N * M)
    wxo_q8.matmul_q8_multi_device(wxo_q8.DeviceBuffer.from_array(a), [(bw, bs, out, M)], N, K)
    wxo_q8.synchronize()
    assert " D256 " in wxo_q8.last_variant(), wxo_q8.last_variant()
    got = out.download(np.float32, N * M)
    assert_matmul(got, a, w, s, N, M, K, rows=np.unique(np.r_[np.arange(0, N, 41), N - 1]))
    n = 1280
    half = wxo_q8.DeviceBuffer(4 * n * M)
    wxo_q8.matmul_q8_multi_device(wxo_q8.DeviceBuffer.from_array(a[:n * K]), [(bw, bs, half, M)], n, K)
    wxo_q8.synchronize()
    variant = wxo_q8.last_variant()
    assert " D128 " in variant, variant
    assert_bits_equal(got[:n * M], half.download(np.float32, n * M), "256-row tiles vs the one-group 128-row form")


def test_matmul_256_row_tiles_ragged():
    """256-row tiles with partial row tiles (two projections of 728 and 200
    rows: 3 + 1 row tiles, 216 and 200 rows in the last), a partial last token
    tile (4066 tokens) and a ragged K (2061): 64 token tiles x 4 row tiles =
    256 tiles,
    Inf and NaN among the activations; sentinels after the outputs untouched,
    every 37th token against the oracle."""
    N, K = 4066, 2061
    Ms = [728, 200]
    rng = np.random.default_rng(984)
    a = rng.standard_normal(N * K).astype(np.float32)
    a[5 * K + 7] = np.inf
    a[9 * K + 100] = np.nan
    ba = wxo_q8.DeviceBuffer.from_array(a)
    host, bufs = [], []
    for M in Ms:
        w = oracle.pack_q8(rng.integers(-128, 128, (M, K)).astype(np.int32).reshape(-1), M, K)
        s = rng.uniform(0.001, 0.05, M).astype(np.float32)
        o = wxo_q8.DeviceBuffer(4 * (N * M + 64))
        o.upload(np.full(N * M + 64, 7.5, np.float32))
        host.append((w, s, M))
        bufs.append((wxo_q8.DeviceBuffer.from_array(w), wxo_q8.DeviceBuffer.from_array(s), o, M))
    wxo_q8.matmul_q8_multi_device(ba, bufs, N, K)
    wxo_q8.synchronize()
    assert " D256 " in wxo_q8.last_variant(), wxo_q8.last_variant()
    rows = np.unique(np.r_[np.arange(0, N, 37), 5, 9, N - 1])
    for (w, s, M), (_, _, o, _) in zip(host, bufs):
        got = o.download(np.float32, N * M + 64)
        assert np.all(got[N * M:] == np.float32(7.5)), f"M={M}: written past the output"
        assert_matmul(got[:N * M], a, w, s, N, M, K, rows=rows)


def test_matmul_weight_past_4_gib():
    """64 tokens against a 4.6 GB packed weight (4.5M rows of K = 1024):
    the tiles address their weight rows and output columns from 64-bit bases,
    so columns past the first 4 GiB of weight are their own rows' sums.
    Sampled weight rows (output columns) at both ends and at random against
    the oracle; the weight is one random 4096-row block repeated."""
    T, M, K, W = 64, 4_500_000, 1024, 256
    rng = np.random.default_rng(64)
    block = rng.integers(0, 2 ** 32, 4096 * W, dtype=np.uint64).astype(np.uint32).reshape(4096, W)
    w = np.ascontiguousarray(np.tile(block, ((M + 4095) // 4096, 1))[:M]).reshape(-1)
    s = rng.uniform(1e-3, 1e-1, M).astype(np.float32)
    a = rng.standard_normal((T, K)).astype(np.float32)
    y = np.asarray(wxo_q8.matmulQ8(a=a, weight=w, scale=s, N=T, M=M, K=K)).reshape(T, M)
    print(wxo_q8.last_variant(), flush=True)
    cols = np.unique(np.concatenate([np.arange(64), np.arange(M - 100, M), rng.integers(0, M, 256)]))
    wsub = w.reshape(M, W)[cols].reshape(-1)
    assert_matmul(np.ascontiguousarray(y[:, cols]), a, wsub, s[cols], T, len(cols), K)
