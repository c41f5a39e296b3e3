"""Pins the oracle's matmulQ8, dequantizePackedQ8, dequantTranspose and
gatherDequantRows (oracle/q8_oracle.c) before the GPU is compared with them.

  * known answers from the reference's tests (tests/golden/kat.json);
  * closed forms computed by another mechanism: numpy's f32 multiply (correctly
    rounded, hence bit-equal to the reference's f64 product stored to f32),
    numpy's f64 matrix product, transposition, row selection;
  * the ECMAScript restatement (oracle/q8_oracle.mjs under node) against the C
    one, bit for bit;
  * mutants (transposed operand, a neighbour's scale, a mis-signed byte, a read
    past K) that each of those checks must reject.
"""
import base64
import json
import math
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
NODE = shutil.which("node")


def kat():
    with open(os.path.join(GOLDEN, "kat.json")) as f:
        return json.load(f)


def f32(x):
    return np.asarray(x, dtype=np.float32)


def dequant_np(codes2d, scale):
    """codes [rows, K] int -> f32 codes * scale via numpy's f32 multiply."""
    return codes2d.astype(np.float32) * f32(scale)[:, None]


def js_sin_wave(n, k, mul, phase=0.0):
    # Math.sin(i * k + phase) * mul, stored to Float32Array (the reference
    # tests' generators); libm's sin agrees with V8's to the f32 rounding here.
    return np.array([math.sin(i * k + phase) * mul for i in range(n)], dtype=np.float32)


def js_code_wave(n, k):
    # Math.round(Math.sin(i * k) * 100) into an Int32Array
    return np.array([int(oracle.js_round(math.sin(i * k) * 100)) for i in range(n)], dtype=np.int32)


def scale_wave(n):
    return np.array([0.02 * (i + 1) + 0.007 for i in range(n)], dtype=np.float32)


# ------------------------------------------------------------ dequantizePackedQ8

def test_dequantize_packed_kats():
    cases = kat()["dequantize_packed_q8"]
    N, K = cases[0]["N"], cases[0]["K"]
    codes = np.array([-128 if i == 0 else ((i * 37) % 255) - 127 for i in range(N * K)], dtype=np.int8)
    scale = f32([0.01 * (r + 1) + 0.003 for r in range(N)])
    w = oracle.pack_int8_rows(codes, N, K)
    got = oracle.dequantize_packed_q8(w, scale, N, K)
    want = dequant_np(codes.reshape(N, K), scale).reshape(-1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert got[0] == np.float32(-128) * scale[0]  # the one byte (0x80) a >= 129 sign test mis-signs

    c = cases[1]
    w = oracle.pack_int8_rows(np.array(c["codes"], np.int8), c["N"], c["K"])
    assert oracle.dequantize_packed_q8(w, f32(c["scale"]), c["N"], c["K"]).tolist() == c["want"]


@pytest.mark.parametrize("N,K", [(1, 1), (3, 5), (7, 64), (5, 1027)])
def test_dequantize_packed_closed_form_and_pad_lanes(N, K):
    rng = np.random.default_rng(N * 1000 + K)
    codes = rng.integers(-128, 128, (N, K)).astype(np.int8)
    scale = rng.uniform(-2, 2, N).astype(np.float32)
    w = oracle.pack_int8_rows(codes, N, K)
    if K % 4:  # garbage in the pad lanes must not leak
        W = oracle.words_per_row(K)
        w = w.reshape(N, W).copy()
        w[:, -1] |= np.uint32(0x7f7f7f7f) & ~np.uint32((1 << (8 * (K % 4))) - 1)
        w = w.reshape(-1)
    got = oracle.dequantize_packed_q8(w, scale, N, K)
    assert np.array_equal(got.view(np.uint32), dequant_np(codes, scale).reshape(-1).view(np.uint32))


# ------------------------------------------------------------ dequantTranspose

def test_dequant_transpose_is_the_transpose_of_dequantize():
    shapes = kat()["dequant_transpose"][0]["shapes"]
    for outF, inF in shapes:
        codes = np.array([((i * 37) % 200) - 100 for i in range(outF * inF)], dtype=np.int8)
        scale = np.array([0.01 + i * 1e-4 for i in range(outF)], dtype=np.float32)
        w = oracle.pack_int8_rows(codes, outF, inF)
        got = oracle.dequant_transpose(w, scale, outF, inF).reshape(inF, outF)
        want = dequant_np(codes.reshape(outF, inF), scale).T
        assert np.array_equal(got.view(np.uint32), np.ascontiguousarray(want).view(np.uint32)), (outF, inF)


# ------------------------------------------------------------ gatherDequantRows

def test_gather_dequant_rows_kats():
    for c in kat()["gather_dequant_rows"]:
        rows = len(c["scale"])
        got = oracle.gather_dequant_rows(np.array(c["codes"], np.int8), f32(c["scale"]), rows, c["D"], c["indices"])
        assert got.tolist() == c["want"], c["source"]


def test_gather_dequant_rows_is_row_selection():
    rng = np.random.default_rng(3)
    rows, D = 37, 70
    codes = rng.integers(-128, 128, (rows, D)).astype(np.int8)
    scale = rng.uniform(0.001, 0.1, rows).astype(np.float32)
    idx = np.array([0, 36, 5, 5, -1, 37, 2 ** 40, -(2 ** 40), 17], dtype=np.int64)
    got = oracle.gather_dequant_rows(codes, scale, rows, D, idx).reshape(len(idx), D)
    table = dequant_np(codes, scale)
    for i, r in enumerate(idx):
        want = table[r] if 0 <= r < rows else np.zeros(D, np.float32)
        assert np.array_equal(got[i].view(np.uint32), want.view(np.uint32)), (i, r)


# ------------------------------------------------------------ matmulQ8

def test_matmul_q8_hand_computed_kat():
    c = kat()["matmul_q8"][1]
    w = oracle.pack_q8(np.array(c["codes"], np.int32), c["M"], c["K"])
    got = oracle.matmul_q8(f32(c["a"]), w, f32(c["scale"]), c["N"], c["M"], c["K"])
    assert got.reshape(-1).tolist() == c["want"]


def test_matmul_q8_empty_k_is_zero():
    w = np.zeros(0, np.uint32)
    got = oracle.matmul_q8(np.zeros(0, np.float32), w, f32([np.inf, 1, np.nan, 2, 3]), 3, 5, 0)
    assert got.shape == (3, 5) and np.array_equal(got, np.zeros((3, 5), np.float32))
    assert not np.signbit(got).any()


def _ref_shapes_inputs(N, M, K):
    a = js_sin_wave(N * K, 0.37, 1.5)
    codes = js_code_wave(M * K, 0.19)
    w = oracle.pack_q8(codes, M, K)
    return a, codes, w, scale_wave(M)


def test_matmul_q8_reference_shapes_match_f64_matrix_product():
    # The oracle's left-to-right f64 loops against numpy's f64 matrix product of
    # a and the f32 dequantized weight (exact products; any summation order is
    # within a few f64 ulps of the sum, far below one f32 step).
    for N, M, K in kat()["matmul_q8"][0]["shapes"]:
        a, codes, w, scale = _ref_shapes_inputs(N, M, K)
        got = oracle.matmul_q8(a, w, scale, N, M, K)
        b = dequant_np(codes.reshape(M, K), scale).astype(np.float64)
        want = (a.reshape(N, K).astype(np.float64) @ b.T).astype(np.float32)
        bound = oracle.matmul_absterm(a, w, scale, N, M, K)
        assert np.all(np.abs(got.astype(np.float64) - want) <= 1e-12 * bound + np.spacing(np.abs(want))), (N, M, K)


def test_matmul_q8_is_n_matvec_calls_within_one_rounding_per_term():
    # ops/matmul/reference.ts:76-77: "N independent matvecQ8 calls".  The two
    # definitions differ only by the f32 rounding of each dequantized term.
    rng = np.random.default_rng(5)
    N, M, K = 6, 9, 301
    codes = rng.integers(-127, 128, M * K).astype(np.int32)
    w = oracle.pack_q8(codes, M, K)
    scale = rng.uniform(0.001, 0.05, M).astype(np.float32)
    a = rng.standard_normal(N * K).astype(np.float32)
    got = oracle.matmul_q8(a, w, scale, N, M, K)
    bound = oracle.matmul_absterm(a, w, scale, N, M, K)
    for n in range(N):
        mv = oracle.matvec_q8(w, scale, a[n * K:(n + 1) * K], M, K)
        assert np.all(np.abs(got[n].astype(np.float64) - mv) <= 2.0 ** -23 * bound[n] + np.spacing(np.abs(mv)))


def test_matmul_q8_edge_cases_and_mutants():
    # q8-edges.wgsl.test.ts:110-139: identical code rows, own scales -> the
    # outputs' ratio is exactly the scales' ratio in f64 terms
    c = kat()["matmul_q8"][2]
    N, M, K = c["N"], c["M"], c["K"]
    shared = js_code_wave(K, 0.27)
    codes = np.concatenate([shared, shared])
    w = oracle.pack_q8(codes, M, K)
    a = js_sin_wave(N * K, 0.5, 1.5)
    s = f32(c["scale"])
    got = oracle.matmul_q8(a, w, s, N, M, K)
    b = dequant_np(codes.reshape(M, K), s).astype(np.float64)
    want = (a.reshape(N, K).astype(np.float64) @ b.T).astype(np.float32)
    assert np.array_equal(got, want)
    assert not np.allclose(got[:, 0], got[:, 1])
    # mutants that the closed form rejects
    bound = oracle.matmul_absterm(a, w, s, N, M, K)
    tol = 1e-5 * bound + 1e-7
    swapped = oracle.matmul_q8(a, w, s[::-1].copy(), N, M, K)  # a neighbour's scale
    assert np.any(np.abs(swapped - want) > tol)
    rng = np.random.default_rng(9)
    N2, M2, K2 = 5, 7, 19
    codes2 = rng.integers(-127, 128, M2 * K2).astype(np.int32)
    w2 = oracle.pack_q8(codes2, M2, K2)
    a2 = rng.standard_normal(N2 * K2).astype(np.float32)
    s2 = rng.uniform(0.01, 0.1, M2).astype(np.float32)
    ref = oracle.matmul_q8(a2, w2, s2, N2, M2, K2)
    tol2 = 1e-5 * oracle.matmul_absterm(a2, w2, s2, N2, M2, K2) + 1e-7
    # the weight read as if it were already [K, M] (matmul's own b layout)
    b_wrong = codes2.reshape(K2, M2).astype(np.float32) * s2[None, :]
    transposed = (a2.reshape(N2, K2).astype(np.float64) @ b_wrong.astype(np.float64)).astype(np.float32)
    assert np.any(np.abs(ref - transposed) > tol2)
    # a mis-signed byte (>= 129 instead of >= 128 as the sign test): 0x80 read as +128
    codes3 = codes2.copy()
    codes3[0] = -128
    w3 = oracle.pack_q8(codes3, M2, K2)
    ref3 = oracle.matmul_q8(a2, w3, s2, N2, M2, K2)
    codes_wrong = codes3.copy()
    codes_wrong[0] = 128
    b_mis = codes_wrong.reshape(M2, K2).astype(np.float32) * s2[:, None]
    mis = (a2.reshape(N2, K2).astype(np.float64) @ b_mis.astype(np.float64).T).astype(np.float32)
    tol3 = 1e-5 * oracle.matmul_absterm(a2, w3, s2, N2, M2, K2) + 1e-7
    assert np.any(np.abs(ref3 - mis) > tol3)
    # reading one word past the row (the sentinel of q8-edges.wgsl.test.ts:29-74)
    padded = np.concatenate([w2, np.full(64, 0x7f7f7f7f, np.uint32)])
    assert np.array_equal(oracle.matmul_q8(a2, padded, s2, N2, M2, K2), ref)
    W2 = oracle.words_per_row(K2)
    shifted = padded[1:1 + M2 * W2]  # rows read with an off-by-one word stride
    assert np.any(np.abs(oracle.matmul_q8(a2, shifted, s2, N2, M2, K2) - ref) > tol2)


# ------------------------------------------------------------ C against ECMAScript

def enc(arr, dtype):
    return {"dtype": dtype, "b64": base64.b64encode(np.ascontiguousarray(arr).tobytes()).decode()}


def dec(b64, dtype):
    return np.frombuffer(base64.b64decode(b64), dtype=dtype)


def run_js(job):
    proc = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "oracle_job.mjs")], input=json.dumps(job),
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stderr
    return json.loads(proc.stdout)


@pytest.mark.skipif(NODE is None, reason="node not on PATH")
def test_c_oracle_matches_ecmascript_oracle_prefill_ops():
    rng = np.random.default_rng(21)
    N, M, K = 7, 13, 67
    a = rng.standard_normal(N * K).astype(np.float32)
    a[3] = np.inf
    a[K + 1] = 0.0
    codes = rng.integers(-128, 128, M * K).astype(np.int32)
    w = oracle.pack_q8(codes, M, K)
    s = rng.uniform(0.001, 0.1, M).astype(np.float32)
    s[4] = np.inf
    js = run_js({"op": "matmulQ8", "N": N, "M": M, "K": K,
                 "arrays": {"a": enc(a, "f32"), "weight": enc(w, "u32"), "scale": enc(s, "f32")}})
    js_y = dec(js["output"], np.float32)
    c_y = oracle.matmul_q8(a, w, s, N, M, K).reshape(-1)
    assert np.array_equal(np.isnan(js_y), np.isnan(c_y))
    ok = ~np.isnan(c_y)
    assert np.array_equal(js_y[ok].view(np.uint32), c_y[ok].view(np.uint32))

    js = run_js({"op": "dequantizePackedQ8", "N": M, "K": K, "arrays": {"weight": enc(w, "u32"), "scale": enc(s, "f32")}})
    assert np.array_equal(dec(js["output"], np.float32).view(np.uint32),
                          oracle.dequantize_packed_q8(w, s, M, K).view(np.uint32))
    js = run_js({"op": "dequantTranspose", "N": M, "K": K, "arrays": {"weight": enc(w, "u32"), "scale": enc(s, "f32")}})
    assert np.array_equal(dec(js["output"], np.float32).view(np.uint32),
                          oracle.dequant_transpose(w, s, M, K).view(np.uint32))
    i8 = codes.astype(np.int8)
    idx = np.array([3, 0, 12, -1, 13, 3], dtype=np.float64)
    js = run_js({"op": "gatherDequantRows", "D": K,
                 "arrays": {"codes": enc(i8, "i8"), "scale": enc(s, "f32"), "indices": enc(idx, "f64")}})
    assert np.array_equal(dec(js["output"], np.float32).view(np.uint32),
                          oracle.gather_dequant_rows(i8, s, M, K, idx.astype(np.int64)).view(np.uint32))


def test_threaded_rows_give_the_same_bits():
    """The C oracle splits matvec and matmul output rows over threads; each
    output is one f64 sum in the reference's order, so the bits do not depend
    on the thread count (OMP_NUM_THREADS is read at each call)."""
    rng = np.random.default_rng(3)
    N, M, K = 64, 515, 1031
    W = (K + 3) // 4
    w = rng.integers(0, 2 ** 32, M * W, dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(1e-3, 5e-2, M).astype(np.float32)
    a = rng.standard_normal(N * K).astype(np.float32)
    a[17] = np.inf
    N2 = 20000  # matvec rows: enough work for the threads
    w2 = rng.integers(0, 2 ** 32, N2 * W, dtype=np.uint64).astype(np.uint32)
    s2 = rng.uniform(1e-3, 5e-2, N2).astype(np.float32)
    old = os.environ.get("OMP_NUM_THREADS")
    runs = []
    try:
        for threads in ("1", "3", "7"):
            os.environ["OMP_NUM_THREADS"] = threads
            runs.append((oracle.matmul_q8(a, w, s, N, M, K), oracle.matmul_absterm(a, w, s, N, M, K),
                         oracle.matvec_q8(w2, s2, a[:K], N2, K), oracle.absterm(w2, s2, a[:K], N2, K)))
    finally:
        if old is None:
            os.environ.pop("OMP_NUM_THREADS", None)
        else:
            os.environ["OMP_NUM_THREADS"] = old
    for other in runs[1:]:
        for x, y in zip(runs[0], other):
            assert np.array_equal(np.asarray(x).view(np.uint8), np.asarray(y).view(np.uint8))
