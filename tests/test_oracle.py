"""Pins the CPU oracle (oracle/) before anything is compared against it.

Checks, in order of strength:
  * the reference's committed fixture pair (llm/fixtures/tiny.weights.bin ->
    tiny_q8.codes.bin + tiny_q8.scales.bin): 16 matrices quantized by the
    reference's own toolchain, bit for bit;
  * the known answers in the reference's tests (tests/golden/kat.json);
  * closed forms the mathematics fixes (packQ8 is the little-endian byte view
    of each row padded to 4 bytes; matvecQ8 is a dot product with exact f64
    products), computed here by a different mechanism than the oracle's;
  * the ECMAScript restatement (oracle/q8_oracle.mjs, run under node) against
    the C restatement, bit for bit, on tie-heavy and edge inputs.
A test at the end shows the KATs reject the plausible mistakes (banker's
rounding, floor(x + 0.5), f32 arithmetic, a wrong byte order).
"""
import base64
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def kat():
    with open(os.path.join(GOLDEN, "kat.json")) as f:
        return json.load(f)


def f32_bits(x):
    return int(np.float32(x).view(np.uint32))


# ---------------------------------------------------------------- Math.round

@pytest.mark.parametrize("v,want", [
    (0.5, 1.0), (-0.5, 0.0), (1.5, 2.0), (-1.5, -1.0), (2.5, 3.0), (-2.5, -2.0),
    (62.5, 63.0), (-62.5, -62.0), (0.49999999999999994, 0.0), (-0.49999999999999994, 0.0),
    (126.49999999999999, 126.0), (126.5, 127.0), (-126.5, -126.0), (3.7, 4.0), (-3.7, -4.0),
    (2.0 ** 52 + 1, 2.0 ** 52 + 1), (-(2.0 ** 53), -(2.0 ** 53)), (1e300, 1e300), (0.0, 0.0),
])
def test_js_round_known_values(v, want):
    # ECMAScript 21.3.2.28 worked values: ties go toward +Infinity, and the
    # largest double below 0.5 rounds to 0 (floor(x + 0.5) would give 1).
    assert oracle.js_round(v) == want


def test_js_round_specials():
    assert np.isnan(oracle.js_round(float("nan")))
    assert oracle.js_round(float("inf")) == float("inf")
    assert oracle.js_round(float("-inf")) == float("-inf")


# ---------------------------------------------------------------- quantize

@pytest.mark.parametrize("case", kat()["quantize"], ids=lambda c: c["source"].split(" ")[0])
def test_quantize_kat(case):
    x = np.array(case["input"], dtype=np.float32)
    codes, scales = oracle.quantize(x, 1, x.size)
    assert codes.tolist() == case["codes"]
    assert f32_bits(scales[0]) == int(case["scale_bits"], 16)


def _tiny_q8_pairs():
    with open(os.path.join(GOLDEN, "tiny.manifest.json")) as f:
        f32_manifest = {w["name"]: w for w in json.load(f)["weights"]}
    with open(os.path.join(GOLDEN, "tiny_q8.manifest.json")) as f:
        q8_manifest = [w for w in json.load(f)["weights"] if w["kind"] == "quant"]
    weights = np.fromfile(os.path.join(GOLDEN, "tiny.weights.bin"), dtype="<f4")
    codes = np.fromfile(os.path.join(GOLDEN, "tiny_q8.codes.bin"), dtype=np.int8)
    scales = np.fromfile(os.path.join(GOLDEN, "tiny_q8.scales.bin"), dtype="<f4")
    for q in q8_manifest:
        N, K = q["shape"]
        src = f32_manifest[q["name"]]
        assert src["shape"] == [N, K]
        w = weights[src["offset"]: src["offset"] + N * K]
        yield (q["name"], N, K, w,
               codes[q["codesOffset"]: q["codesOffset"] + N * K],
               scales[q["scaleOffset"]: q["scaleOffset"] + N])


def test_quantize_matches_reference_fixture_bit_for_bit():
    # llm/fixtures: the f32 tiny model and its int8 form written by the
    # reference's converter (llm/tools/gen_fixture_q8.py -> quant_common.py,
    # the numpy twin that the reference tests against quantize itself).
    pairs = list(_tiny_q8_pairs())
    assert len(pairs) == 16
    total = 0
    for name, N, K, w, want_codes, want_scales in pairs:
        codes, scales = oracle.quantize(w, N, K)
        assert np.array_equal(codes.astype(np.int8), want_codes), name
        assert np.array_equal(codes, want_codes.astype(np.int32)), name
        assert np.array_equal(scales.view(np.uint32), want_scales.view(np.uint32)), name
        total += N * K
    assert total == 106496


def test_quantize_invariants_and_edges():
    rng = np.random.default_rng(7)
    N, D = 64, 333
    x = (rng.standard_normal((N, D)) * rng.uniform(1e-3, 1e3, (N, 1))).astype(np.float32)
    x[3] = 0.0                    # all-zero row: scale 1, codes 0
    x[4, :] = -0.0
    x[5, 7] = np.nan              # NaN propagates through Math.max: scale NaN, codes 0
    x[6, 9] = np.inf              # absmax Inf: inverse 0, scale Inf, codes 0 (Inf*0 is NaN -> 0)
    x[7, :] = 1e-42               # subnormal f32 absmax
    x[8, 11] = -np.inf
    codes, scales = oracle.quantize(x, N, D)
    codes = codes.reshape(N, D)
    assert np.all(np.abs(codes) <= 127)
    assert np.all(codes[3] == 0) and f32_bits(scales[3]) == f32_bits(1.0)
    assert np.all(codes[4] == 0) and f32_bits(scales[4]) == f32_bits(1.0)
    assert np.all(codes[5] == 0) and np.isnan(scales[5])
    assert np.all(codes[6] == 0) and scales[6] == np.inf
    assert np.all(codes[8] == 0) and scales[8] == np.inf
    assert np.all(codes[7] == 127)
    assert scales[7] == np.float32(np.float64(np.float32(1e-42)) / 127.0)
    for r in (0, 1, 2, 9, 10):
        k = int(np.argmax(np.abs(x[r])))
        assert codes[r, k] == (127 if x[r, k] > 0 else -127)
        assert scales[r] > 0
        # dequantised values sit within half a step of the input
        err = np.abs(codes[r] * np.float64(scales[r]) - x[r])
        assert np.all(err <= 0.5 * np.float64(scales[r]) * (1 + 1e-6))


# ---------------------------------------------------------------- packQ8

@pytest.mark.parametrize("case", kat()["pack_q8"], ids=lambda c: c["source"].split(" ")[0])
def test_pack_q8_kat(case):
    words = oracle.pack_q8(np.array(case["codes"], dtype=np.int32), case["N"], case["K"])
    assert [f"0x{w:08x}" for w in words.tolist()] == case["words"]


@pytest.mark.parametrize("case", kat()["pack_int8_rows"], ids=lambda c: c["source"].split(" ")[0])
def test_pack_int8_rows_equals_pack_q8(case):
    c = np.array(case["codes"])
    a = oracle.pack_int8_rows(c.astype(np.int8), case["N"], case["K"])
    b = oracle.pack_q8(c.astype(np.int32), case["N"], case["K"])
    assert np.array_equal(a, b)


def le_view_pack(codes_i32, N, K):
    """Closed form: each row's int8 bytes, zero-padded to a multiple of 4,
    viewed as little-endian u32 -- computed by byte reinterpretation, not by
    shifting and masking."""
    W = (K + 3) // 4
    b = np.zeros((N, 4 * W), dtype=np.uint8)
    b[:, :K] = (np.asarray(codes_i32).reshape(N, K) & 0xFF).astype(np.uint8)
    return b.view("<u4").reshape(-1)


@pytest.mark.parametrize("N,K", [(1, 1), (3, 4), (5, 7), (7, 1027), (4, 4099), (2, 2)])
def test_pack_q8_is_le_byte_view(N, K):
    rng = np.random.default_rng(N * 1000 + K)
    codes = rng.integers(-300, 300, size=N * K, dtype=np.int32)  # & 0xff wraps out-of-range codes
    assert np.array_equal(oracle.pack_q8(codes, N, K), le_view_pack(codes, N, K))
    i8 = rng.integers(-128, 128, size=N * K).astype(np.int8)
    assert np.array_equal(oracle.pack_int8_rows(i8, N, K), le_view_pack(i8.astype(np.int32), N, K))


# ---------------------------------------------------------------- matvecQ8

@pytest.mark.parametrize("case", kat()["matvec_q8"], ids=lambda c: c["source"].split(" ")[0])
def test_matvec_q8_kat(case):
    N, K = case["N"], case["K"]
    w = oracle.pack_q8(np.array(case["codes"], dtype=np.int32), N, K)
    if "pad_patch" in case:
        w[case["pad_patch"]["word"]] |= np.uint32(int(case["pad_patch"]["or"], 16))
    y = oracle.matvec_q8(w, np.array(case["scale"], np.float32), np.array(case["vector"], np.float32), N, K)
    assert y.tolist() == case["want"]


def _unpack_le(weight, N, K):
    W = (K + 3) // 4
    return np.asarray(weight, dtype="<u4").reshape(N, W).view(np.int8)[:, :K].astype(np.float64)


@pytest.mark.parametrize("N,K", [(1, 3), (1, 8), (5, 1024), (3, 1030), (7, 1027), (2, 2600), (16, 4099)])
def test_matvec_q8_matches_f64_dot_product(N, K):
    # Same shapes as ops/matvec/q8.wgsl.test.ts:48.  The int8 codes come from a
    # byte view of the packed words (not the oracle's shift/mask), and numpy's
    # f64 matmul sums in its own order: both agree with the oracle to within
    # f64 rounding of the magnitude sum.
    rng = np.random.default_rng(K)
    codes = rng.integers(-127, 128, size=N * K, dtype=np.int32)
    w = le_view_pack(codes, N, K)
    s = rng.uniform(0.001, 0.05, N).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    y = oracle.matvec_q8(w, s, x, N, K)
    q = _unpack_le(w, N, K)
    want = (q @ x.astype(np.float64)) * s.astype(np.float64)
    bound = oracle.absterm(w, s, x, N, K)
    assert np.allclose(bound, (np.abs(q) @ np.abs(x.astype(np.float64))) * s, rtol=1e-12)
    assert np.all(np.abs(y.astype(np.float64) - want) <= np.abs(want) * 2.0 ** -23 + 1e-12 * bound + 1e-300)


def test_matvec_q8_structural_cases():
    # ops/matvec/q8.wgsl.test.ts:73-106: only columns past the first 1024 carry terms.
    N, K = 3, 1030
    codes = np.zeros((N, K), np.int32)
    x = np.zeros(K, np.float32)
    x[1027], x[K - 1] = 2, -3
    for r in range(N):
        codes[r, 1027] = 1 + r
        codes[r, K - 1] = 2 * (r + 1)
    s = np.array([0.027, 0.047, 0.067], np.float32)
    y = oracle.matvec_q8(oracle.pack_q8(codes, N, K), s, x, N, K)
    for r in range(N):
        want = ((1 + r) * 2.0 - 3.0 * 2 * (r + 1)) * np.float64(s[r])
        assert y[r] == np.float32(want)
    # q8.wgsl.test.ts:108-149: buffers longer than N*W words and K floats,
    # slack filled with sentinels; the answer must not see them.
    N, K = 4, 1023
    W = (K + 3) // 4
    codes = np.array([(i // K) % 5 + 1 for i in range(N * K)], np.int32)
    w = np.concatenate([oracle.pack_q8(codes, N, K), np.full(256, 0x7F7F7F7F, np.uint32)])
    x = np.concatenate([np.ones(K, np.float32), np.full(256, 1000, np.float32)])
    y = oracle.matvec_q8(w, np.ones(N, np.float32), x, N, K)
    assert y.tolist() == [float(K * (r % 5 + 1)) for r in range(N)]


def test_batched_is_m_independent_calls():
    rng = np.random.default_rng(3)
    N, K, M = 9, 77, 5
    w = le_view_pack(rng.integers(-127, 128, N * K), N, K)
    s = rng.uniform(0.01, 0.02, N).astype(np.float32)
    xs = rng.standard_normal((M, K)).astype(np.float32)
    ys = oracle.matvec_q8_batched(w, s, xs, N, K, M)
    for m in range(M):
        assert np.array_equal(ys[m], oracle.matvec_q8(w, s, xs[m], N, K))


# ---------------------------------------------------------------- fused decode forms

@pytest.mark.parametrize("case", kat()["matvec_q8_ffn"], ids=lambda c: c["source"].split(" ")[0])
def test_matvec_q8_ffn_kat(case):
    N, K = case["N"], case["K"]
    wg = oracle.pack_q8(np.array(case["gate_codes"], np.int32), N, K)
    wu = oracle.pack_q8(np.array(case["up_codes"], np.int32), N, K)
    y = oracle.matvec_q8_ffn(wg, np.array(case["scale_gate"], np.float32), wu, np.array(case["scale_up"], np.float32),
                             np.array(case["vector"], np.float32), N, K)
    assert np.all(np.abs(y.astype(np.float64) - np.array(case["want"])) < case["abs_tol"])


@pytest.mark.parametrize("case", kat()["matvec_q8_residual"], ids=lambda c: c["source"].split(" ")[0])
def test_matvec_q8_residual_kat(case):
    N, K = case["N"], case["K"]
    w = oracle.pack_q8(np.array(case["codes"], np.int32), N, K)
    y = oracle.matvec_q8_residual(w, np.array(case["scale"], np.float32), np.array(case["vector"], np.float32),
                                  np.array(case["residual"], np.float32), N, K)
    assert np.all(np.abs(y.astype(np.float64) - np.array(case["want"])) < case["abs_tol"])


def test_silu_closed_forms():
    # silu(0) = 0; silu is odd-symmetric around x/2: silu(x) - silu(-x) = x;
    # silu(-x) -> -0 for x past the f64 exp overflow; silu(x) -> x for large x.
    assert oracle.silu(0.0) == 0.0
    for x in (0.5, 1.0, 2.5, 7.0, 30.0):
        hi, lo = oracle.silu(x), oracle.silu(-x)
        assert abs((float(hi) - float(lo)) - x) <= 4 * np.spacing(np.float32(x))
    assert oracle.silu(-1000.0) == 0.0 and np.signbit(oracle.silu(-1000.0))
    assert oracle.silu(100.0) == 100.0
    assert np.isnan(oracle.silu(float("nan")))
    # the f32 rounding of the f64 value: 4 / (1 + e^-4)
    assert oracle.silu(4.0) == np.float32(4.0 / (1.0 + 0.01831563888873418))


def test_fused_forms_reduce_to_matvec():
    rng = np.random.default_rng(11)
    N, K = 13, 1031
    w = le_view_pack(rng.integers(-127, 128, N * K), N, K)
    s = rng.uniform(0.01, 0.05, N).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    y = oracle.matvec_q8(w, s, x, N, K)
    # zero residual: exactly the projection
    assert np.array_equal(oracle.matvec_q8_residual(w, s, x, np.zeros(N, np.float32), N, K), y)
    # residual add is an f32-rounded sum of two f32 values
    r = rng.standard_normal(N).astype(np.float32)
    assert np.array_equal(oracle.matvec_q8_residual(w, s, x, r, N, K),
                          (r.astype(np.float64) + y.astype(np.float64)).astype(np.float32))
    # gate == up: silu(y) * y
    f = oracle.matvec_q8_ffn(w, s, w, s, x, N, K)
    sy = np.array([oracle.silu(v) for v in y], np.float32)
    assert np.array_equal(f, (sy.astype(np.float64) * y.astype(np.float64)).astype(np.float32))


def test_fused_checks_reject_plausible_mistakes():
    # The tolerance checks the GPU is judged by must catch a gate/up swap, a
    # dropped residual and a residual added before the scale.
    rng = np.random.default_rng(12)
    N, K = 64, 512
    wg = le_view_pack(rng.integers(-127, 128, N * K), N, K)
    wu = le_view_pack(rng.integers(-127, 128, N * K), N, K)
    sg = rng.uniform(0.01, 0.05, N).astype(np.float32)
    su = rng.uniform(0.01, 0.05, N).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    g, u = oracle.matvec_q8(wg, sg, x, N, K), oracle.matvec_q8(wu, su, x, N, K)
    bg, bu = oracle.absterm(wg, sg, x, N, K), oracle.absterm(wu, su, x, N, K)
    good = oracle.matvec_q8_ffn(wg, sg, wu, su, x, N, K)
    assert oracle.check_ffn(good, g, u, bg, bu)[0]
    swapped = oracle.matvec_q8_ffn(wu, su, wg, sg, x, N, K)
    assert not oracle.check_ffn(swapped, g, u, bg, bu)[0]
    r = rng.standard_normal(N).astype(np.float32)
    res = oracle.matvec_q8_residual(wg, sg, x, r, N, K)
    assert oracle.check_residual(res, res, bg)[0]
    assert not oracle.check_residual(g, res, bg)[0]
    unscaled_first = ((oracle.matvec_q8(wg, np.ones(N, np.float32), x, N, K) + r) * sg).astype(np.float32)
    assert not oracle.check_residual(unscaled_first, res, bg)[0]


# ---------------------------------------------------------------- C vs ECMAScript

NODE = shutil.which("node")


def run_js(job):
    proc = subprocess.run([NODE, os.path.join(os.path.dirname(__file__), "node", "oracle_job.mjs")],
                          input=json.dumps(job).encode(), capture_output=True, check=True, timeout=120)
    return json.loads(proc.stdout)


def enc(a, dtype):
    return {"dtype": dtype, "b64": base64.b64encode(np.ascontiguousarray(a).tobytes()).decode()}


def dec(s, dtype):
    return np.frombuffer(base64.b64decode(s), dtype=dtype)


def tie_heavy_rows(rng, N, D):
    """Rows whose x * (127/absmax) products land on or within an ulp of .5."""
    x = rng.standard_normal((N, D)).astype(np.float32)
    for r in range(0, N, 2):
        absmax = np.float32(rng.uniform(0.5, 4.0))
        step = np.float64(absmax) / 127.0
        k = rng.integers(-126, 126, D).astype(np.float64)
        x[r] = (k + 0.5) * step
        x[r, 0] = absmax
    if N > 1:
        x[1, :min(4, D)] = [127.0, 62.5, -62.5, 0.5][:min(4, D)]
    return x


@pytest.mark.skipif(NODE is None, reason="node not on PATH")
def test_c_oracle_matches_ecmascript_oracle():
    rng = np.random.default_rng(11)
    N, D = 48, 517
    x = tie_heavy_rows(rng, N, D)
    x[5, 3] = np.nan
    x[6, 2] = np.inf
    x[7] = 0.0
    x[8] = 1e-40
    x[9, 1] = 0.005327165126800537
    x[9, 0] = 1.3530999422073364
    js = run_js({"op": "quantize", "N": N, "D": D, "arrays": {"input": enc(x, "f32")}})
    c_codes, c_scales = oracle.quantize(x, N, D)
    assert np.array_equal(dec(js["output"], np.int32), c_codes)
    js_scales = dec(js["scales"], np.float32)
    nan = np.isnan(c_scales)
    assert np.array_equal(np.isnan(js_scales), nan)
    assert np.array_equal(js_scales[~nan].view(np.uint32), c_scales[~nan].view(np.uint32))

    K = D
    codes = rng.integers(-300, 300, N * K, dtype=np.int32)
    js = run_js({"op": "packQ8", "N": N, "K": K, "arrays": {"codes": enc(codes, "i32")}})
    assert np.array_equal(dec(js["packed"], np.uint32), oracle.pack_q8(codes, N, K))
    i8 = codes.astype(np.int8)
    js = run_js({"op": "packInt8Rows", "N": N, "K": K, "arrays": {"codes": enc(i8, "i8")}})
    assert np.array_equal(dec(js["packed"], np.uint32), oracle.pack_int8_rows(i8, N, K))

    w = oracle.pack_q8(c_codes, N, K)
    vec = rng.standard_normal(K).astype(np.float32)
    js = run_js({"op": "matvecQ8", "N": N, "K": K,
                 "arrays": {"weight": enc(w, "u32"), "scale": enc(c_scales, "f32"), "vector": enc(vec, "f32")}})
    js_y = dec(js["output"], np.float32)
    c_y = oracle.matvec_q8(w, c_scales, vec, N, K)
    # Same f64 operations in the same order: equal bit for bit (NaN rows as NaN).
    assert np.array_equal(np.isnan(js_y), np.isnan(c_y))
    ok = ~np.isnan(c_y)
    assert np.array_equal(js_y[ok].view(np.uint32), c_y[ok].view(np.uint32))

    # fused forms: the same compositions (silu through V8's Math.exp and glibc's
    # exp, which agree after the f32 rounding on these rows)
    w2 = oracle.pack_q8(rng.integers(-127, 128, N * K, dtype=np.int32), N, K)
    s2 = rng.uniform(0.01, 0.5, N).astype(np.float32)
    vec = (4 * rng.standard_normal(K)).astype(np.float32)
    res = rng.standard_normal(N).astype(np.float32)
    js = run_js({"op": "matvecQ8Ffn", "N": N, "K": K,
                 "arrays": {"weightGate": enc(w, "u32"), "scaleGate": enc(c_scales, "f32"),
                            "weightUp": enc(w2, "u32"), "scaleUp": enc(s2, "f32"), "vector": enc(vec, "f32")}})
    js_f = dec(js["output"], np.float32)
    c_f = oracle.matvec_q8_ffn(w, c_scales, w2, s2, vec, N, K)
    assert np.array_equal(np.isnan(js_f), np.isnan(c_f))
    ok = ~np.isnan(c_f)
    assert np.array_equal(js_f[ok].view(np.uint32), c_f[ok].view(np.uint32))
    js = run_js({"op": "matvecQ8Residual", "N": N, "K": K,
                 "arrays": {"weight": enc(w2, "u32"), "scale": enc(s2, "f32"), "vector": enc(vec, "f32"),
                            "residual": enc(res, "f32")}})
    assert np.array_equal(dec(js["output"], np.float32).view(np.uint32),
                          oracle.matvec_q8_residual(w2, s2, vec, res, N, K).view(np.uint32))


# ---------------------------------------------------------------- the checks have teeth

def _mutant_quantize(x, rounding, f32_math=False):
    x64 = x.astype(np.float32 if f32_math else np.float64)
    absmax = np.max(np.abs(x64))
    inv = (127 / absmax) if absmax != 0 else 0
    v = x64 * (x64.dtype.type(inv))
    if rounding == "rint":
        c = np.rint(v)
    elif rounding == "floor_half":
        c = np.floor(v + 0.5)
    elif rounding == "away":
        c = np.sign(v) * np.floor(np.abs(v) + 0.5)
    else:
        f = np.floor(v)
        c = f + (v - f >= 0.5)
    return np.clip(c, -127, 127).astype(np.int32)


@pytest.mark.parametrize("mutant", [("rint", False), ("floor_half", False), ("away", False), ("js", True)])
def test_quantize_kats_reject_plausible_mistakes(mutant):
    rounding, f32_math = mutant
    cases = kat()["quantize"]
    failures = 0
    for case in cases:
        x = np.array(case["input"], dtype=np.float32)
        if _mutant_quantize(x, rounding, f32_math).tolist() != case["codes"]:
            failures += 1
    # the faithful rule passes every KAT; each mutant fails at least one
    faithful = all(_mutant_quantize(np.array(c["input"], np.float32), "js").tolist() == c["codes"] for c in cases)
    assert faithful
    if not f32_math:
        assert failures >= 1, rounding
    else:
        # f32 products differ from f64 only in rare rows: the tiny fixture
        # (106,496 codes) is what catches f32 arithmetic.
        caught = 0
        for name, N, K, w, want, _ in _tiny_q8_pairs():
            got = np.concatenate([_mutant_quantize(w[r * K:(r + 1) * K], "js", True) for r in range(N)])
            caught += int(np.sum(got != want))
        assert failures >= 1 or caught >= 1


def test_pack_kats_reject_byte_order_mistakes():
    for case in kat()["pack_q8"]:
        codes = np.array(case["codes"], np.int32)
        N, K = case["N"], case["K"]
        W = (K + 3) // 4
        b = np.zeros((N, 4 * W), np.uint8)
        b[:, :K] = (codes.reshape(N, K) & 0xFF).astype(np.uint8)
        big_endian = b.view(">u4").reshape(-1)
        if case["words"] != [f"0x{w:08x}" for w in big_endian.tolist()]:
            return
    pytest.fail("no packQ8 KAT distinguishes byte order")
