"""numpy front end of the C oracle (oracle/q8_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as the
checker, and by bench.py's cpu_baseline leg.  The product never imports it.

Functions mirror the reference's TypeScript definitions:
  quantize            ops/quantize/reference.ts:13-38
  pack_q8             ops/matvec/reference.ts:267-283
  pack_int8_rows      llm/weights-q8.ts:137-139
  matvec_q8           ops/matvec/reference.ts:113-131
  matvec_q8_batched   M x matvec_q8 (no reference function; defined that way)
  matvec_q8_residual  ops/matvec/reference.ts:235-243 (matvecQ8Residual)
  matvec_q8_ffn       ops/matvec/reference.ts:196-207 (matvecQ8Ffn)
  silu                ops/activation/reference.ts:91-92
  absterm             sum_k |s*q*x| per row in f64 (tolerance base)
  matmul_q8           ops/matmul/reference.ts:124-137 (matmulQ8)
  matmul_absterm      sum_k |a * fround(q*s)| per output in f64 (tolerance base)
  dequantize_packed_q8 llm/weights-q8.ts:161-177 (dequantizePackedQ8)
  dequant_transpose   ops/dequant_transpose/reference.ts:40-59 (dequantTranspose)
  gather_dequant_rows llm/weights-q8.ts:207-222 (gatherDequantRows)
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_q8.so")
_lib = None


def build() -> str:
    """Compiles the oracle with its Makefile (gcc, seconds)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    p = ctypes.c_void_p
    sz = ctypes.c_size_t
    lib.q8o_js_round.argtypes = [ctypes.c_double]
    lib.q8o_js_round.restype = ctypes.c_double
    lib.q8o_quantize.argtypes = [p, sz, sz, p, p]
    lib.q8o_pack_q8.argtypes = [p, sz, sz, p]
    lib.q8o_pack_int8_rows.argtypes = [p, sz, sz, p]
    lib.q8o_matvec_q8.argtypes = [p, p, p, sz, sz, p]
    lib.q8o_matvec_q8_batched.argtypes = [p, p, p, sz, sz, sz, p]
    lib.q8o_matvec_q8_absterm.argtypes = [p, p, p, sz, sz, p]
    lib.q8o_matvec_q8_residual.argtypes = [p, p, p, p, sz, sz, p]
    lib.q8o_matvec_q8_ffn.argtypes = [p, p, p, p, p, sz, sz, p]
    lib.q8o_silu.argtypes = [ctypes.c_float]
    lib.q8o_silu.restype = ctypes.c_float
    lib.q8o_matmul_q8.argtypes = [p, p, p, sz, sz, sz, p]
    lib.q8o_matmul_q8_absterm.argtypes = [p, p, p, sz, sz, sz, p]
    lib.q8o_dequantize_packed_q8.argtypes = [p, p, sz, sz, p]
    lib.q8o_dequant_transpose.argtypes = [p, p, sz, sz, p]
    lib.q8o_gather_dequant_rows.argtypes = [p, p, sz, sz, p, sz, p]
    for name in ("q8o_quantize", "q8o_pack_q8", "q8o_pack_int8_rows", "q8o_matvec_q8",
                 "q8o_matvec_q8_batched", "q8o_matvec_q8_absterm", "q8o_matvec_q8_residual",
                 "q8o_matvec_q8_ffn", "q8o_matmul_q8", "q8o_matmul_q8_absterm", "q8o_dequantize_packed_q8",
                 "q8o_dequant_transpose", "q8o_gather_dequant_rows"):
        getattr(lib, name).restype = None
    _lib = lib
    return lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def words_per_row(K: int) -> int:
    return (K + 3) // 4


def js_round(v: float) -> float:
    return _load().q8o_js_round(float(v))


def quantize(inp: np.ndarray, N: int, D: int) -> tuple[np.ndarray, np.ndarray]:
    x = np.ascontiguousarray(inp, dtype=np.float32).reshape(-1)
    assert x.size >= N * D
    out = np.empty(N * D, dtype=np.int32)
    scales = np.empty(N, dtype=np.float32)
    _load().q8o_quantize(_ptr(x), N, D, _ptr(out), _ptr(scales))
    return out, scales


def pack_q8(codes: np.ndarray, N: int, K: int) -> np.ndarray:
    c = np.ascontiguousarray(codes, dtype=np.int32).reshape(-1)
    assert c.size >= N * K
    out = np.empty(N * words_per_row(K), dtype=np.uint32)
    _load().q8o_pack_q8(_ptr(c), N, K, _ptr(out))
    return out


def pack_int8_rows(codes: np.ndarray, N: int, K: int) -> np.ndarray:
    c = np.ascontiguousarray(codes, dtype=np.int8).reshape(-1)
    assert c.size >= N * K
    out = np.empty(N * words_per_row(K), dtype=np.uint32)
    _load().q8o_pack_int8_rows(_ptr(c), N, K, _ptr(out))
    return out


def matvec_q8(weight: np.ndarray, scale: np.ndarray, vector: np.ndarray, N: int, K: int) -> np.ndarray:
    w = np.ascontiguousarray(weight, dtype=np.uint32).reshape(-1)
    s = np.ascontiguousarray(scale, dtype=np.float32).reshape(-1)
    v = np.ascontiguousarray(vector, dtype=np.float32).reshape(-1)
    assert w.size >= N * words_per_row(K) and s.size >= N and v.size >= K
    out = np.empty(N, dtype=np.float32)
    _load().q8o_matvec_q8(_ptr(w), _ptr(s), _ptr(v), N, K, _ptr(out))
    return out


def matvec_q8_batched(weight, scale, vectors, N: int, K: int, M: int) -> np.ndarray:
    w = np.ascontiguousarray(weight, dtype=np.uint32).reshape(-1)
    s = np.ascontiguousarray(scale, dtype=np.float32).reshape(-1)
    v = np.ascontiguousarray(vectors, dtype=np.float32).reshape(-1)
    assert w.size >= N * words_per_row(K) and s.size >= N and v.size >= M * K
    out = np.empty(M * N, dtype=np.float32)
    _load().q8o_matvec_q8_batched(_ptr(w), _ptr(s), _ptr(v), N, K, M, _ptr(out))
    return out.reshape(M, N)


def matvec_q8_residual(weight, scale, vector, residual, N: int, K: int) -> np.ndarray:
    w = np.ascontiguousarray(weight, dtype=np.uint32).reshape(-1)
    s = np.ascontiguousarray(scale, dtype=np.float32).reshape(-1)
    v = np.ascontiguousarray(vector, dtype=np.float32).reshape(-1)
    r = np.ascontiguousarray(residual, dtype=np.float32).reshape(-1)
    assert w.size >= N * words_per_row(K) and s.size >= N and v.size >= K and r.size >= N
    out = np.empty(N, dtype=np.float32)
    _load().q8o_matvec_q8_residual(_ptr(w), _ptr(s), _ptr(v), _ptr(r), N, K, _ptr(out))
    return out


def matvec_q8_ffn(weight_gate, scale_gate, weight_up, scale_up, vector, N: int, K: int) -> np.ndarray:
    wg = np.ascontiguousarray(weight_gate, dtype=np.uint32).reshape(-1)
    sg = np.ascontiguousarray(scale_gate, dtype=np.float32).reshape(-1)
    wu = np.ascontiguousarray(weight_up, dtype=np.uint32).reshape(-1)
    su = np.ascontiguousarray(scale_up, dtype=np.float32).reshape(-1)
    v = np.ascontiguousarray(vector, dtype=np.float32).reshape(-1)
    W = words_per_row(K)
    assert wg.size >= N * W and wu.size >= N * W and sg.size >= N and su.size >= N and v.size >= K
    out = np.empty(N, dtype=np.float32)
    _load().q8o_matvec_q8_ffn(_ptr(wg), _ptr(sg), _ptr(wu), _ptr(su), _ptr(v), N, K, _ptr(out))
    return out


def silu(x: float) -> float:
    return float(_load().q8o_silu(float(x)))


def absterm(weight, scale, vector, N: int, K: int) -> np.ndarray:
    w = np.ascontiguousarray(weight, dtype=np.uint32).reshape(-1)
    s = np.ascontiguousarray(scale, dtype=np.float32).reshape(-1)
    v = np.ascontiguousarray(vector, dtype=np.float32).reshape(-1)
    out = np.empty(N, dtype=np.float64)
    _load().q8o_matvec_q8_absterm(_ptr(w), _ptr(s), _ptr(v), N, K, _ptr(out))
    return out


def matmul_q8(a, weight, scale, N: int, M: int, K: int) -> np.ndarray:
    """ops/matmul/reference.ts:124-137: a [N, K], weight [M, W] -> f32 [N, M]."""
    av = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
    w = np.ascontiguousarray(weight, dtype=np.uint32).reshape(-1)
    s = np.ascontiguousarray(scale, dtype=np.float32).reshape(-1)
    assert av.size >= N * K and w.size >= M * words_per_row(K) and s.size >= M
    out = np.empty(N * M, dtype=np.float32)
    _load().q8o_matmul_q8(_ptr(av), _ptr(w), _ptr(s), N, M, K, _ptr(out))
    return out.reshape(N, M)


def matmul_absterm(a, weight, scale, N: int, M: int, K: int) -> np.ndarray:
    av = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
    w = np.ascontiguousarray(weight, dtype=np.uint32).reshape(-1)
    s = np.ascontiguousarray(scale, dtype=np.float32).reshape(-1)
    out = np.empty(N * M, dtype=np.float64)
    _load().q8o_matmul_q8_absterm(_ptr(av), _ptr(w), _ptr(s), N, M, K, _ptr(out))
    return out.reshape(N, M)


def dequantize_packed_q8(weight, scale, N: int, K: int) -> np.ndarray:
    w = np.ascontiguousarray(weight, dtype=np.uint32).reshape(-1)
    s = np.ascontiguousarray(scale, dtype=np.float32).reshape(-1)
    assert w.size >= N * words_per_row(K) and s.size >= N
    out = np.empty(N * K, dtype=np.float32)
    _load().q8o_dequantize_packed_q8(_ptr(w), _ptr(s), N, K, _ptr(out))
    return out


def dequant_transpose(weight, scale, out_features: int, in_features: int) -> np.ndarray:
    w = np.ascontiguousarray(weight, dtype=np.uint32).reshape(-1)
    s = np.ascontiguousarray(scale, dtype=np.float32).reshape(-1)
    assert w.size >= out_features * words_per_row(in_features) and s.size >= out_features
    out = np.empty(out_features * in_features, dtype=np.float32)
    _load().q8o_dequant_transpose(_ptr(w), _ptr(s), out_features, in_features, _ptr(out))
    return out


def gather_dequant_rows(codes, scale, rows: int, D: int, indices) -> np.ndarray:
    c = np.ascontiguousarray(codes, dtype=np.int8).reshape(-1)
    s = np.ascontiguousarray(scale, dtype=np.float32).reshape(-1)
    ix = np.ascontiguousarray(indices, dtype=np.int64).reshape(-1)
    assert c.size >= rows * D and s.size >= rows
    out = np.empty(ix.size * D, dtype=np.float32)
    _load().q8o_gather_dequant_rows(_ptr(c), _ptr(s), rows, D, _ptr(ix), ix.size, _ptr(out))
    return out


# Output tolerance of the f32 kernels against the f64 reference, per row:
# |y - y_ref| <= REL * sum_k |s*q*x| + ABS.
REL = 1e-5
ABS = 1e-7


def check_matvec(got: np.ndarray, want: np.ndarray, bound: np.ndarray) -> tuple[bool, str]:
    """Returns (ok, worst-offender report) in the shape of harness/agree.ts:27-46."""
    got = np.asarray(got, dtype=np.float64).reshape(-1)
    want = np.asarray(want, dtype=np.float64).reshape(-1)
    bound = np.asarray(bound, dtype=np.float64).reshape(-1)
    if got.shape != want.shape:
        return False, f"length mismatch: got {got.size}, want {want.size}"
    both_nan = np.isnan(got) & np.isnan(want)
    same_inf = np.isinf(got) & np.isinf(want) & (np.sign(got) == np.sign(want))
    with np.errstate(invalid="ignore"):
        err = np.abs(got - want)
        allowed = REL * bound + ABS
        bad = ~(both_nan | same_inf | (err <= allowed))
    if not bad.any():
        return True, "ok"
    idx = np.flatnonzero(bad)
    with np.errstate(invalid="ignore", divide="ignore"):
        ratio = np.where(np.isfinite(err[idx]), err[idx] / allowed[idx], np.inf)
    worst = idx[int(np.nanargmax(ratio))] if ratio.size else idx[0]
    return False, (f"{idx.size} rows out of tolerance; worst row {worst}: got {got[worst]!r} "
                   f"want {want[worst]!r} |err| {err[worst]:.3e} allowed {allowed[worst]:.3e}")


def _ulp32(v: np.ndarray) -> np.ndarray:
    """Spacing of f32 numbers at |v| (the size of one f32 rounding step)."""
    a = np.abs(np.asarray(v, dtype=np.float64)).astype(np.float32)
    return np.spacing(a).astype(np.float64)


def _report(got, want, allowed, what: str) -> tuple[bool, str]:
    got = np.asarray(got, dtype=np.float64).reshape(-1)
    want = np.asarray(want, dtype=np.float64).reshape(-1)
    if got.shape != want.shape:
        return False, f"length mismatch: got {got.size}, want {want.size}"
    both_nan = np.isnan(got) & np.isnan(want)
    same_inf = np.isinf(got) & np.isinf(want) & (np.sign(got) == np.sign(want))
    with np.errstate(invalid="ignore"):
        err = np.abs(got - want)
        bad = ~(both_nan | same_inf | (err <= allowed))
    if not bad.any():
        return True, "ok"
    idx = np.flatnonzero(bad)
    with np.errstate(invalid="ignore", divide="ignore"):
        ratio = np.where(np.isfinite(err[idx]), err[idx] / allowed[idx], np.inf)
    worst = idx[int(np.nanargmax(ratio))] if ratio.size else idx[0]
    return False, (f"{what}: {idx.size} rows out of tolerance; worst row {worst}: got {got[worst]!r} "
                   f"want {want[worst]!r} |err| {err[worst]:.3e} allowed {allowed[worst]:.3e}")


def check_residual(got, want, bound) -> tuple[bool, str]:
    """matvecQ8Residual: the projection's bar (REL * sum|s q x| + ABS) carried
    through the f32 residual add, plus one f32 rounding step of the output
    (the add may round the other way when the projection differs)."""
    bound = np.asarray(bound, dtype=np.float64).reshape(-1)
    allowed = REL * bound + ABS + _ulp32(want)
    return _report(got, want, allowed, "matvecQ8Residual")


# max |silu'(x)| over the reals (attained near x = 2.40)
SILU_SLOPE = 1.0999


def check_ffn(got, gate, up, bound_gate, bound_up) -> tuple[bool, str]:
    """matvecQ8Ffn against its oracle components (gate, up: the oracle's f32
    matvecQ8 rows; bound_*: sum|s q x| per row).  Each projection may be off by
    its bar e = REL * bound + ABS; through out = silu(g) * u that moves the
    output by at most |silu'| e_g |u| + |silu(g)| e_u + |silu'| e_g e_u, plus
    one f32 rounding step of silu(g) (times |u|) and one of the product."""
    g = np.asarray(gate, dtype=np.float32).reshape(-1)
    u = np.asarray(up, dtype=np.float32).reshape(-1).astype(np.float64)
    eg = REL * np.asarray(bound_gate, dtype=np.float64).reshape(-1) + ABS
    eu = REL * np.asarray(bound_up, dtype=np.float64).reshape(-1) + ABS
    sg = np.array([silu(v) for v in g], dtype=np.float32)
    want = (sg.astype(np.float64) * u).astype(np.float32)
    allowed = (SILU_SLOPE * eg * np.abs(u) + np.abs(sg.astype(np.float64)) * eu + SILU_SLOPE * eg * eu
               + _ulp32(sg) * np.abs(u) + _ulp32(want))
    return _report(got, want, allowed, "matvecQ8Ffn")
