"""Python host binding of the gfx950 matvecQ8 library (ctypes over include/wxo_q8.h).

Mirrors the reference's TypeScript op API for this path, same names and
argument meaning:

    matvecQ8(weight=, scale=, vector=, N=, K=)  -> f32 [N]     ops/matvec/reference.ts:117
    packQ8(codes=, N=, K=)                      -> u32 [N*W]   ops/matvec/reference.ts:267
    quantize(input=, N=, D=)                    -> (i32 codes, f32 scales)  ops/quantize/reference.ts:13
    packInt8Rows(codes, N, K)                   -> u32 [N*W]   llm/weights-q8.ts:137
    matmulQ8(a=, weight=, scale=, N=, M=, K=)   -> f32 [N, M]  ops/matmul/reference.ts:124
    dequantizePackedQ8(weight, scale, N, K)     -> f32 [N*K]   llm/weights-q8.ts:161
    dequantTranspose(weight=, scale=, outFeatures=, inFeatures=) -> f32 [inF*outF]
                                                               ops/dequant_transpose/reference.ts:40
    gatherDequantRows(table, indices, D)        -> f32 [len*D] llm/weights-q8.ts:207

plus the batched form matvecQ8Batched (M vectors), the fused
quantizePackQ8, and device-resident buffers (DeviceBuffer) with
stream-ordered entry points for callers that keep weights in HBM
(harness/resident.ts:98-145).

There is no CPU fallback: without the built library or a gfx950 GPU every
call raises WxoError.  The one difference from the reference's behaviour is
deliberate: argument sizes are validated (the reference reads `undefined` ->
NaN on short inputs); a mismatch raises WxoError instead.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG, "lib", "libwxo_q8.so")

WXO_OK = 0
WXO_ERR_INVALID = 1
WXO_ERR_NO_DEVICE = 2
WXO_ERR_DEVICE = 3
WXO_ERR_OOM = 4

# Every symbol include/wxo_q8.h declares, with its ctypes signature.
_P, _U32, _SZ, _I = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_size_t, ctypes.c_int
SIGNATURES = {
    "wxo_abi_version": ([], _I),
    "wxo_last_error": ([], ctypes.c_char_p),
    "wxo_last_variant": ([], ctypes.c_char_p),
    "wxo_init": ([], _I),
    "wxo_describe": ([], ctypes.c_char_p),
    "wxo_device_count": ([ctypes.POINTER(_I)], _I),
    "wxo_set_device": ([_I], _I),
    "wxo_malloc": ([ctypes.POINTER(_P), _SZ], _I),
    "wxo_free": ([_P], _I),
    "wxo_memcpy_htod": ([_P, _P, _SZ, _P], _I),
    "wxo_memcpy_dtoh": ([_P, _P, _SZ, _P], _I),
    "wxo_memcpy_dtoh_async": ([_P, _P, _SZ, _P], _I),
    "wxo_host_malloc": ([ctypes.POINTER(_P), _SZ], _I),
    "wxo_host_free": ([_P], _I),
    "wxo_memcpy_dtod": ([_P, _P, _SZ, _P], _I),
    "wxo_memset": ([_P, _I, _SZ, _P], _I),
    "wxo_synchronize": ([], _I),
    "wxo_stream_create": ([ctypes.POINTER(_P)], _I),
    "wxo_stream_destroy": ([_P], _I),
    "wxo_stream_synchronize": ([_P], _I),
    "wxo_event_create": ([ctypes.POINTER(_P)], _I),
    "wxo_event_create_timer": ([ctypes.POINTER(_P)], _I),
    "wxo_spin": ([ctypes.c_uint32, _P], _I),
    "wxo_gate_hold": ([ctypes.c_uint32, _P, ctypes.POINTER(ctypes.c_uint32)], _I),
    "wxo_gate_release": ([ctypes.c_uint32], _I),
    "wxo_roofline": ([ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)], _I),
    "wxo_roofline_matrix": ([ctypes.POINTER(ctypes.c_double)], _I),
    "wxo_matmul_q8_multi": ([_P, _P, _P, _P, _P, _U32, _U32, _U32, _P], _I),
    "wxo_matmul_q8_multi_ws": ([_P, _P, _P, _P, _P, _U32, _U32, _U32, _P, _SZ, _P], _I),
    "wxo_matmul_q8_workspace_bytes": ([ctypes.POINTER(_SZ)], _I),
    "wxo_matmul_q8_multi_static": ([_P, _P, _P, _P, _P, _U32, _U32, _U32, _P], _I),
    "wxo_graph_capture_begin": ([_P], _I),
    "wxo_graph_capture_end": ([_P, ctypes.POINTER(_P)], _I),
    "wxo_graph_launch": ([_P, _P], _I),
    "wxo_graph_destroy": ([_P], _I),
    "wxo_event_destroy": ([_P], _I),
    "wxo_event_record": ([_P, _P], _I),
    "wxo_event_synchronize": ([_P], _I),
    "wxo_event_elapsed_ms": ([ctypes.POINTER(ctypes.c_float), _P, _P], _I),
    "wxo_matvec_q8": ([_P, _P, _P, _P, _U32, _U32, _U32, _P], _I),
    "wxo_matvec_q8_multi": ([_P, _P, _P, _P, _U32, _P, _U32, _P], _I),
    "wxo_matvec_q8_residual": ([_P, _P, _P, _P, _P, _U32, _U32, _P], _I),
    "wxo_matvec_q8_ffn": ([_P, _P, _P, _P, _P, _P, _U32, _U32, _P], _I),
    "wxo_quantize": ([_P, _U32, _U32, _P, _P, _P], _I),
    "wxo_pack_q8": ([_P, _U32, _U32, _P, _P], _I),
    "wxo_pack_int8_rows": ([_P, _U32, _U32, _P, _P], _I),
    "wxo_quantize_pack_q8": ([_P, _U32, _U32, _P, _P, _P], _I),
    "wxo_matvec_q8_host": ([_P, _P, _P, _P, _U32, _U32, _U32], _I),
    "wxo_matvec_q8_residual_host": ([_P, _P, _P, _P, _P, _U32, _U32], _I),
    "wxo_matvec_q8_ffn_host": ([_P, _P, _P, _P, _P, _P, _U32, _U32], _I),
    "wxo_quantize_host": ([_P, _U32, _U32, _P, _P], _I),
    "wxo_pack_q8_host": ([_P, _U32, _U32, _P], _I),
    "wxo_pack_int8_rows_host": ([_P, _U32, _U32, _P], _I),
    "wxo_quantize_pack_q8_host": ([_P, _U32, _U32, _P, _P], _I),
    "wxo_matmul_q8": ([_P, _P, _P, _P, _U32, _U32, _U32, _P], _I),
    "wxo_quantize_pack_q8_multi": ([_P, _P, _P, _P, _U32, _U32, _P], _I),
    "wxo_dequantize_packed_q8": ([_P, _P, _U32, _U32, _P, _P], _I),
    "wxo_dequant_transpose": ([_P, _P, _U32, _U32, _P, _P], _I),
    "wxo_gather_dequant_rows": ([_P, _P, _U32, _U32, _P, _U32, _P, _P], _I),
    "wxo_matmul_q8_host": ([_P, _P, _P, _P, _U32, _U32, _U32], _I),
    "wxo_dequantize_packed_q8_host": ([_P, _P, _U32, _U32, _P], _I),
    "wxo_dequant_transpose_host": ([_P, _P, _U32, _U32, _P], _I),
    "wxo_gather_dequant_rows_host": ([_P, _P, _U32, _U32, _P, _U32, _P], _I),
}


class WxoError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"wxo status {status}: {message}")
        self.status = status


_lib = None


def lib():
    """Loads lib/libwxo_q8.so (built by web-xpu-ops_amd/build.py)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise WxoError(WXO_ERR_NO_DEVICE, f"{LIB_PATH} is not built; run web-xpu-ops_amd/build.py "
                                              "(the matvecQ8 path has no CPU fallback)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        _lib = handle
    return _lib


def _check(status: int) -> None:
    if status != WXO_OK:
        raise WxoError(status, lib().wxo_last_error().decode(errors="replace"))


def describe() -> str:
    return lib().wxo_describe().decode()


def last_variant() -> str:
    """The kernel instance this thread's last successful op launched."""
    return lib().wxo_last_variant().decode()


def device_count() -> int:
    n = ctypes.c_int(0)
    _check(lib().wxo_device_count(ctypes.byref(n)))
    return n.value


def init() -> None:
    _check(lib().wxo_init())


def roofline(bandwidth: bool = True, compute: bool = True) -> dict:
    """This device's own ceilings, measured now (harness/roofline.ts:162-198):
    {"bandwidth": best sustained HBM read bytes/s, "compute": best sustained
    one-wide f32 FMA flop/s}; a part not asked for is None."""
    bw, fl = ctypes.c_double(0.0), ctypes.c_double(0.0)
    _check(lib().wxo_roofline(ctypes.byref(bw) if bandwidth else None, ctypes.byref(fl) if compute else None))
    return {"bandwidth": bw.value if bandwidth else None, "compute": fl.value if compute else None}


def roofline_matrix() -> float:
    """The sustained bf16 matrix-core rate in flop/s with matmulQ8-like
    operands, measured now (wxo_roofline_matrix)."""
    fl = ctypes.c_double(0.0)
    _check(lib().wxo_roofline_matrix(ctypes.byref(fl)))
    return fl.value


def words_per_row(K: int) -> int:
    return (int(K) + 3) // 4


# ------------------------------------------------------------------ device memory

class DeviceBuffer:
    """A device allocation (hipMalloc) with explicit free; `ptr` is the device address."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p(0)
        _check(lib().wxo_malloc(ctypes.byref(p), self.nbytes))
        self.ptr = p.value or 0

    @classmethod
    def from_array(cls, arr: np.ndarray, stream=None) -> "DeviceBuffer":
        a = np.ascontiguousarray(arr)
        buf = cls(a.nbytes)
        buf.upload(a, stream)
        return buf

    def upload(self, arr: np.ndarray, stream=None, offset: int = 0) -> None:
        a = np.ascontiguousarray(arr)
        if offset + a.nbytes > self.nbytes:
            raise WxoError(WXO_ERR_INVALID, f"upload of {a.nbytes} B at {offset} overflows {self.nbytes} B buffer")
        _check(lib().wxo_memcpy_htod(self.ptr + offset, a.ctypes.data, a.nbytes, _stream_ptr(stream)))

    def download(self, dtype, count: int, stream=None, offset: int = 0) -> np.ndarray:
        out = np.empty(int(count), dtype=dtype)
        if offset + out.nbytes > self.nbytes:
            raise WxoError(WXO_ERR_INVALID, f"download of {out.nbytes} B at {offset} overflows {self.nbytes} B buffer")
        _check(lib().wxo_memcpy_dtoh(out.ctypes.data, self.ptr + offset, out.nbytes, _stream_ptr(stream)))
        return out

    def free(self) -> None:
        if self.ptr:
            _check(lib().wxo_free(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            if self.ptr and _lib is not None:
                _lib.wxo_free(self.ptr)
        except Exception:
            pass


class Stream:
    def __init__(self):
        p = ctypes.c_void_p(0)
        _check(lib().wxo_stream_create(ctypes.byref(p)))
        self.handle = p.value

    def synchronize(self) -> None:
        _check(lib().wxo_stream_synchronize(self.handle))

    def destroy(self) -> None:
        if self.handle:
            _check(lib().wxo_stream_destroy(self.handle))
            self.handle = None


class Graph:
    """Ops of this library captured once on a stream and replayed
    (wxo_graph_capture_begin/_end, wxo_graph_launch)."""

    def __init__(self, handle):
        self.handle = handle

    @staticmethod
    def capture(stream: "Stream", record) -> "Graph":
        """Runs `record()` with `stream` capturing, and returns the graph; the
        capture is closed whatever `record` does."""
        _check(lib().wxo_graph_capture_begin(stream.handle))
        p = ctypes.c_void_p(0)
        try:
            record()
        except BaseException:
            # Close the capture and free whatever it instantiated; the error
            # raised by `record` is the one reported.
            if lib().wxo_graph_capture_end(stream.handle, ctypes.byref(p)) == WXO_OK and p.value:
                lib().wxo_graph_destroy(p)
            raise
        _check(lib().wxo_graph_capture_end(stream.handle, ctypes.byref(p)))
        return Graph(p.value)

    def launch(self, stream: "Stream") -> None:
        _check(lib().wxo_graph_launch(self.handle, stream.handle))

    def destroy(self) -> None:
        if self.handle:
            _check(lib().wxo_graph_destroy(self.handle))
            self.handle = None


class Event:
    def __init__(self, timer: bool = False):
        """timer=True: a timing-only event (wxo_event_create_timer, no fence)."""
        p = ctypes.c_void_p(0)
        _check((lib().wxo_event_create_timer if timer else lib().wxo_event_create)(ctypes.byref(p)))
        self.handle = p.value

    def record(self, stream=None) -> None:
        _check(lib().wxo_event_record(self.handle, _stream_ptr(stream)))

    def synchronize(self) -> None:
        _check(lib().wxo_event_synchronize(self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float(0)
        _check(lib().wxo_event_elapsed_ms(ctypes.byref(ms), self.handle, end.handle))
        return float(ms.value)

    def destroy(self) -> None:
        if self.handle:
            _check(lib().wxo_event_destroy(self.handle))
            self.handle = None


def _stream_ptr(stream) -> int | None:
    if stream is None:
        return None
    return stream.handle if isinstance(stream, Stream) else int(stream)


def synchronize() -> None:
    _check(lib().wxo_synchronize())


def _addr(x) -> int:
    if isinstance(x, DeviceBuffer):
        return x.ptr
    return int(x)


# ------------------------------------------------------------------ device-pointer ops

def matvec_q8_device(weight, scale, vector, output, N: int, K: int, M: int = 1, stream=None) -> None:
    _check(lib().wxo_matvec_q8(_addr(weight), _addr(scale), _addr(vector), _addr(output), N, K, M,
                               _stream_ptr(stream)))


def matmul_q8_multi_device(a, projections, N: int, K: int, stream=None, workspace=None,
                           workspace_bytes: int = 0) -> None:
    """projections: a sequence of (weight, scale, output, M) on the same
    activations a [N, K]; one launch per 4.  With a workspace (a device buffer
    or address and its size in bytes), short prompts split each tile's K steps
    between workgroups (wxo_matmul_q8_multi_ws)."""
    n = len(projections)
    ws = (ctypes.c_void_p * max(n, 1))(*[_addr(p[0]) for p in projections])
    ss = (ctypes.c_void_p * max(n, 1))(*[_addr(p[1]) for p in projections])
    ys = (ctypes.c_void_p * max(n, 1))(*[_addr(p[2]) for p in projections])
    ms = (ctypes.c_uint32 * max(n, 1))(*[int(p[3]) for p in projections])
    if workspace is None:
        _check(lib().wxo_matmul_q8_multi(_addr(a), ws, ss, ys, ms, n, N, K, _stream_ptr(stream)))
    else:
        _check(lib().wxo_matmul_q8_multi_ws(_addr(a), ws, ss, ys, ms, n, N, K, _addr(workspace), workspace_bytes,
                                            _stream_ptr(stream)))


def matmul_q8_multi_static_device(a, projections, N: int, K: int, stream=None) -> None:
    """matmul_q8_multi_device with the library's own workspace
    (wxo_matmul_q8_multi_static): allocates nothing; calls that overlap in
    time on one GPU race."""
    n = len(projections)
    ws = (ctypes.c_void_p * max(n, 1))(*[_addr(p[0]) for p in projections])
    ss = (ctypes.c_void_p * max(n, 1))(*[_addr(p[1]) for p in projections])
    ys = (ctypes.c_void_p * max(n, 1))(*[_addr(p[2]) for p in projections])
    ms = (ctypes.c_uint32 * max(n, 1))(*[int(p[3]) for p in projections])
    _check(lib().wxo_matmul_q8_multi_static(_addr(a), ws, ss, ys, ms, n, N, K, _stream_ptr(stream)))


def matmul_q8_workspace_bytes() -> int:
    """The workspace size that allows every split of wxo_matmul_q8_multi_ws on the current device."""
    b = ctypes.c_size_t(0)
    _check(lib().wxo_matmul_q8_workspace_bytes(ctypes.byref(b)))
    return b.value


def matvec_q8_multi_device(projections, vector, K: int, stream=None) -> None:
    """projections: a sequence of (weight, scale, output, N); one launch per 4."""
    n = len(projections)
    ws = (ctypes.c_void_p * max(n, 1))(*[_addr(p[0]) for p in projections])
    ss = (ctypes.c_void_p * max(n, 1))(*[_addr(p[1]) for p in projections])
    ys = (ctypes.c_void_p * max(n, 1))(*[_addr(p[2]) for p in projections])
    ns = (ctypes.c_uint32 * max(n, 1))(*[int(p[3]) for p in projections])
    _check(lib().wxo_matvec_q8_multi(ws, ss, ys, ns, n, _addr(vector), K, _stream_ptr(stream)))


def matvec_q8_residual_device(weight, scale, vector, residual, output, N: int, K: int, stream=None) -> None:
    _check(lib().wxo_matvec_q8_residual(_addr(weight), _addr(scale), _addr(vector), _addr(residual),
                                        _addr(output), N, K, _stream_ptr(stream)))


def matvec_q8_ffn_device(weight_gate, scale_gate, weight_up, scale_up, vector, output, N: int, K: int,
                         stream=None) -> None:
    _check(lib().wxo_matvec_q8_ffn(_addr(weight_gate), _addr(scale_gate), _addr(weight_up), _addr(scale_up),
                                   _addr(vector), _addr(output), N, K, _stream_ptr(stream)))


def quantize_device(inp, N: int, D: int, output, scales, stream=None) -> None:
    _check(lib().wxo_quantize(_addr(inp), N, D, _addr(output), _addr(scales), _stream_ptr(stream)))


def quantize_pack_q8_multi_device(matrices, K: int, stream=None) -> None:
    """matrices: a sequence of (input, N, packed, scales); one launch per 8."""
    n = len(matrices)
    ins = (ctypes.c_void_p * max(n, 1))(*[_addr(m[0]) for m in matrices])
    ns = (ctypes.c_uint32 * max(n, 1))(*[int(m[1]) for m in matrices])
    ps = (ctypes.c_void_p * max(n, 1))(*[_addr(m[2]) for m in matrices])
    ss = (ctypes.c_void_p * max(n, 1))(*[_addr(m[3]) for m in matrices])
    _check(lib().wxo_quantize_pack_q8_multi(ins, ns, ps, ss, n, K, _stream_ptr(stream)))


def pack_q8_device(codes, N: int, K: int, packed, stream=None) -> None:
    _check(lib().wxo_pack_q8(_addr(codes), N, K, _addr(packed), _stream_ptr(stream)))


def pack_int8_rows_device(codes, N: int, K: int, packed, stream=None) -> None:
    _check(lib().wxo_pack_int8_rows(_addr(codes), N, K, _addr(packed), _stream_ptr(stream)))


def quantize_pack_q8_device(inp, N: int, K: int, packed, scales, stream=None) -> None:
    _check(lib().wxo_quantize_pack_q8(_addr(inp), N, K, _addr(packed), _addr(scales), _stream_ptr(stream)))


# ------------------------------------------------------------------ the reference's op API

def _need(arr, dtype, count: int, name: str) -> np.ndarray:
    a = np.ascontiguousarray(arr, dtype=dtype).reshape(-1)
    if a.size < count:
        raise WxoError(WXO_ERR_INVALID, f"{name} has {a.size} elements, {count} needed")
    return a


def matvecQ8(*, weight, scale, vector, N: int, K: int) -> np.ndarray:
    """ops/matvec/reference.ts:117 -- y[n] = (sum_k q[n,k] x[k]) * scale[n], f32 [N]."""
    return matvecQ8Batched(weight=weight, scale=scale, vectors=vector, N=N, K=K, M=1).reshape(-1)


def matvecQ8Batched(*, weight, scale, vectors, N: int, K: int, M: int) -> np.ndarray:
    """M independent matvecQ8 calls on one weight: vectors [M, K] -> f32 [M, N]."""
    w = _need(weight, np.uint32, N * words_per_row(K), "weight")
    s = _need(scale, np.float32, N, "scale")
    x = _need(vectors, np.float32, M * K, "vector")
    out = np.empty(M * N, dtype=np.float32)
    _check(lib().wxo_matvec_q8_host(w.ctypes.data, s.ctypes.data, x.ctypes.data, out.ctypes.data, N, K, M))
    return out.reshape(M, N)


def matvecQ8Residual(*, weight, scale, vector, residual, N: int, K: int) -> np.ndarray:
    """ops/matvec/reference.ts:235 -- residual[n] + matvecQ8 row n, f32 [N]."""
    w = _need(weight, np.uint32, N * words_per_row(K), "weight")
    s = _need(scale, np.float32, N, "scale")
    x = _need(vector, np.float32, K, "vector")
    r = _need(residual, np.float32, N, "residual")
    out = np.empty(N, dtype=np.float32)
    _check(lib().wxo_matvec_q8_residual_host(w.ctypes.data, s.ctypes.data, x.ctypes.data, r.ctypes.data,
                                             out.ctypes.data, N, K))
    return out


def matvecQ8Ffn(*, weightGate, scaleGate, weightUp, scaleUp, vector, N: int, K: int) -> np.ndarray:
    """ops/matvec/reference.ts:196 -- silu(gate row n) * up row n, f32 [N]."""
    W = words_per_row(K)
    wg = _need(weightGate, np.uint32, N * W, "weightGate")
    sg = _need(scaleGate, np.float32, N, "scaleGate")
    wu = _need(weightUp, np.uint32, N * W, "weightUp")
    su = _need(scaleUp, np.float32, N, "scaleUp")
    x = _need(vector, np.float32, K, "vector")
    out = np.empty(N, dtype=np.float32)
    _check(lib().wxo_matvec_q8_ffn_host(wg.ctypes.data, sg.ctypes.data, wu.ctypes.data, su.ctypes.data,
                                        x.ctypes.data, out.ctypes.data, N, K))
    return out


def quantize(*, input, N: int, D: int) -> tuple[np.ndarray, np.ndarray]:
    """ops/quantize/reference.ts:13 -- (codes int32 [N*D], scales f32 [N])."""
    x = _need(input, np.float32, N * D, "input")
    codes = np.empty(N * D, dtype=np.int32)
    scales = np.empty(N, dtype=np.float32)
    _check(lib().wxo_quantize_host(x.ctypes.data, N, D, codes.ctypes.data, scales.ctypes.data))
    return codes, scales


def packQ8(*, codes, N: int, K: int) -> np.ndarray:
    """ops/matvec/reference.ts:267 -- int32 codes [N*K] -> u32 [N*ceil(K/4)]."""
    c = _need(codes, np.int32, N * K, "codes")
    out = np.empty(N * words_per_row(K), dtype=np.uint32)
    _check(lib().wxo_pack_q8_host(c.ctypes.data, N, K, out.ctypes.data))
    return out


def packInt8Rows(codes, N: int, K: int) -> np.ndarray:
    """llm/weights-q8.ts:137 -- int8 codes [N*K] -> u32 [N*ceil(K/4)]."""
    c = _need(codes, np.int8, N * K, "codes")
    out = np.empty(N * words_per_row(K), dtype=np.uint32)
    _check(lib().wxo_pack_int8_rows_host(c.ctypes.data, N, K, out.ctypes.data))
    return out


def quantizePackQ8(*, input, N: int, K: int) -> tuple[np.ndarray, np.ndarray]:
    """packQ8(quantize(w).output, N, K) and quantize(w).scales in one GPU pass."""
    x = _need(input, np.float32, N * K, "input")
    packed = np.empty(N * words_per_row(K), dtype=np.uint32)
    scales = np.empty(N, dtype=np.float32)
    _check(lib().wxo_quantize_pack_q8_host(x.ctypes.data, N, K, packed.ctypes.data, scales.ctypes.data))
    return packed, scales


def matmul_q8_device(a, weight, scale, output, N: int, M: int, K: int, stream=None) -> None:
    _check(lib().wxo_matmul_q8(_addr(a), _addr(weight), _addr(scale), _addr(output), N, M, K, _stream_ptr(stream)))


def dequantize_packed_q8_device(weight, scale, N: int, K: int, output, stream=None) -> None:
    _check(lib().wxo_dequantize_packed_q8(_addr(weight), _addr(scale), N, K, _addr(output), _stream_ptr(stream)))


def dequant_transpose_device(weight, scale, out_features: int, in_features: int, output, stream=None) -> None:
    _check(lib().wxo_dequant_transpose(_addr(weight), _addr(scale), out_features, in_features, _addr(output),
                                       _stream_ptr(stream)))


def gather_dequant_rows_device(codes, scale, rows: int, D: int, indices, count: int, output, stream=None) -> None:
    _check(lib().wxo_gather_dequant_rows(_addr(codes), _addr(scale), rows, D, _addr(indices), count, _addr(output),
                                         _stream_ptr(stream)))


def matmulQ8(*, a, weight, scale, N: int, M: int, K: int) -> np.ndarray:
    """ops/matmul/reference.ts:124 -- a [N, K] against the packed weight [M, ceil(K/4)]: f32 [N, M]."""
    av = _need(a, np.float32, N * K, "a")
    w = _need(weight, np.uint32, M * words_per_row(K), "weight")
    s = _need(scale, np.float32, M, "scale")
    out = np.empty(N * M, dtype=np.float32)
    _check(lib().wxo_matmul_q8_host(av.ctypes.data, w.ctypes.data, s.ctypes.data, out.ctypes.data, N, M, K))
    return out.reshape(N, M)


def dequantizePackedQ8(weight, scale, N: int, K: int) -> np.ndarray:
    """llm/weights-q8.ts:161 -- packed [N, ceil(K/4)] -> f32 [N*K]."""
    w = _need(weight, np.uint32, N * words_per_row(K), "weight")
    s = _need(scale, np.float32, N, "scale")
    out = np.empty(N * K, dtype=np.float32)
    _check(lib().wxo_dequantize_packed_q8_host(w.ctypes.data, s.ctypes.data, N, K, out.ctypes.data))
    return out


def dequantTranspose(*, weight, scale, outFeatures: int, inFeatures: int) -> np.ndarray:
    """ops/dequant_transpose/reference.ts:40 -- f32 [inFeatures * outFeatures].  Like the
    reference, the weight and scale lengths must match exactly."""
    w = np.ascontiguousarray(weight, dtype=np.uint32).reshape(-1)
    s = np.ascontiguousarray(scale, dtype=np.float32).reshape(-1)
    if w.size != outFeatures * words_per_row(inFeatures):
        raise WxoError(WXO_ERR_INVALID, f"dequantTranspose(): expected {outFeatures * words_per_row(inFeatures)} "
                                        f"packed words, got {w.size}")
    if s.size != outFeatures:
        raise WxoError(WXO_ERR_INVALID, f"dequantTranspose(): expected {outFeatures} scales, got {s.size}")
    out = np.empty(outFeatures * inFeatures, dtype=np.float32)
    _check(lib().wxo_dequant_transpose_host(w.ctypes.data, s.ctypes.data, outFeatures, inFeatures, out.ctypes.data))
    return out


def gatherDequantRows(table, indices, D: int) -> np.ndarray:
    """llm/weights-q8.ts:207 -- table = (codes int8 [rows*D], scale f32 [rows]); rows of the
    table in request order, zeros for indices outside [0, rows)."""
    codes, scale = table
    s = np.ascontiguousarray(scale, dtype=np.float32).reshape(-1)
    rows = s.size
    c = _need(codes, np.int8, rows * D, "codes")
    ix = np.ascontiguousarray(indices, dtype=np.int64).reshape(-1)
    out = np.empty(ix.size * D, dtype=np.float32)
    _check(lib().wxo_gather_dequant_rows_host(c.ctypes.data, s.ctypes.data, rows, D, ix.ctypes.data, ix.size,
                                              out.ctypes.data))
    return out
