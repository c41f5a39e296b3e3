"""wxo_matmul_q8_multi_static, the allocation-free matmulQ8 over the library's
own scratch array, against wxo_matmul_q8_multi_ws with a caller-owned
workspace of the same size: the same bits (the same split, the same sums in
the same order), within the matmulQ8 bar of the oracle (|y - y_ref| <= 1e-5 *
sum_k |a * fround(q * s)| + 1e-7, ops/matmul/reference.ts:124-137), nothing
written past the outputs, on calls in a row, each smaller than the one
before (none may read what an earlier one left in the array)."""
import numpy as np
import pytest

import oracle
import wxo_q8

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 256 * 65536  # the library's array: 64 KiB per CU of a 256-CU device


@pytest.fixture(scope="module", autouse=True)
def device():
    wxo_q8.init()


def check_matmul(got, a, w, s, N, M, K, rows):
    """Output rows (tokens) `rows` against the oracle."""
    asub = np.ascontiguousarray(np.asarray(a, np.float32).reshape(N, K)[rows])
    want = oracle.matmul_q8(asub, w, s, len(rows), M, K)
    bound = oracle.matmul_absterm(asub, w, s, len(rows), M, K)
    ok, msg = oracle.check_matvec(np.asarray(got).reshape(N, M)[rows].reshape(-1), want.reshape(-1),
                                  bound.reshape(-1))
    assert ok, f"N={N} M={M} K={K}: {msg}"


def test_no_alloc_matches_the_workspace_entry():
    rng = np.random.default_rng(2024)
    ws_bytes = min(wxo_q8.matmul_q8_workspace_bytes(), SCRATCH_BYTES)
    ws = wxo_q8.DeviceBuffer(ws_bytes)
    # 700 tokens over two projections (204 of their 308 tiles split in two:
    # 6.4 MiB of the array), then a 64-token projection (every tile in four
    # parts), then a smaller one over two projections (two parts)
    for N, Ms, K, form in [(700, [2048, 1500], 1030, "balance2"), (64, [2048], 2048, "wgsplit4"),
                           (40, [512, 256], 1030, "wgsplit2")]:
        a = rng.standard_normal(N * K).astype(np.float32)
        a[1] = np.inf
        ba = wxo_q8.DeviceBuffer.from_array(a)
        host, with_ws, without = [], [], []
        for M in Ms:
            codes = rng.integers(-128, 128, (M, K)).astype(np.int32)
            w = oracle.pack_q8(codes.reshape(-1), M, K)
            s = rng.uniform(0.001, 0.05, M).astype(np.float32)
            bw, bs = wxo_q8.DeviceBuffer.from_array(w), wxo_q8.DeviceBuffer.from_array(s)
            outs = []
            for _ in range(2):
                o = wxo_q8.DeviceBuffer(4 * (N * M + 64))
                o.upload(np.full(N * M + 64, 7.5, np.float32))
                outs.append(o)
            host.append((w, s, M))
            with_ws.append((bw, bs, outs[0], M))
            without.append((bw, bs, outs[1], M))
        wxo_q8.matmul_q8_multi_device(ba, with_ws, N, K, workspace=ws, workspace_bytes=ws_bytes)
        wxo_q8.synchronize()
        assert wxo_q8.last_variant().split()[1].endswith(form), wxo_q8.last_variant()
        wxo_q8.matmul_q8_multi_static_device(ba, without, N, K)
        wxo_q8.synchronize()
        assert wxo_q8.last_variant().split()[1].endswith(form), wxo_q8.last_variant()
        for (w, s, M), p, q in zip(host, with_ws, without):
            ref = p[2].download(np.float32, N * M + 64)
            got = q[2].download(np.float32, N * M + 64)
            assert np.all(got[N * M:] == np.float32(7.5)), f"M={M}: written past the output"
            bad = np.flatnonzero(got[:N * M].view(np.uint32) != ref[:N * M].view(np.uint32))
            assert bad.size == 0, f"N={N} M={M}: {bad.size} outputs differ from the workspace entry's, first {bad[0]}"
            check_matmul(got[:N * M], a, w, s, N, M, K, np.unique(np.r_[np.arange(0, N, 7), N - 1]))


def test_no_alloc_entry_in_a_captured_graph():
    """The callers the entry point is for include code under HIP graph
    capture.  A 64-token projection through it (every tile's K steps in four
    parts through the array) is captured once and replayed on new
    activations, with an eager call of another shape through the same array
    between replays: every replay gives the bits of the workspace entry issued
    eagerly on the same inputs."""
    rng = np.random.default_rng(77)
    ws_bytes = min(wxo_q8.matmul_q8_workspace_bytes(), SCRATCH_BYTES)
    ws = wxo_q8.DeviceBuffer(ws_bytes)

    def projection(N, M, K):
        w = oracle.pack_q8(rng.integers(-128, 128, (M, K)).astype(np.int32).reshape(-1), M, K)
        s = rng.uniform(0.001, 0.05, M).astype(np.float32)
        return w, s, wxo_q8.DeviceBuffer.from_array(w), wxo_q8.DeviceBuffer.from_array(s)

    N, M, K = 64, 2048, 2048
    w, s, bw, bs = projection(N, M, K)
    ba, out, ref = wxo_q8.DeviceBuffer(4 * N * K), wxo_q8.DeviceBuffer(4 * N * M), wxo_q8.DeviceBuffer(4 * N * M)
    N2, M2, K2 = 40, 512, 1030  # the eager call between replays: two parts per tile
    _, _, bw2, bs2 = projection(N2, M2, K2)
    ba2 = wxo_q8.DeviceBuffer.from_array(rng.standard_normal(N2 * K2).astype(np.float32))
    out2 = wxo_q8.DeviceBuffer(4 * N2 * M2)
    st = wxo_q8.Stream()
    g = wxo_q8.Graph.capture(st, lambda: wxo_q8.matmul_q8_multi_static_device(ba, [(bw, bs, out, M)], N, K, stream=st))
    try:
        for step in range(4):
            a = rng.standard_normal(N * K).astype(np.float32)
            ba.upload(a)
            wxo_q8.synchronize()
            g.launch(st)
            st.synchronize()
            got = out.download(np.float32, N * M)
            wxo_q8.matmul_q8_multi_device(ba, [(bw, bs, ref, M)], N, K, stream=st, workspace=ws,
                                          workspace_bytes=ws_bytes)
            st.synchronize()
            assert "wgsplit4" in wxo_q8.last_variant(), wxo_q8.last_variant()
            want = ref.download(np.float32, N * M)
            bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
            assert bad.size == 0, f"replay {step}: {bad.size} outputs differ from the eager workspace entry's"
            if step == 0:
                check_matmul(got, a, w, s, N, M, K, np.arange(0, N, 9))
            wxo_q8.matmul_q8_multi_static_device(ba2, [(bw2, bs2, out2, M2)], N2, K2, stream=st)
            st.synchronize()
            assert "wgsplit2" in wxo_q8.last_variant(), wxo_q8.last_variant()
    finally:
        g.destroy()
        st.destroy()
