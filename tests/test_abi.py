"""The C ABI library on a machine without a GPU: it loads, exports every
symbol include/wxo_q8.h declares, validates arguments before touching a
device, and fails loudly (no CPU fallback) when no gfx950 is visible.
Also checks the built device code for packed-FP32 instructions."""
import ctypes
import os
import re
import subprocess
import tempfile

import numpy as np
import pytest

import wxo_q8

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "wxo_q8.h")
CSRC = os.path.join(ROOT, "web-xpu-ops_amd", "csrc")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wxo_[a-z0-9_]+)\s*\(", text)))


def have_gpu():
    try:
        return wxo_q8.device_count() > 0
    except wxo_q8.WxoError:
        return False


def test_library_is_built():
    assert os.path.exists(wxo_q8.LIB_PATH), "run __graft_entry__.build() first"


def test_exports_every_declared_symbol():
    names = declared_symbols()
    assert len(names) >= 25
    lib = ctypes.CDLL(wxo_q8.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding covers exactly the declared surface
    assert sorted(wxo_q8.SIGNATURES) == names


def test_abi_version_and_describe():
    assert wxo_q8.lib().wxo_abi_version() == 1
    text = wxo_q8.describe()
    assert text.startswith("wxo_q8 abi=1")
    if not have_gpu():
        assert "device=none" in text


def test_validation_happens_before_device_access():
    L = wxo_q8.lib()
    # M = 0
    assert L.wxo_matvec_q8(None, None, None, None, 4, 8, 0, None) == wxo_q8.WXO_ERR_INVALID
    assert "M (vectors)" in L.wxo_last_error().decode()
    # NULL operand with work to do
    assert L.wxo_matvec_q8(None, None, None, None, 4, 8, 1, None) == wxo_q8.WXO_ERR_INVALID
    assert "weight is NULL" in L.wxo_last_error().decode()
    # size overflow (N * ceil(K/4) > 2^40)
    big = 0xFFFFFFFF
    assert L.wxo_matvec_q8(1, 1, 1, 1, big, big, 1, None) == wxo_q8.WXO_ERR_INVALID
    assert L.wxo_quantize(None, 3, 5, None, None, None) == wxo_q8.WXO_ERR_INVALID
    assert L.wxo_pack_q8(None, 3, 5, None, None) == wxo_q8.WXO_ERR_INVALID
    assert L.wxo_pack_int8_rows(None, 3, 5, None, None) == wxo_q8.WXO_ERR_INVALID
    assert L.wxo_quantize_pack_q8(None, 3, 5, None, None, None) == wxo_q8.WXO_ERR_INVALID
    # the measurement spin refuses more than a second before touching a device
    assert L.wxo_spin(1000001, None) == wxo_q8.WXO_ERR_INVALID
    assert "spin longer than 1 s" in L.wxo_last_error().decode()
    g = ctypes.c_uint32(0)
    assert L.wxo_gate_hold(1000001, None, ctypes.byref(g)) == wxo_q8.WXO_ERR_INVALID
    assert "gate held longer than 1 s" in L.wxo_last_error().decode()
    assert L.wxo_gate_release(0) == wxo_q8.WXO_ERR_INVALID
    # the calibrated ceiling needs at least one output
    assert L.wxo_roofline(None, None) == wxo_q8.WXO_ERR_INVALID
    assert "roofline" in L.wxo_last_error().decode()
    assert L.wxo_roofline_matrix(None) == wxo_q8.WXO_ERR_INVALID
    assert "roofline_matrix" in L.wxo_last_error().decode()
    # graph capture needs a stream of its own
    assert L.wxo_graph_capture_begin(None) == wxo_q8.WXO_ERR_INVALID
    assert "not the null stream" in L.wxo_last_error().decode()
    assert L.wxo_graph_launch(None, None) == wxo_q8.WXO_ERR_INVALID
    assert L.wxo_graph_destroy(None) == wxo_q8.WXO_OK
    # multi-projection: arrays, per-projection sizes, overlapping outputs
    assert L.wxo_matvec_q8_multi(None, None, None, None, 0, None, 8, None) == wxo_q8.WXO_OK
    assert L.wxo_matvec_q8_multi(None, None, None, None, 2, None, 8, None) == wxo_q8.WXO_ERR_INVALID
    with pytest.raises(wxo_q8.WxoError, match="projection 1: weight is NULL"):
        wxo_q8.matvec_q8_multi_device([(16, 16, 0x10000, 4), (0, 16, 0x20000, 4)], 0x30000, 8)
    with pytest.raises(wxo_q8.WxoError, match="outputs of projections 0 and 2 overlap"):
        wxo_q8.matvec_q8_multi_device([(16, 16, 0x10000, 4), (16, 16, 0x20000, 4), (16, 16, 0x1000c, 4)],
                                      0x30000, 8)
    with pytest.raises(wxo_q8.WxoError, match="projection 0: output overlaps the vector"):
        wxo_q8.matvec_q8_multi_device([(16, 16, 0x3001c, 4)], 0x30000, 8)
    # multi-projection matmul: outputs disjoint from the activations and each other
    assert L.wxo_matmul_q8_multi(None, None, None, None, None, 0, 4, 8, None) == wxo_q8.WXO_OK
    with pytest.raises(wxo_q8.WxoError, match="outputs of projections 0 and 1 overlap"):
        wxo_q8.matmul_q8_multi_device(0x30000, [(0x10000, 0x20000, 0x40000, 4), (0x11000, 0x21000, 0x40010, 4)], 2, 8)
    with pytest.raises(wxo_q8.WxoError, match="projection 0: output overlaps the activations"):
        wxo_q8.matmul_q8_multi_device(0x30000, [(0x10000, 0x20000, 0x30010, 4)], 2, 8)
    with pytest.raises(wxo_q8.WxoError, match="projection 1: output overlaps the weight or scale of projection 0"):
        wxo_q8.matvec_q8_multi_device([(0x50000, 0x60000, 0x10000, 4), (16, 16, 0x50004, 4)], 0x30000, 8)
    # the matmul workspace touches no input or output, and is what it says it is
    proj = [(0x10000, 0x20000, 0x40000, 4)]
    with pytest.raises(wxo_q8.WxoError, match="workspace overlaps projection 0's weight, scale or output"):
        wxo_q8.matmul_q8_multi_device(0x30000, proj, 2, 8, workspace=0x40010, workspace_bytes=64)
    with pytest.raises(wxo_q8.WxoError, match="workspace overlaps the activations"):
        wxo_q8.matmul_q8_multi_device(0x30000, proj, 2, 8, workspace=0x2ff00, workspace_bytes=0x200)
    with pytest.raises(wxo_q8.WxoError, match="workspace is NULL with 64 bytes"):
        wxo_q8.matmul_q8_multi_device(0x30000, proj, 2, 8, workspace=0, workspace_bytes=64)
    with pytest.raises(wxo_q8.WxoError, match="workspace is not 16-byte aligned"):
        wxo_q8.matmul_q8_multi_device(0x30000, proj, 2, 8, workspace=0x70004, workspace_bytes=64)
    with pytest.raises(wxo_q8.WxoError):  # bytes = NULL
        wxo_q8._check(L.wxo_matmul_q8_workspace_bytes(None))
    assert L.wxo_quantize_pack_q8_multi(None, None, None, None, 0, 8, None) == wxo_q8.WXO_OK
    with pytest.raises(wxo_q8.WxoError, match="matrix 1: input is NULL"):
        wxo_q8.quantize_pack_q8_multi_device([(0x10000, 2, 0x20000, 0x30000), (0, 2, 0x40000, 0x50000)], 8)
    with pytest.raises(wxo_q8.WxoError, match="outputs of matrix 1 overlap the input of matrix 0"):
        wxo_q8.quantize_pack_q8_multi_device([(0x10000, 2, 0x20000, 0x30000), (0x40000, 2, 0x10010, 0x50000)], 8)
    with pytest.raises(wxo_q8.WxoError, match="packed and scales overlap"):
        wxo_q8.quantize_pack_q8_multi_device([(0x10000, 2, 0x20000, 0x20004)], 8)
    with pytest.raises(wxo_q8.WxoError, match="weight has 3 elements"):
        wxo_q8.matvecQ8(weight=np.zeros(3, np.uint32), scale=np.ones(2, np.float32),
                        vector=np.ones(8, np.float32), N=2, K=8)


@pytest.mark.skipif(have_gpu(), reason="checks the no-GPU failure path")
def test_no_gpu_fails_loudly():
    with pytest.raises(wxo_q8.WxoError) as e:
        wxo_q8.init()
    assert e.value.status == wxo_q8.WXO_ERR_NO_DEVICE
    assert "no CPU fallback" in str(e.value)
    with pytest.raises(wxo_q8.WxoError):
        wxo_q8.matvecQ8(weight=np.zeros(2, np.uint32), scale=np.ones(2, np.float32),
                        vector=np.ones(4, np.float32), N=2, K=4)
    with pytest.raises(wxo_q8.WxoError):
        wxo_q8.quantize(input=np.ones(8, np.float32), N=2, D=4)


def _device_asm(tmp, src):
    """gfx950 assembly of one HIP source, built with the library's own flags."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("wxo_build", os.path.join(ROOT, "web-xpu-ops_amd", "build.py"))
    build = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(build)
    out = os.path.join(tmp, src + ".s")
    flags = [f for f in build.HIP_FLAGS if f != "-fPIC"] + build.PER_FILE_FLAGS.get(src, [])
    subprocess.run(["/opt/rocm/bin/hipcc", *flags, "--cuda-device-only", "-S",
                    "-I", os.path.join(ROOT, "include"), "-I", CSRC, os.path.join(CSRC, src), "-o", out],
                   check=True, capture_output=True)
    return open(out).read()


def test_device_code_has_no_packed_fp32():
    # Every HIP source compiled to gfx950 assembly: no v_pk_add/mul/fma_f32.
    with tempfile.TemporaryDirectory() as tmp:
        for src in ("matvec_q8.hip", "quantize_q8.hip", "matmul_q8.hip", "dequant_q8.hip"):
            asm = _device_asm(tmp, src)
            assert re.search(r"v_pk_(add|mul|fma)_f32", asm) is None, src
            # no register spills in any kernel
            spills = [int(v) for v in re.findall(r"\.vgpr_spill_count:\s+(\d+)", asm)]
            assert spills and max(spills) == 0, src


def test_single_vector_kernel_arguments_are_preloaded():
    # The M = 1 kernels take scalar arguments so that the weight, scale,
    # vector and output pointers and N, K, W arrive in SGPRs at wave launch.
    with tempfile.TemporaryDirectory() as tmp:
        asm = _device_asm(tmp, "matvec_q8.hip")
    lengths = {}
    kernel = None
    for line in asm.splitlines():
        m = re.match(r"\s*\.amdhsa_kernel\s+(\S+)", line)
        if m:
            kernel = m.group(1)
        m = re.match(r"\s*\.amdhsa_user_sgpr_kernarg_preload_length\s+(\d+)", line)
        if m and kernel:
            lengths[kernel] = int(m.group(1))
    m1 = {k: v for k, v in lengths.items() if "matvec_q8_m1_kernel" in k}
    assert m1, "no single-vector kernels found"
    # 4 pointers + N, K, W = 11 SGPRs at least
    assert min(m1.values()) >= 11, m1
