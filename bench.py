#!/usr/bin/env python3
"""bench.py -- matvecQ8 on one MI355X at the headline shape N=11008, K=4096.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one matvecQ8 call (M=1) on HBM-resident packed weights
(Llama-7B MLP up projection).  Inputs are seeded
synthetic data: W ~ N(0, 0.02) quantized and packed on the GPU by the fused
quantize+packQ8 kernel, x ~ N(0, 1).  Every working set here fits in the
256 MB Infinity Cache, so the timed loop rotates over --copies distinct
copies of the packed weight (> 512 MB in all) and each call streams from HBM.

Prints one JSON line:
  value          algorithmic GB/s over the whole timed region (K back-to-back calls)
  ms_per_step    timed region / K
  roofline       the matvec kernel: algorithmic bytes per launch / mean launch
                 duration (HIP events on the launch stream around the K
                 dispatches, which are all that stream holds); traffic = HBM
                 bytes per launch from the committed rocprofv3 counter
                 summary, if present (taken in its own profiler run)
  config.variant the kernel instance that ran (wxo_last_variant)

Every rotated copy is read once during set-up; the timed launches queue
behind LEAD_STEPS untimed calls and are bracketed by timing-only events, so
neither first touches, nor the host's launch latency, nor the events' own
cache fences fall inside the timed region.
  cpu_baseline   the ECMAScript oracle's matvecQ8 under node on one core, on a
                 bounded row sample of the same inputs
"""
from __future__ import annotations

import argparse
import ctypes
import itertools
import json
import os
import re
import shutil
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "web-xpu-ops_amd", "python"))

import wxo_q8  # noqa: E402
import wxo_workloads as wl  # noqa: E402

PEAK_HBM_GBS = 8000.0
# MI355X's published FP32 vector peak.  This build disables packed FP32
# instructions, but one-wide v_fma_f32 chains already run at 125 TFLOP/s on
# gfx950 (wxo_roofline), well past half of it, so the published figure stays
# the bound.
PEAK_FP32_FMA_TFLOPS = 157.3
# Dense bf16 matrix-core peak (the batched path splits x into three bf16 parts
# and runs 16-wide vector tiles, so it issues 3 x 2 x N x K x 16 flops per tile).
PEAK_BF16_MFMA_TFLOPS = 2500.0
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "matvec_q8_cfg2_traffic.txt")
TRAFFIC_NOTE = ("HBM bytes per launch from the committed rocprofv3 --pmc summary "
                "profiles/matvec_q8_cfg2_traffic.txt: TCC_EA0 read and write requests x request size, taken "
                "in its own profiler run (counters need their own process), not in this one")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def read_traffic():
    """HBM bytes per launch from the committed counter summary (key: value lines)."""
    if not os.path.exists(TRAFFIC_SUMMARY):
        return None
    vals = {}
    for line in open(TRAFFIC_SUMMARY):
        m = re.match(r"^\s*([a-z_]+)\s*:\s*([0-9.eE+-]+)\s*$", line)
        if m:
            vals[m.group(1)] = float(m.group(2))
    return vals.get("hbm_bytes_per_launch")


def calibrated_ceiling():
    """This device's own ceilings, measured now by wxo_roofline (the
    reference's harness/roofline.ts method: 512 MiB hashed buffers swept once
    per launch, fastest of several attempts; FMA chains from registers)."""
    r = wxo_q8.roofline()
    cal = {"GB/s": round(r["bandwidth"] / 1e9, 1), "fma_TFLOP/s": round(r["compute"] / 1e12, 2),
           "source": "wxo_roofline: two 512 MiB hash-filled buffers swept alternately with dwordx4 loads, fastest of "
                     "3 regions of 8 back-to-back sweeps (launch cost included); one-wide f32 FMA chains"}
    log(f"calibrated ceiling: {cal['GB/s']} GB/s HBM read ({100 * cal['GB/s'] / PEAK_HBM_GBS:.1f}% of 8 TB/s), "
        f"{cal['fma_TFLOP/s']} TFLOP/s one-wide f32 FMA")
    return cal


def add_calibrated(table, cal):
    """Every GPU row measured against HBM also as a % of the calibrated read
    ceiling; the ceiling itself heads the table."""
    for row in table:
        if "pct_hbm" in row and "GB/s" in row:
            row["pct_of_calibrated"] = round(100.0 * row["GB/s"] / cal["GB/s"], 1)
    table.insert(0, {"case": "calibrated ceiling (wxo_roofline): HBM read stream and f32 FMA", "GB/s": cal["GB/s"],
                     "pct_hbm": round(100.0 * cal["GB/s"] / PEAK_HBM_GBS, 1), "fma_TFLOP/s": cal["fma_TFLOP/s"],
                     "source": cal["source"]})


def calibrated_matrix_ceiling():
    """The bf16 matrix cores' sustained rate on every CU with operands of
    matmulQ8's kinds, measured now by wxo_roofline_matrix (the clock sags under
    matrix work, so the nominal peak is not what real operands get)."""
    tf = wxo_q8.roofline_matrix() / 1e12
    cal = {"TFLOP/s": round(tf, 1),
           "source": "wxo_roofline_matrix: v_mfma_f32_16x16x32_bf16 on every CU, two waves per SIMD, int8 codes x "
                     "bf16 parts of random sign/mantissa/exponent, fastest of 3 ~1 ms launches"}
    log(f"calibrated matrix ceiling: {cal['TFLOP/s']} TFLOP/s bf16 ({100 * tf / PEAK_BF16_MFMA_TFLOPS:.1f}% of "
        f"{PEAK_BF16_MFMA_TFLOPS:.0f})")
    return cal


def add_calibrated_matrix(table, calm):
    """Every matmulQ8 row also as a % of the calibrated matrix-core rate (its
    matrix work is 3x its useful flops: the exact three-part split); the
    ceiling itself heads the table."""
    for row in table:
        if row.get("case", "").startswith("prefill matmulQ8") and "TFLOP/s" in row:
            row["pct_of_calibrated_matrix"] = round(100.0 * 3.0 * row["TFLOP/s"] / calm["TFLOP/s"], 1)
    table.insert(0, {"case": "calibrated ceiling (wxo_roofline_matrix): bf16 matrix cores on matmulQ8-like operands",
                     "TFLOP/s": calm["TFLOP/s"],
                     "pct_of_peak": round(100.0 * calm["TFLOP/s"] / PEAK_BF16_MFMA_TFLOPS, 1), "source": calm["source"]})


def cpu_baseline(packed, scales, x, N, K, budget_s):
    node = shutil.which("node")
    if node is None:
        return None
    rows = 2048  # bounded sample: ~1/5 of the rows per run
    with tempfile.TemporaryDirectory() as tmp:
        packed.tofile(os.path.join(tmp, "weight.bin"))
        scales.tofile(os.path.join(tmp, "scale.bin"))
        x.tofile(os.path.join(tmp, "vector.bin"))
        proc = subprocess.run([node, os.path.join(ROOT, "oracle", "cpu_baseline.mjs"), tmp, str(N), str(K),
                               str(budget_s), str(rows)], capture_output=True, text=True, timeout=budget_s + 120)
    if proc.returncode != 0:
        log(f"cpu baseline failed: {proc.stderr.strip()[-300:]}")
        return None
    r = json.loads(proc.stdout.strip().splitlines()[-1])
    sample_bytes = wl.matvec_bytes(r["rows"], K)
    gbs = sample_bytes / (r["median_us"] * 1e-6) / 1e9
    return {
        "value": round(gbs, 4), "unit": "GB/s", "cores": 1, "kind": "port",
        "us_per_call_full_shape": round(r["median_us"] * N / r["rows"], 1),
        "sample": (f"oracle/q8_oracle.mjs matvecQ8 under node {r['node']} (V8, single thread) on rows 0..{r['rows']-1} "
                   f"of the same N={N},K={K} inputs, median of {r['runs']} runs ({r['median_us']:.0f} us each); "
                   f"host has {os.cpu_count()} cores"),
    }


# Untimed steps enqueued after the synchronisation that opens a timed
# sequence and before its first event: the timed launches queue behind
# running work, so neither the host's latency to the first launch nor an idle
# GPU's state at the start falls inside the events' interval.
LEAD_STEPS = 10


# Every launch of one measured case takes the next index of ONE sequence, from
# the first set-up call through the last timed call.  A launch that picks its
# weight copy as index % copies therefore reads each copy exactly `copies`
# launches after its previous read, i.e. after every other copy has streamed
# through the caches in between.  Restarting the index at the timed region
# would re-read the copies the lead calls had just streamed (a few tens of MB
# back, well inside the 256 MB Infinity Cache).


def time_loop(stream, launch, steps, warmup, seq=None, setup=0):
    """Mean us per step over `steps` back-to-back steps (timing-only events on
    the stream).  `seq` continues the case's launch index sequence; `setup`
    untimed launches (one per rotated copy) run before the warm-up, so no copy
    is first read inside the timed region."""
    seq = itertools.count() if seq is None else seq
    for _ in range(setup + warmup):
        launch(next(seq))
    stream.synchronize()
    e0, e1 = wxo_q8.Event(timer=True), wxo_q8.Event(timer=True)
    for _ in range(LEAD_STEPS):
        launch(next(seq))
    e0.record(stream)
    for _ in range(steps):
        launch(next(seq))
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_ms(e1) * 1e3 / steps


# Host-issued time_loop measures what a caller issuing one call at a time
# sees: for a kernel shorter than the host's issue cost per call (~3 us from
# Python through ctypes, ~2.8 us from C) that is the host's rate, not the
# GPU's.  time_loop_queued puts a fixed-length spin kernel ahead of the timed
# launches, so the host has queued them all before the GPU reaches the first:
# the events then bracket back-to-back execution on the GPU alone.


def _spin(stream, us):
    """A spin kernel of `us` microseconds (the GPU's 100 MHz clock) on `stream`."""
    _check(wxo_q8.lib().wxo_spin(int(us), stream.handle))


def time_loop_queued(stream, launch, steps, seq=None):
    """GPU-side mean us per step: `steps` launches queued behind a spin kernel
    long enough for the host to issue them all, between timing-only events.
    Returns None if the host did not finish issuing inside the spin.  `seq`
    continues the case's launch index sequence."""
    seq = itertools.count() if seq is None else seq
    stream.synchronize()
    t0 = time.perf_counter()
    for _ in range(5):  # the host's issue time per step, to size the spin
        launch(next(seq))
    per_step_us = (time.perf_counter() - t0) * 1e6 / 5
    stream.synchronize()
    e0, e1 = wxo_q8.Event(timer=True), wxo_q8.Event(timer=True)
    spin_us = min(900000.0, 2.0 * per_step_us * steps + 1000.0)
    _spin(stream, spin_us)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        launch(next(seq))
    e1.record(stream)
    host_us = (time.perf_counter() - t0) * 1e6
    e1.synchronize()
    if host_us > 0.8 * spin_us:
        log(f"queued timing: the host took {host_us:.0f} us to issue {steps} steps (spin {spin_us:.0f} us); dropped")
        return None
    return e0.elapsed_ms(e1) * 1e3 / steps


def time_both(stream, launch, steps, warmup, setup=0):
    """(host-issued us per step, GPU-side queued us per step or None), one
    launch index sequence across both (`setup`: see time_loop)."""
    seq = itertools.count()
    us = time_loop(stream, launch, steps, warmup, seq, setup)
    return us, time_loop_queued(stream, launch, steps, seq)


def _q(usq):
    return None if usq is None else round(usq, 3)


def _qs(usq):
    return "" if usq is None else f"  (queued: {usq:.2f} us)"


ROT_TARGET = 600 * 1024 * 1024  # > 2x the 256 MB Infinity Cache


def _check(st):
    if st != 0:
        raise wxo_q8.WxoError(st, wxo_q8.lib().wxo_last_error().decode())


def prepare_weights(stream, w_f32, N, K, copies):
    """Quantize+pack `w_f32` on the GPU into `copies` consecutive copies (rotation)."""
    L = wxo_q8.lib()
    W = (K + 3) // 4
    src = wxo_q8.DeviceBuffer.from_array(w_f32, stream)
    packed = wxo_q8.DeviceBuffer(N * W * 4 * copies)
    scale = wxo_q8.DeviceBuffer(N * 4)
    wxo_q8.quantize_pack_q8_device(src, N, K, packed, scale, stream)
    for i in range(1, copies):
        _check(L.wxo_memcpy_dtod(packed.ptr + i * N * W * 4, packed.ptr, N * W * 4, stream.handle))
    stream.synchronize()
    src.free()
    return packed, scale


def timed_headline(stream, call, copies, warmup, steps, event=None, sync=None):
    """The headline's timed region: `steps` back-to-back calls between two
    timing-only events (recording them fences nothing, so no cache write-back
    or invalidation lands inside the interval), synchronised on both sides.
    Returns the interval in ms.

    Before it, on one continuing index sequence (call(i) reads copy i % copies):
    one set-up call per copy, so every copy's pages have been read once before
    any is timed; `warmup` untimed calls; then LEAD_STEPS untimed calls
    enqueued just ahead of the first event, so the timed launches queue behind
    running work and the host's latency to the first launch stays outside the
    interval.  Every timed call reads the copy read longest ago."""
    event = event or wxo_q8.Event
    sync = sync or wxo_q8.synchronize
    seq = itertools.count()
    for _ in range(copies):
        call(next(seq))
    stream.synchronize()
    for _ in range(warmup):
        call(next(seq))
    stream.synchronize()
    e0, e1 = event(timer=True), event(timer=True)
    sync()
    for _ in range(LEAD_STEPS):
        call(next(seq))
    e0.record(stream)
    for _ in range(steps):
        call(next(seq))
    e1.record(stream)
    e1.synchronize()
    sync()
    return e0.elapsed_ms(e1)


def measure_matvec(stream, name, N, K, M, w_f32, x, steps, warmup, queued=False):
    """One matvecQ8 configuration on rotated weights: us per call, algorithmic
    GB/s, the bound (HBM, or the compute rate of the path that runs: one-wide
    FP32 FMA for one vector, bf16 matrix cores at three products per code for
    batched vectors) and the kernel instance."""
    L = wxo_q8.lib()
    sp = stream.handle
    W = (K + 3) // 4
    nbytes = wl.matvec_bytes(N, K, M)
    copies = max(1, -(-ROT_TARGET // (N * W * 4)))
    packed, scale = prepare_weights(stream, w_f32, N, K, copies)
    vec = wxo_q8.DeviceBuffer.from_array(x, stream)
    out = wxo_q8.DeviceBuffer(N * M * 4)
    ptrs = [packed.ptr + i * N * W * 4 for i in range(copies)]

    def call(i):
        _check(L.wxo_matvec_q8(ptrs[i % copies], scale.ptr, vec.ptr, out.ptr, N, K, M, sp))
    seq = itertools.count()
    for _ in range(copies):  # every copy read once before timing
        call(next(seq))
    us = time_loop(stream, call, steps, warmup, seq)
    usq = time_loop_queued(stream, call, steps, seq) if queued else None
    variant = wxo_q8.last_variant()
    gbs = nbytes / (us * 1e-6) / 1e9
    flops = 2.0 * N * K * M
    tflops = flops / (us * 1e-6) / 1e12
    hbm_us = nbytes / (PEAK_HBM_GBS * 1e9) * 1e6
    if M == 1:  # one FMA per code on the VALU
        comp_us, comp_name = flops / (PEAK_FP32_FMA_TFLOPS * 1e12) * 1e6, "valu_fp32"
    else:  # matrix cores: three bf16 products per code, 16 vectors per tile
        mflops = 3.0 * 2.0 * N * K * 16 * (-(-M // 16))
        comp_us, comp_name = mflops / (PEAK_BF16_MFMA_TFLOPS * 1e12) * 1e6, "mfma_bf16"
    bound = "hbm" if hbm_us >= comp_us else comp_name
    log(f"{name}: {us:.2f} us  {gbs:.0f} GB/s  {100*gbs/PEAK_HBM_GBS:.1f}% HBM  bound={bound}  [{variant}]{_qs(usq)}")
    for b in (packed, scale, vec, out):
        b.free()
    r = {"case": name, "N": N, "K": K, "M": M, "us": round(us, 3), "GB/s": round(gbs, 1),
         "pct_hbm": round(100 * gbs / PEAK_HBM_GBS, 1), "TFLOP/s": round(tflops, 2),
         "bound": bound, "pct_of_bound": round(100 * max(hbm_us, comp_us) / us, 1),
         "weight_copies": copies, "variant": variant}
    if queued:
        r["us_queued"] = _q(usq)
    return r


def run_case(stream, spec, steps, warmup):
    """`--case cfgN[:M]`: one BASELINE matvecQ8 configuration alone (M vectors)."""
    name, _, m = spec.partition(":")
    M = int(m) if m else 1
    if name not in wl.CONFIGS:
        raise SystemExit(f"--case: unknown configuration {name!r} (one of {', '.join(wl.CONFIGS)})")
    c = wl.make_config(name, M=M)
    return measure_matvec(stream, f"{name} matvecQ8 M={M}", c["N"], c["K"], M, c["w"], c["x"], steps, warmup)


def run_suite(stream, steps, warmup, napi=True):
    """Every BASELINE configuration on one GPU: us/step, algorithmic GB/s and
    the fraction of the bound that applies (HBM, or the compute rate of the
    path that runs when that is lower: one-wide FP32 FMA for one vector, bf16
    matrix cores for batched vectors)."""
    L = wxo_q8.lib()
    sp = stream.handle
    results = []
    rot_target = ROT_TARGET
    check = _check

    def prepare(w_f32, N, K, copies):
        return prepare_weights(stream, w_f32, N, K, copies)

    def matvec_case(name, N, K, M, w_f32, x):
        results.append(measure_matvec(stream, "suite " + name, N, K, M, w_f32, x, steps, warmup, queued=True))
        results[-1]["case"] = name

    c1 = wl.make_config("cfg1")
    matvec_case("cfg1 matvecQ8", c1["N"], c1["K"], 1, c1["w"], c1["x"])
    c3 = wl.make_config("cfg3")
    matvec_case("cfg3 matvecQ8 ragged K=4099", c3["N"], c3["K"], 1, c3["w"], c3["x"])
    c2 = wl.make_config("cfg2")
    matvec_case("cfg2 matvecQ8", c2["N"], c2["K"], 1, c2["w"], c2["x"])
    del c1, c2, c3

    # cfg4: one decoder layer's 7 projections back to back on resident weights,
    # rotating over enough layers' worth of weights to stream from HBM.
    mats, xh, xf = wl.make_decoder_layer()
    layer_bytes = sum(wl.matvec_bytes(N, K) for _, N, K, _ in mats)
    layers = max(1, -(-rot_target // layer_bytes))
    prepared = [prepare(wf, N, K, layers) for _, N, K, wf in mats]
    vh = wxo_q8.DeviceBuffer.from_array(xh, stream)
    vf = wxo_q8.DeviceBuffer.from_array(xf, stream)
    outb = wxo_q8.DeviceBuffer(5632 * 4)

    def layer_step(i):
        li = i % layers
        for (name, N, K, _), (packed, scale) in zip(mats, prepared):
            W = (K + 3) // 4
            check(L.wxo_matvec_q8(packed.ptr + li * N * W * 4, scale.ptr, (vf if K == 5632 else vh).ptr, outb.ptr,
                                  N, K, 1, sp))
    us, usq = time_both(stream, layer_step, max(1, steps // 7), max(1, warmup // 7), layers)
    gbs = layer_bytes / (us * 1e-6) / 1e9
    results.append({"case": "cfg4 decoder layer: 7 matvecQ8 calls", "bytes": layer_bytes, "us": round(us, 3),
                    "GB/s": round(gbs, 1), "pct_hbm": round(100 * gbs / PEAK_HBM_GBS, 1), "layers_rotated": layers,
                    "us_queued": _q(usq)})
    log(f"suite cfg4 layer: {us:.2f} us/layer  {gbs:.0f} GB/s{_qs(usq)}")

    # The same layer as the resident engine runs its decode projections
    # (llm/engine-q8-resident.ts:1843-1869): q/k/v plain, o_proj and down_proj
    # as matvecQ8Residual into the residual stream, gate/up as one
    # matvecQ8Ffn: 6 launches, and the 3 elementwise passes folded in.
    by = {name: i for i, (name, _, _, _) in enumerate(mats)}
    resid = wxo_q8.DeviceBuffer.from_array(np.zeros(2048, np.float32), stream)
    hidden = wxo_q8.DeviceBuffer(5632 * 4)

    def fused_step(i):
        li = i % layers

        def wp(name):
            _, N, K, _ = mats[by[name]]
            packed, scale = prepared[by[name]]
            return packed.ptr + li * N * ((K + 3) // 4) * 4, scale.ptr

        for name in ("wq", "wk", "wv"):
            w, sc = wp(name)
            check(L.wxo_matvec_q8(w, sc, vh.ptr, outb.ptr, 2048, 2048, 1, sp))
        w, sc = wp("wo")
        check(L.wxo_matvec_q8_residual(w, sc, vh.ptr, resid.ptr, resid.ptr, 2048, 2048, sp))
        (wg, sg), (wu, su) = wp("wGate"), wp("wUp")
        check(L.wxo_matvec_q8_ffn(wg, sg, wu, su, vh.ptr, hidden.ptr, 5632, 2048, sp))
        w, sc = wp("wDown")
        check(L.wxo_matvec_q8_residual(w, sc, vf.ptr, resid.ptr, resid.ptr, 2048, 5632, sp))
    us, usq = time_both(stream, fused_step, max(1, steps // 7), max(1, warmup // 7), layers)
    gbs = layer_bytes / (us * 1e-6) / 1e9
    results.append({"case": "cfg4 decoder layer as the resident engine runs it: 3 matvecQ8 + 2 matvecQ8Residual "
                            "+ 1 matvecQ8Ffn", "bytes": layer_bytes, "us": round(us, 3), "GB/s": round(gbs, 1),
                    "pct_hbm": round(100 * gbs / PEAK_HBM_GBS, 1), "layers_rotated": layers, "us_queued": _q(usq)})
    log(f"suite cfg4 layer fused: {us:.2f} us/layer  {gbs:.0f} GB/s{_qs(usq)}")

    # The same again as the resident batch issues it: the three same-vector
    # projections wq/wk/wv coalesced into one wxo_matvec_q8_multi launch.
    P3 = ctypes.c_void_p * 3
    ns3 = (ctypes.c_uint32 * 3)(2048, 2048, 2048)
    qkv_out = wxo_q8.DeviceBuffer(3 * 2048 * 4)
    outs3 = P3(qkv_out.ptr, qkv_out.ptr + 2048 * 4, qkv_out.ptr + 2 * 2048 * 4)

    def coalesced_step(i):
        li = i % layers

        def wp(name):
            _, N, K, _ = mats[by[name]]
            packed, scale = prepared[by[name]]
            return packed.ptr + li * N * ((K + 3) // 4) * 4, scale.ptr

        q, k, v = wp("wq"), wp("wk"), wp("wv")
        check(L.wxo_matvec_q8_multi(P3(q[0], k[0], v[0]), P3(q[1], k[1], v[1]), outs3, ns3, 3, vh.ptr, 2048, sp))
        w, sc = wp("wo")
        check(L.wxo_matvec_q8_residual(w, sc, vh.ptr, resid.ptr, resid.ptr, 2048, 2048, sp))
        (wg, sg), (wu, su) = wp("wGate"), wp("wUp")
        check(L.wxo_matvec_q8_ffn(wg, sg, wu, su, vh.ptr, hidden.ptr, 5632, 2048, sp))
        w, sc = wp("wDown")
        check(L.wxo_matvec_q8_residual(w, sc, vf.ptr, resid.ptr, resid.ptr, 2048, 5632, sp))
    us, usq = time_both(stream, coalesced_step, max(1, steps // 7), max(1, warmup // 7),
                       layers)
    gbs = layer_bytes / (us * 1e-6) / 1e9
    results.append({"case": "cfg4 decoder layer as the resident batch issues it: wq/wk/wv in one matvecQ8 multi "
                            "launch + 2 matvecQ8Residual + 1 matvecQ8Ffn", "bytes": layer_bytes, "us": round(us, 3),
                    "GB/s": round(gbs, 1), "pct_hbm": round(100 * gbs / PEAK_HBM_GBS, 1), "layers_rotated": layers,
                    "us_queued": _q(usq)})
    log(f"suite cfg4 layer coalesced: {us:.2f} us/layer  {gbs:.0f} GB/s{_qs(usq)}")
    qkv_out.free()
    resid.free()
    hidden.free()
    for packed, scale in prepared:
        packed.free()
        scale.free()

    # cfg4: quantize + packQ8 (fused) of the seven f32 matrices.
    srcs = [(N, K, wxo_q8.DeviceBuffer.from_array(wf, stream)) for _, N, K, wf in mats]
    outs = [(wxo_q8.DeviceBuffer(N * ((K + 3) // 4) * 4), wxo_q8.DeviceBuffer(N * 4)) for _, N, K, _ in mats]
    qbytes = sum(wl.quantize_pack_bytes(N, K) for _, N, K, _ in mats)

    def quant_step(i):
        for (N, K, src), (packed, scale) in zip(srcs, outs):
            wxo_q8.quantize_pack_q8_device(src, N, K, packed, scale, stream)
    us, usq = time_both(stream, quant_step, max(1, steps // 20), 2)
    gbs = qbytes / (us * 1e-6) / 1e9
    results.append({"case": "cfg4 quantize+packQ8 (fused) of the 7 matrices", "bytes": qbytes, "us": round(us, 3),
                    "GB/s": round(gbs, 1), "pct_hbm": round(100 * gbs / PEAK_HBM_GBS, 1), "us_queued": _q(usq)})
    log(f"suite cfg4 quantize+pack: {us:.2f} us  {gbs:.0f} GB/s{_qs(usq)}")

    # The same seven as the resident batch issues them: matrices with one K
    # in one wxo_quantize_pack_q8_multi launch (K = 2048 x 6, K = 5632 x 1).
    by_k = {}
    for (N, K, src), (packed, scale) in zip(srcs, outs):
        by_k.setdefault(K, []).append((src, N, packed, scale))

    def quant_multi_step(i):
        for K, group in by_k.items():
            wxo_q8.quantize_pack_q8_multi_device(group, K, stream)
    us, usq = time_both(stream, quant_multi_step, max(1, steps // 20), 2)
    gbs = qbytes / (us * 1e-6) / 1e9
    results.append({"case": f"cfg4 quantize+packQ8 of the 7 matrices as the resident batch issues them "
                            f"({len(by_k)} launches, one per K)", "bytes": qbytes, "us": round(us, 3),
                    "GB/s": round(gbs, 1), "pct_hbm": round(100 * gbs / PEAK_HBM_GBS, 1), "us_queued": _q(usq)})
    log(f"suite cfg4 quantize+pack coalesced: {us:.2f} us  {gbs:.0f} GB/s{_qs(usq)}")
    for (_, _, src), (packed, scale) in zip(srcs, outs):
        src.free()
        packed.free()
        scale.free()
    del mats, srcs, outs

    # Resident weight load (the engine's create(): llm/engine-q8-resident.ts:521-538
    # packs each projection on the CPU, ~0.62 GB/s per README.md:1809-1813): the
    # seven cfg4 matrices' int8 codes from host memory to packed resident
    # weights.  K % 4 == 0 here, so the packed layout is the codes' bytes and
    # the upload is the pack; wall clock, pageable host memory, then the
    # packInt8Rows kernel alone on a ragged device-resident matrix (cfg3 shape).
    mats, _, _ = wl.make_decoder_layer()
    host_codes = []
    for _, N, K, wf in mats:
        host_codes.append((N, K, np.ascontiguousarray(
            np.random.default_rng(N + K).integers(-127, 128, N * K).astype(np.int8))))
    dev_w = [wxo_q8.DeviceBuffer(N * ((K + 3) // 4) * 4) for N, K, _ in host_codes]
    code_bytes = sum(c.nbytes for _, _, c in host_codes)
    reps = 20
    for r in range(reps + 2):
        if r == 2:
            stream.synchronize()
            t0 = time.perf_counter()
        for (N, K, c), d in zip(host_codes, dev_w):
            check(L.wxo_memcpy_htod(d.ptr, c.ctypes.data, c.nbytes, sp))
    stream.synchronize()
    us = (time.perf_counter() - t0) * 1e6 / reps
    gbs = code_bytes / (us * 1e-6) / 1e9
    results.append({"case": "resident load: cfg4's 7 matrices, int8 codes on the host -> packed resident weights "
                            "(upload is the pack for K % 4 == 0; pageable host memory)", "bytes": code_bytes,
                    "us": round(us, 3), "GB/s": round(gbs, 2), "reference_cpu_packInt8Rows_GB/s": 0.62})
    log(f"suite resident load cfg4: {us:.1f} us  {gbs:.1f} GB/s (reference CPU packInt8Rows 0.62 GB/s)")
    for d in dev_w:
        d.free()
    N3, K3 = 4096, 4099
    W3 = (K3 + 3) // 4
    copies3 = max(1, -(-rot_target // (N3 * W3 * 4)))
    src3 = wxo_q8.DeviceBuffer.from_array(np.random.default_rng(3).integers(-127, 128, N3 * K3 * copies3)
                                          .astype(np.int8), stream)
    dst3 = wxo_q8.DeviceBuffer(N3 * W3 * 4 * copies3)
    us, usq = time_both(stream, lambda i: check(L.wxo_pack_int8_rows(src3.ptr + (i % copies3) * N3 * K3, N3, K3,
                                                                     dst3.ptr + (i % copies3) * N3 * W3 * 4, sp)),
                        max(1, steps // 4), max(1, warmup // 4), copies3)
    pbytes = N3 * K3 + N3 * W3 * 4
    gbs = pbytes / (us * 1e-6) / 1e9
    results.append({"case": "packInt8Rows on the GPU, device-resident codes, N=4096 K=4099 (ragged)", "bytes": pbytes,
                    "us": round(us, 3), "GB/s": round(gbs, 1), "pct_hbm": round(100 * gbs / PEAK_HBM_GBS, 1),
                    "us_queued": _q(usq)})
    log(f"suite packInt8Rows ragged 4096x4099: {us:.2f} us  {gbs:.0f} GB/s  {100*gbs/PEAK_HBM_GBS:.1f}% HBM{_qs(usq)}")
    src3.free()
    dst3.free()
    del mats, host_codes

    # cfg5: vocab head N=151936, K=1024, M in {1, 4, 8, 16}.
    for M in (1, 4, 8, 16):
        c5 = wl.make_config("cfg5", M=M)
        matvec_case(f"cfg5 LM head M={M}", c5["N"], c5["K"], M, c5["w"], c5["x"])
        del c5

    run_prefill_suite(stream, steps, warmup, results, check)
    if napi:
        results.extend(napi_end_to_end())
    results.extend(cpu_reference_ops(budget_s=1.0))
    return results


def napi_end_to_end():
    """What a JavaScript caller sees through the Node-API addon (launch plus
    stream synchronisation per call, readback, the PCIe-inclusive host call and
    a whole resident decode step): bench_napi.mjs, run
    as a child process.  Reported beside the kernel-only event timings."""
    node = shutil.which("node")
    if node is None:
        return []
    proc = subprocess.run([node, os.path.join(ROOT, "bench_napi.mjs")],
                          capture_output=True, text=True, timeout=300)
    if proc.returncode != 0:
        raise RuntimeError(f"bench_napi.mjs failed: {proc.stderr.strip()[-500:]}")
    r = json.loads(proc.stdout.strip().splitlines()[-1])
    for e in r["results"]:
        e["node"] = r["node"]
        log(f"suite {e['case']}: {e['us']} us")
    return r["results"]


def cpu_reference_ops(budget_s):
    """The reference's CPU path for each measured op, restated in ECMAScript
    (oracle/q8_oracle.mjs) and timed under node on one host core over a
    bounded sample of the suite's shapes (oracle/cpu_baseline_ops.mjs).
    Reported beside the GPU numbers; not a target."""
    node = shutil.which("node")
    if node is None:
        return []
    out = []
    # op -> (algorithmic bytes of the sample, useful flops of the sample)
    for op in ("quantize_pack", "pack_int8_rows", "ffn", "matmul", "dequantize", "dequant_transpose", "gather"):
        proc = subprocess.run([node, os.path.join(ROOT, "oracle", "cpu_baseline_ops.mjs"), op, str(budget_s)],
                              capture_output=True, text=True, timeout=budget_s * 20 + 120)
        if proc.returncode != 0:
            log(f"cpu reference {op} failed: {proc.stderr.strip()[-200:]}")
            continue
        r = json.loads(proc.stdout.strip().splitlines()[-1])
        us = r["median_us"]
        entry = {"case": f"CPU reference, one core (node {r['node']}): {r['op']}", "us": round(us, 1),
                 "sample": {k: r[k] for k in ("N", "M", "K", "rows", "D", "T") if k in r}, "runs": r["runs"],
                 "cores": 1}
        if op == "quantize_pack":
            entry["GB/s"] = round(wl.quantize_pack_bytes(r["N"], r["K"]) / (us * 1e-6) / 1e9, 3)
        elif op == "pack_int8_rows":
            entry["GB/s"] = round((r["N"] * r["K"] + r["N"] * ((r["K"] + 3) // 4) * 4) / (us * 1e-6) / 1e9, 3)
        elif op == "ffn":
            entry["GB/s"] = round(2 * wl.matvec_bytes(r["N"], r["K"]) / (us * 1e-6) / 1e9, 3)
        elif op == "matmul":
            entry["GFLOP/s"] = round(2.0 * r["N"] * r["M"] * r["K"] / (us * 1e-6) / 1e9, 3)
        elif op in ("dequantize", "dequant_transpose"):
            W = (r["K"] + 3) // 4
            entry["GB/s"] = round((r["N"] * W * 4 + 4 * r["N"] + 4 * r["N"] * r["K"]) / (us * 1e-6) / 1e9, 3)
        elif op == "gather":
            entry["GB/s"] = round(r["T"] * (r["D"] + 4 + 8 + 4 * r["D"]) / (us * 1e-6) / 1e9, 3)
        out.append(entry)
        log(f"cpu reference {op}: {us:.0f} us per call ({entry.get('GB/s', entry.get('GFLOP/s'))} "
            f"{'GB/s' if 'GB/s' in entry else 'GFLOP/s'}) on {entry['sample']}")
    return out


def run_prefill_suite(stream, steps, warmup, results, check):
    """The prefill side (the next rows after the decode path): matmulQ8 over
    one decoder layer's seven projections for a 512-token prompt, then the
    dequant / gather ops.  matmulQ8 is compute-bound: its bound is the bf16
    matrix-core rate at three products per code (the exact split of each
    activation), i.e. 3 x 2 N M K flops; TFLOP/s counts the 2 N M K useful
    flops."""
    L = wxo_q8.lib()
    sp = stream.handle
    T = wl.PREFILL_TOKENS
    mats, _, _ = wl.make_decoder_layer()
    rng = np.random.default_rng(7)
    a_h = wxo_q8.DeviceBuffer.from_array(rng.standard_normal(T * 2048, dtype=np.float32), stream)
    a_f = wxo_q8.DeviceBuffer.from_array(rng.standard_normal(T * 5632, dtype=np.float32), stream)
    out = wxo_q8.DeviceBuffer(T * 5632 * 4)
    prepared = []
    for name, N, K, wf in mats:
        src = wxo_q8.DeviceBuffer.from_array(wf, stream)
        packed = wxo_q8.DeviceBuffer(N * ((K + 3) // 4) * 4)
        scale = wxo_q8.DeviceBuffer(N * 4)
        wxo_q8.quantize_pack_q8_device(src, N, K, packed, scale, stream)
        stream.synchronize()
        src.free()
        prepared.append((name, N, K, packed, scale))
    total_flops = 0.0
    total_us = 0.0
    for name, N, K, packed, scale in prepared:
        a = a_f if K == 5632 else a_h
        us = time_loop(stream, lambda i: check(L.wxo_matmul_q8(a.ptr, packed.ptr, scale.ptr, out.ptr, T, N, K, sp)),
                       max(1, steps // 20), max(1, warmup // 20))  # 25+ us per call: never host-bound
        flops = 2.0 * T * N * K
        bound_us = 3.0 * flops / (PEAK_BF16_MFMA_TFLOPS * 1e12) * 1e6
        total_flops += flops
        total_us += us
        results.append({"case": f"prefill matmulQ8 {name}: tokens={T} M={N} K={K}", "us": round(us, 3),
                        "TFLOP/s": round(flops / (us * 1e-6) / 1e12, 1), "bound": "mfma_bf16 (x3 exact split)",
                        "pct_of_bound": round(100 * bound_us / us, 1)})
        log(f"suite prefill matmulQ8 {name} {T}x{N}x{K}: {us:.2f} us  {flops / (us * 1e-6) / 1e12:.1f} TFLOP/s  "
            f"{100 * bound_us / us:.1f}% of the x3 bf16 bound")
    bound_us = 3.0 * total_flops / (PEAK_BF16_MFMA_TFLOPS * 1e12) * 1e6
    results.append({"case": f"prefill matmulQ8: one decoder layer's 7 projections, {T} tokens", "us": round(total_us, 3),
                    "TFLOP/s": round(total_flops / (total_us * 1e-6) / 1e12, 1),
                    "pct_of_bound": round(100 * bound_us / total_us, 1)})
    log(f"suite prefill layer: {total_us:.1f} us  {total_flops / (total_us * 1e-6) / 1e12:.1f} TFLOP/s")

    # The same layer as the resident batch issues it: projections of the same
    # activations (q, k, v; gate, up) in one wxo_matmul_q8_multi_ws launch
    # each, with the device's workspace (short prompts split their tiles' K
    # steps between workgroups).
    by = {name: (N, K, packed, scale) for name, N, K, packed, scale in prepared}
    ws_bytes = wxo_q8.matmul_q8_workspace_bytes()
    ws = wxo_q8.DeviceBuffer(ws_bytes)
    outs = {name: wxo_q8.DeviceBuffer(T * N * 4) for name, N, _, _, _ in prepared}
    groups = [(a_h, ("wq", "wk", "wv")), (a_h, ("wo",)), (a_h, ("wGate", "wUp")), (a_f, ("wDown",))]
    layer_us = 0.0
    for act, names in groups:
        K = by[names[0]][1]
        projs = [(by[n][2].ptr, by[n][3].ptr, outs[n].ptr, by[n][0]) for n in names]
        us = time_loop(stream, lambda i: wxo_q8.matmul_q8_multi_device(act, projs, T, K, stream, ws, ws_bytes),
                       max(1, steps // 20), max(1, warmup // 20))
        flops = sum(2.0 * T * by[n][0] * K for n in names)
        layer_us += us
        results.append({"case": f"prefill matmulQ8 {'+'.join(names)} in one launch: tokens={T} K={K}",
                        "us": round(us, 3), "TFLOP/s": round(flops / (us * 1e-6) / 1e12, 1),
                        "variant": wxo_q8.last_variant()})
        log(f"suite prefill {'+'.join(names)} one launch: {us:.2f} us  {flops / (us * 1e-6) / 1e12:.1f} TFLOP/s")
    results.append({"case": f"prefill matmulQ8: one decoder layer, {T} tokens, as the resident batch issues it "
                            f"(q/k/v and gate/up each in one launch: 4 launches)", "us": round(layer_us, 3),
                    "TFLOP/s": round(total_flops / (layer_us * 1e-6) / 1e12, 1),
                    "pct_of_bound": round(100 * bound_us / layer_us, 1)})
    log(f"suite prefill layer, coalesced: {layer_us:.1f} us  {total_flops / (layer_us * 1e-6) / 1e12:.1f} TFLOP/s")
    # Short prompts: the same four launches over the first Ts tokens (the
    # dispatch picks its tile shape from the tile count).
    for Ts in (64, 128, 256):
        short_us = 0.0
        variants = []
        for act, names in groups:
            K = by[names[0]][1]
            projs = [(by[n][2].ptr, by[n][3].ptr, outs[n].ptr, by[n][0]) for n in names]
            short_us += time_loop(stream, lambda i: wxo_q8.matmul_q8_multi_device(act, projs, Ts, K, stream, ws,
                                                                                  ws_bytes),
                                  max(1, steps // 20), max(1, warmup // 20))
            variants.append(wxo_q8.last_variant())
        short_flops = total_flops * Ts / T
        results.append({"case": f"prefill matmulQ8: one decoder layer, {Ts} tokens, as the resident batch issues it "
                                f"(4 launches)", "us": round(short_us, 3),
                        "TFLOP/s": round(short_flops / (short_us * 1e-6) / 1e12, 1), "variants": variants})
        log(f"suite prefill layer, {Ts} tokens, coalesced: {short_us:.1f} us  "
            f"{short_flops / (short_us * 1e-6) / 1e12:.1f} TFLOP/s")
    # A long prompt: the same four launches over 2048 tokens, where the
    # 256-row tiles fill the CUs in whole rounds (or 5.5 of them for gate/up).
    TL = 4 * T
    a_hl = wxo_q8.DeviceBuffer.from_array(rng.standard_normal(TL * 2048, dtype=np.float32), stream)
    a_fl = wxo_q8.DeviceBuffer.from_array(rng.standard_normal(TL * 5632, dtype=np.float32), stream)
    outs_l = {name: wxo_q8.DeviceBuffer(TL * N * 4) for name, N, _, _, _ in prepared}
    long_us = 0.0
    variants = []
    for act, names in ((a_hl, ("wq", "wk", "wv")), (a_hl, ("wo",)), (a_hl, ("wGate", "wUp")), (a_fl, ("wDown",))):
        K = by[names[0]][1]
        projs = [(by[n][2].ptr, by[n][3].ptr, outs_l[n].ptr, by[n][0]) for n in names]
        long_us += time_loop(stream, lambda i: wxo_q8.matmul_q8_multi_device(act, projs, TL, K, stream, ws, ws_bytes),
                             max(1, steps // 40), max(1, warmup // 40))
        variants.append(wxo_q8.last_variant())
    long_flops = total_flops * TL / T
    results.append({"case": f"prefill matmulQ8: one decoder layer, {TL} tokens, as the resident batch issues it "
                            f"(4 launches)", "us": round(long_us, 3),
                    "TFLOP/s": round(long_flops / (long_us * 1e-6) / 1e12, 1),
                    "pct_of_bound": round(100 * 3.0 * long_flops / (PEAK_BF16_MFMA_TFLOPS * 1e12) * 1e6 / long_us, 1),
                    "variants": variants})
    log(f"suite prefill layer, {TL} tokens, coalesced: {long_us:.1f} us  {long_flops / (long_us * 1e-6) / 1e12:.1f} "
        f"TFLOP/s")
    for b in list(outs_l.values()) + [a_hl, a_fl]:
        b.free()
    # The same four launches without a workspace (wxo_matmul_q8_multi: no K
    # split between workgroups), at every prompt length, beside the above.
    for Ts in (64, 128, 256, T):
        plain_us = 0.0
        for act, names in groups:
            K = by[names[0]][1]
            projs = [(by[n][2].ptr, by[n][3].ptr, outs[n].ptr, by[n][0]) for n in names]
            plain_us += time_loop(stream, lambda i: wxo_q8.matmul_q8_multi_device(act, projs, Ts, K, stream),
                                  max(1, steps // 20), max(1, warmup // 20))
        results.append({"case": f"prefill matmulQ8: one decoder layer, {Ts} tokens, 4 launches without a workspace",
                        "us": round(plain_us, 3),
                        "TFLOP/s": round(total_flops * Ts / T / (plain_us * 1e-6) / 1e12, 1)})
        log(f"suite prefill layer, {Ts} tokens, 4 launches without a workspace: {plain_us:.1f} us")
    for b in outs.values():
        b.free()
    ws.free()

    # dequantizePackedQ8 and dequantTranspose of the gate projection, gather of
    # the prompt's rows from a 32000 x 2048 int8 embedding table
    _, N, K, packed, scale = prepared[4]
    W = (K + 3) // 4
    dq_bytes = N * W * 4 + 4 * N + 4 * N * K
    for case, fn in (("dequantizePackedQ8", lambda i: check(L.wxo_dequantize_packed_q8(packed.ptr, scale.ptr, N, K,
                                                                                         out2.ptr, sp))),
                     ("dequantTranspose", lambda i: check(L.wxo_dequant_transpose(packed.ptr, scale.ptr, N, K,
                                                                                    out2.ptr, sp)))):
        out2 = wxo_q8.DeviceBuffer(N * K * 4)
        us, usq = time_both(stream, fn, max(1, steps // 20), max(1, warmup // 20))
        gbs = dq_bytes / (us * 1e-6) / 1e9
        results.append({"case": f"{case} N={N} K={K}", "bytes": dq_bytes, "us": round(us, 3), "GB/s": round(gbs, 1),
                        "pct_hbm": round(100 * gbs / PEAK_HBM_GBS, 1), "us_queued": _q(usq)})
        log(f"suite {case} {N}x{K}: {us:.2f} us  {gbs:.0f} GB/s  {100 * gbs / PEAK_HBM_GBS:.1f}% HBM{_qs(usq)}")
        out2.free()
    rows, D = 32000, 2048
    table = wxo_q8.DeviceBuffer.from_array(rng.integers(-127, 128, rows * D).astype(np.int8), stream)
    tscale = wxo_q8.DeviceBuffer.from_array(rng.uniform(0.001, 0.02, rows).astype(np.float32), stream)
    idx = wxo_q8.DeviceBuffer.from_array(rng.integers(0, rows, T).astype(np.int64), stream)
    g_bytes = T * (D + 4 + 8 + 4 * D)
    us, usq = time_both(stream, lambda i: check(L.wxo_gather_dequant_rows(table.ptr, tscale.ptr, rows, D, idx.ptr, T,
                                                                          out.ptr, sp)),
                        max(1, steps // 20), max(1, warmup // 20))
    gbs = g_bytes / (us * 1e-6) / 1e9
    results.append({"case": f"gatherDequantRows {T} rows of a {rows}x{D} table", "bytes": g_bytes, "us": round(us, 3),
                    "GB/s": round(gbs, 1), "us_queued": _q(usq)})
    log(f"suite gatherDequantRows {T} of {rows}x{D}: {us:.2f} us  {gbs:.0f} GB/s{_qs(usq)}")
    for b in (a_h, a_f, out, table, tscale, idx):
        b.free()
    for _, _, _, packed, scale in prepared:
        packed.free()
        scale.free()


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--copies", type=int, default=12, help="distinct weight copies rotated through (HBM, not MALL)")
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--suite", metavar="PATH", default=None,
                    help="also measure every BASELINE configuration and write the table (JSON) to PATH")
    ap.add_argument("--prefill-suite", metavar="PATH", default=None,
                    help="measure only the prefill-side ops (matmulQ8, dequant, gather) and write them to PATH")
    ap.add_argument("--case", metavar="CFG[:M]", default=None,
                    help="measure one BASELINE configuration alone (e.g. cfg5:16) and print its line (diagnostics, "
                         "profiling)")
    ap.add_argument("--no-napi", action="store_true",
                    help="leave the Node-API end-to-end rows out of --suite (kernel traces: the tracer would follow "
                         "the node child too)")
    ap.add_argument("--calibrate-copy", type=int, default=0,
                    help="after timing, run this many device copies of the packed weight (counter calibration)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU only: the matvecQ8 path runs on one MI355X; "
                                   "multi-GPU row sharding is a design note, not a measured configuration",
                          "n_gpus": args.gpus}))
        return 2

    wxo_q8.init()
    log(wxo_q8.describe())
    if args.case:
        print(json.dumps(run_case(wxo_q8.Stream(), args.case, args.steps, args.warmup)), flush=True)
        return 0
    if args.prefill_suite:
        stream = wxo_q8.Stream()
        table = []

        def check(st):
            if st != 0:
                raise wxo_q8.WxoError(st, wxo_q8.lib().wxo_last_error().decode())
        run_prefill_suite(stream, args.steps, args.warmup, table, check)
        add_calibrated_matrix(table, calibrated_matrix_ceiling())
        add_calibrated(table, calibrated_ceiling())
        if not args.no_cpu_baseline:
            table.extend(cpu_reference_ops(budget_s=1.0))
        with open(args.prefill_suite, "w") as f:
            json.dump(table, f, indent=1)
        return 0
    cfg = wl.CONFIGS["cfg2"]
    N, K, M = cfg["N"], cfg["K"], 1
    W = (K + 3) // 4
    c = wl.make_config("cfg2")
    stream = wxo_q8.Stream()

    # quantize + pack on the GPU (the product path), then replicate.
    bw_f32 = wxo_q8.DeviceBuffer.from_array(c["w"], stream)
    packed0 = wxo_q8.DeviceBuffer(N * W * 4)
    scale = wxo_q8.DeviceBuffer(N * 4)
    wxo_q8.quantize_pack_q8_device(bw_f32, N, K, packed0, scale, stream)
    stream.synchronize()
    bw_f32.free()
    row_bytes = N * W * 4
    copies = max(1, args.copies)
    rot = wxo_q8.DeviceBuffer(row_bytes * copies)
    for i in range(copies):
        wxo_q8.lib().wxo_memcpy_dtod(rot.ptr + i * row_bytes, packed0.ptr, row_bytes, stream.handle)
    vec = wxo_q8.DeviceBuffer.from_array(c["x"], stream)
    out = wxo_q8.DeviceBuffer(N * M * 4)
    stream.synchronize()
    weights = [rot.ptr + i * row_bytes for i in range(copies)]
    launch = wxo_q8.lib().wxo_matvec_q8
    sp = stream.handle

    def call(i):
        st = launch(weights[i % copies], scale.ptr, vec.ptr, out.ptr, N, K, M, sp)
        if st != 0:
            raise wxo_q8.WxoError(st, wxo_q8.lib().wxo_last_error().decode())

    total_ms = timed_headline(stream, call, copies, args.warmup, args.steps)
    variant = wxo_q8.last_variant()
    ms_per_step = total_ms / args.steps
    bytes_per_call = wl.matvec_bytes(N, K, M)
    value = bytes_per_call / (ms_per_step * 1e-3) / 1e9

    # The launch stream holds nothing but these K matvec dispatches between
    # the events, so the timed region / K is the mean launch duration,
    # back to back (events around single launches would add ~2 us each).
    launch_us = ms_per_step * 1e3
    achieved = bytes_per_call / (launch_us * 1e-6) / 1e9
    log(f"timed region {total_ms:.3f} ms / {args.steps} calls = {launch_us:.3f} us/call ({variant})")

    cal = calibrated_ceiling()

    if args.calibrate_copy:
        # Plain device copies of one weight copy into another (rocclr's
        # copyBuffer kernel), source and destination rotating through the
        # copies like the timed calls, so neither is cache-resident: the
        # known-size reference for the traffic counters.
        for i in range(args.calibrate_copy):
            src, dst = (2 * i) % copies, (2 * i + 1) % copies
            wxo_q8.lib().wxo_memcpy_dtod(rot.ptr + dst * row_bytes, rot.ptr + src * row_bytes, row_bytes, sp)
        stream.synchronize()
        log(f"calibration: {args.calibrate_copy} device copies of {row_bytes} B")

    baseline = None
    if not args.no_cpu_baseline:
        packed_host = packed0.download(np.uint32, N * W)
        scales_host = scale.download(np.float32, N)
        baseline = cpu_baseline(packed_host, scales_host, c["x"], N, K, args.cpu_budget)

    if args.suite:
        table = run_suite(stream, args.steps, args.warmup, napi=not args.no_napi)
        add_calibrated(table, cal)
        with open(args.suite, "w") as f:
            json.dump(table, f, indent=1)

    line = {
        "metric": "matvecQ8 achieved HBM GB/s (% of 8 TB/s peak; us/call) at N=11008, K=4096",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "us_per_call": round(ms_per_step * 1e3, 3),
        "pct_of_peak": round(100.0 * value / PEAK_HBM_GBS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 weights x f32 vector, f32 accumulate",
        "data": "synthetic (seeded numpy PCG64: W~N(0,0.02) quantized+packed on GPU, x~N(0,1))",
        "config": {"workload": "matvecQ8 Llama-7B MLP up N=11008 K=4096 M=1 (BASELINE configs[1])",
                   "N": N, "K": K, "M": M, "variant": variant, "weight_copies_rotated": copies,
                   "rotated_bytes": row_bytes * copies, "bytes_per_call": bytes_per_call},
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": read_traffic(),
            "traffic_source": TRAFFIC_NOTE,
            "launch_us_events": round(launch_us, 3),
            "calibrated": {"GB/s": cal["GB/s"], "frac": round(achieved / cal["GB/s"], 4),
                           "fma_TFLOP/s": cal["fma_TFLOP/s"], "source": cal["source"]},
        },
        "cpu_baseline": baseline,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
