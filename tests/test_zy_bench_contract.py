"""bench.py's output contract: one JSON line with the fields the round's
driver reads, a roofline object for the dominant kernel and the CPU baseline
beside it; one GPU only; no CPU fallback when no gfx950 is visible."""
import json
import os
import subprocess
import sys

import pytest

import wxo_q8

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def have_gpu():
    try:
        return wxo_q8.device_count() > 0
    except wxo_q8.WxoError:
        return False


def run_bench(*args, timeout=600):
    return subprocess.run([sys.executable, BENCH, *args], capture_output=True, text=True, timeout=timeout, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    p = run_bench("--gpus", "2")
    assert p.returncode == 2
    msg = json.loads(p.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"] and msg["n_gpus"] == 2


@pytest.mark.skipif(have_gpu(), reason="checks the no-GPU failure path")
def test_no_gpu_fails_loudly():
    p = run_bench("--steps", "5", "--warmup", "1")
    assert p.returncode != 0
    assert "no CPU fallback" in p.stderr


@pytest.mark.gpu
def test_json_line_contract():
    print("bench.py --steps 200 --warmup 20 --cpu-budget 1", flush=True)
    p = run_bench("--steps", "200", "--warmup", "20", "--cpu-budget", "1")
    assert p.returncode == 0, p.stderr[-2000:]
    lines = [l for l in p.stdout.splitlines() if l.strip()]
    assert len(lines) == 1, lines
    r = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in r, key
    assert r["n_gpus"] == 1 and r["steps"] == 200 and r["warmup"] == 20
    assert r["unit"] == "GB/s" and r["higher_is_better"] is True and r["vs_baseline"] is None
    assert "workload" in r["config"] and r["config"]["N"] == 11008 and r["config"]["K"] == 4096
    # value is algorithmic bytes over the measured time per call
    assert abs(r["value"] - r["config"]["bytes_per_call"] / (r["ms_per_step"] * 1e-3) / 1e9) <= 0.01 * r["value"]
    rl = r["roofline"]
    assert rl["bound"] == "hbm" and rl["unit"] == "GB/s" and rl["peak"] == 8000.0
    assert abs(rl["frac"] - rl["achieved"] / rl["peak"]) < 1e-3
    assert 0.3 < rl["frac"] < 1.0
    assert rl["traffic"] is None or rl["traffic"] >= r["config"]["bytes_per_call"] * 0.99
    assert abs(rl["launch_us_events"] - r["ms_per_step"] * 1e3) < 1e-2
    assert "profiles/" in rl["traffic_source"]
    # the kernel instance that ran is named
    assert r["config"]["variant"].startswith("matvec_q8_m1 ") and "waves=4" in r["config"]["variant"]
    cb = r["cpu_baseline"]
    assert cb is not None and cb["kind"] in ("port", "reference") and cb["cores"] >= 1 and cb["value"] > 0


@pytest.mark.gpu
def test_short_and_long_runs_agree():
    """The driver's short run (20 steps after 5 warmups) and a 2000-step run
    measure the same per-call time: no first touches, no host launch latency,
    no event fences and no re-read of a recently streamed weight copy inside
    the timed region (one launch index runs from the set-up through the
    timed calls).  Each bench process places its buffers anew, which moves a
    run by up to about 1 %, so short and long runs alternate, seven of each,
    and their medians must agree within 2 %.  A cache re-read of weight copies
    would show as more than that; what remains is the box: sustained 17 ms
    streams ran 0.5 % slower than 0.17 ms bursts on one MI355X and 1.5 % on
    another (medians 8.69 against 8.56 us), so a 1 % bar fails by the box.
    The rotation itself is pinned exactly on the CPU (test_bench_rotation)."""
    runs = {20: [], 2000: []}
    for _ in range(7):
        for steps, warmup in ((20, 5), (2000, 200)):
            print(f"bench.py --steps {steps} --warmup {warmup} --no-cpu-baseline", flush=True)
            p = run_bench("--steps", str(steps), "--warmup", str(warmup), "--no-cpu-baseline")
            assert p.returncode == 0, p.stderr[-2000:]
            runs[steps].append(json.loads(p.stdout.strip().splitlines()[-1])["ms_per_step"])
            print(f"  ms_per_step {runs[steps][-1]}", flush=True)
    res = {k: sorted(v)[3] for k, v in runs.items()}
    assert abs(res[20] - res[2000]) <= 0.02 * res[2000], runs
