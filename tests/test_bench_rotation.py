"""The timed loops of bench.py rotate weight copies so that every timed call
streams its weights from HBM: each call reads copy (index % copies), and the
index runs on from the set-up calls through the timed ones.  These tests drive
the loops with a recording launch and stand-in events (no GPU) and check the
index sequence they issue: every timed call reads the copy whose previous read
is the furthest back (exactly `copies` calls earlier), and no copy is first
read inside a timed region."""
import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


class Recorder:
    """One log of launches and event records in issue order."""

    def __init__(self):
        self.log = []
        self.handle = 0

    def launch(self, i):
        self.log.append(("call", i))

    def synchronize(self):
        self.log.append(("sync", None))

    def event_type(self):
        rec = self

        class Event:
            def __init__(self, timer=False):
                assert timer, "timed regions use timing-only events"

            def record(self, stream):
                rec.log.append(("event", None))

            def synchronize(self):
                pass

            def elapsed_ms(self, end):
                return 1.0

        return Event

    def timed_regions(self):
        """[(calls before the region, calls inside it)] for each event pair."""
        marks = [n for n, (kind, _) in enumerate(self.log) if kind == "event"]
        assert len(marks) % 2 == 0
        out = []
        for a, b in zip(marks[::2], marks[1::2]):
            before = [i for kind, i in self.log[:a] if kind == "call"]
            inside = [i for kind, i in self.log[a:b] if kind == "call"]
            out.append((before, inside))
        return out


def check_rotation(calls_before, timed, copies):
    """Every timed call's copy was last read exactly `copies` calls earlier,
    and was read at least once before the region opened."""
    seq = calls_before + timed
    last = {}
    for pos, i in enumerate(seq):
        c = i % copies
        if pos >= len(calls_before):
            assert c in last, f"copy {c} first read inside the timed region (call {pos})"
            assert pos - last[c] == copies, (
                f"timed call {pos - len(calls_before)} reads copy {c}, last read {pos - last[c]} calls earlier "
                f"(fewer than the {copies} copies rotated)")
        last[c] = pos


@pytest.mark.parametrize("copies,warmup,steps", [(12, 5, 20), (12, 200, 2000), (12, 0, 7), (5, 3, 40), (1, 2, 3),
                                                 (13, 11, 1)])
def test_headline_timed_calls_read_the_oldest_copy(bench, copies, warmup, steps):
    rec = Recorder()
    bench.timed_headline(rec, rec.launch, copies, warmup, steps, event=rec.event_type(), sync=lambda: None)
    (before, timed), = rec.timed_regions()
    assert len(timed) == steps
    assert len(before) == copies + warmup + bench.LEAD_STEPS
    check_rotation(before, timed, copies)


def test_driver_short_run_sequence(bench):
    """The driver's run (--steps 20 --warmup 5, 12 copies): the exact copies of
    the timed calls, none of them read in the 11 calls before it."""
    rec = Recorder()
    bench.timed_headline(rec, rec.launch, 12, 5, 20, event=rec.event_type(), sync=lambda: None)
    (before, timed), = rec.timed_regions()
    assert [i % 12 for i in timed] == [(27 + n) % 12 for n in range(20)]
    for n, i in enumerate(timed):
        window = (before + timed)[len(before) + n - 11:len(before) + n]
        assert i % 12 not in [j % 12 for j in window]


@pytest.mark.parametrize("copies,setup,warmup,steps", [(12, 12, 5, 20), (82, 82, 28, 285), (34, 34, 50, 500)])
def test_suite_loops_continue_the_rotation(bench, monkeypatch, copies, setup, warmup, steps):
    """time_both: the host-issued loop then the queued loop, one sequence."""
    rec = Recorder()
    monkeypatch.setattr(bench.wxo_q8, "Event", rec.event_type())
    monkeypatch.setattr(bench, "_spin", lambda stream, us: None)
    bench.time_both(rec, rec.launch, steps, warmup, setup)
    regions = rec.timed_regions()
    assert len(regions) == 2
    for before, timed in regions:
        assert len(timed) == steps
        check_rotation(before, timed, copies)


def test_measure_matvec_style_setup_then_loops(bench, monkeypatch):
    """measure_matvec's order: one set-up call per copy on the case's sequence,
    then time_loop and time_loop_queued continuing it."""
    import itertools
    rec = Recorder()
    monkeypatch.setattr(bench.wxo_q8, "Event", rec.event_type())
    monkeypatch.setattr(bench, "_spin", lambda stream, us: None)
    copies = 12
    seq = itertools.count()
    for _ in range(copies):
        rec.launch(next(seq))
    bench.time_loop(rec, rec.launch, 20, 5, seq)
    bench.time_loop_queued(rec, rec.launch, 20, seq)
    for before, timed in rec.timed_regions():
        check_rotation(before, timed, copies)


def test_a_restarted_index_is_caught(bench):
    """The check itself: the sequence the loops issued before (lead calls at
    warmup + i, timed calls from 0) fails it."""
    copies, warmup, steps = 12, 5, 20
    before = list(range(copies)) + list(range(warmup)) + [warmup + i for i in range(bench.LEAD_STEPS)]
    timed = list(range(steps))
    with pytest.raises(AssertionError, match="last read"):
        check_rotation(before, timed, copies)


def test_prefill_rows_against_the_calibrated_matrix_rate(bench):
    """Every matmulQ8 row of the prefill suite gets its share of the calibrated
    matrix-core rate at three matrix flops per useful one; other rows are left
    alone, and the ceiling itself heads the table."""
    table = [{"case": "prefill matmulQ8 wq: tokens=512 M=2048 K=2048", "us": 25.0, "TFLOP/s": 170.0},
             {"case": "prefill matmulQ8: one decoder layer, 512 tokens", "us": 200.0, "TFLOP/s": 250.0},
             {"case": "dequantizePackedQ8 N=5632 K=2048", "us": 9.5, "GB/s": 6000.0}]
    bench.add_calibrated_matrix(table, {"TFLOP/s": 1750.0, "source": "test"})
    assert table[0]["case"].startswith("calibrated ceiling (wxo_roofline_matrix)")
    assert table[0]["TFLOP/s"] == 1750.0 and table[0]["pct_of_peak"] == 70.0
    assert table[1]["pct_of_calibrated_matrix"] == round(100 * 3 * 170.0 / 1750.0, 1)
    assert table[2]["pct_of_calibrated_matrix"] == round(100 * 3 * 250.0 / 1750.0, 1)
    assert "pct_of_calibrated_matrix" not in table[3]
