"""The timeline tool's stamp analysis (juno_amd/timeline.py) on synthetic
stamps whose intervals are known: the staged walk's four stamps per wave and
the batched walk's per-step and epilogue stamps.  The instrumented GPU builds
themselves run only on the GPU box (never the shipped library)."""
import numpy as np
import pytest

from juno_amd import timeline as TL


def test_staged_stats_known_intervals():
    # 2 workgroups x 16 waves; ticks of 10 ns; waves start 0..31 ticks apart
    nw, wgs = 16, 2
    t = np.zeros((wgs * nw, 4), dtype=np.uint64)
    for i in range(wgs * nw):
        t0 = 1000 + i
        t[i] = [t0, t0 + 200, t0 + 300, t0 + 1500 + (i // nw) * 100]
    d = TL.staged_launch_stats(t.reshape(-1))
    assert d["waves"] == 32
    assert d["start_max"] == pytest.approx(0.31)
    assert d["prologue_p50"] == pytest.approx(2.155, abs=1e-9)  # (200 + 15.5 ticks) -> us
    assert d["wg_end_min"] == pytest.approx((15 + 1500) * 0.01)
    assert d["end"] == pytest.approx((31 + 1600) * 0.01)


def test_staged_stats_ignore_waves_that_did_not_run():
    t = np.zeros((32, 4), dtype=np.uint64)
    t[:16] = [[1000 + i, 1100 + i, 1200 + i, 2000 + i] for i in range(16)]
    d = TL.staged_launch_stats(t.reshape(-1))
    assert d["waves"] == 16 and d["end"] == pytest.approx(10.15)


def test_mfma_stats_known_intervals():
    # 8 waves, 3 steps: barrier 50, park 10, stage 40, fold 70 ticks; the
    # first step's barrier 300 ticks after entry; epilogue 20 / 30 / 60 ticks
    waves, steps = 8, 3
    t = np.zeros((waves, TL.MFMA_PER_WAVE), dtype=np.uint64)
    for w in range(waves):
        now = 5000 + w
        t[w, 0] = now
        for sidx in range(steps):
            now += 300 if sidx == 0 else 50
            t[w, 1 + 4 * sidx] = now
            now += 10
            t[w, 2 + 4 * sidx] = now
            now += 40
            t[w, 3 + 4 * sidx] = now
            now += 70
            t[w, 4 + 4 * sidx] = now
        t[w, 65] = now + 20
        t[w, 66] = now + 50
        if w < 4:  # the waves of the last split
            t[w, 67] = now + 110
    d = TL.mfma_launch_stats(t.reshape(-1))
    assert d["steps"] == steps and d["waves"] == waves
    assert d["barrier_first"] == pytest.approx(3.0)
    assert d["barrier_rest"] == pytest.approx(0.5)
    assert d["park_rest"] == pytest.approx(0.1)
    assert d["stage_issue_rest"] == pytest.approx(0.4)
    assert d["mfma_fold_rest"] == pytest.approx(0.7)
    assert d["acked_p50"] == pytest.approx(0.2)
    assert d["counted_p50"] == pytest.approx(0.3)
    assert d["sum_store_p50"] == pytest.approx(0.6)
    assert d["walk_end_max"] == pytest.approx((7 + 300 + 120 + 2 * 170) * 0.01)


def test_mfma_stats_unsplit_launch_has_no_epilogue_figures():
    t = np.zeros((8, TL.MFMA_PER_WAVE), dtype=np.uint64)
    for w in range(8):
        t[w, :9] = 1000 + w + np.arange(9) * 10
    d = TL.mfma_launch_stats(t.reshape(-1))
    assert d["steps"] == 2 and "acked_p50" not in d and "sum_store_p50" not in d
    text = TL.summary_mfma({"launches": [dict(d, event_us=1.0)], "B": 32, "kernel": 1, "ksplit": 1})
    assert "| park |" in text
