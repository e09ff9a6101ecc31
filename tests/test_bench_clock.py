"""bench.py's shader-clock summary (CPU only: samples are given, amdsmi is
not read)."""

from __future__ import annotations

import importlib.util
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def sampler_with(bench, rows_by_gpu):
    s = bench.ClockSampler.__new__(bench.ClockSampler)
    s.error = None
    s.samples = rows_by_gpu
    return s


def test_idle_samples_do_not_lower_the_kernel_clock(bench):
    # 40 busy samples at 2400 MHz, 30 idle ones parked at 1200 MHz
    rows = [(2400.0, 100.0)] * 40 + [(1200.0, 0.0)] * 30
    r = sampler_with(bench, {0: rows}).result()
    assert r["mean_mhz"] == pytest.approx((40 * 2400 + 30 * 1200) / 70, abs=0.1)
    assert r["busy_samples"] == 40 and r["busy_mean_mhz"] == 2400.0
    assert bench.ClockSampler.kernel_mhz(r) == 2400.0


def test_few_busy_samples_fall_back_to_the_median(bench):
    rows = [(2000.0, 10.0)] * 20 + [(2400.0, 90.0)] * 5 + [(1500.0, 0.0)] * 4
    r = sampler_with(bench, {0: rows}).result()
    assert r["busy_samples"] == 5
    assert bench.ClockSampler.kernel_mhz(r) == 2000.0


def test_busiest_gpu_is_reported(bench):
    rows = {0: [(1000.0, 5.0)] * 12, 1: [(2100.0, 95.0)] * 12}
    r = sampler_with(bench, rows).result()
    assert r["busy_mean_mhz"] == 2100.0


def test_no_samples(bench):
    r = sampler_with(bench, {}).result()
    assert "error" in r and bench.ClockSampler.kernel_mhz(r) is None
    assert bench.ClockSampler.kernel_mhz(None) is None
