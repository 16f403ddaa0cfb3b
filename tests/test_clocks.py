"""CPU tests of the clock/power telemetry, the row gates and the between-run
comparison (``tritonkv_amd/clocks.py``), on fake sysfs trees."""

from __future__ import annotations

import json
import os
import subprocess
import sys
import time

import pytest

from tritonkv_amd import clocks

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _write(path, text):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w") as f:
        f.write(text)


def _fake_card(root, sclk="0: 500Mhz\n1: 2105Mhz *\n2: 2400Mhz\n"):
    dev = os.path.join(root, "card0", "device")
    _write(os.path.join(dev, "pp_dpm_sclk"), sclk)
    _write(os.path.join(dev, "pp_dpm_mclk"), "0: 2000Mhz *\n")
    _write(os.path.join(dev, "gpu_busy_percent"), "97\n")
    hw = os.path.join(dev, "hwmon", "hwmon0")
    _write(os.path.join(hw, "power1_input"), "1012000000\n")
    _write(os.path.join(hw, "temp2_label"), "junction\n")
    _write(os.path.join(hw, "temp2_input"), "71000\n")
    _write(os.path.join(hw, "temp3_label"), "mem\n")
    _write(os.path.join(hw, "temp3_input"), "55000\n")
    return dev


def test_parse_dpm():
    assert clocks.parse_dpm("0: 500Mhz\n1: 2105Mhz *\n2: 2400Mhz\n") == (2105.0, 2400.0)
    assert clocks.parse_dpm("0: 2000Mhz *\n") == (2000.0, 2000.0)
    assert clocks.parse_dpm("0: 0.5GHz\n1: 1.9GHz *\n") == (1900.0, 1900.0)
    assert clocks.parse_dpm("0: 500Mhz\n1: 2400Mhz\n") == (None, 2400.0)   # no current mark
    assert clocks.parse_dpm("") == (None, None)
    assert clocks.parse_dpm("garbage\nS: nothing\n") == (None, None)


def test_sysfs_reader_on_a_fake_card(tmp_path):
    dev = _fake_card(str(tmp_path))
    assert clocks.find_device(str(tmp_path)) == dev
    r = clocks.SysfsReader(dev)
    assert r.gfx_max_mhz == 2400.0
    s = r.sample()
    assert s == {"gfx_mhz": 2105.0, "mem_mhz": 2000.0, "busy_pct": 97.0,
                 "power_w": pytest.approx(1012.0), "junction_c": 71.0, "hbm_c": 55.0}
    assert clocks.find_device(str(tmp_path / "none")) is None


def test_monitor_windows_and_gates(tmp_path):
    dev = _fake_card(str(tmp_path))
    mon = clocks.ClockMonitor(interval_s=0.005, device_dir=dev, allow_amdsmi=False)
    assert mon.start()
    assert mon.source == "sysfs" and mon.gfx_max_mhz == 2400.0
    t0 = time.time()
    time.sleep(0.08)
    t1 = time.time()
    # throttle: the current level drops to 1500 MHz (< 0.7 x 2400)
    _write(os.path.join(dev, "pp_dpm_sclk"), "0: 500Mhz\n1: 1500Mhz *\n2: 2400Mhz\n")
    time.sleep(0.08)
    t2 = time.time()
    mon.stop()
    early = mon.window(t0, t1)
    assert early["enough_samples"] and early["boosted"] and early["stable"]
    assert early["gfx_mhz_min"] == 2105.0 and early["junction_c_max"] == 71.0
    assert early["mem_clock_constant"]
    whole = mon.window(t0, t2)
    assert whole["gfx_mhz_min"] == 1500.0 and not whole["boosted"] and not whole["stable"]
    assert mon.window(t2 + 10, t2 + 11) is None


def test_monitor_without_telemetry(tmp_path):
    mon = clocks.ClockMonitor(device_dir=str(tmp_path / "absent"), allow_amdsmi=False)
    assert not mon.start() and not mon.available


def test_hot_junction_fails_the_thermal_gate():
    vals = [{"gfx_mhz": 2400.0, "junction_c": 96.0}] * 5
    w = clocks.summarize(vals, 2400.0)
    assert w["boosted"] and not w["thermal_headroom"] and not w["stable"]
    w = clocks.summarize(vals[:3], 2400.0)
    assert not w["enough_samples"]


def test_amdsmi_csv_line():
    header = ("gpu,xcp,power_usage,max_power,hotspot_temperature,memory_temperature,"
              "gfx_clk,gfx,mem,mem_clock").split(",")
    s = clocks.parse_amdsmi_csv_line(header, "0,0,250,1400,46,33,157,0,0,2000")
    assert s == {"gfx_mhz": 157.0, "mem_mhz": 2000.0, "busy_pct": 0.0, "power_w": 250.0,
                 "junction_c": 46.0, "hbm_c": 33.0}
    assert clocks.parse_amdsmi_csv_line(header, "0,0,250") is None


def test_spread_and_row_gate():
    assert clocks.spread_frac([100.0, 101.0, 104.0]) == pytest.approx(0.04 / 1.01)
    # 8 or more timings: IQR (inclusive quartiles) over the median, outliers ignored
    xs = [100.0] * 4 + [101.0] * 4 + [200.0]
    assert clocks.spread_frac(xs) == pytest.approx(1.0 / 101.0)
    assert clocks.timing_is_tight(xs)
    assert not clocks.timing_is_tight([100.0, 110.0])
    assert clocks.spread_frac([]) is None
    stable = {"stable": True}
    assert clocks.row_gate(stable, [100.0, 101.0])["quotable"]
    assert not clocks.row_gate({"stable": False}, [100.0, 101.0])["quotable"]
    assert not clocks.row_gate(stable, [100.0, 120.0])["quotable"]
    g = clocks.row_gate(None, [100.0, 101.0])   # no sampler: the timing gate alone
    assert g["quotable"] and g["clocks_stable"] is None


def _line(value, fp16_split, fused2_split, gfx=2100.0):
    return {"metric": "m", "value": value, "unit": "us", "steps": 100,
            "cpu_baseline": {"value": 5.0},
            "clocks": {"gfx_mhz_mean": gfx},
            "detail": {"fp16": {"us_per_step": fp16_split + 5, "split_kernel_us": fp16_split,
                                "cache_bytes": 123, "clocks": {"gfx_mhz_mean": gfx}},
                       "fused2": {"split_kernel_us": fused2_split}}}


def test_compare_runs():
    a, b = _line(200.0, 620.0, 150.0), _line(204.0, 690.0, 151.0, gfx=1900.0)
    recs = {r["key"]: r for r in clocks.compare_runs([a, b], ["a", "b"])}
    assert set(recs) == {"value", "detail.fp16.us_per_step", "detail.fp16.split_kernel_us",
                         "detail.fused2.split_kernel_us"}            # timings only
    assert recs["value"]["spread_frac"] == pytest.approx(0.02) and not recs["value"]["moved"]
    assert recs["detail.fp16.split_kernel_us"]["moved"]
    assert recs["detail.fp16.split_kernel_us"]["gfx_mhz_mean"] == {"a": 2100.0, "b": 1900.0}
    assert recs["value"]["gfx_mhz_mean"] == {"a": 2100.0, "b": 1900.0}
    assert recs["detail.fused2.split_kernel_us"]["gfx_mhz_mean"] is None


def test_load_run_and_bench_compare(tmp_path):
    pa, pb = tmp_path / "a.json", tmp_path / "b.json"
    pa.write_text("# llama 4-bit: step 200 us\n" + json.dumps(_line(200.0, 620.0, 150.0)) + "\n")
    pb.write_text(json.dumps({"round": 1, "bench": _line(230.0, 621.0, 150.0)}))
    assert clocks.load_run(str(pa))["value"] == 200.0
    assert clocks.load_run(str(pb))["value"] == 230.0
    bad = tmp_path / "bad.json"
    bad.write_text("nothing here\n")
    with pytest.raises(ValueError):
        clocks.load_run(str(bad))
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--compare", str(pa),
                        str(pb)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["runs"] == ["a.json", "b.json"] and out["moved"] == ["value"]
    assert out["max_spread_frac"] == pytest.approx(0.15)
