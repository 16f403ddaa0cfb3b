"""Clock, power and temperature telemetry around timed measurements, and the
gates that decide whether a timing is quotable.

The reference samples ``nvidia-smi -lms`` in a background process and gates
each benchmark row on the samples taken while the row was timed
(``benchmark.py:130-296``), and compares complete runs against each other
(``between_run.py:113-217``).  On MI355X the same facts are plain reads of the amdgpu
driver's sysfs files, so the sampler here is a thread that reads them, with no
subprocess per sample:

* ``pp_dpm_sclk`` / ``pp_dpm_mclk``: the DPM levels, the current one marked
  ``*`` (under load the middle line carries the live graphics clock, e.g.
  ``1: 2105Mhz *``; the last line is the maximum);
* ``gpu_busy_percent``;
* ``hwmon*/power1_input`` (microwatts), ``temp2_input`` (junction) and
  ``temp3_input`` (HBM), in millidegrees.

When sysfs is not readable, :class:`ClockMonitor` falls back to one
long-lived ``amd-smi monitor --csv`` process (whose period is whole seconds,
so only long windows gather enough samples).  Telemetry is an annotation:
when neither source works the monitor reports ``available = False`` and the
measurement goes on without it.

A row is *stable* when every graphics-clock sample is at least
``BOOST_FLOOR_FRAC`` of the maximum level, the junction stays below
``JUNCTION_LIMIT_C`` and there are at least ``MIN_SAMPLES`` samples; it is
*tight* when its own timings agree (IQR, or for fewer than 8 timings the full
range, within ``MAX_SPREAD_FRAC`` of the median, ``benchmark.py:298``, ``:316-322``).
*Quotable* means both.
"""

from __future__ import annotations

import csv
import glob
import io
import json
import os
import statistics
import subprocess
import threading
import time

BOOST_FLOOR_FRAC = 0.70      # every graphics-clock sample >= this fraction of the top DPM level
JUNCTION_LIMIT_C = 95.0      # junction temperature above which throttling is assumed
MAX_SPREAD_FRAC = 0.05       # a quotable timing's IQR (or range) is within 5% of its median
MIN_SAMPLES = 4              # fewer samples than this prove nothing about the window
KEYS = ("gfx_mhz", "mem_mhz", "busy_pct", "power_w", "junction_c", "hbm_c")


# --------------------------------------------------------------------------
# sysfs parsing (pure functions, tested on the CPU)
# --------------------------------------------------------------------------

def parse_dpm(text: str) -> tuple[float | None, float | None]:
    """(current MHz, top-level MHz) of a ``pp_dpm_*clk`` file.

    Lines read ``<level>: <freq>Mhz`` with ``*`` after the current level;
    frequencies may also be given in GHz.  Returns ``(None, None)`` for text
    with no level line.
    """
    cur, top = None, None
    for line in text.splitlines():
        if ":" not in line:
            continue
        _, rest = line.split(":", 1)
        tok = rest.split()
        if not tok:
            continue
        f = tok[0].lower()
        try:
            if f.endswith("mhz"):
                mhz = float(f[:-3])
            elif f.endswith("ghz"):
                mhz = float(f[:-3]) * 1e3
            else:
                continue
        except ValueError:
            continue
        top = mhz if top is None else max(top, mhz)
        if "*" in rest:
            cur = mhz
    return cur, top


def find_device(root: str = "/sys/class/drm") -> str | None:
    """The sysfs ``device`` directory of the first amdgpu card that exposes
    ``pp_dpm_sclk``, or None.  (A box here has one GPU.)"""
    for d in sorted(glob.glob(os.path.join(root, "card*", "device"))):
        if os.path.exists(os.path.join(d, "pp_dpm_sclk")):
            return d
    return None


def _read(path: str) -> str | None:
    try:
        with open(path) as f:
            return f.read()
    except OSError:
        return None


def _num(text: str | None, scale: float = 1.0) -> float | None:
    if text is None:
        return None
    try:
        return float(text.strip()) * scale
    except ValueError:
        return None


class SysfsReader:
    """One telemetry sample per call from a card's sysfs directory."""

    def __init__(self, device_dir: str):
        self.dev = device_dir
        hw = sorted(glob.glob(os.path.join(device_dir, "hwmon", "hwmon*")))
        self.hwmon = hw[0] if hw else None
        _, self.gfx_max_mhz = parse_dpm(_read(os.path.join(device_dir, "pp_dpm_sclk")) or "")
        self.temps = {}
        if self.hwmon:
            for lab in glob.glob(os.path.join(self.hwmon, "temp*_label")):
                name = (_read(lab) or "").strip().lower()
                self.temps[name] = lab[:-len("_label")] + "_input"

    def sample(self) -> dict:
        gfx, _ = parse_dpm(_read(os.path.join(self.dev, "pp_dpm_sclk")) or "")
        mem, _ = parse_dpm(_read(os.path.join(self.dev, "pp_dpm_mclk")) or "")
        s = {"gfx_mhz": gfx, "mem_mhz": mem,
             "busy_pct": _num(_read(os.path.join(self.dev, "gpu_busy_percent"))),
             "power_w": None, "junction_c": None, "hbm_c": None}
        if self.hwmon:
            p = _num(_read(os.path.join(self.hwmon, "power1_input")), 1e-6)
            if p is None:
                p = _num(_read(os.path.join(self.hwmon, "power1_average")), 1e-6)
            s["power_w"] = p
            for key, name in (("junction_c", "junction"), ("hbm_c", "mem")):
                if name in self.temps:
                    s[key] = _num(_read(self.temps[name]), 1e-3)
        return s


def parse_amdsmi_csv_line(header: list[str], line: str) -> dict | None:
    """One ``amd-smi monitor -p -t -u -m --csv`` data line as a sample."""
    row = next(csv.reader(io.StringIO(line)), None)
    if not row or len(row) != len(header):
        return None
    d = dict(zip(header, row))
    names = {"gfx_mhz": "gfx_clk", "mem_mhz": "mem_clock", "busy_pct": "gfx",
             "power_w": "power_usage", "junction_c": "hotspot_temperature",
             "hbm_c": "memory_temperature"}
    out = {k: _num(d.get(v)) for k, v in names.items()}
    return out if out["gfx_mhz"] is not None else None


def amdsmi_gfx_max_mhz(timeout_s: float = 20.0) -> float | None:
    """The top graphics clock from ``amd-smi metric -c --json`` (GPU 0)."""
    try:
        r = subprocess.run(["amd-smi", "metric", "-c", "--json"], capture_output=True,
                           text=True, timeout=timeout_s)
        data = json.loads(r.stdout)
        gpus = data.get("gpu_data", data) if isinstance(data, dict) else data
        clk = gpus[0]["clock"]
        return float(clk["gfx_0"]["max_clk"]["value"])
    except (OSError, ValueError, KeyError, IndexError, TypeError, subprocess.SubprocessError):
        return None


# --------------------------------------------------------------------------
# the sampler
# --------------------------------------------------------------------------

class ClockMonitor:
    """Background sampler.  ``window(t0, t1)`` summarises the samples taken
    while [t0, t1] (``time.time()`` stamps) was being measured."""

    def __init__(self, interval_s: float = 0.02, device_dir: str | None = None,
                 allow_amdsmi: bool = True):
        self.interval_s = interval_s
        self.device_dir = device_dir
        self.allow_amdsmi = allow_amdsmi
        self.samples: list[tuple[float, dict]] = []
        self.source = None
        self.gfx_max_mhz = None
        self.available = False
        self._stop = threading.Event()
        self._thread = None
        self._proc = None
        self._lock = threading.Lock()

    # -- life cycle --------------------------------------------------------
    def start(self, settle_s: float = 0.25) -> bool:
        dev = self.device_dir or find_device()
        if dev is not None:
            reader = SysfsReader(dev)
            if reader.sample()["gfx_mhz"] is not None:
                self.source, self.gfx_max_mhz = "sysfs", reader.gfx_max_mhz
                self._thread = threading.Thread(target=self._poll, args=(reader,), daemon=True)
        if self._thread is None and self.allow_amdsmi:
            self._start_amdsmi()
        if self._thread is None:
            return False
        self._thread.start()
        deadline = time.time() + max(settle_s, 5 * self.interval_s)
        while time.time() < deadline and not self.samples:
            time.sleep(self.interval_s)
        self.available = bool(self.samples)
        return self.available

    def _start_amdsmi(self):
        period = max(1, round(self.interval_s))
        try:
            self._proc = subprocess.Popen(
                ["amd-smi", "monitor", "-p", "-t", "-u", "-m", "--csv", "-w", str(period)],
                stdout=subprocess.PIPE, stderr=subprocess.DEVNULL, text=True, bufsize=1)
        except OSError:
            self._proc = None
            return
        self.source = "amd-smi"
        self.gfx_max_mhz = amdsmi_gfx_max_mhz()
        self._thread = threading.Thread(target=self._read_amdsmi, daemon=True)

    def stop(self):
        self._stop.set()
        if self._proc is not None:
            try:
                self._proc.terminate()
                self._proc.wait(timeout=5)
            except Exception:
                pass
        if self._thread is not None and self._thread.is_alive():
            self._thread.join(timeout=2)

    def __enter__(self):
        self.start()
        return self

    def __exit__(self, *exc):
        self.stop()

    # -- sampling threads --------------------------------------------------
    def _add(self, s: dict):
        with self._lock:
            self.samples.append((time.time(), s))

    def _poll(self, reader: SysfsReader):
        while not self._stop.is_set():
            self._add(reader.sample())
            self._stop.wait(self.interval_s)

    def _read_amdsmi(self):
        header = None
        for line in self._proc.stdout:
            if self._stop.is_set():
                break
            line = line.strip()
            if not line:
                continue
            if line.startswith("gpu,"):
                header = line.split(",")
                continue
            if header is not None:
                s = parse_amdsmi_csv_line(header, line)
                if s is not None:
                    self._add(s)

    # -- queries -------------------------------------------------------------
    def latest(self) -> dict | None:
        with self._lock:
            return self.samples[-1][1] if self.samples else None

    def window(self, t0: float, t1: float) -> dict | None:
        with self._lock:
            vals = [s for (t, s) in self.samples if t0 <= t <= t1]
        if not vals:
            return None
        return summarize(vals, self.gfx_max_mhz, self.source)


def summarize(vals: list[dict], gfx_max_mhz: float | None, source: str | None = None) -> dict:
    """Min/mean/max of every sampled quantity plus the stability gates."""
    out = {"n_samples": len(vals), "source": source}
    for k in KEYS:
        xs = [v[k] for v in vals if v.get(k) is not None]
        if xs:
            out[f"{k}_min"] = round(min(xs), 1)
            out[f"{k}_mean"] = round(statistics.fmean(xs), 1)
            out[f"{k}_max"] = round(max(xs), 1)
    gmin = out.get("gfx_mhz_min")
    out["gfx_max_level_mhz"] = gfx_max_mhz
    out["boosted"] = bool(gfx_max_mhz and gmin is not None
                          and gmin >= BOOST_FLOOR_FRAC * gfx_max_mhz)
    jmax = out.get("junction_c_max")
    out["thermal_headroom"] = jmax is None or jmax < JUNCTION_LIMIT_C
    out["enough_samples"] = len(vals) >= MIN_SAMPLES
    out["mem_clock_constant"] = out.get("mem_mhz_min") == out.get("mem_mhz_max")
    out["stable"] = bool(out["boosted"] and out["thermal_headroom"] and out["enough_samples"])
    return out


# --------------------------------------------------------------------------
# gates on the timings themselves
# --------------------------------------------------------------------------

def spread_frac(xs: list[float]) -> float | None:
    """IQR / median for 8 or more timings, (max - min) / median for fewer."""
    xs = sorted(float(x) for x in xs)
    if not xs:
        return None
    med = statistics.median(xs)
    if med <= 0:
        return None
    if len(xs) >= 8:
        q = statistics.quantiles(xs, n=4, method="inclusive")
        return (q[2] - q[0]) / med
    return (xs[-1] - xs[0]) / med


def timing_is_tight(xs: list[float]) -> bool:
    f = spread_frac(xs)
    return f is not None and f <= MAX_SPREAD_FRAC


def row_gate(clock_window: dict | None, timings: list[float]) -> dict:
    """The verdict for one measured row."""
    f = spread_frac(timings)
    tight = f is not None and f <= MAX_SPREAD_FRAC
    stable = bool(clock_window and clock_window.get("stable"))
    return {"spread_frac": None if f is None else round(f, 4), "tight": tight,
            "clocks_stable": stable if clock_window else None,
            "quotable": tight and (stable if clock_window else True)}


# --------------------------------------------------------------------------
# between-run comparison
# --------------------------------------------------------------------------

TIME_KEYS = ("value", "us_per_step", "split_kernel_us", "step_us", "kernel_us")


def _leaves(d, prefix=""):
    if isinstance(d, dict):
        for k, v in d.items():
            yield from _leaves(v, f"{prefix}.{k}" if prefix else str(k))
    elif isinstance(d, (int, float)) and not isinstance(d, bool):
        yield prefix, float(d)


def load_run(path: str) -> dict:
    """A bench JSON line from a file: the last line that parses as an object
    with a ``metric`` key (a driver record wrapping it under ``bench`` or
    ``result`` is unwrapped)."""
    with open(path) as f:
        text = f.read()
    cands = []
    try:
        cands.append(json.loads(text))
    except ValueError:
        for line in text.splitlines():
            line = line.strip()
            if line.startswith("{"):
                try:
                    cands.append(json.loads(line))
                except ValueError:
                    pass
    for obj in reversed(cands):
        if not isinstance(obj, dict):
            continue
        for key in (None, "bench", "result", "parsed"):
            o = obj if key is None else obj.get(key)
            if isinstance(o, dict) and "metric" in o:
                return o
    raise ValueError(f"{path}: no bench JSON line with a 'metric' key")


def compare_runs(runs: list[dict], names: list[str] | None = None,
                 threshold: float = MAX_SPREAD_FRAC) -> list[dict]:
    """One record per timing present in every run: the per-run values, the
    run-to-run spread ``max / min - 1``, and whether it exceeds ``threshold``.
    Timings are the leaves named in ``TIME_KEYS``; clock means of the rows
    that carry them ride along so a moved row can be read against its clock."""
    names = names or [f"run{i}" for i in range(len(runs))]
    flat = [dict(_leaves(r)) for r in runs]
    keys = set(flat[0])
    for f in flat[1:]:
        keys &= set(f)
    recs = []
    for k in sorted(keys):
        if k.rsplit(".", 1)[-1] not in TIME_KEYS or k.startswith("cpu_baseline"):
            continue
        xs = [f[k] for f in flat]
        lo, hi = min(xs), max(xs)
        spread = hi / lo - 1.0 if lo > 0 else float("inf")
        base = k.rsplit(".", 1)[0] if "." in k else ""
        gfx = [f.get(f"{base}.clocks.gfx_mhz_mean" if base else "clocks.gfx_mhz_mean")
               for f in flat]
        recs.append({"key": k, "values": dict(zip(names, xs)), "spread_frac": round(spread, 4),
                     "moved": spread > threshold,
                     "gfx_mhz_mean": dict(zip(names, gfx)) if any(g is not None for g in gfx)
                     else None})
    return recs
