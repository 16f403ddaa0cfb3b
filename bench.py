#!/usr/bin/env python
"""Decode-step benchmark of the MI355X fused quantized-KV attention.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]

Headline workload (``config.workload``): BASELINE.json config 4, the
Llama-3-8B attention shape -- B=32, HQ=32, HKV=8, D=128, ctx 32768, fp16 q,
K/V N(0,1) with 4 seeded x8 outlier channels per KV head, 4-bit group-size-32
split-P caches.  One step = one decode step over the whole batch (split kernel
+ combine).  Two independently seeded cache copies (1.34 GB each, together
more than 10x the 256 MB Infinity Cache) alternate step by step, so every step
streams its cache from HBM ("cold cache").  Inputs are resident in HBM before
the timed region starts.

Prints ONE JSON line.  ``value`` is microseconds per decode step (lower is
better), measured with HIP events on torch's current stream around the replay
of a HIP graph holding exactly K steps, after W untimed warmup steps.
``roofline`` relates the split kernel's algorithmic bytes (cache + q + out)
to its own average duration (a graph of split-kernel launches only) and
MI355X's 8 TB/s HBM peak.  ``cpu_baseline`` times the oracle's scalar C
restatement of the reference's CPU path on a bounded sample of the same step.
Unless ``--quick``, the line also carries the 2-bit and fp16-control numbers of
the same shape, the same 4-bit step over shuffled page pools (page sizes 32
and 256), and the Qwen2.5-1.5B table of BASELINE.json configs 2-3
(cache-resident and DRAM-resident, ctx 512..16384).

A background sampler reads the GPU's clocks, power and temperatures while the
Llama-shape legs run (``clocks``: per-leg windows and the quotable gate).
``python bench.py --compare A.json B.json ...`` compares complete runs row by
row instead of measuring.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "µs/decode step + achieved HBM GB/s (% peak), 4/2-bit vs fp16 control, cold cache"
HBM_PEAK_GBS = 8000.0
INFINITY_CACHE = 256 * 2 ** 20


def _args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=1000,
                    help="untimed steps (graph replays) right before the timed ones")
    ap.add_argument("--min-warmup-s", type=float, default=None,
                    help="seconds of warm-up replays at least (default: timing.MIN_WARMUP_S; "
                         "0 for counter runs, where every dispatch is serialised)")
    ap.add_argument("--quick", action="store_true",
                    help="headline workload only (no 2-bit / control / Qwen table / CPU baseline)")
    ap.add_argument("--num-splits", type=int, default=None)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--rocprof-summary", metavar="TRACE_DIR", default=None,
                    help="no GPU work: summarise a rocprofv3 --kernel-trace --stats "
                         "--output-format csv directory (plus --pmc-fetch/--pmc-write "
                         "counter directories) as the text kept under profiles/")
    ap.add_argument("--pmc-fetch", default=None)
    ap.add_argument("--pmc-write", default=None)
    ap.add_argument("--kernel", default=None,
                    help="full kernel name the summary and traffic figures are for (default: "
                         "the headline's split kernel instantiation)")
    ap.add_argument("--command", default="", help="command line recorded in the summary")
    ap.add_argument("--title", default="", help="first line of the summary (default: the headline)")
    ap.add_argument("--rows", type=int, default=8, help="kernels listed in the summary")
    ap.add_argument("--no-clocks", action="store_true",
                    help="do not sample clocks/power/temperature during the timed legs")
    ap.add_argument("--compare", nargs="+", metavar="RUN_JSON", default=None,
                    help="no timing: compare the bench JSON lines of complete runs row by row")
    ap.add_argument("--kernel-probe", choices=sorted(KERNEL_PROBES), default=None,
                    help="no timing: a few eager launches of one split kernel at its benchmark "
                         "shape, for rocprofv3 --pmc counter runs")
    ap.add_argument("--counter-summary", nargs="+", metavar="PMC_DIR", default=None,
                    help="no GPU work: per-kernel table of the SQ/GRBM counters of rocprofv3 "
                         "--pmc output directories (one per pass)")
    ap.add_argument("--skip-dispatches", type=int, default=0,
                    help="with --counter-summary: leave out the first N dispatches of each kernel")
    ap.add_argument("--regime-probe", choices=("hot", "cold"), default=None,
                    help="no timing: 60 eager Qwen2.5-1.5B ctx-16384 4-bit decode calls on one "
                         "cache (hot) or rotating copies >= 768 MB (cold), for rocprofv3 --pmc")
    ap.add_argument("--order-sweep", action="store_true",
                    help="the dispatch-order measurements: the 70B-style ragged batch's decode "
                         "and read probe at 1-16 splits in grid and longest-first order, and "
                         "the Llama-3-8B step with equal lengths passed as seq_lens")
    ap.add_argument("--qwen-trace", type=int, metavar="CTX", default=None,
                    help="no timing: 200 eager hot decode calls each of the fused 4-bit, fused "
                         "2-bit and fp16 control paths at the Qwen2.5-1.5B shape and context "
                         "CTX (default splits, combine launch included), for a rocprofv3 "
                         "kernel trace")
    return ap.parse_args()


# ---------------------------------------------------------------------------
# workload construction
# ---------------------------------------------------------------------------


def algorithmic_bytes(B, HQ, HKV, S, D, kbits, vbits, gs):
    """Cache bytes + q (fp16) + out (fp32) of one decode step."""
    from tritonkv_amd.quantize import cache_row_bytes

    cache = B * HKV * S * (cache_row_bytes(D, kbits, gs) + cache_row_bytes(D, vbits, gs))
    return cache, cache + B * HQ * D * (2 + 4)


def llama_inputs(seed, B=32, HQ=32, HKV=8, S=32768, D=128):
    """BASELINE.json config 4's inputs: fp16 N(0,1) q/K/V with 4 seeded x8
    outlier channels per KV head (``tritonkv_amd.synthetic``, the generator
    the full-size GPU parity tests check the kernels on)."""
    from tritonkv_amd import synthetic

    q, k, v, _ = synthetic.outlier_channel_kv(B, HQ, HKV, S, D, seed=seed)
    return q, k, v


# The split kernel's paired-tile form runs for GQA groups of at most 8 heads
# and splits of at least this many tokens (kPairedTilesMinSplit in
# tritonkv_amd/csrc/quant_split.h).
PAIRED_TILES_MIN_SPLIT = 8192


def split_kernel_name(D, kbits, vbits, gs, waves, G, split_size, paged=False, kch=False,
                      ordered=False, vsplit=1, small_grid=False):
    """The demangled name (as rocprofv3 prints it) of the quantized split
    kernel instantiation that a launch with these arguments runs (``vsplit``:
    2 or 4 for the dims-split kernels of small grids, ``small_grid`` for their
    layout on fewer than 8 tuples)."""
    pt = not kch and G <= 8 and split_size >= PAIRED_TILES_MIN_SPLIT
    hs = 16 if D // gs < 2 else 4 if G <= 4 else 8 if G <= 8 else 16  # head columns
    b = lambda x: "true" if x else "false"  # noqa: E731
    return (f"void tkv::quant_split_lds_kernel<{D}, {kbits}, {vbits}, {gs}, {waves}, 2, "
            f"{b(paged)}, {b(pt)}, {b(kch)}, {hs}, {b(ordered)}, {vsplit}, {b(small_grid)}>"
            "(tkv::SplitParams)")


# ---------------------------------------------------------------------------
# timing
# ---------------------------------------------------------------------------


_CLOCKS = None          # the running clocks.ClockMonitor, if any
_LAST_WINDOW = None     # (t0, t1): the last timed_steps' timed replays plus a lead-in
CLOCK_LEAD_IN_S = 0.1   # warm-up time before the timed replays that the clock window includes


def clock_record(timings, full=False):
    """Clock window of the last ``timed_steps`` call plus the row gate, or None
    without a sampler."""
    from tritonkv_amd import clocks

    if _CLOCKS is None or _LAST_WINDOW is None:
        return None
    win = _CLOCKS.window(*_LAST_WINDOW)
    gate = clocks.row_gate(win, timings)
    if win is None:
        return gate
    if not full:
        win = {k: win[k] for k in ("n_samples", "gfx_mhz_min", "gfx_mhz_mean", "power_w_mean",
                                   "junction_c_max", "stable") if k in win}
    return {**win, **gate}


_LAST_WARMUP = None      # (replays, seconds) of the last timed_steps' warm-up
MIN_WARMUP_S = None      # --min-warmup-s


def timed_steps(copies, steps, warmup, reps=3):
    """µs per step of ``steps`` rotating calls in one graph (``timing.timed_steps``:
    the mean over ``reps`` timed replays, after at least ``warmup`` steps and
    ``timing.MIN_WARMUP_S`` seconds of warm-up replays of the same graph), plus
    the wall-clock ms per step of the first timed replay and the per-replay
    figures.  Records the clock window and the warm-up of the call."""
    from tritonkv_amd import timing

    global _LAST_WINDOW, _LAST_WARMUP
    floor = timing.MIN_WARMUP_S if MIN_WARMUP_S is None else MIN_WARMUP_S
    t = timing.timed_steps(copies, steps, warmup, reps=reps, min_warmup_s=floor)
    _LAST_WINDOW = (t.timed_start - CLOCK_LEAD_IN_S, t.timed_end)
    _LAST_WARMUP = (t.warmup_replays, t.warmup_s)
    return t.us, t.wall_ms, t.per_replay_us


def per_call_us(calls, reps=5):
    from tritonkv_amd import timing

    return timing.per_call_us(calls, reps=reps)


def capture(calls):
    from tritonkv_amd import timing

    return timing.capture(calls)


# ---------------------------------------------------------------------------
# callables
# ---------------------------------------------------------------------------


def fused_call(q, kq, vq, num_splits=None, split_only=False, waves=None, fused_combine=False,
               probe=False):
    """One decode step as a callable (``probe``: the read-ceiling probe of the
    split kernel's access pattern instead, ``tkv_read_probe``)."""
    import torch

    from tritonkv_amd import _lib
    from tritonkv_amd.kernels.fused_decode_attn import _workspace_for, choose_waves, plan_splits

    B, HQ, D = q.shape
    _, HKV, S, _ = kq.packed.shape
    _, ns, size = plan_splits(S, 64, num_splits, B, HKV, HQ // HKV)
    out = torch.empty(B, HQ, D, device=q.device)
    acc, mx, sm, cnt = _workspace_for({}, B, HQ, ns, D, q.device, HKV)
    wv = choose_waves(B, HKV, HQ // HKV, size, ns, D=D, k_nbits=kq.nbits, v_nbits=vq.nbits,
                      group_size=kq.group_size) if waves is None else waves
    args = _lib.DecodeArgs(
        q=q.data_ptr(), k=kq.packed.data_ptr(), k_scale=kq.scale.data_ptr(),
        k_zero=kq.zero.data_ptr(), v=vq.packed.data_ptr(), v_scale=vq.scale.data_ptr(),
        v_zero=vq.zero.data_ptr(), acc=_lib.ptr(acc), maxs=_lib.ptr(mx), sums=_lib.ptr(sm),
        out=out.data_ptr(), B=B, HQ=HQ, HKV=HKV, S=S, D=D, k_nbits=kq.nbits, v_nbits=vq.nbits,
        group_size=kq.group_size, sm_scale=D ** -0.5, split_size=size, num_splits=ns,
        counters=_lib.ptr(cnt) if (fused_combine and not split_only) else None, waves=wv)
    lib = _lib.load()
    fn = lib.tkv_fused_decode_split if split_only else lib.tkv_fused_decode_attention
    if probe:
        fn = lib.tkv_read_probe

    def call():
        _lib.check(fn(args, torch.cuda.current_stream().cuda_stream), "fused")
    call.keep = (out, acc, mx, sm, cnt, q, kq, vq)
    call.num_splits = ns
    call.kernel = split_kernel_name(D, kq.nbits, vq.nbits, kq.group_size, wv, HQ // HKV, size)
    return call


def to_pool(qt, page_size, seed):
    """``qt`` scattered page by page into a pool in random page order, with
    the block table that maps it back: ``(pool, table)``."""
    import torch

    from tritonkv_amd.paged import empty_paged_pool

    B, H, S, _ = qt.packed.shape
    mp = S // page_size
    g = torch.Generator().manual_seed(seed)
    table = torch.randperm(B * mp, generator=g).reshape(B, mp).to(torch.int32).to(qt.device)
    pool = empty_paged_pool(B * mp, H, page_size, qt.head_dim, qt.nbits, qt.group_size, qt.device)
    for src, dst in ((qt.packed, pool.packed), (qt.scale, pool.scale), (qt.zero, pool.zero)):
        dst[table.long()] = src.reshape(B, H, mp, page_size, -1).permute(0, 2, 1, 3, 4)
    return pool, table


def paged_call(q, kp, vp, table, split_only=False):
    import torch

    from tritonkv_amd import _lib
    from tritonkv_amd.kernels.fused_decode_attn import _workspace_for, choose_waves, plan_splits

    B, HQ, D = q.shape
    num_pages, HKV, page, _ = kp.packed.shape
    S = table.shape[1] * page
    _, ns, size = plan_splits(S, 64, None, B, HKV, HQ // HKV)
    out = torch.empty(B, HQ, D, device=q.device)
    acc, mx, sm, _ = _workspace_for({}, B, HQ, ns, D, q.device, HKV)
    args = _lib.DecodeArgs(
        q=q.data_ptr(), k=kp.packed.data_ptr(), k_scale=kp.scale.data_ptr(),
        k_zero=kp.zero.data_ptr(), v=vp.packed.data_ptr(), v_scale=vp.scale.data_ptr(),
        v_zero=vp.zero.data_ptr(), acc=_lib.ptr(acc), maxs=_lib.ptr(mx), sums=_lib.ptr(sm),
        out=out.data_ptr(), B=B, HQ=HQ, HKV=HKV, S=S, D=D, k_nbits=kp.nbits, v_nbits=vp.nbits,
        group_size=kp.group_size, sm_scale=D ** -0.5, split_size=size, num_splits=ns,
        waves=choose_waves(B, HKV, HQ // HKV, size, ns, paged=True), block_table=table.data_ptr(),
        block_table_stride=table.shape[1], page_size=page, num_pages=num_pages)
    lib = _lib.load()
    fn = lib.tkv_fused_decode_split if split_only else lib.tkv_fused_decode_attention

    def call():
        _lib.check(fn(args, torch.cuda.current_stream().cuda_stream), "paged")
    call.keep = (out, acc, mx, sm, q, kp, vp, table)
    return call


def fp16_call(q, k, v, num_splits=None, split_only=False, waves=None, fused_combine=False):
    import torch

    from tritonkv_amd import _lib
    from tritonkv_amd.kernels.fused_decode_attn import (TOKENS_PER_WORKGROUP_FP16, _workspace_for,
                                                        choose_waves, plan_splits)

    B, HQ, D = q.shape
    _, HKV, S, _ = k.shape
    _, ns, size = plan_splits(S, 64, num_splits, B, HKV, HQ // HKV, TOKENS_PER_WORKGROUP_FP16)
    out = torch.empty(B, HQ, D, device=q.device)
    acc, mx, sm, cnt = _workspace_for({}, B, HQ, ns, D, q.device, HKV)
    wv = choose_waves(B, HKV, HQ // HKV, size, ns) if waves is None else waves
    args = _lib.DecodeArgs(
        q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), acc=_lib.ptr(acc), maxs=_lib.ptr(mx),
        sums=_lib.ptr(sm), out=out.data_ptr(), B=B, HQ=HQ, HKV=HKV, S=S, D=D, k_nbits=16,
        v_nbits=16, group_size=D, sm_scale=D ** -0.5, split_size=size, num_splits=ns,
        counters=_lib.ptr(cnt) if (fused_combine and not split_only) else None, waves=wv)
    lib = _lib.load()
    fn = lib.tkv_fp16_decode_split if split_only else lib.tkv_fp16_decode_attention

    def call():
        _lib.check(fn(args, torch.cuda.current_stream().cuda_stream), "fp16")
    call.keep = (out, acc, mx, sm, cnt, q, k, v)
    call.num_splits = ns
    return call


def torch_nosplit_call(q, k, v):
    """No-split fp16 baseline in plain torch: one batched GEMM for the scores
    (K pre-transposed once, outside the timed region, so the right operand is
    contiguous), an fp32 softmax, one batched GEMM for the output."""
    import torch

    B, HQ, D = q.shape
    _, HKV, S, _ = k.shape
    G = HQ // HKV
    kT = k.transpose(-1, -2).contiguous()  # (B, HKV, D, S)
    vc = v.contiguous()
    qg = q.view(B, HKV, G, D)
    scale = D ** -0.5

    def call():
        s = torch.matmul(qg, kT)  # (B, HKV, G, S)
        p = torch.softmax(s.float() * scale, dim=-1).half()
        return torch.matmul(p, vc).view(B, HQ, D)
    call.keep = (q, kT, vc)
    call.num_splits = 1
    return call


def copy_probe(nbytes=1 << 30, reps=5):
    """Device-to-device copy bandwidth (read + write bytes / time), median of reps.

    Also the calibration kernel for rocprofv3 FETCH_SIZE / WRITE_SIZE: it reads
    and writes exactly ``nbytes`` per dispatch.
    """
    import torch

    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    out = []
    for _ in range(reps):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        dst.copy_(src)
        e.record()
        torch.cuda.synchronize()
        out.append(2 * nbytes / (s.elapsed_time(e) * 1e-3) / 1e9)
    del src, dst
    return statistics.median(out)


# ---------------------------------------------------------------------------
# rocprofv3 summaries (text kept under profiles/) and the traffic figure
# ---------------------------------------------------------------------------

COPY_PROBE_BYTES = 1 << 30
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "quant_split_kernel_llama3_8b_4bit.txt")


def _csv_rows(directory, suffix):
    import csv
    import glob

    files = sorted(glob.glob(os.path.join(directory, f"*{suffix}")))
    if not files:
        raise FileNotFoundError(f"no *{suffix} under {directory}")
    with open(files[0], newline="") as fh:
        return list(csv.DictReader(fh))


def _short(name, width=96):
    return name if len(name) <= width else name[:width - 3] + "..."


def _counter_per_dispatch(directory, kernel):
    """(mean counter value of ``kernel``'s largest-grid dispatches, n, name,
    mean value of the 1 GiB copy-probe dispatches) from a --pmc directory."""
    rows = _csv_rows(directory, "counter_collection.csv")
    by = {}
    for r in rows:
        by.setdefault((r["Kernel_Name"], int(r["Grid_Size"])), []).append(float(r["Counter_Value"]))
    mine = [(g, n, v) for (n, g), v in by.items() if n == kernel]
    if not mine:
        raise ValueError(f"no dispatch of {kernel!r} in {directory}")
    g, name, vals = max(mine)
    copies = [v for (n, _), v in by.items() if "copyBuffer" in n]
    copy_kib = max(statistics.mean(v) for v in copies) if copies else None
    return statistics.mean(vals), len(vals), name, copy_kib


def rocprof_summary(a) -> int:
    if a.kernel is None:
        a.kernel = split_kernel_name(128, 4, 4, 32, 8, 4, 32768)
    out = []
    out.append(a.title or f"# rocprofv3 summary -- kernel {a.kernel}..., Llama-3-8B decode step "
               f"(B=32 HQ=32 HKV=8 D=128 ctx=32768, 4-bit gs32), bench.py --quick")
    if a.command:
        out.append(f"command: {a.command}")
    trace = _csv_rows(a.rocprof_summary, "kernel_trace.csv")
    stats = _csv_rows(a.rocprof_summary, "kernel_stats.csv")
    out.append("")
    out.append("## kernel stats (rocprofv3 --stats, all dispatches of the run)")
    out.append(f"{'calls':>6} {'avg_us':>10} {'min_us':>10} {'max_us':>10} {'pct':>6}  kernel")
    for r in sorted(stats, key=lambda r: -float(r["TotalDurationNs"]))[:a.rows]:
        out.append(f"{int(r['Calls']):>6} {float(r['AverageNs']) / 1e3:>10.2f} "
                   f"{float(r['MinNs']) / 1e3:>10.2f} {float(r['MaxNs']) / 1e3:>10.2f} "
                   f"{float(r['Percentage']):>6.2f}  {_short(r['Name'])}")
    out.append("")
    out.append("## per-dispatch durations by grid (kernel trace)")
    groups = {}
    for r in trace:
        grid = (int(r["Grid_Size_X"]), int(r["Grid_Size_Y"]), int(r["Grid_Size_Z"]))
        wg = int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) * int(r["Workgroup_Size_Z"])
        dur = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        groups.setdefault((r["Kernel_Name"], grid, wg), []).append(dur)
    out.append(f"{'calls':>6} {'avg_us':>10} {'median_us':>10} {'grid':>18} {'wg':>5}  kernel")
    for (name, grid, wg), d in sorted(groups.items(), key=lambda kv: -sum(kv[1]))[:a.rows + 2]:
        out.append(f"{len(d):>6} {statistics.mean(d):>10.2f} {statistics.median(d):>10.2f} "
                   f"{'x'.join(map(str, grid)):>18} {wg:>5}  {_short(name)}")
    if a.pmc_fetch and a.pmc_write:
        f_kib, nf, name, f_copy = _counter_per_dispatch(a.pmc_fetch, a.kernel)
        w_kib, nw, _, w_copy = _counter_per_dispatch(a.pmc_write, a.kernel)
        copy_kib = COPY_PROBE_BYTES / 1024
        ff = copy_kib / f_copy if f_copy else 1.0
        fw = copy_kib / w_copy if w_copy else 1.0
        traffic = int(round((f_kib * ff + w_kib * fw) * 1024))
        out.append("")
        out.append("## HBM traffic (rocprofv3 --pmc FETCH_SIZE, then --pmc WRITE_SIZE; KiB/dispatch)")
        out.append(f"kernel: {name}")
        out.append(f"FETCH_SIZE  {f_kib:14.1f} KiB over {nf} dispatches; copy probe "
                   f"({COPY_PROBE_BYTES} B read+write) reads {f_copy:.1f} KiB -> factor {ff:.4f}")
        out.append(f"WRITE_SIZE  {w_kib:14.1f} KiB over {nw} dispatches; copy probe "
                   f"writes {w_copy:.1f} KiB -> factor {fw:.4f}")
        out.append(f"traffic_bytes_per_launch: {traffic}")
    print("\n".join(out))
    return 0


def measured_traffic(kernel_name):
    """HBM bytes per launch from the committed --pmc summary, if it was taken
    of the same kernel instantiation; else None."""
    try:
        with open(TRAFFIC_PROFILE) as fh:
            text = fh.read()
    except OSError:
        return None
    kern = [ln.split(":", 1)[1].strip() for ln in text.splitlines() if ln.startswith("kernel: ")]
    vals = [ln.split(":", 1)[1].strip() for ln in text.splitlines()
            if ln.startswith("traffic_bytes_per_launch:")]
    if not kern or not vals or kern[-1] != kernel_name:
        return None
    return int(vals[-1])


# ---------------------------------------------------------------------------
# CPU baseline: the oracle's scalar C restatement on a bounded sample
# ---------------------------------------------------------------------------


def cpu_baseline(q, kq, vq, got, threads=None, one_thread_units=16):
    """The oracle's scalar C restatement (``oracle/tkv_oracle.c``: dequantise K
    and V to fp32, then fp32 attention) timed over the whole decode step on the
    host's cores, one (batch row, kv head) unit per task (ctypes releases the
    GIL for the C call), plus a one-thread figure on a few units.

    Doubles as the benchmark's correctness snapshot: every unit's oracle
    output is compared with ``got``, the GPU output of the timed step on the
    same cache, against the 2e-3 max-abs / 1e-3 mean-abs tolerance."""
    import concurrent.futures as cf

    import numpy as np

    from oracle import c_oracle

    B, HQ, D = q.shape
    _, HKV, S, _ = kq.packed.shape
    G = HQ // HKV
    host = [t.cpu().numpy() for t in (kq.packed, kq.scale, kq.zero, vq.packed, vq.scale, vq.zero)]
    qf = q.float().cpu().numpy()
    units = [(b, h) for b in range(B) for h in range(HKV)]

    def run(u):
        b, h = u
        sub = [a[b:b + 1, h:h + 1] for a in host]
        return c_oracle.quantized_decode_attention(
            qf[b:b + 1, h * G:(h + 1) * G], (sub[0], sub[1], sub[2], kq.nbits, kq.group_size),
            (sub[3], sub[4], sub[5], vq.nbits, vq.group_size), D ** -0.5)

    run(units[0])  # load the library, touch the pages
    n = threads or min(16, len(os.sched_getaffinity(0)))
    t0 = time.perf_counter()
    with cf.ThreadPoolExecutor(max_workers=n) as ex:
        refs = list(ex.map(run, units))
    t_all = time.perf_counter() - t0
    t0 = time.perf_counter()
    for u in units[:one_thread_units]:
        run(u)
    t_one = (time.perf_counter() - t0) / one_thread_units
    max_abs, sum_abs, count, worst = 0.0, 0.0, 0, None
    for (b, h), ref in zip(units, refs):
        d = np.abs(got[b, h * G:(h + 1) * G].astype(np.float64) - ref[0])
        if d.max() > max_abs:
            max_abs, worst = float(d.max()), [b, h]
        sum_abs += float(d.sum())
        count += d.size
    check = {"units": len(units), "max_abs_err": max_abs, "mean_abs_err": sum_abs / count,
             "worst_unit": worst, "tolerance": {"max_abs": 2e-3, "mean_abs": 1e-3},
             "ok": bool(max_abs <= 2e-3 and sum_abs / count <= 1e-3),
             "reference": "oracle/tkv_oracle.c fp32 dequantise-then-attend on the timed cache"}
    try:
        cpu = next(ln.split(":", 1)[1].strip() for ln in open("/proc/cpuinfo")
                   if ln.startswith("model name"))
    except (OSError, StopIteration):
        cpu = "unknown"
    base = {"value": round(t_all * 1e6, 1), "unit": "us/decode step", "cores": n, "kind": "port",
            "sample": (f"the whole decode step: all {len(units)} (batch row, kv head) units, "
                       f"oracle/tkv_oracle.c (scalar C: dequantize K,V to fp32 + fp32 attention), "
                       f"one unit per task on {n} threads ({t_all:.2f} s)"),
            "one_thread_us_per_step": round(t_one * len(units) * 1e6, 1),
            "one_thread_sample": f"{one_thread_units} units on 1 thread, x{len(units) / one_thread_units:.0f}",
            "cpu": cpu}
    return base, check


# ---------------------------------------------------------------------------
# correctness snapshot: the checker of every timed leg (oracle/, outside every
# timed region, as the reference re-checks what it times: benchmark.py:1050-1110)
# ---------------------------------------------------------------------------

CHECK_TOL = {"max_abs": 2e-3, "mean_abs": 1e-3}


def _host_rows(t, b, h, L=None):
    x = t[b, h] if L is None else t[b, h, :L]
    return x.contiguous().cpu().numpy()


def _qnp(qt, b, h, L=None):
    """One (batch row, kv head) block of a device QuantizedTensor as the oracle's container."""
    from oracle import quant as oq

    return oq.QuantNP(_host_rows(qt.packed, b, h, L), _host_rows(qt.scale, b, h, L),
                      _host_rows(qt.zero, b, h, L), qt.nbits, qt.group_size, qt.head_dim)


def _attend(qrows, krows, vrows):
    """fp32 attention of G query rows over one block's fp32 K/V rows
    (oracle/tkv_oracle.c, sums in binary64)."""
    from oracle import c_oracle

    D = qrows.shape[-1]
    return c_oracle.decode_attention(qrows[None], krows[None, None], vrows[None, None],
                                     D ** -0.5)[0]


def unit_refs(q, kq, vq, units, lens=None, fp16_dequant=False):
    """The oracle's fp32 dequantise-then-attend of (batch row, kv head) units of
    device caches (K and V may differ in bit width), or with ``fp16_dequant``
    the reference's fp16 dequant baseline (``reference.py:96-108``) then fp32
    attention.  -> {unit: (G, D) float32}"""
    import numpy as np

    from oracle import quant as oq

    B, HQ, D = q.shape
    G = HQ // kq.packed.shape[1]
    qf = q.float().cpu().numpy()
    out = {}
    for b, h in units:
        L = None if lens is None else int(lens[b])
        kn, vn = _qnp(kq, b, h, L), _qnp(vq, b, h, L)
        if fp16_dequant:
            kd = oq.dequantize_fp16(kn).astype(np.float32)
            vd = oq.dequantize_fp16(vn).astype(np.float32)
        else:
            kd, vd = oq.dequantize_groupwise(kn), oq.dequantize_groupwise(vn)
        out[(b, h)] = _attend(qf[b, h * G:(h + 1) * G], kd, vd)
    return out


def truth_refs(q, k, v, units, lens=None):
    """fp32 attention over the unquantized fp16 K/V: the end-to-end "truth" of
    the reference's snapshot (``benchmark.py:1058-1062``)."""
    B, HQ, D = q.shape
    G = HQ // k.shape[1]
    qf = q.float().cpu().numpy()
    out = {}
    for b, h in units:
        L = None if lens is None else int(lens[b])
        out[(b, h)] = _attend(qf[b, h * G:(h + 1) * G], _host_rows(k, b, h, L).astype("float32"),
                              _host_rows(v, b, h, L).astype("float32"))
    return out


def unit_check(got, refs, G, what):
    """Max-abs and mean-abs of the GPU output rows of each unit against the
    oracle's, over all the units, and whether they meet the tolerance."""
    import numpy as np

    max_abs, sum_abs, count, worst = 0.0, 0.0, 0, None
    for (b, h), ref in refs.items():
        d = np.abs(got[b, h * G:(h + 1) * G].astype(np.float64) - ref)
        if float(d.max()) >= max_abs:
            max_abs, worst = float(d.max()), [b, h]
        sum_abs += float(d.sum())
        count += d.size
    mean = sum_abs / max(count, 1)
    return {"units": len(refs), "max_abs_err": max_abs, "mean_abs_err": mean, "worst_unit": worst,
            "ok": bool(max_abs <= CHECK_TOL["max_abs"] and mean <= CHECK_TOL["mean_abs"]),
            "reference": what}


def rel_l2_units(got, refs, G):
    """Relative L2 error of the GPU rows of the units against ``refs`` (one
    norm over all of them)."""
    import numpy as np

    num = den = 0.0
    for (b, h), ref in refs.items():
        g = got[b, h * G:(h + 1) * G].astype(np.float64)
        num += float(((g - ref) ** 2).sum())
        den += float((ref.astype(np.float64) ** 2).sum())
    return (num / max(den, 1e-300)) ** 0.5


# the sampled (batch row, kv head) units of the Llama-3-8B-shape legs
LLAMA_UNITS = [(b, (5 * b) % 8) for b in range(0, 32, 4)]


def llama_leg_check(got, q, kq, vq, truth):
    """Check of one Llama-3-8B-shape leg on its first cache copy: the sampled
    units against the oracle, plus the end-to-end rel-L2 against fp32
    attention over the unquantized K/V next to the fp16 dequant baseline's
    (``truth``: the units' reference rows)."""
    G = q.shape[1] // kq.packed.shape[1]
    chk = unit_check(got, unit_refs(q, kq, vq, LLAMA_UNITS), G,
                     "oracle fp32 dequantise-then-attend, sampled units")
    chk["kernel_rel_l2_vs_fp16_truth"] = round(rel_l2_units(got, truth, G), 5)
    chk["fp16_baseline_rel_l2_vs_fp16_truth"] = round(rel_l2_units(
        _stack(unit_refs(q, kq, vq, LLAMA_UNITS, fp16_dequant=True), q.shape), truth, G), 5)
    return chk


def _stack(refs, shape):
    """Unit rows back into a (B, HQ, D) array (zeros elsewhere)."""
    import numpy as np

    B, HQ, D = shape
    out = np.zeros((B, HQ, D), np.float32)
    for (b, h), r in refs.items():
        g = r.shape[0]
        out[b, h * g:(h + 1) * g] = r
    return out


def qwen_snapshot(ctxs=(512, 2048, 8192, 16384), seeds=(0, 1, 2)):
    """The reference's correctness snapshot (``benchmark.py:1050-1110``) on the
    Qwen2.5-1.5B shape: per (ctx, nbits) and seeds 0-2, the reference's own
    inputs (``make_random_kv``: N(0,1) with 1% x8 outliers), quantized on the
    GPU and decoded with the default plan the table times; kernel against the
    fp32 dequantise-then-attend oracle (max/mean abs, rel-L2, cosine), and
    end-to-end rel-L2 against fp32 attention over the fp16 K/V, for the kernel
    and for the fp16 dequant baseline.  The fp16 control is checked against the
    same truth.  ``published`` holds the reference's table
    (``README.md:286-295``): rel-L2 vs fp16 truth, kernel / baseline."""
    import numpy as np
    import torch

    from oracle import attention as oatt
    from oracle import inputs as oinp
    from tritonkv_amd.kernels import fp16_decode_attention, fused_decode_attention
    from tritonkv_amd.quantize import quantize_kv

    published = {(512, 4): (0.1207, 0.1208), (2048, 4): (0.1396, 0.1397),
                 (8192, 4): (0.1251, 0.1249), (16384, 4): (0.1509, 0.1514),
                 (512, 2): (0.6558, 0.6560), (2048, 2): (0.8110, 0.8105),
                 (8192, 2): (0.6589, 0.6585), (16384, 2): (0.7560, 0.7557)}
    B, HQ, HKV, D = 1, 12, 2, 128
    units = [(0, 0), (0, 1)]
    rows, ctrl = [], []
    for S in ctxs:
        ctrl_max = 0.0
        for nbits in (4, 2):
            per = []
            for seed in seeds:
                q, k, v = oinp.make_random_kv(B, HQ, HKV, S, D, seed=seed)
                qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
                kq, vq = quantize_kv(kd, vd, nbits, 32)
                got = fused_decode_attention(qd, kq, vq).cpu().numpy()
                ref = _stack(unit_refs(qd, kq, vq, units), q.shape)
                base = _stack(unit_refs(qd, kq, vq, units, fp16_dequant=True), q.shape)
                truth = _stack(truth_refs(qd, kd, vd, units), q.shape)
                m = oatt.metrics(got, ref)
                per.append({"seed": seed, "max_abs_err": m["max_abs_err"],
                            "mean_abs_err": m["mean_abs_err"], "rel_l2": m["rel_l2"],
                            "cosine": m["cosine"],
                            "kernel_rel_l2_vs_fp16_truth": oatt.metrics(got, truth)["rel_l2"],
                            "baseline_rel_l2_vs_fp16_truth": oatt.metrics(base, truth)["rel_l2"]})
                if nbits == 4:  # the control on the same inputs, once per seed
                    gc = fp16_decode_attention(qd, kd, vd).cpu().numpy()
                    ctrl_max = max(ctrl_max, oatt.metrics(gc, truth)["max_abs_err"])
                del qd, kd, vd, kq, vq
            mean = lambda key: float(np.mean([p[key] for p in per]))
            pub = published.get((S, nbits))
            rows.append({
                "ctx": S, "nbits": nbits, "seeds": per,
                "max_abs_err": max(p["max_abs_err"] for p in per),
                "mean_abs_err": max(p["mean_abs_err"] for p in per),
                "min_cosine": min(p["cosine"] for p in per),
                "mean_kernel_rel_l2_vs_fp16_truth": round(mean("kernel_rel_l2_vs_fp16_truth"), 5),
                "mean_baseline_rel_l2_vs_fp16_truth": round(mean("baseline_rel_l2_vs_fp16_truth"), 5),
                "published_kernel_baseline_rel_l2": pub,
                "ok": bool(max(p["max_abs_err"] for p in per) <= CHECK_TOL["max_abs"]
                           and max(p["mean_abs_err"] for p in per) <= CHECK_TOL["mean_abs"])})
            print(f"# qwen snapshot ctx={S} {nbits}-bit: max abs {rows[-1]['max_abs_err']:.2e}, "
                  f"rel-L2 vs fp16 truth {rows[-1]['mean_kernel_rel_l2_vs_fp16_truth']} "
                  f"(published {pub})", file=sys.stderr, flush=True)
        ctrl.append({"ctx": S, "max_abs_err_vs_fp32_attention": ctrl_max,
                     "ok": bool(ctrl_max <= CHECK_TOL["max_abs"])})
        torch.cuda.empty_cache()
    return {"fused": rows, "fp16_control": ctrl,
            "inputs": "oracle.inputs.make_random_kv (the reference's generator: N(0,1), "
                      "1% of values x8), seeds 0-2; units: both kv heads"}


def cpu_config1(reps=50):
    """the reference's CPU decode step at the Qwen shape,
    ctx 512 -- dequantise K, V (4-bit gs32) to fp32, then fp32 attention -- as
    restated by the oracle (numpy dequantise, torch CPU attention), timed on
    this host with all its cores and with one thread; median of ``reps``."""
    import numpy as np
    import torch

    from oracle import inputs as oinp
    from oracle import quant as oq

    q, k, v = oinp.make_random_kv(1, 12, 2, 512, 128, seed=0, outlier_frac=0.0)
    kq, vq = oq.quantize_kv(k.numpy(), v.numpy(), 4, 32)
    qf = torch.from_numpy(q.float().numpy())

    def step():
        kd = torch.from_numpy(oq.dequantize_groupwise(kq))
        vd = torch.from_numpy(oq.dequantize_groupwise(vq))
        kd = kd.repeat_interleave(6, dim=1)
        vd = vd.repeat_interleave(6, dim=1)
        s_ = torch.einsum("bhd,bhsd->bhs", qf, kd) * (128 ** -0.5)
        return torch.einsum("bhs,bhsd->bhd", torch.softmax(s_, dim=-1), vd)

    out = {}
    threads0 = torch.get_num_threads()
    ncores = len(os.sched_getaffinity(0))
    for name, nt in (("all_cores", ncores), ("one_thread", 1)):
        torch.set_num_threads(nt)
        for _ in range(5):
            step()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter_ns()
            step()
            ts.append((time.perf_counter_ns() - t0) / 1e3)
        ts.sort()
        out[name] = {"us_median": round(statistics.median(ts), 1),
                     "us_iqr": round(ts[3 * len(ts) // 4] - ts[len(ts) // 4], 1), "threads": nt}
    torch.set_num_threads(threads0)
    try:
        cpu = next(ln.split(":", 1)[1].strip() for ln in open("/proc/cpuinfo") if ln.startswith("model name"))
    except (OSError, StopIteration):
        cpu = "unknown"
    out["cpu"] = cpu
    out["sample"] = ("Qwen2.5-1.5B attention, B=1 HQ=12 HKV=2 D=128 ctx=512, N(0,1) fp16 q/K/V seed 0, "
                     "4-bit gs32 split-P; numpy dequantise + torch CPU fp32 attention")
    return out


# ---------------------------------------------------------------------------
# 70B-style ragged batch
# ---------------------------------------------------------------------------


def ragged_70b(steps, warmup, seed=2024, check=False):
    """B=64, HQ=64, HKV=8, D=128; per-sequence length S_b ~ U[1024, 131072]
    (seeded); K 4-bit / V 2-bit, group 32; inputs from
    ``tritonkv_amd.synthetic.ragged_batch`` (the full-size GPU parity test's).
    One step appends one new token per sequence (GPU quantize + pack of K and
    V at position S_b) and then decodes over S_b + 1 tokens.  Storage is padded
    to 131072 + 64 tokens; only the sum of S_b + 1 counts as cache bytes."""
    import torch

    from tritonkv_amd import synthetic
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.quantize import append_kv, cache_row_bytes

    B, HQ, HKV, D, gs, cap = 64, 64, 8, 128, 32, 131072 + 64
    lens = synthetic.ragged_lengths(B, 1024, 131072, seed=seed)
    q, kc, vc, k_new, v_new = synthetic.ragged_batch(B, HQ, HKV, D, lens, cap, 4, 2, gs, seed=seed)
    pos = lens.to("cuda")
    lens1 = (lens + 1).to("cuda")
    out = torch.empty(B, HQ, D, device="cuda")
    ws = {}

    def decode():
        fused_decode_attention(q, kc, vc, seq_lens=lens1, allow_mixed_bits=True, out=out, _workspace=ws)

    def step():
        append_kv(kc, k_new, pos)
        append_kv(vc, v_new, pos)
        decode()

    def fused_step():  # the append inside the split kernel: one launch
        fused_decode_attention(q, kc, vc, seq_lens=lens1, allow_mixed_bits=True, out=out,
                               _workspace=ws, k_new=k_new, v_new=v_new)

    def decode_natural():  # split workgroups in grid order, no longest-first order
        fused_decode_attention(q, kc, vc, seq_lens=lens1, allow_mixed_bits=True, out=out,
                               _workspace=ws, dispatch_order=False)

    torch.cuda.synchronize()
    row = cache_row_bytes(D, 4, gs) + cache_row_bytes(D, 2, gs)
    tokens = int(lens1.sum())
    decode_bytes = tokens * HKV * row + B * HQ * D * (2 + 4)
    append_bytes = B * HKV * (2 * D * 2 + row)
    us, _, _ = timed_steps([step], steps, warmup)
    dus, _, _ = timed_steps([decode], steps, warmup)
    fus, _, _ = timed_steps([fused_step], steps, warmup)
    nus, _, _ = timed_steps([decode_natural], steps, warmup)
    total = decode_bytes + append_bytes
    if check:  # out: the last timed call's decode over S_b + 1 tokens
        lh = lens1.cpu()
        rows = sorted({int(lh.argmax()), int(lh.argmin()), 0, 17, 33, 50})
        units = [(b, b % HKV) for b in rows]
        chk = unit_check(out.cpu().numpy(), unit_refs(q, kc, vc, units, lens=lh), HQ // HKV,
                         "oracle fp32 dequantise-then-attend (K 4-bit, V 2-bit), rows of "
                         "the longest and shortest sequences among the sampled units")
        chk["row_lengths"] = [int(lh[b]) for b in rows]
    res = {"us_per_step": round(us, 2), "decode_us": round(dus, 2),
           "append_us": round(us - dus, 2), "fused_append_step_us": round(fus, 2),
           "decode_us_natural_order": round(nus, 2),
           "sum_tokens": tokens,
           "algorithmic_bytes": total,
           "gbps_step": round(total / us / 1e3, 1),
           "frac_of_hbm_peak_step": round(total / us / 1e3 / HBM_PEAK_GBS, 4),
           "frac_of_hbm_peak_decode": round(decode_bytes / dus / 1e3 / HBM_PEAK_GBS, 4),
           "lengths": "S_b ~ U[1024, 131072], torch.Generator().manual_seed(%d)" % seed}
    if check:
        res["check"] = chk
    print(f"# ragged 70b K4/V2: step {us:.1f} us (decode {dus:.1f} us, natural order "
          f"{nus:.1f} us, fused append+decode {fus:.1f} us), {total / us / 1e3:.0f} GB/s",
          file=sys.stderr, flush=True)
    del kc, vc, ws
    torch.cuda.empty_cache()
    return res


def channel_unit_check(out, q, ck, vq, kr, vr, S, window, units=((0, 0), (9, 3), (21, 5), (31, 7))):
    """The per-channel step's output on sampled units against the oracle
    (``oracle/channel.py``: per-channel keys and per-token values dequantized,
    then the fp16 window, fp32 attention)."""
    from oracle import channel as och

    G = q.shape[1] // ck.packed.shape[1]
    qf = q.float().cpu().numpy()
    refs = {}
    for b, h in units:
        ckn = och.ChannelKeysNP(_host_rows(ck.packed, b, h)[None, None],
                                _host_rows(ck.scale, b, h)[None, None],
                                _host_rows(ck.zero, b, h)[None, None], ck.nbits, 32, ck.head_dim)
        vqn = _qnp(vq, b, h)
        vqn.packed, vqn.scale, vqn.zero = vqn.packed[None, None], vqn.scale[None, None], \
            vqn.zero[None, None]
        kk, vv, _ = och.history(ckn, vqn, _host_rows(kr, b, h)[None, None],
                                _host_rows(vr, b, h)[None, None], [S], [window])
        refs[(b, h)] = _attend(qf[b, h * G:(h + 1) * G], kk[0, 0], vv[0, 0])
    return unit_check(out.cpu().numpy(), refs, G, "oracle per-channel keys + per-token values "
                      "+ fp16 window, fp32 attention, sampled units")


def channel_keys(steps, warmup, B=32, HQ=32, HKV=8, S=32768, D=128, window=16,
                 check=False):
    """Per-channel (KIVI-style) keys at the Llama-3-8B shape: keys quantized per
    (32-token block, channel), values per token (group 32), a 16-token fp16
    window; one step = split kernel (per-channel key path) + fp16 window split
    + combine.  Accuracy on the same synthetic keys (4 x8 outlier channels per
    KV head): relative L2 error of dequantized keys and of the attention output
    of batch rows 0-3 against fp32 attention over the original fp16 K/V, for
    per-token and per-channel keys (values per token either way)."""
    import torch

    from tritonkv_amd.channel import channel_decode_attention, quantize_keys_per_channel
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.quantize import (dequantize_groupwise, quantize_groupwise, unpack_codes)

    res = {}
    for nb in (2, 4):
        calls, first = [], None
        for c in range(2):
            q, k, v = llama_inputs(seed=10 + c, B=B, HQ=HQ, HKV=HKV, S=S, D=D)
            g = torch.Generator(device="cuda").manual_seed(50 + c)
            kr = torch.randn(B, HKV, 32, D, device="cuda", generator=g, dtype=torch.float16)
            vr = torch.randn(B, HKV, 32, D, device="cuda", generator=g, dtype=torch.float16)
            ck = quantize_keys_per_channel(k, nb)
            vq = quantize_groupwise(v, nb, 32)
            ql = torch.full((B,), S, dtype=torch.int32, device="cuda")
            rl = torch.full((B,), window, dtype=torch.int32, device="cuda")
            out = torch.empty(B, HQ, D, device="cuda")
            ws = {}

            def step(q=q, ck=ck, vq=vq, kr=kr, vr=vr, ql=ql, rl=rl, out=out, ws=ws):
                channel_decode_attention(q, ck, vq, kr, vr, q_lens=ql, res_lens=rl, out=out,
                                         _workspace=ws, equal_lengths=True)
            step()
            calls.append(step)
            if c == 0:
                first = (q, k, v, ck, vq, kr, vr, out)
            else:
                del k, v
        us, _, _ = timed_steps(calls, steps, warmup)
        krow = D * nb // 8 + 4 * D // 32
        vrow = D * nb // 8 + 4 * (D // 32)
        nbytes = B * HKV * (S * (krow + vrow) + window * 2 * D * 2) + B * HQ * D * (2 + 4)
        entry = {"us_per_step": round(us, 2), "algorithmic_bytes": nbytes,
                 "gbps_step": round(nbytes / us / 1e3, 1),
                 "frac_of_hbm_peak_step": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
        # accuracy, batch rows 0-3
        q, k, v, ck, vq, kr, vr, out0 = first
        if check:
            entry["check"] = channel_unit_check(out0, q, ck, vq, kr, vr, S, window)
        r = slice(0, 4)
        kf, vf = k[r].float(), v[r].float()
        codes = unpack_codes(ck.packed[r], nb, D).float()
        kd_ch = codes * ck.scale[r].float().repeat_interleave(32, dim=2) + \
            ck.zero[r].float().repeat_interleave(32, dim=2)
        kq_tok = quantize_groupwise(k[r].contiguous(), nb, 32)
        kd_tok = dequantize_groupwise(kq_tok)
        rel = lambda a, b: float((a - b).norm() / b.norm())
        entry["key_rel_l2_per_token"] = round(rel(kd_tok, kf), 4)
        entry["key_rel_l2_per_channel"] = round(rel(kd_ch, kf), 4)

        def truth(qr):
            G = HQ // HKV
            qg = qr.float().reshape(4, HKV, G, D)
            sc = torch.matmul(qg, kf.transpose(-1, -2)) / math.sqrt(D)
            return torch.matmul(torch.softmax(sc, dim=-1), vf).reshape(4, HQ, D)

        ref = truth(q[r])
        vq4 = type(vq)(vq.packed[r].contiguous(), vq.scale[r].contiguous(),
                       vq.zero[r].contiguous(), vq.nbits, vq.group_size, D)
        ck4 = type(ck)(ck.packed[r].contiguous(), ck.scale[r].contiguous(),
                       ck.zero[r].contiguous(), ck.nbits, D)
        kr0 = torch.zeros(4, HKV, 32, D, device="cuda", dtype=torch.float16)
        got_ch = channel_decode_attention(q[r].contiguous(), ck4, vq4, kr0, kr0.clone(),
                                          res_lens=torch.zeros(4, dtype=torch.int32, device="cuda"))
        got_tok = fused_decode_attention(q[r].contiguous(), kq_tok, vq4)
        entry["attn_rel_l2_per_token_keys"] = round(rel(got_tok, ref), 4)
        entry["attn_rel_l2_per_channel_keys"] = round(rel(got_ch, ref), 4)
        res[f"k{nb}v{nb}"] = entry
        print(f"# llama per-channel keys {nb}-bit: step {us:.2f} us; key rel-L2 per-token "
              f"{entry['key_rel_l2_per_token']} vs per-channel {entry['key_rel_l2_per_channel']}; "
              f"attention rel-L2 {entry['attn_rel_l2_per_token_keys']} vs "
              f"{entry['attn_rel_l2_per_channel_keys']}", file=sys.stderr, flush=True)
        del calls, first, q, k, v, ck, vq, kf, vf, codes, kd_ch, kd_tok, kq_tok
        torch.cuda.empty_cache()
    return res


# ---------------------------------------------------------------------------
# Qwen2.5-1.5B table (BASELINE.json configs 2 and 3)
# ---------------------------------------------------------------------------


def qwen_table(ctxs=(512, 2048, 8192, 16384), check=False):
    """The Qwen2.5-1.5B batch-1 table (configs 2 and 3): hot and cold µs per
    call of each method at each context; with ``check``, each row also
    carries the check of its first cache copy's output (both kv heads):
    against the oracle's fp32 dequantise-then-attend (fused), or fp32
    attention over the fp16 K/V (fp16 control, torch)."""
    import torch

    from tritonkv_amd.quantize import QuantizedTensor, quantize_groupwise
    from tritonkv_amd.timing import per_call, replicas_for

    B, HQ, HKV, D, gs = 1, 12, 2, 128, 32
    rows = []
    for S in ctxs:
        g = torch.Generator(device="cuda").manual_seed(1000 + S)
        q = torch.randn(B, HQ, D, device="cuda", generator=g, dtype=torch.float16)
        ns_fused4 = None
        for method in ("fused4", "fused2", "fp16", "fp16_fused_split", "fp16_nosplit",
                       "torch_fp16"):
            nbits = {"fused4": 4, "fused2": 2}.get(method, 16)
            cache, step_bytes = algorithmic_bytes(B, HQ, HKV, S, D, nbits, nbits, gs)
            R = replicas_for(cache)
            kv = torch.randn(2, R, B, HKV, S, D, device="cuda", generator=g, dtype=torch.float16)
            calls = []
            if method == "fp16":
                for i in range(R):
                    calls.append(fp16_call(q, kv[0, i], kv[1, i]))
            elif method == "fp16_fused_split":  # the fused 4-bit kernel's split count
                for i in range(R):
                    calls.append(fp16_call(q, kv[0, i], kv[1, i], num_splits=ns_fused4))
            elif method == "fp16_nosplit":
                for i in range(R):
                    calls.append(fp16_call(q, kv[0, i], kv[1, i], num_splits=1))
            elif method == "torch_fp16":
                for i in range(R):
                    calls.append(torch_nosplit_call(q, kv[0, i], kv[1, i]))
            else:
                kq = quantize_groupwise(kv[0], nbits, gs)
                vq = quantize_groupwise(kv[1], nbits, gs)
                del kv
                for i in range(R):
                    ki = QuantizedTensor(kq.packed[i], kq.scale[i], kq.zero[i], nbits, gs, D)
                    vi = QuantizedTensor(vq.packed[i], vq.scale[i], vq.zero[i], nbits, gs, D)
                    calls.append(fused_call(q, ki, vi))
            if method == "fused4":
                ns_fused4 = calls[0].num_splits
            hot_t = per_call([calls[0]] * 50)
            cold_t = per_call(calls)
            hot, cold = hot_t.us, cold_t.us
            rows.append({"ctx": S, "method": method, "cache_bytes": cache, "replicas": R,
                         "splits": calls[0].num_splits,
                         "hot_us": round(hot, 3), "cold_us": round(cold, 3),
                         "cold_gbps": round(step_bytes / cold / 1e3, 1),
                         "cold_frac_of_hbm_peak": round(step_bytes / cold / 1e3 / HBM_PEAK_GBS, 4),
                         "hot_effective_gbps": round(step_bytes / hot / 1e3, 1),
                         "warmup": {"hot_replays": hot_t.warmup_replays,
                                    "hot_s": round(hot_t.warmup_s, 3),
                                    "cold_replays": cold_t.warmup_replays,
                                    "cold_s": round(cold_t.warmup_s, 3)}})
            if check:
                units = [(0, 0), (0, 1)]
                c0 = calls[0]
                if method.startswith("fused"):
                    got = c0.keep[0].cpu().numpy()
                    refs = unit_refs(c0.keep[5], c0.keep[6], c0.keep[7], units)
                    what = "oracle fp32 dequantise-then-attend"
                else:
                    got = (c0() if method == "torch_fp16" else c0.keep[0]).float().cpu().numpy()
                    qq, kk, vv = (q, c0.keep[1].transpose(-1, -2), c0.keep[2]) \
                        if method == "torch_fp16" else (q, c0.keep[6], c0.keep[7])
                    refs = truth_refs(qq, kk, vv, units)
                    what = "fp32 attention over the fp16 K/V"
                rows[-1]["check"] = unit_check(got, refs, HQ // HKV, what)
            print(f"# qwen ctx={S} {method}: hot {hot:.2f} us  cold {cold:.2f} us  (R={R})",
                  file=sys.stderr, flush=True)
            del calls
            torch.cuda.empty_cache()
    by = {(r["ctx"], r["method"]): r for r in rows}

    def ratio(S, num, den, col):
        return round(by[(S, num)][col] / by[(S, den)][col], 3)

    effects = {str(S): {"quant_effect_cold_4b": ratio(S, "fp16", "fused4", "cold_us"),
                        "quant_effect_cold_4b_same_split": ratio(S, "fp16_fused_split", "fused4",
                                                                 "cold_us"),
                        "quant_effect_hot_4b_same_split": ratio(S, "fp16_fused_split", "fused4",
                                                                "hot_us"),
                        "quant_effect_cold_2b": ratio(S, "fp16", "fused2", "cold_us"),
                        "quant_effect_hot_4b": ratio(S, "fp16", "fused4", "hot_us"),
                        "flash_decode_effect_cold_vs_torch": ratio(S, "torch_fp16", "fp16", "cold_us"),
                        "flash_decode_effect_cold_vs_nosplit": ratio(S, "fp16_nosplit", "fp16", "cold_us"),
                        "flash_decode_effect_hot_vs_torch": ratio(S, "torch_fp16", "fp16", "hot_us")}
               for S in ctxs}
    return {"rows": rows, "effects": effects}


def qwen_eager(ctxs=(512, 2048, 8192, 16384), check=False):
    """Eager per-call latency at the Qwen2.5-1.5B shape (B=1, 4-bit gs32, one
    cache): ``fused_decode_attention`` / ``fp16_decode_attention`` called from
    Python with no graph, back to back (the reference's pipelined timing,
    ``benchmark.py:532-553``), next to the same Python call replayed from a
    graph; ``launch_overhead_us`` = eager - graph (``:1542-1545``).
    ``host_us`` is what issuing one call costs the host (validation, split
    plan, argument block, ctypes): while it exceeds the GPU time of a call the
    eager stream waits on Python."""
    import torch

    from tritonkv_amd.kernels import fp16_decode_attention, fused_decode_attention
    from tritonkv_amd.quantize import quantize_kv
    from tritonkv_amd.timing import eager_per_call, per_call

    B, HQ, HKV, D, gs = 1, 12, 2, 128, 32
    res = {}
    for S in ctxs:
        g = torch.Generator(device="cuda").manual_seed(3000 + S)
        q = torch.randn(B, HQ, D, device="cuda", generator=g, dtype=torch.float16)
        k = torch.randn(B, HKV, S, D, device="cuda", generator=g, dtype=torch.float16)
        v = torch.randn(B, HKV, S, D, device="cuda", generator=g, dtype=torch.float16)
        kq, vq = quantize_kv(k, v, 4, gs)
        row = {}
        for name, fn in (("fused4", lambda o, w: fused_decode_attention(q, kq, vq, out=o,
                                                                       _workspace=w)),
                         ("fp16", lambda o, w: fp16_decode_attention(q, k, v, out=o,
                                                                     _workspace=w))):
            out, ws = torch.empty(B, HQ, D, device="cuda"), {}
            call = lambda fn=fn, out=out, ws=ws: fn(out, ws)  # noqa: E731
            call()
            e = eager_per_call(call)
            gr = per_call([call] * 50).us
            row[name] = {"eager_us": round(e.us, 3), "graph_us": round(gr, 3),
                         "launch_overhead_us": round(e.us - gr, 3),
                         "host_us_per_call": round(e.host_us, 3)}
            if check:
                units = [(0, 0), (0, 1)]
                refs = (unit_refs(q, kq, vq, units) if name == "fused4"
                        else truth_refs(q, k, v, units))
                row[name]["check"] = unit_check(out.cpu().numpy(), refs, HQ // HKV,
                                                "oracle (as the Qwen table)")
        res[str(S)] = row
        print(f"# qwen eager ctx={S}: fused4 {row['fused4']['eager_us']} us eager vs "
              f"{row['fused4']['graph_us']} graph (host {row['fused4']['host_us_per_call']} us); "
              f"fp16 {row['fp16']['eager_us']} vs {row['fp16']['graph_us']}",
              file=sys.stderr, flush=True)
        del kq, vq, k, v
        torch.cuda.empty_cache()
    return res


def qwen_serving_steps(ctxs=(2048, 16384), check=False):
    """A whole decode step at the Qwen2.5-1.5B shape (B=1, 4-bit gs32, one
    cache): append the new token's K and V, then attend over it -- as three
    launches (two appends + decode) and as one (the append fused into the split
    kernel).  Per-step µs of a graph of 50 steps."""
    import torch

    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.quantize import append_kv, quantize_groupwise

    B, HQ, HKV, D, gs = 1, 12, 2, 128, 32
    res = {}
    for S in ctxs:
        g = torch.Generator(device="cuda").manual_seed(2000 + S)
        q = torch.randn(B, HQ, D, device="cuda", generator=g, dtype=torch.float16)
        kq = quantize_groupwise(torch.randn(B, HKV, S, D, device="cuda", generator=g,
                                            dtype=torch.float16), 4, gs)
        vq = quantize_groupwise(torch.randn(B, HKV, S, D, device="cuda", generator=g,
                                            dtype=torch.float16), 4, gs)
        k_new = torch.randn(B, HKV, 1, D, device="cuda", generator=g, dtype=torch.float16)
        v_new = torch.randn(B, HKV, 1, D, device="cuda", generator=g, dtype=torch.float16)
        lens = torch.full((B,), S, dtype=torch.int32, device="cuda")
        pos = lens - 1
        out = torch.empty(B, HQ, D, device="cuda")
        ws = {}

        def three():
            append_kv(kq, k_new, pos)
            append_kv(vq, v_new, pos)
            fused_decode_attention(q, kq, vq, seq_lens=lens, out=out, _workspace=ws)

        def one():
            fused_decode_attention(q, kq, vq, seq_lens=lens, out=out, _workspace=ws,
                                   k_new=k_new, v_new=v_new)

        t3 = per_call_us([three] * 50)
        t1 = per_call_us([one] * 50)
        res[str(S)] = {"three_launches_us": round(t3, 3), "fused_us": round(t1, 3),
                       "speedup": round(t3 / t1, 3)}
        if check:  # the fused step's output over the cache its own append wrote
            res[str(S)]["check"] = unit_check(
                out.cpu().numpy(), unit_refs(q, kq, vq, [(0, 0), (0, 1)]), HQ // HKV,
                "oracle fp32 dequantise-then-attend over the cache after the fused append")
        print(f"# qwen serving step ctx={S}: append+append+decode {t3:.2f} us, fused {t1:.2f} us",
              file=sys.stderr, flush=True)
        del kq, vq
        torch.cuda.empty_cache()
    return res


def qwen_e2e(ctxs=(8192, 32768), B=16, steps=8, seed=11, check=False):
    """End-to-end decode tokens/s of a random-initialised Qwen2.5-1.5B-architecture
    model (transformers, fp16 weights, 28 layers, HQ=12, HKV=2, D=128) at batch B
    with the cache pre-filled to ctx tokens of synthetic K/V: stock transformers
    (SDPA + DynamicCache, eager), the fp16 control kernel and the fused 4-bit
    kernel (``tritonkv_amd.hf``, eager and as one captured HIP graph per step),
    and 2-bit per-channel keys with an fp16 window (the same two ways)."""
    import torch
    from transformers import DynamicCache, Qwen2Config, Qwen2ForCausalLM

    from tritonkv_amd import hf

    hf.register()
    cfg = Qwen2Config(vocab_size=151936, hidden_size=1536, intermediate_size=8960,
                      num_hidden_layers=28, num_attention_heads=12, num_key_value_heads=2,
                      max_position_embeddings=65536, rope_theta=1e6, tie_word_embeddings=True)
    torch.manual_seed(seed)
    model = Qwen2ForCausalLM(cfg).half().cuda().eval()
    HKV, D = 2, 128
    res = {}

    def fill(cache, L):
        g = torch.Generator(device="cuda").manual_seed(seed)
        for i in range(cfg.num_hidden_layers):
            k = torch.randn(B, HKV, L, D, device="cuda", generator=g, dtype=torch.float16)
            v = torch.randn(B, HKV, L, D, device="cuda", generator=g, dtype=torch.float16)
            cache.update(k, v, i)
            del k, v

    def timed(fn, n):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s.record()
        for _ in range(n):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) * 1e3 / n

    with torch.no_grad():
        for L in ctxs:
            row, logits = {}, {}
            for name in ("stock_sdpa", "tkv_fp16", "tkv_4bit", "tkv_2bit_channel"):
                if name == "stock_sdpa":
                    model.set_attn_implementation("sdpa")
                    cache = DynamicCache(config=model.config)
                else:
                    model.set_attn_implementation(hf.ATTN_NAME)
                    nb = {"tkv_fp16": 16, "tkv_4bit": 4, "tkv_2bit_channel": 2}[name]
                    cache = hf.TkvCache(model.config, capacity=L + 4 * steps + 8, nbits=nb,
                                        keys="channel" if name == "tkv_2bit_channel" else "token")
                fill(cache, L)
                ids = torch.zeros(B, 1, dtype=torch.long, device="cuda")
                pos = torch.full((B, 1), L, dtype=torch.long, device="cuda")

                def step():
                    lg = model(input_ids=ids, position_ids=pos, past_key_values=cache,
                               use_cache=True, logits_to_keep=1).logits
                    pos.add_(1)
                    return lg

                logits[name] = step()[:, -1].float()  # warm-up; every variant's first step
                entry = {"eager_us": round(timed(step, steps), 1)}
                if name != "stock_sdpa":
                    try:
                        g = capture([step])
                        entry["graph_us"] = round(timed(g.replay, steps), 1)
                        del g
                    except Exception as exc:  # report, do not fail the bench
                        entry["graph_error"] = f"{type(exc).__name__}: {exc}"[:200]
                best = min(v for k, v in entry.items() if k.endswith("_us"))
                entry["tokens_per_s"] = round(B / best * 1e6, 1)
                if name != "stock_sdpa":
                    entry["cache_bytes"] = cache.nbytes
                row[name] = entry
                print(f"# e2e qwen2.5-1.5b B={B} ctx={L} {name}: {entry}", file=sys.stderr,
                      flush=True)
                del cache
                torch.cuda.empty_cache()
            if check:  # first decode step's logits against stock transformers (SDPA)
                ref = logits["stock_sdpa"]
                chk = {}
                for name in ("tkv_fp16", "tkv_4bit", "tkv_2bit_channel"):
                    d = logits[name] - ref
                    chk[name] = {"logits_rel_l2_vs_stock": round(float(d.norm() / ref.norm()), 5),
                                 "top1_agreement": round(float((logits[name].argmax(-1) ==
                                                                ref.argmax(-1)).float().mean()), 4)}
                # the fp16 control attends in fp32 over the same fp16 cache as SDPA
                chk["ok"] = bool(chk["tkv_fp16"]["logits_rel_l2_vs_stock"] < 1e-2)
                chk["reference"] = ("stock transformers (SDPA, DynamicCache) on the same weights "
                                    "and pre-filled cache; only the fp16 control is held to a "
                                    "bound (rel-L2 < 1e-2), the quantized rows are recorded")
                row["check"] = chk
            row["speedup_4bit_vs_fp16_control"] = round(
                row["tkv_4bit"]["tokens_per_s"] / row["tkv_fp16"]["tokens_per_s"], 3)
            row["speedup_4bit_vs_stock"] = round(
                row["tkv_4bit"]["tokens_per_s"] / row["stock_sdpa"]["tokens_per_s"], 3)
            res[str(L)] = row
    del model
    torch.cuda.empty_cache()
    return {"batch": B, "model": "Qwen2.5-1.5B architecture, random init, fp16", "ctx": res}


# ---------------------------------------------------------------------------


# name -> (K bits, V bits, group size, per-channel keys): the Llama-3-8B-shape
# split kernels of the benchmark's legs.
KERNEL_PROBES = {"k4v4g32": (4, 4, 32, False), "k4v4g128": (4, 4, 128, False),
                 "k2v2g32": (2, 2, 32, False), "k2v2g128": (2, 2, 128, False),
                 "ch2": (2, 2, 32, True), "ch4": (4, 4, 32, True)}


def kernel_probe(name, launches=6):
    """``launches`` eager split-kernel launches (no combine) of one format at the
    Llama-3-8B shape on the benchmark's first cache copy, plus the read probe of
    the same access pattern (not for per-channel keys)."""
    import torch

    from tritonkv_amd import _lib
    from tritonkv_amd.channel import BLOCK, quantize_keys_per_channel
    from tritonkv_amd.kernels.fused_decode_attn import choose_waves, plan_splits
    from tritonkv_amd.quantize import quantize_groupwise, quantize_kv

    kb, vb, gs, ch = KERNEL_PROBES[name]
    q, k, v = llama_inputs(seed=10)
    calls = []
    if ch:
        ck = quantize_keys_per_channel(k, kb)
        vq = quantize_groupwise(v, vb, gs)
        del k, v
        B, HQ, D = q.shape
        _, HKV, S, _ = vq.packed.shape
        _, ns, size = plan_splits(S, 64, None, B, HKV, HQ // HKV)
        out = torch.empty(B, HQ, D, device="cuda")
        acc = torch.empty(B, HQ, ns + 1, D, device="cuda")
        ml = torch.empty(2, B, HQ, ns + 1, device="cuda")
        args = _lib.DecodeArgs(
            q=q.data_ptr(), k=ck.packed.data_ptr(), k_scale=ck.scale.data_ptr(),
            k_zero=ck.zero.data_ptr(), v=vq.packed.data_ptr(), v_scale=vq.scale.data_ptr(),
            v_zero=vq.zero.data_ptr(), acc=acc.data_ptr(), maxs=ml[0].data_ptr(),
            sums=ml[1].data_ptr(), out=out.data_ptr(), B=B, HQ=HQ, HKV=HKV, S=S, D=D,
            k_nbits=kb, v_nbits=vb, group_size=gs, sm_scale=D ** -0.5, split_size=size,
            num_splits=ns, waves=choose_waves(B, HKV, HQ // HKV, size, ns, D=D, k_nbits=kb,
                                              v_nbits=vb, group_size=gs), key_block=BLOCK,
            split_base=0, num_splits_total=ns + 1)
        lib = _lib.load()

        def call():
            _lib.check(lib.tkv_fused_decode_split(args, torch.cuda.current_stream().cuda_stream),
                       "per-channel split")
        call.keep = (q, ck, vq, out, acc, ml)
        calls.append(call)
    else:
        kq, vq = quantize_kv(k, v, kb, gs)
        del k, v
        calls.append(fused_call(q, kq, vq, split_only=True))
        calls.append(fused_call(q, kq, vq, probe=True))
    for f in calls:
        for _ in range(launches):
            f()
    torch.cuda.synchronize()
    print(json.dumps({"kernel_probe": name, "launches": launches, "kernels": len(calls)}))
    return 0


def counter_summary(dirs, skip=0) -> int:
    """Mean value per dispatch of every counter in the --pmc directories, per
    kernel (largest grid of each kernel name), with per-wave instruction counts;
    the first ``skip`` dispatches of each kernel and counter are left out
    (warm-up calls)."""
    rows = {}
    for d in dirs:
        for r in _csv_rows(d, "counter_collection.csv"):
            key = r["Kernel_Name"]
            grid = int(r["Grid_Size"])
            ent = rows.setdefault(key, {})
            ent.setdefault((grid, r["Counter_Name"]), []).append(float(r["Counter_Value"]))
    for ent in rows.values():
        for k in ent:
            if len(ent[k]) > skip:
                ent[k] = ent[k][skip:]
    out = []
    for name, ent in rows.items():
        if "tkv::" not in name:
            continue
        gmax = max(g for g, _ in ent)
        vals = {c: statistics.mean(v) for (g, c), v in ent.items() if g == gmax}
        out.append(f"kernel: {name}  (grid {gmax} work-items)")
        for c in sorted(vals):
            out.append(f"  {c:28s} {vals[c]:18.1f}")
        waves = vals.get("SQ_WAVES")
        if waves:
            per = ", ".join(f"{c[len('SQ_INSTS_'):]} {vals[c] / waves:.0f}"
                            for c in sorted(vals) if c.startswith("SQ_INSTS_"))
            out.append(f"  per wave: {per}")
        if vals.get("SQ_BUSY_CYCLES") and vals.get("SQ_ACTIVE_INST_VALU") and vals.get("SQ_WAVE_CYCLES"):
            out.append(f"  SQ_ACTIVE_INST_VALU / SQ_WAVE_CYCLES = "
                       f"{vals['SQ_ACTIVE_INST_VALU'] / vals['SQ_WAVE_CYCLES']:.3f}")
        out.append("")
    print("\n".join(out))
    return 0


def order_sweep(steps=30, warmup=200):
    """Longest-piece-first dispatch order against the grid order (one JSON line).

    * the 70B-style ragged batch of ``ragged_70b`` (K4/V2, lengths U[1024,
      131072], seed 2024): decode and ``tkv_read_probe`` at 1, 2, 3, 4, 6, 8
      and 16 splits per row, each in both orders;
    * the Llama-3-8B step (4-bit gs32, B=32, ctx 32768) with every length
      passed as ``seq_lens``: grid order, the order, and no ``seq_lens``."""
    import torch

    from tritonkv_amd import _lib, synthetic
    from tritonkv_amd.kernels import fused_decode_attention
    from tritonkv_amd.kernels.fused_decode_attn import _workspace_for, plan_splits
    from tritonkv_amd.quantize import quantize_groupwise

    B, HQ, HKV, D, gs, S = 64, 64, 8, 128, 32, 131072 + 64
    lens = synthetic.ragged_lengths(B, 1024, 131072, seed=2024)
    q, kc, vc, _, _ = synthetic.ragged_batch(B, HQ, HKV, D, lens, S, 4, 2, gs, seed=2024)
    lens1 = (lens + 1).to("cuda")
    out = torch.empty(B, HQ, D, device="cuda")
    lib = _lib.load()
    rows = []
    for ns in (1, 2, 3, 4, 6, 8, 16):
        _, n, size = plan_splits(S, 64, ns, B, HKV, HQ // HKV, ragged=True)
        acc, mx, sm, _ = _workspace_for({}, B, HQ, n, D, q.device, HKV)
        order = torch.empty(2 * B * HKV * n, dtype=torch.int32, device="cuda")
        row = {"splits": n, "split_size": size}
        for use in (False, True):
            ws = {}

            def decode():
                fused_decode_attention(q, kc, vc, seq_lens=lens1, allow_mixed_bits=True,
                                       out=out, _workspace=ws, num_splits=ns,
                                       dispatch_order=use)
            args = _lib.DecodeArgs(
                q=q.data_ptr(), k=kc.packed.data_ptr(), k_scale=kc.scale.data_ptr(),
                k_zero=kc.zero.data_ptr(), v=vc.packed.data_ptr(), v_scale=vc.scale.data_ptr(),
                v_zero=vc.zero.data_ptr(), seq_lens=lens1.data_ptr(), acc=_lib.ptr(acc),
                maxs=_lib.ptr(mx), sums=_lib.ptr(sm), out=out.data_ptr(), B=B, HQ=HQ, HKV=HKV,
                S=S, D=D, k_nbits=4, v_nbits=2, group_size=gs, sm_scale=D ** -0.5,
                split_size=size, num_splits=n, waves=8,
                work_order=order.data_ptr() if use else None)

            def probe(args=args):
                _lib.check(lib.tkv_read_probe(args, torch.cuda.current_stream().cuda_stream),
                           "tkv_read_probe")
            key = "longest_first" if use else "grid"
            row[key + "_decode_us"] = round(timed_steps([decode], steps, warmup)[0], 1)
            row[key + "_probe_us"] = round(timed_steps([probe], steps, warmup)[0], 1)
        print(f"# ragged 70b {json.dumps(row)}", file=sys.stderr, flush=True)
        rows.append(row)
    del q, kc, vc, out
    torch.cuda.empty_cache()

    Bq, HQq, Sq = 32, 32, 32768
    g = torch.Generator(device="cuda").manual_seed(7)
    qq = torch.randn(Bq, HQq, D, device="cuda", generator=g).half()
    kq = quantize_groupwise(torch.randn(Bq, HKV, Sq, D, device="cuda", generator=g).half(), 4, gs)
    vq = quantize_groupwise(torch.randn(Bq, HKV, Sq, D, device="cuda", generator=g).half(), 4, gs)
    eq = torch.full((Bq,), Sq, dtype=torch.int32, device="cuda")
    outq = torch.empty(Bq, HQq, D, device="cuda")
    equal = {}
    for name, kw in (("no_seq_lens", {}), ("seq_lens_grid_order", dict(seq_lens=eq, dispatch_order=False)),
                     ("seq_lens_longest_first", dict(seq_lens=eq))):
        ws = {}

        def step(kw=kw, ws=ws):
            fused_decode_attention(qq, kq, vq, out=outq, _workspace=ws, **kw)
        equal[name + "_us"] = round(timed_steps([step], steps, warmup)[0], 1)
    print(f"# llama equal lengths {json.dumps(equal)}", file=sys.stderr, flush=True)
    print(json.dumps({"order_sweep": {"ragged_70b_k4v2": rows, "llama3_8b_equal_lengths": equal}}))
    return 0


def regime_probe(mode):
    """Eager decode calls at the Qwen2.5-1.5B shape, ctx 16384, 4-bit gs32, on one
    cache ('hot') or on rotating copies totalling >= 768 MB ('cold')."""
    import torch

    from tritonkv_amd.quantize import QuantizedTensor, quantize_groupwise
    from tritonkv_amd.timing import replicas_for

    B, HQ, HKV, D, S, gs = 1, 12, 2, 128, 16384, 32
    g = torch.Generator(device="cuda").manual_seed(7)
    q = torch.randn(B, HQ, D, device="cuda", generator=g, dtype=torch.float16)
    cache, _ = algorithmic_bytes(B, HQ, HKV, S, D, 4, 4, gs)
    R = 1 if mode == "hot" else replicas_for(cache)
    kv = torch.randn(2, R, B, HKV, S, D, device="cuda", generator=g, dtype=torch.float16)
    kq, vq = quantize_groupwise(kv[0], 4, gs), quantize_groupwise(kv[1], 4, gs)
    del kv
    calls = [fused_call(q, QuantizedTensor(kq.packed[i], kq.scale[i], kq.zero[i], 4, gs, D),
                        QuantizedTensor(vq.packed[i], vq.scale[i], vq.zero[i], 4, gs, D))
             for i in range(R)]
    for c in calls[:min(R, 8)]:
        c()
    torch.cuda.synchronize()
    for i in range(60):
        calls[i % R]()
    torch.cuda.synchronize()
    print(json.dumps({"regime": mode, "replicas": R, "calls": 60}))
    return 0


def qwen_trace(S, calls_each=200):
    """Eager hot decode calls at the Qwen2.5-1.5B shape (B=1, HQ=12, HKV=2,
    D=128, gs32): fp16 control, fused 4-bit, fused 2-bit, in that order."""
    import torch

    from tritonkv_amd.quantize import quantize_groupwise

    B, HQ, HKV, D, gs = 1, 12, 2, 128, 32
    g = torch.Generator(device="cuda").manual_seed(7)
    q = torch.randn(B, HQ, D, device="cuda", generator=g, dtype=torch.float16)
    k = torch.randn(B, HKV, S, D, device="cuda", generator=g, dtype=torch.float16)
    v = torch.randn(B, HKV, S, D, device="cuda", generator=g, dtype=torch.float16)
    calls = [fp16_call(q, k, v)] + [
        fused_call(q, quantize_groupwise(k, nb, gs), quantize_groupwise(v, nb, gs))
        for nb in (4, 2)]
    for c in calls:
        for _ in range(calls_each):
            c()
        torch.cuda.synchronize()
    print(json.dumps({"qwen_trace": S, "calls_each": calls_each,
                      "splits": [c.num_splits for c in calls]}))
    return 0


def main() -> int:
    a = _args()
    if a.rocprof_summary:
        return rocprof_summary(a)
    if a.counter_summary:
        return counter_summary(a.counter_summary, a.skip_dispatches)
    if a.kernel_probe:
        return kernel_probe(a.kernel_probe)
    if a.regime_probe:
        return regime_probe(a.regime_probe)
    if a.qwen_trace:
        return qwen_trace(a.qwen_trace)
    if a.order_sweep:
        return order_sweep()
    if a.compare:
        return compare(a.compare)
    global MIN_WARMUP_S
    MIN_WARMUP_S = a.min_warmup_s
    if a.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU per box; the decode step shards "
                          "by (batch, kv head) with no communication, and no figure at "
                          f"{a.gpus} GPUs is produced"}))
        return 2
    import torch

    from tritonkv_amd.kernels import triton_available
    from tritonkv_amd.quantize import quantize_kv
    from tritonkv_amd.timing import empty_kernel_floor

    ok, why = triton_available()
    if not ok:
        print(json.dumps({"error": why}))
        return 1
    torch.backends.cuda.matmul.allow_tf32 = False
    B, HQ, HKV, S, D, gs = 32, 32, 8, 32768, 128, 32
    detail = {}
    global _CLOCKS
    if not a.no_clocks:
        from tritonkv_amd.clocks import ClockMonitor

        mon = ClockMonitor(interval_s=0.01)
        _CLOCKS = mon if mon.start() else None

    def build_copies(nbits, g_s=gs):
        out = []
        for c in range(2):
            q, k, v = llama_inputs(seed=10 + c)
            if nbits == 16:
                out.append((q, k, v))
            else:
                kq, vq = quantize_kv(k, v, nbits, g_s)
                del k, v
                out.append((q, kq, vq))
        torch.cuda.synchronize()
        return out

    # ---- headline: 4-bit --------------------------------------------------
    copies4 = build_copies(4)
    cache4, bytes4 = algorithmic_bytes(B, HQ, HKV, S, D, 4, 4, gs)
    steps4 = [fused_call(*c, num_splits=a.num_splits) for c in copies4]
    us4, wall4, samples4 = timed_steps(steps4, a.steps, a.warmup)
    warm4 = _LAST_WARMUP
    clocks4 = clock_record(samples4, full=True)
    split4 = [fused_call(*c, num_splits=a.num_splits, split_only=True) for c in copies4]
    split_us4, _, split_samples4 = timed_steps(split4, a.steps, a.warmup)
    clocks_split4 = clock_record(split_samples4)
    kernel4 = split4[0].kernel
    achieved = bytes4 / split_us4 / 1e3
    probe4 = [fused_call(*c, num_splits=a.num_splits, probe=True) for c in copies4]
    probe_us4, _, _ = timed_steps(probe4, a.steps, a.warmup)
    ceiling4 = cache4 / probe_us4 / 1e3
    print(f"# llama 4-bit read-ceiling probe: {probe_us4:.2f} us = {ceiling4:.0f} GB/s; split "
          f"kernel at {probe_us4 / split_us4:.1%} of it", file=sys.stderr, flush=True)
    del probe4
    print(f"# llama 4-bit: step {us4:.2f} us, split kernel {split_us4:.2f} us, "
          f"{achieved:.0f} GB/s ({achieved / HBM_PEAK_GBS:.1%} of 8 TB/s), "
          f"splits={steps4[0].num_splits}", file=sys.stderr, flush=True)
    copy_gbs = copy_probe()
    print(f"# device copy probe: {copy_gbs:.0f} GB/s (read+write)", file=sys.stderr, flush=True)
    detail["device_copy_gbps"] = round(copy_gbs, 1)
    detail["fused4"] = {"us_per_step": round(us4, 2), "split_kernel_us": round(split_us4, 2),
                        "frac_of_copy_bw": round(achieved / copy_gbs, 4),
                        "cache_bytes": cache4, "algorithmic_bytes": bytes4,
                        "gbps_step": round(bytes4 / us4 / 1e3, 1),
                        "num_splits": steps4[0].num_splits,
                        "step_us_per_replay": [round(x, 2) for x in samples4],
                        "split_kernel_us_per_replay": [round(x, 2) for x in split_samples4],
                        "read_ceiling": {"probe_us": round(probe_us4, 2),
                                         "gbps": round(ceiling4, 1),
                                         "frac_of_hbm_peak": round(ceiling4 / HBM_PEAK_GBS, 4),
                                         "kernel_frac_of_ceiling": round(probe_us4 / split_us4, 4)},
                        "clocks": clocks_split4}
    cpu, checks, truth = None, {}, None
    q0, kq0, vq0 = copies4[0]
    got0 = steps4[0].keep[0].cpu().numpy()  # copy 0's output of the last timed replay
    checking = not a.quick and not a.no_cpu_baseline
    if checking:
        cpu, check = cpu_baseline(q0, kq0, vq0, got0)
        print(f"# cpu baseline {cpu['value'] / 1e3:.0f} ms/step on {cpu['cores']} threads; "
              f"check vs oracle: max abs {check['max_abs_err']:.2e}, mean abs "
              f"{check['mean_abs_err']:.2e} over {check['units']} units", file=sys.stderr,
              flush=True)
        cpu["config1_reference_cpu_step"] = cpu_config1()
        # end-to-end: fp32 attention over copy 0's unquantized K/V, sampled units
        qt, kt, vt = llama_inputs(seed=10)
        truth = truth_refs(qt, kt, vt, LLAMA_UNITS)
        del qt, kt, vt
        G4 = HQ // HKV
        check["kernel_rel_l2_vs_fp16_truth"] = round(rel_l2_units(got0, truth, G4), 5)
        check["fp16_baseline_rel_l2_vs_fp16_truth"] = round(rel_l2_units(
            _stack(unit_refs(q0, kq0, vq0, LLAMA_UNITS, fp16_dequant=True), q0.shape), truth,
            G4), 5)
        checks["llama_fused4"] = check
    del steps4, split4
    if not a.quick:
        # the headline step with every row's length passed as seq_lens: with
        # equal_lengths the unragged plan (the headline's), without it the
        # ragged rule's two pieces per row
        from tritonkv_amd.kernels import fused_decode_attention

        lens = torch.full((B,), S, dtype=torch.int32, device="cuda")
        eq = {}
        for key, flag in (("equal_lengths", True), ("ragged_plan", False)):
            calls = []
            for q, kq, vq in copies4:
                out, ws = torch.empty(B, HQ, D, device="cuda"), {}

                def f(q=q, kq=kq, vq=vq, out=out, ws=ws, flag=flag):
                    fused_decode_attention(q, kq, vq, seq_lens=lens, equal_lengths=flag,
                                           out=out, _workspace=ws)
                f()  # workspace allocated outside the captured graph
                f.out = out
                calls.append(f)
            t, _, _ = timed_steps(calls, a.steps, a.warmup)
            eq[key] = {"us_per_step": round(t, 2), "vs_no_seq_lens": round(t / us4, 4)}
            if key == "equal_lengths" and checking:
                same = bool((calls[0].out.cpu().numpy() == got0).all())
                checks["llama_equal_lens"] = {"bitwise_equal_to_no_seq_lens_step": same,
                                              "ok": same,
                                              "reference": "the headline step without seq_lens"}
            del calls
        eq["no_seq_lens_us"] = round(us4, 2)
        detail["llama_equal_lens"] = eq
        print(f"# llama 4-bit, equal seq_lens: {eq['equal_lengths']['us_per_step']} us with "
              f"equal_lengths, {eq['ragged_plan']['us_per_step']} us with the ragged plan, "
              f"{us4:.2f} us without seq_lens", file=sys.stderr, flush=True)
    torch.cuda.empty_cache()
    if not a.quick:
        # the same step over page pools in shuffled page order (serving layout)
        detail["paged4"] = {}
        for page in (32, 256):
            pools = []
            for i, (q, kq, vq) in enumerate(copies4):
                kp, table = to_pool(kq, page, seed=100 + i)
                vp, _ = to_pool(vq, page, seed=100 + i)
                pools.append((q, kp, vp, table))
            pcalls = [paged_call(*p) for p in pools]
            us, _, _ = timed_steps(pcalls, a.steps, a.warmup)
            if checking:  # the paged step reads the same tokens: bit-identical output
                gp = pcalls[0].keep[0].cpu().numpy()
                checks[f"paged4_page{page}"] = {
                    "bitwise_equal_to_contiguous_step": bool((gp == got0).all()),
                    "ok": bool((gp == got0).all()),
                    "reference": "the contiguous headline step's output on the same tokens"}
            del pcalls
            sp, _, sps = timed_steps([paged_call(*p, split_only=True) for p in pools], a.steps,
                                     a.warmup)
            detail["paged4"][f"page{page}"] = {
                "us_per_step": round(us, 2), "split_kernel_us": round(sp, 2),
                "frac_of_hbm_peak": round(bytes4 / sp / 1e3 / HBM_PEAK_GBS, 4),
                "vs_contiguous_step": round(us / us4, 4), "clocks": clock_record(sps)}
            print(f"# llama 4-bit paged (page {page}, shuffled): step {us:.2f} us, split "
                  f"{sp:.2f} us", file=sys.stderr, flush=True)
            del pools
            torch.cuda.empty_cache()
    del copies4
    torch.cuda.empty_cache()

    if not a.quick:
        for nbits, g_s, name in ((2, 32, "fused2"), (16, 32, "fp16"), (4, 128, "fused4_gs128"),
                                 (2, 128, "fused2_gs128")):
            cps = build_copies(nbits, g_s)
            cache, nbytes = algorithmic_bytes(B, HQ, HKV, S, D, nbits, nbits, g_s)
            mk = fp16_call if nbits == 16 else fused_call
            lcalls = [mk(*c) for c in cps]
            us, _, _ = timed_steps(lcalls, a.steps, a.warmup)
            if checking:
                got = lcalls[0].keep[0].cpu().numpy()
                if nbits == 16:
                    checks[name] = unit_check(got, truth, HQ // HKV,
                                              "fp32 attention over the fp16 K/V, sampled units")
                else:
                    checks[name] = llama_leg_check(got, *cps[0], truth)
            del lcalls
            sp, _, sps = timed_steps([mk(*c, split_only=True) for c in cps], a.steps, a.warmup)
            detail[name] = {"us_per_step": round(us, 2), "split_kernel_us": round(sp, 2),
                            "cache_bytes": cache, "algorithmic_bytes": nbytes,
                            "gbps_split_kernel": round(nbytes / sp / 1e3, 1),
                            "frac_of_hbm_peak": round(nbytes / sp / 1e3 / HBM_PEAK_GBS, 4),
                            "clocks": clock_record(sps)}
            if nbits != 16:
                pu, _, _ = timed_steps([mk(*c, probe=True) for c in cps], a.steps, a.warmup)
                detail[name]["read_ceiling"] = {
                    "probe_us": round(pu, 2), "gbps": round(cache / pu / 1e3, 1),
                    "kernel_frac_of_ceiling": round(pu / sp, 4)}
            print(f"# llama {name}: step {us:.2f} us, split {sp:.2f} us", file=sys.stderr, flush=True)
            del cps
            torch.cuda.empty_cache()
        detail["quant_effect_4b"] = round(detail["fp16"]["us_per_step"] / us4, 3)
        detail["quant_effect_2b"] = round(detail["fp16"]["us_per_step"] / detail["fused2"]["us_per_step"], 3)
        detail["empty_graph_node_us"] = round(empty_kernel_floor(), 2)
        detail["qwen2.5-1.5b"] = qwen_table(check=checking)
        detail["qwen2.5-1.5b_eager"] = qwen_eager(check=checking)
        detail["qwen2.5-1.5b_serving_step"] = qwen_serving_steps(check=checking)
        detail["qwen2.5-1.5b_e2e_decode"] = qwen_e2e(check=checking)
        detail["ragged_70b_k4v2"] = ragged_70b(a.steps, a.warmup, check=checking)
        detail["channel_keys"] = channel_keys(a.steps, a.warmup, check=checking)
        if checking:
            # one check record per timed leg, gathered from the legs
            checks["qwen_table"] = {f"{r['ctx']}/{r['method']}": r.pop("check")
                                    for r in detail["qwen2.5-1.5b"]["rows"]}
            checks["qwen_eager"] = {f"{S_}/{m}": row[m].pop("check")
                                    for S_, row in detail["qwen2.5-1.5b_eager"].items()
                                    for m in ("fused4", "fp16")}
            checks["qwen_serving_step"] = {S_: r.pop("check") for S_, r in
                                           detail["qwen2.5-1.5b_serving_step"].items()}
            checks["qwen_e2e"] = {L_: r.pop("check") for L_, r in
                                  detail["qwen2.5-1.5b_e2e_decode"]["ctx"].items()}
            checks["ragged_70b_k4v2"] = detail["ragged_70b_k4v2"].pop("check")
            checks["channel_keys"] = {k_: e.pop("check") for k_, e in
                                      detail["channel_keys"].items()}
            # the reference's own snapshot: its inputs, seeds 0-2, every (ctx, nbits)
            checks["qwen_reference_snapshot"] = qwen_snapshot()

    line = {
        "metric": METRIC,
        "value": round(us4, 2),
        "unit": "us/decode step",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(wall4, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 codes x fp16 q (fp16 MFMA, fp32 accumulate)",
        "data": "synthetic: seeded N(0,1) fp16 q/K/V, 4 x8 outlier channels per KV head",
        "config": {"workload": "llama-3-8b attention decode step, B=32 HQ=32 HKV=8 D=128 ctx=32768, "
                               "4-bit gs32 split-P K/V, DRAM-resident (2 rotating cache copies)",
                   "batch": B, "ctx": S, "q_heads": HQ, "kv_heads": HKV, "head_dim": D,
                   "nbits": 4, "group_size": gs, "cache_bytes_per_step": cache4,
                   "parallelism": "single GPU (flash-decoding splits x kv heads)"},
        "gbps": round(bytes4 / us4 / 1e3, 1),
        "hbm_frac": round(bytes4 / us4 / 1e3 / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(kernel4),
                     "kernel": kernel4, "kernel_us": round(split_us4, 2),
                     "algorithmic_bytes": bytes4,
                     "read_ceiling_gbps": round(ceiling4, 1),
                     "frac_of_read_ceiling": round(probe_us4 / split_us4, 4)},
        "cpu_baseline": cpu,
        "check": checks or None,
        "check_ok": all(c.get("ok", True) for c in _check_leaves(checks)) if checks else None,
        "warmup_replays": warm4[0],
        "warmup_s": round(warm4[1], 3),
        "clocks": clocks4,
        "detail": detail,
    }
    if _CLOCKS is not None:
        _CLOCKS.stop()
    print(json.dumps(line))
    return 0


def _check_leaves(checks):
    """Every check record (a dict carrying "ok") of the nested check field."""
    if isinstance(checks, dict):
        if "ok" in checks:
            yield checks
        else:
            for v in checks.values():
                yield from _check_leaves(v)
    elif isinstance(checks, list):
        for v in checks:
            yield from _check_leaves(v)


def compare(paths) -> int:
    """Row-by-row comparison of complete runs' bench lines (one JSON per run):
    prints one JSON object; the rows whose run-to-run spread exceeds 5% are
    listed under ``moved``."""
    from tritonkv_amd import clocks

    runs = [clocks.load_run(p) for p in paths]
    names = [os.path.basename(p) for p in paths]
    recs = clocks.compare_runs(runs, names)
    print(json.dumps({"runs": names, "rows": len(recs),
                      "moved": [r["key"] for r in recs if r["moved"]],
                      "max_spread_frac": max((r["spread_frac"] for r in recs), default=None),
                      "records": recs}))
    return 0


if __name__ == "__main__":
    sys.exit(main())
