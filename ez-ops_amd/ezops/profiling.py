"""Kernel profiling on MI355X: wave-level timelines exported to Perfetto, and
a rocprofv3 harness per op.

The reference advertises SM-level profiling with a Perfetto /
chrome://tracing export (README.md:13) but implements only an Nsight Compute
wrapper (scripts/ncu_profile.py).  Both exist here, for gfx950:

* Wave timelines.  ``libezops_hip_prof.so`` is the library built with
  ``-DEZ_PROFILE=1``: every wave of the hot kernels records its begin / end
  time (s_memrealtime, 100 MHz) and where it ran (XCD, shader engine, CU,
  SIMD).  ``WaveTrace`` runs the ops inside its ``with`` block through that
  build and collects the records::

      with WaveTrace() as tr:
          op(*data)
      tr.chrome_trace("layer.json")   # open in ui.perfetto.dev or chrome://tracing
      print(tr.summary())

  One Perfetto process per XCD, one track per (SE, CU, SIMD).

* ``python -m ezops.profiling rocprof <op> -p <params>`` runs the op under
  ``rocprofv3 --kernel-trace --stats`` (CSV + a ``.pftrace`` Perfetto file),
  optionally ``--pmc`` counter passes (one run per group, never combined
  with a trace domain), and prints each kernel's time with the op's
  speed-of-light figures from ``Op.get_roofline()``.
  ``python -m ezops.profiling trace <op> -p <params>`` writes the wave
  timeline of one call.  Params follow the reference's ncu_profile.py:
  ``-p M=5,N=10`` or ``-p 5,10``.
"""

from __future__ import annotations

import argparse
import csv
import importlib
import json
import os
import shutil
import subprocess
import sys
import textwrap
from pathlib import Path

import numpy as np

from . import _hip

PROF_LIB = Path(os.environ.get("EZOPS_HIP_PROF_LIB", Path(__file__).resolve().parent / "_lib" / "libezops_hip_prof.so"))

RECORD_DTYPE = np.dtype([("t0", "<u8"), ("t1", "<u8"), ("hw_id", "<u4"), ("xcc_id", "<u4"), ("kernel", "<u2"),
                         ("wave", "<u2"), ("block", "<u4")])
assert RECORD_DTYPE.itemsize == 32

KERNEL_NAMES = {
    1: "gemv_rows", 2: "gemv_valu", 3: "linear_scalar", 4: "linear_mfma", 5: "attn_split", 6: "attn_combine",
    7: "prefill_attn", 8: "silu_mul", 9: "qk_norm_rope", 10: "rmsnorm_f32", 11: "rmsnorm_bf16", 12: "softmax",
    13: "sum", 14: "gemm",
}
TICKS_PER_US = 100.0  # s_memrealtime runs at 100 MHz
MAX_RECORDS = 1 << 21  # host buffer of a WaveTrace (64 MiB)


def decode_hw_id(hw_id) -> dict:
    """Fields of the HW_ID register (gfx9 layout)."""
    hw = np.asarray(hw_id, dtype=np.uint32)
    return {"slot": hw & 0xF, "simd": (hw >> 4) & 0x3, "cu": (hw >> 8) & 0xF, "sh": (hw >> 12) & 0x1,
            "se": (hw >> 13) & 0x7}


def chrome_trace(records: np.ndarray) -> dict:
    """Chrome trace-event JSON (Perfetto reads it): one complete event per wave."""
    events = []
    if len(records) == 0:
        return {"traceEvents": events, "displayTimeUnit": "ns"}
    t_min = int(records["t0"].min())
    f = decode_hw_id(records["hw_id"])
    xcc = (records["xcc_id"] & 0xF).astype(int)
    track = (f["se"].astype(int) * 2 + f["sh"].astype(int)) * 64 + f["cu"].astype(int) * 4 + f["simd"].astype(int)
    seen = set()
    for i, r in enumerate(records):
        pid, tid = int(xcc[i]), int(track[i])
        if (pid, tid) not in seen:
            seen.add((pid, tid))
            events.append({"name": "thread_name", "ph": "M", "pid": pid, "tid": tid,
                           "args": {"name": f"SE{int(f['se'][i])} SH{int(f['sh'][i])} CU{int(f['cu'][i])} "
                                            f"SIMD{int(f['simd'][i])}"}})
        events.append({
            "name": KERNEL_NAMES.get(int(r["kernel"]), f"kernel{int(r['kernel'])}"), "ph": "X", "pid": pid,
            "tid": tid, "ts": (int(r["t0"]) - t_min) / TICKS_PER_US,
            "dur": max(int(r["t1"]) - int(r["t0"]), 0) / TICKS_PER_US,
            "args": {"block": int(r["block"]), "wave": int(r["wave"]), "slot": int(f["slot"][i])},
        })
    for pid in sorted({int(x) for x in xcc}):
        events.append({"name": "process_name", "ph": "M", "pid": pid, "args": {"name": f"XCD {pid}"}})
    return {"traceEvents": events, "displayTimeUnit": "ns"}


def summarize(records: np.ndarray) -> list[dict]:
    """Per kernel: waves, wall span, mean wave time, and the XCD balance
    (waves and busy time per XCD, and the spread of the XCDs' last wave)."""
    out = []
    for k in sorted({int(x) for x in records["kernel"]}):
        r = records[records["kernel"] == k]
        dur = (r["t1"].astype(np.int64) - r["t0"].astype(np.int64)) / TICKS_PER_US
        xcc = (r["xcc_id"] & 0xF).astype(int)
        ends = {int(x): float((r["t1"][xcc == x].max() - r["t0"].min()) / TICKS_PER_US) for x in sorted(set(xcc))}
        out.append({
            "kernel": KERNEL_NAMES.get(k, f"kernel{k}"), "waves": int(len(r)),
            "span_us": float((r["t1"].max() - r["t0"].min()) / TICKS_PER_US),
            "mean_wave_us": float(dur.mean()), "max_wave_us": float(dur.max()),
            "waves_per_xcd": {int(x): int((xcc == x).sum()) for x in sorted(set(xcc))},
            "busy_us_per_xcd": {int(x): round(float(dur[xcc == x].sum()), 2) for x in sorted(set(xcc))},
            "xcd_end_spread_us": float(max(ends.values()) - min(ends.values())),
        })
    return out


class WaveTrace:
    """Run the ops called inside the block through the profiling build and
    collect one record per wave (see the module docstring)."""

    def __init__(self, path: Path | str = PROF_LIB, capacity: int = MAX_RECORDS):
        self.path, self.capacity = Path(path), capacity
        self.records = np.zeros(0, dtype=RECORD_DTYPE)
        self._lib = self._saved = None

    def __enter__(self) -> "WaveTrace":
        import torch

        self._lib = _hip.load(self.path)
        torch.cuda.synchronize()
        rc = self._lib.ezops_profile_reset()
        if rc != 0:
            raise RuntimeError(f"ezops_profile_reset failed ({rc}): {self._lib.ezops_hip_last_error().decode()}")
        self._saved, _hip._lib = _hip._lib, self._lib
        return self

    def __exit__(self, *exc) -> None:
        import torch

        try:
            torch.cuda.synchronize()
            buf = np.zeros(self.capacity, dtype=RECORD_DTYPE)
            n = self._lib.ezops_profile_read(buf.ctypes.data, self.capacity)
            if n < 0:
                raise RuntimeError(f"ezops_profile_read failed ({n}): {self._lib.ezops_hip_last_error().decode()}")
            self.records = np.sort(buf[:n], order="t0")
        finally:
            _hip._lib = self._saved

    def chrome_trace(self, path: Path | str | None = None) -> dict:
        doc = chrome_trace(self.records)
        if path is not None:
            Path(path).write_text(json.dumps(doc))
        return doc

    def summary(self) -> list[dict]:
        return summarize(self.records)


# ---------------------------------------------------------------- CLI
def op_class(op_name: str):
    mod = importlib.import_module("ezops")
    name = "".join(p.capitalize() for p in op_name.split("_")) + "Op"
    if not hasattr(mod, name):
        raise SystemExit(f"unknown op {op_name!r} (no ezops.{name})")
    return getattr(mod, name)


def parse_params(text: str) -> tuple[list, dict]:
    """'M=5,N=10' -> ([], {'M': 5, 'N': 10}); '5,10' -> ([5, 10], {})."""
    def num(v: str):
        v = v.strip()
        try:
            return int(v)
        except ValueError:
            return float(v)

    if not text:
        return [], {}
    if "=" in text:
        return [], {k.strip(): num(v) for k, v in (p.split("=") for p in text.split(","))}
    return [num(v) for v in text.split(",")], {}


def run_script(op_name: str, args: list, kwargs: dict, warmup: int, iters: int) -> str:
    """Python source of the profiled program: the op on the hip backend."""
    params = ", ".join([repr(a) for a in args] + [f"{k}={v!r}" for k, v in kwargs.items()] + ["backend='hip'"])
    cls = op_class(op_name).__name__
    pkg = Path(__file__).resolve().parent.parent
    return textwrap.dedent(f"""\
        import sys
        sys.path.insert(0, {str(pkg)!r})
        import torch
        from ezops import {cls}

        op = {cls}({params})
        data = op.gen_data()
        for _ in range({warmup}):
            op(*data)
        torch.cuda.synchronize()
        for _ in range({iters}):
            op(*data)
        torch.cuda.synchronize()
        print("profiled {op_name}: {warmup} warmup + {iters} calls", flush=True)
    """)


def read_kernel_stats(path: Path) -> list[dict]:
    """rocprofv3 ``*_kernel_stats.csv`` rows as dicts with float times (us)."""
    rows = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            rows.append({"name": r["Name"], "calls": int(r["Calls"]), "total_us": float(r["TotalDurationNs"]) / 1e3,
                         "avg_us": float(r["AverageNs"]) / 1e3, "min_us": float(r["MinNs"]) / 1e3,
                         "max_us": float(r["MaxNs"]) / 1e3, "percent": float(r["Percentage"])})
    return rows


def sol_report(rows: list[dict], calls: int, nbytes: float, nflops: float, peak_gbps: float,
               peak_tflops: float) -> dict:
    """Per-call kernel time of the op and its speed-of-light fractions."""
    total_us = sum(r["total_us"] for r in rows) / max(calls, 1)
    gbps = nbytes / (total_us * 1e-6) / 1e9 if total_us else 0.0
    tflops = nflops / (total_us * 1e-6) / 1e12 if total_us else 0.0
    return {"kernel_us_per_call": total_us, "GBps": gbps, "TFLOPs": tflops,
            "frac_hbm": gbps / peak_gbps, "frac_mfma": tflops / peak_tflops}


def _rocprof(args) -> int:
    exe = shutil.which("rocprofv3")
    if exe is None:
        print("rocprofv3 not found (ROCm profiler)", file=sys.stderr)
        return 1
    pos, kw = parse_params(args.params)
    out = Path(args.output_dir).resolve()
    out.mkdir(parents=True, exist_ok=True)
    script = out / f"_run_{args.op_name}.py"
    script.write_text(run_script(args.op_name, pos, kw, args.warmup, args.iters))
    env = dict(os.environ, TMPDIR="/tmp")
    base = [exe, "--kernel-trace", "--stats", "--output-format", "csv", "pftrace", "-d", str(out), "-o", args.op_name,
            "--", sys.executable, str(script)]
    print(" ".join(base), flush=True)
    r = subprocess.run(base, cwd="/tmp", env=env, timeout=args.timeout)
    if r.returncode != 0:
        return r.returncode
    for i, group in enumerate(args.pmc or []):
        cmd = [exe, "--pmc", *group.split(","), "--output-format", "csv", "-d", str(out), "-o",
               f"{args.op_name}_pmc{i}", "--", sys.executable, str(script)]
        print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, cwd="/tmp", env=env, timeout=args.timeout)
        if r.returncode != 0:
            return r.returncode
    stats = next(out.glob(f"**/{args.op_name}_kernel_stats.csv"), None)
    if stats is None:
        print(f"no kernel stats under {out}", file=sys.stderr)
        return 1
    rows = read_kernel_stats(stats)
    op = op_class(args.op_name)(*pos, **kw)
    rf = op.get_roofline()
    rep = sol_report(rows, args.warmup + args.iters, rf.fused_bytes, rf.flops, args.peak_gbps, args.peak_tflops)
    for r in rows:
        print(f"{r['avg_us']:10.2f} us x {r['calls']:4d}  {r['name'][:100]}")
    print(json.dumps({"op": args.op_name, "params": args.params, **rep,
                      "pftrace": [str(p) for p in out.glob(f"**/{args.op_name}*.pftrace")]}))
    return 0


def _trace(args) -> int:
    import torch

    pos, kw = parse_params(args.params)
    op = op_class(args.op_name)(*pos, **kw, backend="hip")
    data = op.gen_data()
    with WaveTrace():  # warm-up through the profiling build itself (its first launches load its code)
        for _ in range(args.warmup):
            op(*data)
    with WaveTrace() as tr:
        for _ in range(args.iters):
            op(*data)
    tr.chrome_trace(args.output)
    print(json.dumps({"op": args.op_name, "waves": int(len(tr.records)), "trace": str(args.output),
                      "kernels": tr.summary()}))
    return 0


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(prog="python -m ezops.profiling", description=__doc__.split("\n\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    a = sub.add_parser("rocprof", help="rocprofv3 kernel trace + stats (+ Perfetto file, + counter passes)")
    a.add_argument("op_name")
    a.add_argument("-p", "--params", default="")
    a.add_argument("-o", "--output-dir", default=".profiles")
    a.add_argument("-w", "--warmup", type=int, default=3)
    a.add_argument("-n", "--iters", type=int, default=10)
    a.add_argument("--pmc", action="append", help="comma-separated counter group; repeat for more passes")
    a.add_argument("--peak-gbps", type=float, default=8000.0)
    a.add_argument("--peak-tflops", type=float, default=2500.0)
    a.add_argument("--timeout", type=int, default=600)
    t = sub.add_parser("trace", help="wave-level timeline of the op (profiling build) as Chrome/Perfetto JSON")
    t.add_argument("op_name")
    t.add_argument("-p", "--params", default="")
    t.add_argument("-o", "--output", default="wave_trace.json")
    t.add_argument("-w", "--warmup", type=int, default=2)
    t.add_argument("-n", "--iters", type=int, default=1)
    args = ap.parse_args(argv)
    return _rocprof(args) if args.cmd == "rocprof" else _trace(args)


if __name__ == "__main__":
    sys.exit(main())
