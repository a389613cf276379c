"""MI355X hardware profile for roofline analysis.

Mirrors the reference's hardware-profile tooling:
* ``SPECS`` / ``detect_profile`` / ``get_specs`` — the spec database
  (benchmarks/hardware/gpu_specs.py), here with the one chip this backend runs on;
* ``measure_hbm`` / ``measure_mfma`` — the calibration microbenchmarks
  (benchmarks/hardware/memory/hbm_bandwidth.py, benchmarks/hardware/compute/matmul_peak.py),
  here the library's own STREAM probe (``ezops_hbm_probe``) and MFMA chain probe
  (``ezops_mfma_probe``) instead of CUDA kernels / torch matmuls;
* ``generate_yaml`` / ``main`` — the profile writer (scripts/roofline_profile.py:72-241),
  same YAML layout (theoretical + calibration; effective = theoretical * calibration);
* ``load_profile`` — the loader the reference benches use (benchmarks/bench_gemv.py ``_load_profile``).

Run ``python -m ezops.hardware`` on an MI355X to (re)write ``ezops/assets/mi355x.yaml``.
"""

from __future__ import annotations

import argparse
import math
from pathlib import Path

ASSETS = Path(__file__).resolve().parent / "assets"

# Published dense peaks (no sparsity), FMA counted as 2 flops.
SPECS = {
    "mi355x": {
        "names": ["AMD Instinct MI355X", "AMD Instinct MI350X"],
        "arch": "gfx950",
        "cu_count": 256,
        "l2_cache_size": 4 * 1024 * 1024,      # per XCD (8 XCDs)
        "mall_size": 256 * 1024 * 1024,        # Infinity Cache
        "lds_per_cu": 160 * 1024,
        "hbm_bw_gb": 8000.0,
        "tensor_core_tflops": {"bf16": 2500.0, "fp16": 2500.0, "fp8": 5000.0, "fp32": 157.3},
    },
}

_MFMA_KINDS = {"bf16": 0, "fp16": 1, "bf16_32x32": 2, "fp32": 3}
_MFMA_FLOPS_PER_INSTR = {0: 2 * 16 * 16 * 32, 1: 2 * 16 * 16 * 32, 2: 2 * 16 * 16 * 32, 3: 2 * 16 * 16 * 4}


def detect_profile(name: str = "", arch: str = "") -> str | None:
    """Profile key for a device name / gcnArchName, or None."""
    for key, spec in SPECS.items():
        if spec["arch"] and arch and arch.split(":")[0] == spec["arch"]:
            return key
        if any(n.lower() in name.lower() for n in spec["names"]):
            return key
    return None


def get_specs(profile: str) -> dict:
    return SPECS[profile]


def measure_hbm(n_bytes_per_array: int = 2 << 30, reps: int = 10) -> dict:
    """STREAM triad (a = b + s*c) and streaming read over arrays >> MALL: best GB/s
    (the read: the better of the looping and the one-shot-block patterns)."""
    import torch

    from . import _hip

    n = n_bytes_per_array // 4
    a = torch.empty(n, dtype=torch.float32, device="cuda")
    b = torch.rand(n, device="cuda")
    c = torch.rand(n, device="cuda")
    s = _hip.stream()
    out = {}
    for kind, name, nbytes in ((3, "triad", 12 * n), (4, "read", 4 * n), (5, "read_blocks", 4 * n)):
        best = math.inf
        for _ in range(reps + 2):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            _hip.call("ezops_hbm_probe", kind, a.data_ptr(), b.data_ptr(), c.data_ptr(), n, 1.5, s)
            e1.record()
            torch.cuda.synchronize()
            best = min(best, e0.elapsed_time(e1))
        out[name] = nbytes / (best * 1e-3) / 1e9
    out["read"] = max(out["read"], out.pop("read_blocks"))
    del a, b, c
    torch.cuda.empty_cache()
    return out


def measure_mfma(dtype: str = "bf16", iters: int = 4096, reps: int = 10) -> float:
    """Dense MFMA throughput (TFLOP/s) of independent MFMA chains on every SIMD
    (16x16x32 for bf16 / fp16, 32x32x16 for "bf16_32x32", 16x16x4 for fp32)."""
    import torch

    from . import _hip

    blocks = torch.cuda.get_device_properties(0).multi_processor_count * 8
    sink = torch.zeros(4, device="cuda")
    s = _hip.stream()
    flops = blocks * 4 * iters * 8 * _MFMA_FLOPS_PER_INSTR[_MFMA_KINDS[dtype]]
    best = math.inf
    for _ in range(reps + 2):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        _hip.call("ezops_mfma_probe", _MFMA_KINDS[dtype], sink.data_ptr(), blocks, iters, s)
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1))
    return flops / (best * 1e-3) / 1e12


def _fmt(coeff: float, unit_exp: int) -> str:
    """`coeff` x 10^unit_exp in the reference's notation ('8000e9'); YAML reads it as text,
    load_profile() converts."""
    return f"{coeff:.1f}e{unit_exp}" if coeff != int(coeff) else f"{int(coeff)}e{unit_exp}"


def generate_yaml(profile: str, gpu_name: str, hbm: dict, mfma_tflops: dict) -> str:
    """Profile YAML in the reference's layout (assets/rtx_5060_ti.yaml).

    ``hbm.calibration`` is the best sustained rate measured (the streaming
    read when it is given, else the triad): the reference's benches divide by
    ``theoretical * calibration`` (benchmarks/bench_gemv.py:62-86), and a
    denominator that the chip's own read-only kernels beat is not a peak.
    The triad is kept as ``triad_calibration``.

    ``tensor_core.tf32``: gfx950 has no TF32 matrix type (xf32 was dropped
    after CDNA3); fp32 GEMMs run on the fp32 MFMA at the fp32 rate, so the
    tf32 entry -- the FP32 compute ceiling the reference's ``_compute_sol``
    reads -- carries the fp32 matrix peak and its calibration."""
    spec = SPECS[profile]
    best = max(hbm.values())
    src = "streaming read (non-temporal, one-shot blocks)" if "read" in hbm and hbm["read"] >= best else "STREAM Triad"
    lines = [
        f"# GPU Profile: {gpu_name}",
        "# Calibration: ezops_hbm_probe (STREAM probes over 2 GiB arrays) and ezops_mfma_probe",
        "# Written by: cd ez-ops_amd && python -m ezops.hardware",
        "#",
        "# Only store theoretical + calibration here.",
        "# effective = theoretical * calibration is computed by load_profile().",
        "",
        f"gpu: {gpu_name}",
        f"compute_capability: {spec['arch']}",
        "",
        f"sm_count: {spec['cu_count']}            # compute units",
        f"l2_cache_size: {spec['l2_cache_size']}       # {spec['l2_cache_size'] >> 20} MB per XCD",
        f"mall_size: {spec['mall_size']}       # {spec['mall_size'] >> 20} MB Infinity Cache",
        f"shared_memory_per_sm: {spec['lds_per_cu']}       # {spec['lds_per_cu'] >> 10} KB LDS",
        "",
        "hbm:",
        f"  theoretical: {_fmt(spec['hbm_bw_gb'], 9)}        # bytes/s, spec sheet",
        f"  calibration: {best / spec['hbm_bw_gb']:.3f}         # best sustained: {src}",
    ]
    if "triad" in hbm:
        lines.append(f"  triad_calibration: {hbm['triad'] / spec['hbm_bw_gb']:.3f}   # STREAM Triad")
    if "read" in hbm:
        lines.append(f"  read_calibration: {hbm['read'] / spec['hbm_bw_gb']:.3f}    # streaming read (non-temporal, one-shot blocks)")
    lines += ["", "tensor_core:"]
    entries = dict(spec["tensor_core_tflops"])
    entries["tf32"] = entries["fp32"]
    for dtype, theo in entries.items():
        meas = mfma_tflops.get("fp32" if dtype == "tf32" else dtype)
        note = "  (no TF32 type on gfx950: the fp32 MFMA peak)" if dtype == "tf32" else ""
        lines.append(f"  {dtype}:")
        lines.append(f"    theoretical: {_fmt(theo, 12)}     # FLOPS, spec sheet (dense){note}")
        if meas is not None:
            lines.append(f"    calibration: {meas / theo:.2f}")
        lines.append("")
    return "\n".join(lines)


def load_profile(name_or_path: str | Path = "mi355x") -> dict:
    """Parse a profile YAML and add effective peaks (theoretical * calibration)."""
    import yaml

    path = Path(name_or_path)
    if not path.suffix:
        path = ASSETS / f"{name_or_path}.yaml"
    prof = yaml.safe_load(path.read_text())
    hbm = prof["hbm"]
    hbm["effective"] = float(hbm["theoretical"]) * float(hbm.get("calibration", 1.0))
    for key in ("read", "triad"):
        if f"{key}_calibration" in hbm:
            hbm[f"{key}_effective"] = float(hbm["theoretical"]) * float(hbm[f"{key}_calibration"])
    for entry in prof.get("tensor_core", {}).values():
        entry["effective"] = float(entry["theoretical"]) * float(entry.get("calibration", 1.0))
    return prof


def compute_sol(roofline, profile: dict, input_bytes: int) -> dict | None:
    """Speed-of-light times of one op call (the reference benches' rule,
    benchmarks/bench_gemv.py:62-86): compute time at the calibrated tf32
    tensor-core rate (the fp32 MFMA peak on gfx950), memory time of the
    inputs at the calibrated HBM rate ("fused": the op reads each input
    once) and of every ``_ref_forward`` intermediate ("unfused"); the
    theoretical minimum is the larger of compute and fused memory.  None when
    the profile lacks an HBM or tf32 peak.  Times in µs, ``theo_min_s`` in s."""
    hbm = profile.get("hbm", {})
    tc = profile.get("tensor_core", {}).get("tf32")
    if not hbm.get("theoretical") or not tc or not tc.get("theoretical"):
        return None
    bw = float(hbm["theoretical"]) * float(hbm.get("calibration", 1.0))
    fl = float(tc["theoretical"]) * float(tc.get("calibration", 1.0))
    t_c, t_m = roofline.flops / fl, input_bytes / bw
    t_min = max(t_c, t_m)
    return {"compute_us": t_c * 1e6, "mem_fused_us": t_m * 1e6, "mem_unfused_us": roofline.bytes / bw * 1e6,
            "theo_min_us": t_min * 1e6, "theo_min_s": t_min}


def device_profile() -> dict | None:
    """The loaded profile of GPU 0 (None for a device without one)."""
    import torch

    props = torch.cuda.get_device_properties(0)
    key = detect_profile(props.name, getattr(props, "gcnArchName", ""))
    return load_profile(key) if key else None


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Generate the MI355X roofline profile YAML")
    ap.add_argument("--output-dir", default=str(ASSETS))
    ap.add_argument("--dtypes", default="bf16,fp32")
    args = ap.parse_args(argv)

    import torch

    props = torch.cuda.get_device_properties(0)
    profile = detect_profile(props.name, getattr(props, "gcnArchName", ""))
    if profile is None:
        print(f"unknown device {props.name!r}: only the MI355X profile is defined")
        return 2
    hbm = measure_hbm()
    print(f"HBM triad {hbm['triad']:.0f} GB/s, streaming read {hbm['read']:.0f} GB/s (calibration: the best)")
    mfma = {}
    for dtype in [d.strip() for d in args.dtypes.split(",") if d.strip()]:
        mfma[dtype] = measure_mfma(dtype)
        print(f"MFMA {dtype}: {mfma[dtype]:.0f} TFLOP/s")
        if dtype == "bf16":  # the larger tile shape can issue denser; keep the faster
            big = measure_mfma("bf16_32x32")
            print(f"MFMA bf16 32x32x16: {big:.0f} TFLOP/s")
            mfma[dtype] = max(mfma[dtype], big)
    text = generate_yaml(profile, SPECS[profile]["names"][0], hbm, mfma)
    out = Path(args.output_dir) / f"{profile}.yaml"
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(text + "\n")
    print(f"saved {out}")
    print(text)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
