"""Hardware profile (reference: scripts/roofline_profile.py, assets/rtx_5060_ti.yaml)."""
import pytest
import yaml

from ezops import hardware


def test_detect_profile():
    assert hardware.detect_profile("AMD Instinct MI355X") == "mi355x"
    assert hardware.detect_profile("AMD Radeon Graphics", "gfx950:sramecc+:xnack-") == "mi355x"
    assert hardware.detect_profile("NVIDIA H100", "sm_90") is None


def test_yaml_roundtrip(tmp_path):
    text = hardware.generate_yaml("mi355x", "AMD Instinct MI355X", {"triad": 5400.0, "read": 6400.0},
                                  {"bf16": 2000.0})
    data = yaml.safe_load(text)
    assert float(data["hbm"]["theoretical"]) == pytest.approx(8000e9)
    assert data["hbm"]["calibration"] == pytest.approx(6400 / 8000, abs=1e-3)  # the best probe
    assert data["hbm"]["triad_calibration"] == pytest.approx(5400 / 8000, abs=1e-3)
    assert data["tensor_core"]["bf16"]["calibration"] == pytest.approx(0.8)
    assert "calibration" not in data["tensor_core"]["fp8"]  # not measured: theoretical only
    p = tmp_path / "x.yaml"
    p.write_text(text)
    prof = hardware.load_profile(p)
    assert prof["hbm"]["effective"] == pytest.approx(6400e9, rel=1e-3)
    assert prof["hbm"]["triad_effective"] == pytest.approx(5400e9, rel=1e-3)
    assert prof["hbm"]["read_effective"] == pytest.approx(6400e9, rel=1e-3)
    assert prof["tensor_core"]["bf16"]["effective"] == pytest.approx(2000e12, rel=1e-2)
    assert prof["tensor_core"]["fp8"]["effective"] == pytest.approx(5000e12)


def test_committed_profile_loads():
    prof = hardware.load_profile("mi355x")
    assert prof["compute_capability"] == "gfx950"
    assert 3000e9 < prof["hbm"]["effective"] < 8000e9
    assert 0 < prof["tensor_core"]["bf16"]["effective"] <= 2500e12


@pytest.mark.gpu
def test_probes_measure_plausible_peaks():
    hbm = hardware.measure_hbm(n_bytes_per_array=1 << 30, reps=3)
    assert 2000 < hbm["triad"] < 8000 and 2000 < hbm["read"] < 8000
    tf = hardware.measure_mfma("bf16", iters=1024, reps=3)
    assert 200 < tf < 2600, tf
    tf32 = hardware.measure_mfma("fp32", iters=1024, reps=3)
    assert 20 < tf32 < 160, tf32


def _compute_sol(roofline, profile, input_bytes):
    """Restatement of the reference benches' SOL rule (benchmarks/bench_gemv.py:62-86):
    None without an hbm and a tf32 tensor-core entry, else the compute time at
    the tf32 peak, the memory times at the calibrated HBM rate and their max."""
    hbm = profile.get("hbm", {})
    tc = profile.get("tensor_core", {}).get("tf32")
    if not hbm.get("theoretical") or not tc or not tc.get("theoretical"):
        return None
    eff_hbm = float(hbm["theoretical"]) * float(hbm.get("calibration", 1.0))
    eff_compute = float(tc["theoretical"]) * float(tc.get("calibration", 1.0))
    compute_t = roofline.flops / eff_compute
    mem_fused_t = input_bytes / eff_hbm
    return {"compute_us": compute_t * 1e6, "mem_fused_us": mem_fused_t * 1e6,
            "mem_unfused_us": roofline.bytes / eff_hbm * 1e6, "theo_min_us": max(compute_t, mem_fused_t) * 1e6}


def test_committed_profile_gives_reference_sol():
    """The reference's GEMV bench computes a SOL from this profile (it needs tf32)."""
    from ezops import GemvOp

    with open(hardware.ASSETS / "mi355x.yaml") as f:
        prof = yaml.safe_load(f)  # the reference benches read the raw YAML (bench_gemv.py:55-59)
    assert float(prof["tensor_core"]["tf32"]["theoretical"]) == pytest.approx(157.3e12)
    roof = GemvOp(4096, 4096).get_roofline()
    assert roof.bytes == 33_570_816 and roof.flops == 2 * 4096 * 4096
    sol = _compute_sol(roof, prof, 33_570_816)
    assert sol is not None
    eff = 8000e9 * float(prof["hbm"]["calibration"])
    assert sol["theo_min_us"] == pytest.approx(33_570_816 / eff * 1e6)  # HBM-bound: memory time wins
    assert sol["theo_min_us"] > sol["compute_us"]
    # the calibrated rate is the best measured one, never below the triad
    assert float(prof["hbm"]["calibration"]) >= float(prof["hbm"]["triad_calibration"])
