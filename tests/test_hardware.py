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
    assert data["hbm"]["calibration"] == pytest.approx(5400 / 8000, abs=1e-3)
    assert data["tensor_core"]["bf16"]["calibration"] == pytest.approx(0.8)
    assert "calibration" not in data["tensor_core"]["fp8"]  # not measured: theoretical only
    p = tmp_path / "x.yaml"
    p.write_text(text)
    prof = hardware.load_profile(p)
    assert prof["hbm"]["effective"] == pytest.approx(5400e9, rel=1e-3)
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
