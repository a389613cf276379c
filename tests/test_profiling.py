"""Profiling tooling on the CPU: wave-record export to Chrome/Perfetto JSON,
summaries, the rocprofv3 harness's script generation and CSV parsing, and
that the production library reports profiling as not compiled in."""

import json

import numpy as np
import pytest

from ezops import _hip, profiling


def records():
    r = np.zeros(4, dtype=profiling.RECORD_DTYPE)
    # kernel 1 on XCD 0 (SE 1, CU 3, SIMD 2) and XCD 5; kernel 5 on XCD 5
    hw = (1 << 13) | (3 << 8) | (2 << 4) | 7
    r["t0"] = [1000, 1100, 1200, 1500]
    r["t1"] = [1300, 1900, 1250, 2500]
    r["hw_id"] = [hw, hw, 0, 0]
    r["xcc_id"] = [0, 5, 5, 5]
    r["kernel"] = [1, 1, 5, 5]
    r["wave"] = [0, 1, 0, 3]
    r["block"] = [0, 0, 7, 9]
    return r


def test_record_layout_and_hw_id():
    assert profiling.RECORD_DTYPE.itemsize == 32
    f = profiling.decode_hw_id([(1 << 13) | (3 << 8) | (2 << 4) | 7])
    assert (int(f["se"][0]), int(f["cu"][0]), int(f["simd"][0]), int(f["slot"][0])) == (1, 3, 2, 7)


def test_chrome_trace_export(tmp_path):
    doc = profiling.chrome_trace(records())
    xs = [e for e in doc["traceEvents"] if e["ph"] == "X"]
    assert [e["name"] for e in xs] == ["gemv_rows", "gemv_rows", "attn_split", "attn_split"]
    assert xs[0]["ts"] == 0.0 and xs[0]["dur"] == 3.0  # 300 ticks of 10 ns
    assert xs[1]["pid"] == 5 and xs[3]["args"] == {"block": 9, "wave": 3, "slot": 0}
    assert xs[0]["tid"] == (1 * 2 + 0) * 64 + 3 * 4 + 2
    names = {e["args"]["name"] for e in doc["traceEvents"] if e["name"] == "process_name"}
    assert names == {"XCD 0", "XCD 5"}
    p = tmp_path / "t.json"
    p.write_text(json.dumps(doc))
    assert json.loads(p.read_text())["displayTimeUnit"] == "ns"


def test_summary():
    s = {k["kernel"]: k for k in profiling.summarize(records())}
    assert s["gemv_rows"]["waves"] == 2 and s["gemv_rows"]["span_us"] == 9.0
    assert s["gemv_rows"]["waves_per_xcd"] == {0: 1, 5: 1}
    assert s["gemv_rows"]["xcd_end_spread_us"] == 6.0
    assert s["attn_split"]["mean_wave_us"] == 5.25


def test_cli_helpers(tmp_path):
    assert profiling.parse_params("M=5,N=10") == ([], {"M": 5, "N": 10})
    assert profiling.parse_params("5,10,0.5") == ([5, 10, 0.5], {})
    src = profiling.run_script("gemv", [4096, 4096], {}, 2, 5)
    assert "GemvOp(4096, 4096, backend='hip')" in src and "range(5)" in src
    compile(src, "run", "exec")
    with pytest.raises(SystemExit):
        profiling.op_class("no_such_op")
    csv_path = tmp_path / "x_kernel_stats.csv"
    csv_path.write_text('"Name","Calls","TotalDurationNs","AverageNs","Percentage","MinNs","MaxNs","StdDev"\n'
                        '"k1",10,100000,10000,80.0,9000,12000,1.0\n"k2",10,25000,2500,20.0,2000,3000,1.0\n')
    rows = profiling.read_kernel_stats(csv_path)
    assert rows[0]["avg_us"] == 10.0 and rows[1]["calls"] == 10
    rep = profiling.sol_report(rows, 10, 50e6, 0, 8000.0, 2500.0)
    assert rep["kernel_us_per_call"] == 12.5 and rep["GBps"] == pytest.approx(4000.0) and rep["frac_hbm"] == pytest.approx(0.5)


def test_production_library_has_no_profiling():
    lib = _hip.lib()
    assert lib.ezops_profile_read(None, 0) == profiling_enosys()
    assert b"EZ_PROFILE" in lib.ezops_hip_last_error()
    assert lib.ezops_profile_reset() == profiling_enosys()


def profiling_enosys():
    return -38


def test_wave_trace_needs_the_profiling_build(tmp_path):
    with pytest.raises(RuntimeError, match="not found"):
        with profiling.WaveTrace(tmp_path / "missing.so"):
            pass
