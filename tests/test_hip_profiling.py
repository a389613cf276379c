"""Wave-level timelines on the GPU: the profiling build gives bit-identical
results to the production library, and its records name the kernels each
op launches with sane times and placement."""

import json

import numpy as np
import pytest
import torch

from ezops import GemvOp, Qwen3DenseDecodeOp, Qwen3PrefillOp, profiling

pytestmark = pytest.mark.gpu
QWEN3_8B = dict(hidden_size=4096, intermediate_size=12288, num_heads=32, head_dim=128)


def check_records(rec, kernels):
    assert len(rec) > 0
    names = {profiling.KERNEL_NAMES[int(k)] for k in np.unique(rec["kernel"])}
    assert names == kernels, names
    assert (rec["t1"] >= rec["t0"]).all()
    assert ((rec["xcc_id"] & 0xF) < 8).all()
    span_us = (rec["t1"].max() - rec["t0"].min()) / profiling.TICKS_PER_US
    assert 0 < span_us < 1e6


def test_wave_trace_gemv():
    op = GemvOp(4096, 4096, backend="hip")
    A, B, C = op.gen_data()
    op(A, B, C)
    ref = C.clone()
    with profiling.WaveTrace() as tr:
        op(A, B, C)
    assert torch.equal(C, ref)
    check_records(tr.records, {"gemv_rows"})
    # 4 waves per block, blocks of 1 to 8 weight rows: every wave ran once
    assert len(tr.records) % 4 == 0 and 4096 // 8 * 4 <= len(tr.records) <= 4096 * 4
    assert len(np.unique(tr.records["block"])) * 4 == len(tr.records)


def test_wave_trace_decode_layer(tmp_path):
    op = Qwen3DenseDecodeOp(1, 4096, backend="hip", num_kv_heads=8, kv_lens=[3000], norm_weights=True,
                            rope_theta=1e6, **QWEN3_8B)
    data = op.gen_data()
    ref = op(*data).clone()
    with profiling.WaveTrace() as tr:
        out = op(*data)
    assert torch.equal(out, ref)
    check_records(tr.records, {"gemv_rows", "attn_split", "attn_combine"})
    doc = tr.chrome_trace(tmp_path / "layer.json")
    assert sum(e["ph"] == "X" for e in doc["traceEvents"]) == len(tr.records)
    assert json.loads((tmp_path / "layer.json").read_text())["traceEvents"]
    s = {k["kernel"]: k for k in tr.summary()}
    assert sum(s["gemv_rows"]["waves_per_xcd"].values()) == s["gemv_rows"]["waves"]


def test_wave_trace_prefill():
    op = Qwen3PrefillOp(2, 1024, q_lens=[300, 45], past_lens=[0, 100], backend="hip", num_kv_heads=8,
                        norm_weights=True, rope_theta=1e6, **QWEN3_8B)
    data = op.gen_data()
    K0, V0 = data[1].clone(), data[2].clone()
    ref = op(*data).clone()
    data = (data[0], K0, V0, *data[3:])
    with profiling.WaveTrace() as tr:
        out = op(*data)
    # the same kernels with the wave recorder compiled in: bit-identical results
    assert torch.equal(out, ref)
    # (SwiGLU runs in the gate/up GEMM's epilogue at Qwen3-8B's IS = 12288)
    check_records(tr.records, {"rmsnorm_bf16", "gemm", "qk_norm_rope", "prefill_attn"})
