"""Host-side API: registry, op validation, roofline counts, torch ``ref`` ops vs oracle (CPU)."""

import numpy as np
import pytest
import torch

import oracle
from ezops import (AttnDecodeOp, FusedOProjFfnOp, FusedQkNormRopeOp, GemvOp, PagedAttnDecodeOp, PrefillAttnOp, Qwen3DecodeStepOp, Qwen3PrefillOp,
                   Qwen3DenseDecodeOp,
                   ReduceOp, RmsNormOp, SoftmaxOp, get_kernel, list_backends, list_ops, register_kernel)
from ezops.ops.utils.accuracy import bitwise_equal, sqnr_db
from ezops.ops.utils.roofline import RooflineResult, measure_roofline

OPS = ["attn_decode", "fused_o_proj_ffn", "fused_qk_norm_rope", "gemv", "paged_attn_decode", "prefill_attn", "qwen3_decode_step", "qwen3_dense_decode", "qwen3_dense_prefill",
       "reduce", "rmsnorm", "softmax"]


def n(x):
    return x.float().numpy()


def test_registry_single_hip_backend():
    assert list_ops() == OPS
    for op in OPS:
        assert list_backends(op) == ["hip"]
        cls = get_kernel(op, "hip")
        assert cls.op_name == op and cls.backend == "hip"


def test_registry_errors():
    with pytest.raises(KeyError, match="Available backends for 'gemv': \\['hip'\\]"):
        get_kernel("gemv", "triton")
    with pytest.raises(ValueError, match="already registered"):
        register_kernel("gemv", "hip")(type("Dup", (), {}))


def test_validation_errors():
    with pytest.raises(ValueError, match="power of two"):
        FusedQkNormRopeOp(1, num_heads=16, head_dim=100, max_seq_len=128, position=0)
    with pytest.raises(ValueError, match="position"):
        FusedQkNormRopeOp(1, num_heads=16, head_dim=128, max_seq_len=128, position=128)
    with pytest.raises(ValueError, match="divisible"):
        FusedQkNormRopeOp(1, num_heads=16, head_dim=128, max_seq_len=128, position=0, num_kv_heads=6)
    with pytest.raises(ValueError, match="divisible"):
        Qwen3DenseDecodeOp(1, 128, num_heads=16, head_dim=128, hidden_size=2048, intermediate_size=6144,
                           num_kv_heads=6)
    with pytest.raises(ValueError, match="divisible"):
        AttnDecodeOp(1, 16, 128, 128, num_kv_heads=6)
    # tile divisibility is enforced by the backend kernel (reference test targets its own backend)
    with pytest.raises(ValueError, match="divisible"):
        FusedOProjFfnOp(1, hidden_size=2048, intermediate_size=6200, num_heads=16, head_dim=128, backend="hip")
    with pytest.raises(ValueError, match="seq_len"):
        Qwen3DenseDecodeOp(1, 0, 2048, 6144, 16, 128)
    with pytest.raises(ValueError, match="kv_lens"):
        Qwen3DenseDecodeOp(1, 16, 256, 512, 4, 64, kv_lens=[17])
    with pytest.raises(ValueError, match="head_dim"):
        AttnDecodeOp(1, 4, 16, 96, backend="hip")


def test_roofline_known_answers():
    a, b = torch.randn(32, 64), torch.randn(64, 128)
    r = measure_roofline(lambda x, y: x @ y, (a, b), {})
    assert r.flops == 2 * 32 * 64 * 128 and r.bytes == a.nbytes + b.nbytes + 32 * 128 * 4
    x = torch.randn(1024)
    r = measure_roofline(lambda u, v: u + v, (x, x), {})
    assert r.flops == 1024 and r.bytes == 3 * 4096
    assert RooflineResult(10, 0, 0).arithmetic_intensity == float("inf")
    # decode-path byte counts of the benchmark configs
    assert GemvOp(4096, 4096).get_roofline().bytes == 33_570_816
    assert AttnDecodeOp(32, 32, 8192, 128, num_kv_heads=8).get_roofline().bytes == 1_074_266_112
    assert SoftmaxOp(4096, 32768).get_roofline().bytes == 1_073_741_824
    assert ReduceOp(1 << 28).get_roofline().bytes == 1_073_741_828


def test_accuracy_helpers():
    a = torch.tensor([0.0, 1.0])
    assert bitwise_equal(a, a.clone()) and not bitwise_equal(a, torch.tensor([-0.0, 1.0]))
    assert sqnr_db(a, a) == float("inf")


# --- torch ``ref`` backend (the reference's _ref_forward semantics) vs the numpy oracle

def test_ref_gemv_rms_softmax_reduce():
    torch.manual_seed(0)
    op = GemvOp(64, 96)
    A, B, C = op.gen_data("cpu")
    op(A, B, C)
    np.testing.assert_allclose(n(C), oracle.gemv(n(A), n(B).T.copy()), rtol=1e-2, atol=1e-2)
    op = RmsNormOp(5, 100)
    X, O = op.gen_data("cpu")
    op(X, O)
    np.testing.assert_allclose(n(O), oracle.rmsnorm_f32(n(X)), rtol=1e-5, atol=1e-6)
    op = RmsNormOp(4, 256, dtype=torch.bfloat16, weighted=True)
    X, W, O = op.gen_data("cpu")
    op(X, W, O)
    np.testing.assert_allclose(n(O), oracle.rmsnorm_bf16(n(X), n(W)), rtol=1e-2, atol=2e-2)
    op = SoftmaxOp(3, 1000)
    X, O = op.gen_data("cpu")
    op(X, O)
    np.testing.assert_allclose(n(O), oracle.softmax(n(X)), rtol=1e-5, atol=1e-6)
    op = ReduceOp(10001)
    A, O = op.gen_data("cpu")
    op(A, O)
    assert op.check(O, torch.from_numpy(oracle.reduce_sum(n(A))))


def test_ref_attn_and_qk_rope():
    torch.manual_seed(1)
    op = AttnDecodeOp(2, 8, 40, 64, num_kv_heads=2)
    Q, K, V = op.gen_data("cpu")
    lens = torch.tensor([40, 17], dtype=torch.int32)
    out = op(Q, K, V, lens)
    ref = oracle.attn_decode(n(Q)[:, :, 0], n(K), n(V), lens.numpy())
    np.testing.assert_allclose(n(out)[:, :, 0], ref, rtol=1e-2, atol=1e-2)
    pop = PagedAttnDecodeOp(3, 8, 2, 64, page_size=32, max_pages=3, num_pages=11)
    Q, Kp, Vp, bt, lens = pop.gen_data("cpu")
    out = pop(Q, Kp, Vp, bt, lens)
    ref = oracle.paged_attn_decode(n(Q)[:, :, 0], n(Kp), n(Vp), bt.numpy(), lens.numpy(), 32)
    np.testing.assert_allclose(n(out)[:, :, 0], ref, rtol=1e-2, atol=1e-2)
    with pytest.raises(ValueError, match="power of two"):
        PagedAttnDecodeOp(1, 8, 2, 64, page_size=48, max_pages=2)
    op = FusedQkNormRopeOp(2, 8, 64, 50, position=[3, 49], num_kv_heads=2)
    data = op.gen_data("cpu")
    npy = [n(x) for x in data]
    qo, ko = op(*data)
    q2, k2, Kc, Vc = oracle.qk_norm_rope(*npy, positions=[3, 49])
    np.testing.assert_allclose(n(qo), q2, rtol=1e-2, atol=1e-2)
    np.testing.assert_allclose(n(ko), k2, rtol=1e-2, atol=1e-2)
    np.testing.assert_array_equal(n(data[8]), Vc)


def test_ref_fused_and_layer():
    torch.manual_seed(2)
    op = FusedOProjFfnOp(2, 128, 192, 4, 32)
    data = op.gen_data("cpu")
    out = op(*data)
    ref = oracle.o_proj_ffn(*[n(x) for x in data])
    assert op.check(out, torch.from_numpy(ref))
    op = Qwen3DenseDecodeOp(2, 24, 128, 192, 4, 32, num_kv_heads=2, kv_lens=[24, 9], norm_weights=True,
                            rope_theta=1e6)
    data = op.gen_data("cpu")
    npy = [n(x) for x in data]
    out = op(*data)
    ref, Kc, Vc = oracle.qwen3_layer(*npy[:7], 4, 2, 32, kv_lens=[24, 9], in_norm_w=npy[7], q_norm_w=npy[8],
                                     k_norm_w=npy[9], post_norm_w=npy[10], cos=npy[11], sin=npy[12])
    assert op.check(out, torch.from_numpy(ref))
    np.testing.assert_allclose(n(data[1]), Kc, rtol=1e-2, atol=1e-2)
    np.testing.assert_array_equal(n(data[2]), Vc)


def test_ref_layer_paged_cache():
    """Paged reference layer = oracle layer on the gathered cache; only the
    decoded token's rows change in the pools."""
    torch.manual_seed(3)
    op = Qwen3DenseDecodeOp(2, 64, 128, 192, 4, 32, num_kv_heads=2, kv_lens=[64, 33], norm_weights=True,
                            rope_theta=1e6, page_size=32, num_pages=7)
    data = op.gen_data("cpu")
    bt = data[-1]
    V0 = data[2].clone()
    npy = [n(x) for x in data[:-1]]
    Kc0 = oracle.paged_to_contiguous(npy[1], bt.numpy(), 32)
    Vc0 = oracle.paged_to_contiguous(npy[2], bt.numpy(), 32)
    out = op(*data)
    ref, Kc, Vc = oracle.qwen3_layer(npy[0], Kc0, Vc0, *npy[3:7], 4, 2, 32, kv_lens=[64, 33], in_norm_w=npy[7],
                                     q_norm_w=npy[8], k_norm_w=npy[9], post_norm_w=npy[10], cos=npy[11],
                                     sin=npy[12])
    assert op.check(out, torch.from_numpy(ref))
    np.testing.assert_allclose(oracle.paged_to_contiguous(n(data[1]), bt.numpy(), 32), Kc, rtol=1e-2, atol=1e-2)
    np.testing.assert_array_equal(oracle.paged_to_contiguous(n(data[2]), bt.numpy(), 32), Vc)
    changed = (data[2] != V0).any(dim=(1, 3)).nonzero().tolist()  # (page, row) pairs
    assert sorted(changed) == sorted([[int(bt[0, 1]), 31], [int(bt[1, 1]), 0]])
    with pytest.raises(ValueError, match="kv_lens"):
        Qwen3DenseDecodeOp(1, 64, 128, 192, 4, 32, page_size=32)
    with pytest.raises(ValueError, match="dividing"):
        Qwen3DenseDecodeOp(1, 80, 128, 192, 4, 32, kv_lens=[3], page_size=32)


@pytest.mark.parametrize("paged", [False, True])
def test_ref_decode_step_vs_oracle_chain(paged):
    """Multi-layer step = the oracle layer applied layer by layer, then the
    final RMSNorm and the LM head (bf16 staging of the normed state)."""
    torch.manual_seed(5)
    kw = dict(page_size=32, num_pages=9) if paged else {}
    op = Qwen3DecodeStepOp(2, 64, 128, 192, 4, 32, 3, num_kv_heads=2, vocab_size=50, kv_lens=[64, 40],
                           norm_weights=True, rope_theta=1e6, **kw)
    hidden, layers, cos, sin, fw, lm, bt = op.gen_data("cpu")
    npl = [[n(t) for t in layer] for layer in layers]
    h_ref = n(hidden)
    for L in npl:
        K, V = L[0], L[1]
        if paged:
            K, V = oracle.paged_to_contiguous(K, bt.numpy(), 32), oracle.paged_to_contiguous(V, bt.numpy(), 32)
        h_ref, _, _ = oracle.qwen3_layer(h_ref, K, V, *L[2:6], 4, 2, 32, kv_lens=[64, 40], in_norm_w=L[6],
                                         q_norm_w=L[7], k_norm_w=L[8], post_norm_w=L[9], cos=n(cos), sin=n(sin))
    logits_ref = oracle.linear_bf16(oracle.rmsnorm_bf16(h_ref, n(fw)), n(lm))
    h, logits = op(hidden, layers, cos, sin, fw, lm, bt)
    assert op.check(h, torch.from_numpy(h_ref))
    assert op.check(logits, torch.from_numpy(logits_ref))
    with pytest.raises(ValueError, match="num_layers"):
        Qwen3DecodeStepOp(1, 64, 128, 192, 4, 32, 0)


def test_ref_prefill_attn_vs_oracle():
    torch.manual_seed(6)
    op = PrefillAttnOp(2, 8, 2, 32, 64, q_lens=[9, 4], past_lens=[0, 30])
    Q, K, V = op.gen_data("cpu")
    out = op(Q, K, V)
    ref = oracle.prefill_attn(n(Q), n(K), n(V), [9, 4], [0, 30])
    np.testing.assert_allclose(n(out), ref, rtol=1e-2, atol=1e-2)
    with pytest.raises(ValueError, match="capacity"):
        PrefillAttnOp(1, 8, 2, 32, 64, q_lens=[40], past_lens=[30])


@pytest.mark.parametrize("paged", [False, True])
def test_ref_prefill_layer_vs_oracle(paged):
    torch.manual_seed(8)
    kw = dict(page_size=32, num_pages=5) if paged else {}
    op = Qwen3PrefillOp(2, 64, 128, 192, 4, 32, q_lens=[9, 3], past_lens=[0, 40], num_kv_heads=2,
                        norm_weights=True, rope_theta=1e6, **kw)
    data = op.gen_data("cpu")
    npy = [n(x) for x in data]
    K0, V0 = npy[1], npy[2]
    if paged:
        bt = data[-1].numpy()
        K0, V0 = oracle.paged_to_contiguous(K0, bt, 32), oracle.paged_to_contiguous(V0, bt, 32)
    out = op(*data)
    ref, Kc, Vc = oracle.qwen3_prefill(npy[0], K0, V0, *npy[3:7], 4, 2, 32, [9, 3], [0, 40], in_norm_w=npy[7],
                                       q_norm_w=npy[8], k_norm_w=npy[9], post_norm_w=npy[10], cos=npy[11],
                                       sin=npy[12])
    assert op.check(out, torch.from_numpy(ref))
    K1 = n(data[1]) if not paged else oracle.paged_to_contiguous(n(data[1]), bt, 32)
    np.testing.assert_allclose(K1, Kc, rtol=1e-2, atol=1e-2)


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus N > 1 (or a WORLD_SIZE > 1 launch)
    exits with status 2 and says why, before touching a device."""
    import os
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    for args, env in ((["--gpus", "2"], {}), ([], {"WORLD_SIZE": "2"})):
        r = subprocess.run([sys.executable, str(root / "bench.py"), *args, "--steps", "1", "--warmup", "0"],
                           capture_output=True, text=True, timeout=300, env={**os.environ, **env})
        assert r.returncode == 2, (r.returncode, r.stdout[-500:], r.stderr[-500:])
        assert "one GPU" in r.stdout + r.stderr
