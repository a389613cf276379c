"""Fused decode ops on HIP vs the numpy oracle (GPU).

Mirrors the reference's parity tests (tests/test_fused_qk_norm_rope.py:10-64,
tests/test_fused_o_proj_ffn.py:14-40, tests/test_qwen3_dense_decode.py:17-64)
with the oracle as the checker, plus the Qwen3-8B benchmark shapes.
"""

import numpy as np
import pytest
import torch

import oracle
from ezops import FusedOProjFfnOp, FusedQkNormRopeOp, Qwen3DenseDecodeOp, list_backends

pytestmark = pytest.mark.gpu
BF_TOL = dict(rtol=1e-2, atol=2e-2)


def assert_layer_bar(out, ref):
    """The elementwise bar on all but at most max(2, 1e-4 n) elements, every
    element within twice the bar: legitimate fp32 accumulation orders of the
    oracle already differ past the bar on single elements of the Qwen3-8B
    layer (tests/test_oracle.py::test_layer_bar_order_sensitivity)."""
    d = np.abs(out - ref)
    bar = BF_TOL["atol"] + BF_TOL["rtol"] * np.abs(ref)
    assert (d <= 2 * bar).all(), float((d - 2 * bar).max())
    assert int((d > bar).sum()) <= max(2, int(1e-4 * d.size)), int((d > bar).sum())

QWEN3_VL_2B_HEADS = dict(num_heads=16, head_dim=128, num_kv_heads=8)
QWEN3_VL_2B = dict(hidden_size=2048, intermediate_size=6144, num_heads=16, head_dim=128)
QWEN3_0_6B = dict(hidden_size=1024, intermediate_size=3072, num_heads=16, head_dim=128)
QWEN3_8B = dict(hidden_size=4096, intermediate_size=12288, num_heads=32, head_dim=128)


def n(x):
    return x.detach().float().cpu().numpy()


@pytest.mark.parametrize("batch,max_seq_len,position,num_kv_heads", [
    (1, 128, 0, 8), (1, 1024, 512, 8), (2, 1025, 1024, 8), (1, 4096, 1, 4), (1, 100, 50, 16), (1, 33, 17, 2),
    (4, 2048, [5, 2047, 0, 1000], 8),  # one position per sequence
])
def test_fused_qk_norm_rope(batch, max_seq_len, position, num_kv_heads):
    assert list_backends("fused_qk_norm_rope") == ["hip"]
    kw = {**QWEN3_VL_2B_HEADS, "num_kv_heads": num_kv_heads}
    torch.manual_seed(42)
    op = FusedQkNormRopeOp(batch, max_seq_len=max_seq_len, position=position, backend="hip", **kw)
    data = op.gen_data()
    K0, V0 = data[7].clone(), data[8].clone()
    q_out, k_out = op(*data)
    pos = np.broadcast_to(np.asarray(position), (batch,))
    rq, rk, rK, rV = oracle.qk_norm_rope(*[n(x) for x in data[:7]], n(K0), n(V0), pos)
    np.testing.assert_allclose(n(q_out), rq, **BF_TOL)
    np.testing.assert_allclose(n(k_out), rk, **BF_TOL)
    Kc, Vc = data[7], data[8]
    for b in range(batch):
        p = int(pos[b])
        np.testing.assert_allclose(n(Kc[b, :, p]), rk[b], **BF_TOL)
        assert torch.equal(Vc[b, :, p], data[2][b])
        mask = torch.ones(max_seq_len, dtype=torch.bool, device=Kc.device)
        mask[p] = False
        assert torch.equal(Kc[b][:, mask], K0[b][:, mask])
        assert torch.equal(Vc[b][:, mask], V0[b][:, mask])


@pytest.mark.parametrize("head_dim,num_kv_heads", [(32, 4), (64, 2), (256, 8)])
def test_fused_qk_norm_rope_head_dims(head_dim, num_kv_heads):
    """head_dim 64/256 take the 16-byte-lane kernel, 32 the one-pair-per-lane one."""
    torch.manual_seed(3)
    op = FusedQkNormRopeOp(3, num_heads=16, head_dim=head_dim, max_seq_len=300, position=[0, 299, 17],
                           num_kv_heads=num_kv_heads, backend="hip")
    data = op.gen_data()
    K0, V0 = data[7].clone(), data[8].clone()
    q_out, k_out = op(*data)
    rq, rk, rK, rV = oracle.qk_norm_rope(*[n(x) for x in data[:7]], n(K0), n(V0), np.array([0, 299, 17]))
    np.testing.assert_allclose(n(q_out), rq, **BF_TOL)
    np.testing.assert_allclose(n(k_out), rk, **BF_TOL)
    np.testing.assert_allclose(n(data[7]), rK, **BF_TOL)
    assert torch.equal(data[8].cpu().float(), torch.from_numpy(rV))


@pytest.mark.parametrize("batch,shape", [(1, QWEN3_VL_2B), (1, QWEN3_0_6B), (2, QWEN3_VL_2B), (4, QWEN3_VL_2B),
                                         (1, QWEN3_8B), (16, QWEN3_8B), (7, QWEN3_0_6B)])
def test_fused_o_proj_ffn(batch, shape):
    torch.manual_seed(42)
    op = FusedOProjFfnOp(batch, backend="hip", **shape)
    data = op.gen_data()
    out = op(*data)
    ref = torch.from_numpy(oracle.o_proj_ffn(*[n(x) for x in data])).to(out.device)
    assert op.check(out, ref), (out.float() - ref).norm().item() / ref.norm().item()
    np.testing.assert_allclose(n(out), n(ref), **BF_TOL)


def _misaligned(t):
    """The same values at an address 2 bytes past a 16-byte boundary."""
    buf = torch.empty(t.numel() + 8, dtype=t.dtype, device=t.device)
    v = buf[1:1 + t.numel()].view(t.shape)
    v.copy_(t)
    assert v.data_ptr() % 16 != 0
    return v


def _layer(batch, seq_len, kwargs, misalign=(), **mode):
    torch.manual_seed(42)
    op = Qwen3DenseDecodeOp(batch, seq_len, backend="hip", **kwargs, **mode)
    data = list(op.gen_data())
    for i in misalign:
        data[i] = _misaligned(data[i])
    K0, V0 = data[1].clone(), data[2].clone()
    out = op(*data)
    npy = [n(x) for x in data]
    extra = {}
    if mode.get("norm_weights"):
        extra.update(in_norm_w=npy[7], q_norm_w=npy[8], k_norm_w=npy[9], post_norm_w=npy[10])
    if mode.get("rope_theta"):
        extra.update(cos=npy[-2], sin=npy[-1])
    ref, rK, rV = oracle.qwen3_layer(npy[0], n(K0), n(V0), *npy[3:7], op.num_heads, op.num_kv_heads, op.head_dim,
                                     kv_lens=mode.get("kv_lens"), **extra)
    ref_t = torch.from_numpy(ref).to(out.device)
    assert op.check(out, ref_t), (out.float() - ref_t).norm().item() / ref_t.norm().item()
    assert_layer_bar(n(out), ref)
    Kc, Vc = data[1], data[2]
    for b, L in enumerate(op.lens()):
        np.testing.assert_allclose(n(Kc[b, :, L - 1]), rK[b, :, L - 1], **BF_TOL)
        np.testing.assert_allclose(n(Vc[b, :, L - 1]), rV[b, :, L - 1], **BF_TOL)
        mask = torch.ones(seq_len, dtype=torch.bool, device=Kc.device)
        mask[L - 1] = False
        assert torch.equal(Kc[b][:, mask], K0[b][:, mask])
        assert torch.equal(Vc[b][:, mask], V0[b][:, mask])


@pytest.mark.parametrize("batch,seq_len,num_kv_heads", [(1, 128, 8), (1, 1000, 8), (2, 1025, 8), (1, 4096, 4), (1, 1, 8),
                                                                    (2, 1000, 1)])
def test_qwen3_dense_decode_reference_mode(batch, seq_len, num_kv_heads):
    _layer(batch, seq_len, {**QWEN3_VL_2B, "num_kv_heads": num_kv_heads})


@pytest.mark.parametrize("batch,seq_len", [(1, 16384), (3, 2048), (4, 4096), (16, 4096)])
def test_qwen3_8b_layer_qwen3_mode(batch, seq_len):
    rng = np.random.default_rng(4)
    lens = rng.integers(min(1024, seq_len), seq_len + 1, size=batch).tolist()
    _layer(batch, seq_len, {**QWEN3_8B, "num_kv_heads": 8}, kv_lens=lens, norm_weights=True, rope_theta=1e6)


@pytest.mark.parametrize("misalign", [(4,), (5,), (6,), (4, 5, 6)])  # Wo, Wgu, Wd
def test_batched_layer_unaligned_weights(misalign):
    """At batch > 4 the stages pass activations on in the MFMA-packed layout
    only when the stages on both sides read it with 16-byte loads; an
    unaligned weight selects the row-major hand-off (the layer used to return
    EINVAL from a middle stage after the cache write)."""
    _layer(8, 512, {**QWEN3_0_6B, "num_kv_heads": 8}, misalign=misalign, kv_lens=[500, 17, 300, 512, 1, 64, 255, 400],
           norm_weights=True, rope_theta=1e6)


@pytest.mark.parametrize("misalign", [(2,), (4, 5), (6,)])  # Wo, Wg / Wu, Wd
def test_batched_o_proj_ffn_unaligned_weights(misalign):
    torch.manual_seed(42)
    op = FusedOProjFfnOp(16, backend="hip", **QWEN3_0_6B)
    data = list(op.gen_data())
    for i in misalign:
        data[i] = _misaligned(data[i])
    out = op(*data)
    ref = oracle.o_proj_ffn(*[n(x) for x in data])
    np.testing.assert_allclose(n(out), ref, **BF_TOL)


def test_qwen3_layer_repeated_calls():
    """Split partials and cache slots of one call never leak into the next:
    repeated calls with new hidden states stay correct."""
    torch.manual_seed(7)
    op = Qwen3DenseDecodeOp(1, 4096, backend="hip", kv_lens=[3000], norm_weights=True, rope_theta=1e6,
                            **QWEN3_8B, num_kv_heads=8)
    data = list(op.gen_data())
    npy = [n(x) for x in data]
    for it in range(4):
        data[0] = torch.randn_like(data[0], dtype=torch.float32).to(torch.bfloat16)
        npy[0] = n(data[0])
        out = op(*data)
        ref, _, _ = oracle.qwen3_layer(npy[0], npy[1], npy[2], *npy[3:7], 32, 8, 128, kv_lens=[3000],
                                       in_norm_w=npy[7], q_norm_w=npy[8], k_norm_w=npy[9], post_norm_w=npy[10],
                                       cos=npy[11], sin=npy[12])
        assert op.check(out, torch.from_numpy(ref).to(out.device)), it


@pytest.mark.parametrize("batch,kv_lens", [(1, [3000]), (4, [1, 31, 33, 2049])])
def test_qwen3_layer_ignores_rows_past_lengths(batch, kv_lens):
    """Cache rows past each sequence's length (the decoded token goes to row
    len - 1) are never read: NaN there leaves the output and the written
    rows bit-identical to a run over finite values."""
    torch.manual_seed(13)
    op = Qwen3DenseDecodeOp(batch, 4096, backend="hip", kv_lens=kv_lens, norm_weights=True, rope_theta=1e6,
                            **QWEN3_8B, num_kv_heads=8)
    data = list(op.gen_data())
    ref_K, ref_V = data[1].clone(), data[2].clone()
    out_ref = op(data[0], ref_K, ref_V, *data[3:])
    K, V = data[1].clone(), data[2].clone()
    for b, L in enumerate(kv_lens):
        K[b, :, L:] = float("nan")
        V[b, :, L:] = float("inf")
    out = op(data[0], K, V, *data[3:])
    assert torch.equal(out, out_ref)
    for b, L in enumerate(kv_lens):
        assert torch.equal(K[b, :, :L], ref_K[b, :, :L]) and torch.equal(V[b, :, :L], ref_V[b, :, :L])


@pytest.mark.parametrize("batch", [1, 16])
def test_qwen3_layer_graph_replays(batch):
    """The layer captured once in a HIP graph and replayed: every replay equals
    the eager result (split partials, merge counters and cache slots return to
    their start state within each call)."""
    torch.manual_seed(9)
    rng = np.random.default_rng(9)
    lens = rng.integers(1024, 4096 + 1, size=batch).tolist()
    op = Qwen3DenseDecodeOp(batch, 4096, backend="hip", kv_lens=lens, norm_weights=True, rope_theta=1e6,
                            **QWEN3_8B, num_kv_heads=8)
    data = op.gen_data()
    eager = op(*data).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        op(*data)  # warm the workspace on this stream
        g_ = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_, stream=s):
            out = op(*data)
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(4):
        g_.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        eager2 = op(*data)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(eager2, eager)
