"""HIP kernels vs the numpy oracle and the golden vectors (GPU).

Bars: bf16 outputs allclose(atol=2e-2, rtol=1e-2) against the fp32-accumulated
oracle; fp32 RMSNorm 1e-5; fp32 softmax atol 1e-6 /
rtol 1e-5; sum atol 1e-7 * n (reference ReduceOp tolerance).
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle
from ezops import AttnDecodeOp, GemvOp, ReduceOp, RmsNormOp, SoftmaxOp, _hip
from ezops.kernels.gemv.gemv_hip import linear
from ezops.ops.utils.accuracy import check_determinism, check_input_readonly

pytestmark = pytest.mark.gpu
BF_TOL = dict(rtol=1e-2, atol=2e-2)
DEV = "cuda"


def n(x):
    return x.detach().float().cpu().numpy()


def g(a, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(DEV)


@pytest.mark.parametrize("N,K", [(4096, 4096), (8, 16), (7, 100), (4096, 12288), (6144, 4096), (1, 8), (333, 1032),
                                 (4096, 2048), (2048, 1024), (6144, 2048), (1024, 3072), (2048, 6144)])
def test_gemv(N, K):
    """The reference's GEMV bench shape (4096 x 2048) and the Qwen3-0.6B /
    VL-2B projection widths among them; the reference op's own check too."""
    torch.manual_seed(0)
    op = GemvOp(N, K, backend="hip")
    A, B, C = op.gen_data()
    op(A, B, C)
    ref = oracle.gemv(n(A), n(B))
    np.testing.assert_allclose(n(C), ref, **BF_TOL)
    assert op.check(C, torch.from_numpy(ref).to(torch.bfloat16).to(DEV))
    assert check_determinism(op, (A, B), C) and check_input_readonly(op, (A, B), C)


@pytest.mark.parametrize("M", [2, 3, 4, 5, 8, 16, 17, 32])
@pytest.mark.parametrize("N,K", [(96, 256), (200, 1000), (64, 4096)])
def test_linear_batched(M, N, K):
    rng = np.random.default_rng(M * 1000 + N)
    X = oracle.bf16(rng.standard_normal((M, K)).astype(np.float32))
    W = oracle.bf16(rng.standard_normal((N, K)).astype(np.float32) * K ** -0.5)
    Y = linear(g(X), g(W))
    np.testing.assert_allclose(n(Y), oracle.linear_bf16(X, W), **BF_TOL)


@pytest.mark.parametrize("batch,dim", [(1, 64), (128, 1024), (3, 100), (7, 4097), (4096, 4096), (2, 40000)])
def test_rmsnorm_f32(batch, dim):
    torch.manual_seed(42)
    op = RmsNormOp(batch, dim, backend="hip")
    X, Out = op.gen_data()
    op(X, Out)
    ref = torch.from_numpy(oracle.rmsnorm_f32(n(X))).to(DEV)
    assert op.check(Out, ref), (Out - ref).abs().max().item()
    assert check_determinism(op, (X,), Out) and check_input_readonly(op, (X,), Out)


def test_rmsnorm_f32_custom_eps():
    torch.manual_seed(42)
    op = RmsNormOp(64, 1024, backend="hip", eps=1e-5)
    X, Out = op.gen_data()
    op(X, Out)
    assert op.check(Out, torch.from_numpy(oracle.rmsnorm_f32(n(X), 1e-5)).to(DEV))


@pytest.mark.parametrize("batch,dim", [(64, 4096), (3, 100), (5, 40000), (1, 8)])
def test_rmsnorm_bf16_weighted(batch, dim):
    torch.manual_seed(1)
    op = RmsNormOp(batch, dim, backend="hip", dtype=torch.bfloat16, weighted=True)
    X, W, Out = op.gen_data()
    op(X, W, Out)
    np.testing.assert_allclose(n(Out), oracle.rmsnorm_bf16(n(X), n(W)), **BF_TOL)
    assert check_determinism(op, (X, W), Out) and check_input_readonly(op, (X, W), Out)


@pytest.mark.parametrize("batch,dim", [(1, 64), (128, 1024), (3, 100), (7, 4097), (64, 32768), (2, 40000)])
def test_softmax(batch, dim):
    torch.manual_seed(42)
    op = SoftmaxOp(batch, dim, backend="hip")
    X, Out = op.gen_data()
    X.mul_(3)
    op(X, Out)
    ref = torch.from_numpy(oracle.softmax(n(X))).to(DEV)
    assert op.check(Out, ref), (Out - ref).abs().max().item()
    assert check_determinism(op, (X,), Out) and check_input_readonly(op, (X,), Out)


@pytest.mark.parametrize("size", [1, 37, 1000, (1 << 20) + 3, 1 << 24])
def test_reduce(size):
    torch.manual_seed(3)
    op = ReduceOp(size, backend="hip")
    A, Out = op.gen_data()
    op(A, Out)
    ref = torch.from_numpy(oracle.reduce_sum(n(A))).to(DEV)
    assert op.check(Out, ref), (Out.item(), ref.item())
    assert check_determinism(op, (A,), Out) and check_input_readonly(op, (A,), Out)


def test_reduce_shared_workspace_across_lengths():
    """One workspace serves calls of different lengths through the C ABI: the
    arrival counter sits at a fixed offset, so a short call after a long one
    (different block counts) still finds it at zero."""
    n_big, n_small = 1 << 24, 8192 * 10
    ws_bytes = _hip.size("ezops_reduce_sum_workspace_size", n_big)
    assert ws_bytes >= _hip.size("ezops_reduce_sum_workspace_size", n_small)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(5)
    for size in (n_big, n_small, n_big, 1):
        A = torch.rand(size, generator=gen, device=DEV) * 2 - 1
        out = torch.full((1,), float("nan"), device=DEV)
        _hip.call("ezops_reduce_sum_f32", A.data_ptr(), out.data_ptr(), size, ws.data_ptr(), ws_bytes,
                  _hip.stream())
        torch.cuda.synchronize()
        assert abs(out.item() - oracle.reduce_sum(n(A))[0]) <= 1e-7 * size, (size, out.item())


def test_reduce_unaligned_view():
    base = torch.rand(4097, device=DEV) * 2 - 1
    A = base[1:]  # 4-byte offset: scalar path
    op = ReduceOp(4096, backend="hip")
    Out = torch.empty(1, device=DEV)
    op(A, Out)
    assert abs(Out.item() - oracle.reduce_sum(n(A))[0]) <= 1e-7 * 4096


@pytest.mark.parametrize("B,H,Hkv,S,D,ragged", [
    (2, 8, 2, 1, 128, False),      # cache of one slot
    (1, 32, 8, 1000, 128, False),  # Qwen3-8B heads, non multiple of the tile
    (2, 16, 8, 1025, 128, False),
    (3, 8, 8, 300, 64, False),     # MHA, head_dim 64
    (2, 32, 4, 4097, 128, False),  # group 8
    (1, 16, 1, 32768, 128, False), # group 16: one kv head for 16 query heads (all MFMA columns live)
    (3, 32, 2, 1500, 64, True),    # group 16, head_dim 64, ragged
    (4, 32, 8, 8192, 128, True),   # ragged lengths
    (3, 16, 8, 700, 64, True),
])
def test_attn_decode(B, H, Hkv, S, D, ragged):
    torch.manual_seed(2)
    op = AttnDecodeOp(B, H, S, D, backend="hip", num_kv_heads=Hkv)
    Q, K, V = op.gen_data()
    lens = None
    if ragged:
        lens = torch.randint(1, S + 1, (B,), dtype=torch.int32)
        lens[0] = S
        lens = lens.to(DEV)
    out = op(Q, K, V, lens)
    ref = oracle.attn_decode(n(Q)[:, :, 0], n(K), n(V), None if lens is None else n(lens).astype(np.int64))
    np.testing.assert_allclose(n(out)[:, :, 0], ref, **BF_TOL)
    out2 = op(Q, K, V, lens)  # counters were reset: a second call is identical
    assert torch.equal(out, out2)


@pytest.mark.parametrize("H,Hkv,D", [(32, 8, 128), (16, 16, 64), (32, 4, 128), (16, 1, 128)])
def test_attn_decode_tile_residues_and_nonfinite_tail(H, Hkv, D):
    """Every length residue modulo the 32-position tile (1, 31, 33, ...), with
    NaN / Inf in every cache row at or past the length: those rows are never
    read (tile rows past the length are clamped to the last live row), so the
    result matches the oracle over the live rows."""
    B, S = 8, 160
    op = AttnDecodeOp(B, H, S, D, backend="hip", num_kv_heads=Hkv)
    torch.manual_seed(29)
    Q, K, V = op.gen_data()
    nK, nV = n(K).copy(), n(V).copy()
    for start in (1, 9, 17, 25):
        lens = torch.tensor([start + 4 * b for b in range(B)], dtype=torch.int32)
        lens[-1] = 1
        Kg, Vg = K.clone(), V.clone()
        for b, L in enumerate(lens.tolist()):
            Kg[b, :, L:] = float("nan")
            Vg[b, :, L:] = float("inf")
        out = op(Q, Kg, Vg, lens.to(DEV))
        ref = oracle.attn_decode(n(Q)[:, :, 0], nK, nV, lens.numpy().astype(np.int64))
        assert torch.isfinite(out).all()
        np.testing.assert_allclose(n(out)[:, :, 0], ref, **BF_TOL)


@pytest.mark.parametrize("B,S,bound", [(1, 16384, "max"), (3, 4096, "max"), (4, 8192, "cut"), (2, 3000, "over")])
def test_attn_decode_max_kv_len(B, S, bound):
    """max_kv_len plans the grid on the caller's length bound; lengths above
    it are cut to it, a bound above the capacity means the capacity."""
    torch.manual_seed(3)
    op = AttnDecodeOp(B, 32, S, 128, backend="hip", num_kv_heads=8)
    Q, K, V = op.gen_data()
    lens = torch.randint(S // 8, S + 1, (B,), dtype=torch.int32)
    hint = {"max": int(lens.max()), "cut": int(lens.float().mean()), "over": 2 * S}[bound]
    out = op._kernel(Q, K, V, lens.to(DEV), max_kv_len=hint)
    eff = np.minimum(lens.numpy().astype(np.int64), min(hint, S))
    ref = oracle.attn_decode(n(Q)[:, :, 0], n(K), n(V), eff)
    np.testing.assert_allclose(n(out)[:, :, 0], ref, **BF_TOL)
    with pytest.raises(ValueError):
        op._kernel(Q, K, V, lens.to(DEV), max_kv_len=-1)


@pytest.mark.parametrize("B,S", [(1, 16384), (8, 4096)])
def test_attn_decode_consecutive_calls_fresh_partials(B, S):
    """Split partials are handed between blocks through device-coherent
    accesses; consecutive calls with new inputs must never see the previous
    call's partials."""
    op = AttnDecodeOp(B, 32, S, 128, backend="hip", num_kv_heads=8)
    torch.manual_seed(11)
    Q, K, V = op.gen_data()
    lens = torch.randint(S // 2, S + 1, (B,), dtype=torch.int32).to(DEV)
    nK, nV = n(K), n(V)
    for it in range(4):
        Q = torch.randn_like(Q, dtype=torch.float32).mul_(1 + it).to(torch.bfloat16)
        out = op(Q, K, V, lens)
        ref = oracle.attn_decode(n(Q)[:, :, 0], nK, nV, n(lens).astype(np.int64))
        np.testing.assert_allclose(n(out)[:, :, 0], ref, **BF_TOL)


def test_attn_decode_ragged_splits_follow_lengths():
    """Ragged batches get splits in proportion to each sequence's length;
    consecutive calls whose lengths shrink leave stale partials of the
    previous call in the unused split slots, which must never be merged."""
    B, S = 12, 8192
    op = AttnDecodeOp(B, 32, S, 128, backend="hip", num_kv_heads=8)
    torch.manual_seed(21)
    Q, K, V = op.gen_data()
    nK, nV = n(K), n(V)
    rng = np.random.default_rng(21)
    for it, hi in enumerate([S, S // 2, 600, S]):
        lens = torch.from_numpy(rng.integers(1, hi + 1, size=B).astype(np.int32))
        lens[it % B] = hi
        out = op._kernel(Q, K, V, lens.to(DEV), max_kv_len=S)
        ref = oracle.attn_decode(n(Q)[:, :, 0], nK, nV, lens.numpy().astype(np.int64))
        np.testing.assert_allclose(n(out)[:, :, 0], ref, **BF_TOL)


def test_reduce_consecutive_calls():
    op = ReduceOp(1 << 22, backend="hip")
    Out = torch.empty(1, device=DEV)
    for it in range(4):
        A = (torch.rand(1 << 22, device=DEV) * 2 - 1) * (it + 1)
        op(A, Out)
        assert abs(Out.item() - oracle.reduce_sum(n(A))[0]) <= 1e-7 * (1 << 22)


def test_attn_decode_stream_and_graph():
    torch.manual_seed(5)
    op = AttnDecodeOp(2, 32, 2048, 128, backend="hip", num_kv_heads=8)
    Q, K, V = op.gen_data()
    eager = op(Q, K, V)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        g_ = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_, stream=s):
            out = op(Q, K, V)
    for _ in range(3):
        g_.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


# ---- golden vectors through the C ABI
def test_golden_gemv_rms_softmax_reduce(golden):
    x, W = golden["gemv_x"], golden["gemv_W"]
    C = torch.empty(W.shape[0], dtype=torch.bfloat16, device=DEV)
    GemvOp(*W.shape, backend="hip")(g(x), g(W), C)
    np.testing.assert_allclose(n(C), golden["gemv_y"], **BF_TOL)
    X = g(golden["rms32_X"], torch.float32)
    O = torch.empty_like(X)
    RmsNormOp(*X.shape, backend="hip")(X, O)
    np.testing.assert_allclose(n(O), golden["rms32_out"], rtol=1e-5, atol=1e-6)
    X, w = g(golden["rmsbf_X"]), g(golden["rmsbf_w"])
    O = torch.empty_like(X)
    RmsNormOp(*X.shape, backend="hip", dtype=torch.bfloat16, weighted=True)(X, w, O)
    np.testing.assert_allclose(n(O), golden["rmsbf_out"], **BF_TOL)
    X = g(golden["softmax_X"], torch.float32)
    O = torch.empty_like(X)
    SoftmaxOp(*X.shape, backend="hip")(X, O)
    np.testing.assert_allclose(n(O), golden["softmax_out"], rtol=1e-5, atol=1e-6)
    A = g(golden["reduce_A"], torch.float32)
    O = torch.empty(1, device=DEV)
    ReduceOp(A.numel(), backend="hip")(A, O)
    np.testing.assert_allclose(n(O), golden["reduce_out"], atol=1e-7 * A.numel())


def test_golden_o_proj_ffn_through_abi(golden):
    gd = golden
    attn, res = g(gd["ffn_attn"]), g(gd["ffn_res"])
    Wo, w, Wg, Wu, Wd = (g(gd[k]) for k in ("ffn_Wo", "ffn_w", "ffn_Wg", "ffn_Wu", "ffn_Wd"))
    B, QR = attn.shape
    HS, IS = Wo.shape[0], Wg.shape[0]
    out = torch.empty(B, HS, dtype=torch.bfloat16, device=DEV)
    ws = torch.zeros(_hip.size("ezops_o_proj_ffn_workspace_size", B, HS, IS, QR), dtype=torch.uint8, device=DEV)
    _hip.call("ezops_o_proj_ffn_bf16", attn.data_ptr(), res.data_ptr(), Wo.data_ptr(), w.data_ptr(), Wg.data_ptr(),
              Wu.data_ptr(), Wd.data_ptr(), out.data_ptr(), B, HS, IS, QR, 1e-6, ws.data_ptr(), ws.numel(),
              _hip.stream())
    np.testing.assert_allclose(n(out), gd["ffn_out"], **BF_TOL)


def test_golden_qk_norm_rope_through_abi(golden):
    gd = golden
    q, k, v = g(gd["rope_q"]), g(gd["rope_k"]), g(gd["rope_v"])
    B, H, D = q.shape
    Hkv, S = k.shape[1], gd["rope_cos"].shape[0]
    Kc, Vc = g(gd["rope_Kc"]), g(gd["rope_Vc"])
    qo = torch.empty_like(q)
    ko = torch.empty_like(k)
    pos = torch.from_numpy(gd["rope_pos"]).to(DEV)
    # keep every operand referenced until the kernel has run
    qw, kw, cos, sin = (g(gd[k_]) for k_ in ("rope_qw", "rope_kw", "rope_cos", "rope_sin"))
    _hip.call("ezops_qk_norm_rope_bf16", q.data_ptr(), H * D, k.data_ptr(), Hkv * D, v.data_ptr(), Hkv * D,
              qw.data_ptr(), kw.data_ptr(), cos.data_ptr(), sin.data_ptr(), Kc.data_ptr(), Vc.data_ptr(),
              qo.data_ptr(), ko.data_ptr(),
              B, H, Hkv, D, S, 0, pos.data_ptr(), 0, 1e-6, _hip.stream())
    torch.cuda.synchronize()
    np.testing.assert_allclose(n(qo), gd["rope_qout"], **BF_TOL)
    np.testing.assert_allclose(n(ko), gd["rope_kout"], **BF_TOL)
    for b, p in enumerate(gd["rope_pos"]):
        np.testing.assert_array_equal(n(Vc)[b, :, p], gd["rope_v"][b])
        np.testing.assert_array_equal(n(Kc)[b, :, p], n(ko)[b])


@pytest.mark.parametrize("M", [1, 3, 8, 16, 20])
@pytest.mark.parametrize("epi", [0, 1, 2, 3])
@pytest.mark.parametrize("norm", [0, 1])
@pytest.mark.parametrize("N,K", [(192, 512), (200, 1032), (200, 4096)])
def test_linear_stage_epilogues(M, epi, norm, N, K):
    """ezops_linear_stage_bf16: RMSNorm prologue x epilogues, VALU (M <= 4; K = 4096 takes the
    row-block kernel, one weight row per block at this N) and MFMA (M > 4) paths, with partial
    weight tiles, partial K chunks and partial batch blocks."""
    rng = np.random.default_rng(100 * M + 10 * epi + norm + K)
    X = oracle.bf16(rng.standard_normal((M, K)).astype(np.float32))
    W = oracle.bf16(rng.standard_normal((N, K)).astype(np.float32) * K ** -0.5)
    W2 = oracle.bf16(rng.standard_normal((N, K)).astype(np.float32) * K ** -0.5)
    R = oracle.bf16(rng.standard_normal((M, N)).astype(np.float32))
    w = oracle.bf16(rng.standard_normal(K).astype(np.float32) * 0.1 + 1)
    Xn = oracle.rmsnorm_bf16(X, w) if norm else X
    g_ = oracle.linear_bf16(Xn, W)
    if epi == 0:
        ref = g_
    elif epi == 1:
        ref = oracle.bf16(R + g_)
    elif epi == 2:
        u = oracle.linear_bf16(Xn, W2)
        ref = oracle.bf16(oracle.bf16(g_ / (1 + np.exp(-g_.astype(np.float64)))) * u)
    else:
        ref = Xn @ W.T
    tX, tW, tW2, tR, tw = g(X), g(W), g(W2), g(R), g(w)
    Y = torch.empty(M, N, dtype=torch.float32 if epi == 3 else torch.bfloat16, device=DEV)
    ws = torch.zeros(max(256, _hip.size("ezops_linear_stage_workspace_size", M, K, norm)), dtype=torch.uint8,
                     device=DEV)
    _hip.call("ezops_linear_stage_bf16", tX.data_ptr(), K, tW.data_ptr(), tW2.data_ptr(), Y.data_ptr(), N,
              tR.data_ptr(), N, tw.data_ptr(), norm, 1e-6, epi, M, N, K, ws.data_ptr(), ws.numel(), _hip.stream())
    np.testing.assert_allclose(n(Y), ref, **BF_TOL)


def _stage_ref(X, W, W2, R, w, norm, epi):
    Xn = oracle.rmsnorm_bf16(X, w) if norm else X
    g_ = oracle.linear_bf16(Xn, W)
    if epi == 0:
        return g_
    if epi == 1:
        return oracle.bf16(R + g_)
    u = oracle.linear_bf16(Xn, W2)
    return oracle.bf16(oracle.bf16(g_ / (1 + np.exp(-g_.astype(np.float64)))) * u)


@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("K", [64, 520, 1024, 2048, 3072, 6144, 16384, 16392])
@pytest.mark.parametrize("epi,norm", [(0, 0), (1, 0), (2, 1), (0, 1)])
def test_gemv_rows_widths(M, K, epi, norm):
    """M <= 4 at every row width class: 64- and 128-thread row groups (K <=
    1024), 256-thread groups with 1-8 chunks per thread and a masked last
    chunk (520, 3072), and past 16384 the wave-per-row kernel; with the
    RMSNorm prologue staged in bf16 as the reference stages it.  N = 203
    leaves the last row group partly empty."""
    N = 203
    rng = np.random.default_rng(7 * M + K + 13 * epi + norm)
    X = oracle.bf16(rng.standard_normal((M, K)).astype(np.float32))
    W = oracle.bf16(rng.standard_normal((N, K)).astype(np.float32) * K ** -0.5)
    W2 = oracle.bf16(rng.standard_normal((N, K)).astype(np.float32) * K ** -0.5)
    R = oracle.bf16(rng.standard_normal((M, N)).astype(np.float32))
    w = oracle.bf16(rng.standard_normal(K).astype(np.float32) * 0.1 + 1)
    ref = _stage_ref(X, W, W2, R, w, norm, epi)
    Y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
    ws = torch.zeros(256, dtype=torch.uint8, device=DEV)
    tX, tW, tW2, tR, tw = g(X), g(W), g(W2), g(R), g(w)  # held until the kernel has run
    _hip.call("ezops_linear_stage_bf16", tX.data_ptr(), K, tW.data_ptr(), tW2.data_ptr(), Y.data_ptr(), N,
              tR.data_ptr(), N, tw.data_ptr(), norm, 1e-6, epi, M, N, K, ws.data_ptr(), ws.numel(), _hip.stream())
    np.testing.assert_allclose(n(Y), ref, **BF_TOL)


@pytest.mark.parametrize("M,N", [(16, 12288), (20, 8192), (8, 12288)])
def test_linear_stage_swiglu_multi_tile(M, N):
    """Gate/up shapes whose 16-row tiles are 3x / 2x the CU count run as
    multi-tile blocks (the DMA ring continues across tiles): bit-exact with
    the one-tile-per-block launch on the same rows, and against the oracle."""
    K = 4096
    rng = np.random.default_rng(M + N)
    X = oracle.bf16(rng.standard_normal((M, K)).astype(np.float32))
    W = oracle.bf16(rng.standard_normal((N, K)).astype(np.float32) * K ** -0.5)
    W2 = oracle.bf16(rng.standard_normal((N, K)).astype(np.float32) * K ** -0.5)
    g_, u = oracle.linear_bf16(X, W), oracle.linear_bf16(X, W2)
    ref = oracle.bf16(oracle.bf16(g_ / (1 + np.exp(-g_.astype(np.float64)))) * u)
    tX, tW, tW2 = g(X), g(W), g(W2)
    ws = torch.zeros(256, dtype=torch.uint8, device=DEV)

    def run(rows):  # the first `rows` output rows through ezops_linear_stage_bf16 (SwiGLU epilogue)
        Y = torch.empty(M, rows, dtype=torch.bfloat16, device=DEV)
        _hip.call("ezops_linear_stage_bf16", tX.data_ptr(), K, tW.data_ptr(), tW2.data_ptr(), Y.data_ptr(), rows,
                  None, 0, None, 0, 1e-6, 2, M, rows, K, ws.data_ptr(), ws.numel(), _hip.stream())
        return Y

    Y = run(N)
    np.testing.assert_allclose(n(Y), ref, **BF_TOL)
    # N - 16 rows: not a multiple of the CU count, so one tile per block
    assert torch.equal(Y[:, : N - 16], run(N - 16))


@pytest.mark.parametrize("M", [5, 16, 20])
@pytest.mark.parametrize("extra,K", [(2048, 4096), (2048, 1032), (904, 4096), (8, 512)])
@pytest.mark.parametrize("epi", [0, 1, 3])
def test_linear_stage_24_row_blocks(M, extra, K, epi):
    """M <= 16 with 16 < N / CUs <= 24 (QKV at B=16: 6144 rows over 256
    CUs) runs one block of 16 + 8 rows per CU, the two MFMA tiles sharing
    each X fragment; N = 16 * CUs + extra covers the full case (extra =
    8 * CUs), a partial last block and a block whose second tile is empty.
    M = 20 takes the 16-row tiles (two batch blocks) for comparison."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    N = 16 * cus + (extra if extra < 2048 else 8 * cus)
    rng = np.random.default_rng(M + N + K + epi)
    X = oracle.bf16(rng.standard_normal((M, K)).astype(np.float32))
    W = oracle.bf16(rng.standard_normal((N, K)).astype(np.float32) * K ** -0.5)
    R = oracle.bf16(rng.standard_normal((M, N)).astype(np.float32))
    g_ = oracle.linear_bf16(X, W)
    ref = {0: g_, 1: oracle.bf16(R + g_), 3: X @ W.T}[epi]
    tX, tW, tR = g(X), g(W), g(R)
    Y = torch.full((M, N), float("nan"), dtype=torch.float32 if epi == 3 else torch.bfloat16, device=DEV)
    ws = torch.zeros(256, dtype=torch.uint8, device=DEV)
    _hip.call("ezops_linear_stage_bf16", tX.data_ptr(), K, tW.data_ptr(), None, Y.data_ptr(), N,
              tR.data_ptr(), N, None, 0, 1e-6, epi, M, N, K, ws.data_ptr(), ws.numel(), _hip.stream())
    torch.cuda.synchronize()
    if epi == 3:
        np.testing.assert_allclose(n(Y), ref, rtol=1e-3, atol=1e-3)
    else:
        np.testing.assert_allclose(n(Y), ref, **BF_TOL)


@pytest.mark.parametrize("M,extra,epi", [(16, 37, 0), (5, 0, 1), (20, 1000, 3), (16, 8192, 1)])
def test_linear_stage_streaming_blocks(M, extra, epi):
    """At least four 16-row tiles per CU and K = 4096 (an LM head at batch
    > 4): two streaming blocks per CU walk the tiles with one DMA ring;
    ragged last tiles, partial batch blocks and every store form."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    N, K = 4 * 16 * cus + extra, 4096
    rng = np.random.default_rng(M + N + epi)
    X = oracle.bf16(rng.standard_normal((M, K)).astype(np.float32))
    W = oracle.bf16(rng.standard_normal((N, K)).astype(np.float32) * K ** -0.5)
    R = oracle.bf16(rng.standard_normal((M, N)).astype(np.float32))
    g_ = oracle.linear_bf16(X, W)
    ref = {0: g_, 1: oracle.bf16(R + g_), 3: X @ W.T}[epi]
    tX, tW, tR = g(X), g(W), g(R)
    Y = torch.full((M, N), float("nan"), dtype=torch.float32 if epi == 3 else torch.bfloat16, device=DEV)
    ws = torch.zeros(256, dtype=torch.uint8, device=DEV)
    for _ in range(2):  # the second call on the same output: bitwise the same
        _hip.call("ezops_linear_stage_bf16", tX.data_ptr(), K, tW.data_ptr(), None, Y.data_ptr(), N,
                  tR.data_ptr(), N, None, 0, 1e-6, epi, M, N, K, ws.data_ptr(), ws.numel(), _hip.stream())
        torch.cuda.synchronize()
        if epi == 3:
            np.testing.assert_allclose(n(Y), ref, rtol=1e-3, atol=1e-3)
        else:
            np.testing.assert_allclose(n(Y), ref, **BF_TOL)


@pytest.mark.parametrize("M", [5, 16, 20])
@pytest.mark.parametrize("shape", ["gate_up3", "gate_up2", "qkv24", "tiles"])
def test_linear_stage_norm_in_kernel(M, shape):
    """Batched stages with the RMSNorm prologue at K = 4096 normalise inside
    the X-stationary kernel (no staging pass): gate/up with 3 and 2 tiles per
    CU (multi-tile blocks), the 24-row QKV blocks, and a few 16-row tiles;
    M = 20 spans two batch blocks (multi-tile and one-tile shapes)."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    K = 4096
    N, epi = {"gate_up3": (48 * cus, 2), "gate_up2": (32 * cus, 2), "qkv24": (24 * cus, 0), "tiles": (200, 1)}[shape]
    if shape == "qkv24" and M > 16:
        N = 16 * cus // 2  # M > 16 has no 24-row blocks; one tile per CU at most
    rng = np.random.default_rng(M + N)
    X = oracle.bf16(rng.standard_normal((M, K)).astype(np.float32) * 2)
    W = oracle.bf16(rng.standard_normal((N, K)).astype(np.float32) * K ** -0.5)
    W2 = oracle.bf16(rng.standard_normal((N, K)).astype(np.float32) * K ** -0.5)
    R = oracle.bf16(rng.standard_normal((M, N)).astype(np.float32))
    w = oracle.bf16(rng.standard_normal(K).astype(np.float32) * 0.1 + 1)
    ref = _stage_ref(X, W, W2, R, w, 1, epi)
    tX, tW, tW2, tR, tw = g(X), g(W), g(W2), g(R), g(w)
    Y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
    ws = torch.zeros(_hip.size("ezops_linear_stage_workspace_size", M, K, 1), dtype=torch.uint8, device=DEV)
    _hip.call("ezops_linear_stage_bf16", tX.data_ptr(), K, tW.data_ptr(), tW2.data_ptr(), Y.data_ptr(), N,
              tR.data_ptr(), N, tw.data_ptr(), 1, 1e-6, epi, M, N, K, ws.data_ptr(), ws.numel(), _hip.stream())
    np.testing.assert_allclose(n(Y), ref, **BF_TOL)
