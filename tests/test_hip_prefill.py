"""Prefill attention (GPU) vs the oracle; paged cache bit-exact against the
contiguous kernel on the gathered cache."""

import numpy as np
import pytest
import torch

import oracle
from ezops import PrefillAttnOp
from ezops.ops.paged_attn_decode import paged_to_contiguous

pytestmark = pytest.mark.gpu
BF_TOL = dict(rtol=1e-2, atol=2e-2)


def n(x):
    return x.detach().float().cpu().numpy()


@pytest.mark.parametrize("H,Hkv,S,q_lens,past", [
    (32, 8, 1024, [1024], [0]),                    # fresh prompt, Qwen3-8B heads
    (32, 8, 2048, [100, 1, 333, 0], [0, 500, 1000, 7]),  # ragged chunks over cached prefixes
    (8, 8, 512, [200, 77], [40, 0]),               # MHA
    (16, 8, 512, [130], [3]),                      # group 2
    (32, 4, 512, [64, 65], [0, 447]),              # group 8, second chunk ends at the capacity
])
def test_prefill_attn_vs_oracle(H, Hkv, S, q_lens, past):
    torch.manual_seed(len(q_lens) * 10 + H)
    B = len(q_lens)
    op = PrefillAttnOp(B, H, Hkv, 128, S, q_lens, past, backend="hip")
    Q, K, V = op.gen_data()
    out = op(Q, K, V)
    ref = oracle.prefill_attn(n(Q), n(K), n(V), q_lens, past)
    np.testing.assert_allclose(n(out), ref, **BF_TOL)
    assert torch.equal(out, op(Q, K, V))


@pytest.mark.parametrize("page_size", [32, 64, 256])
def test_prefill_attn_paged_equals_contiguous(page_size):
    torch.manual_seed(page_size)
    q_lens, past = [300, 17, 512], [0, 900, 200]
    B, S = 3, 1024
    pop = PrefillAttnOp(B, 32, 8, 128, S, q_lens, past, backend="hip", page_size=page_size,
                        num_pages=B * S // page_size + 5)
    Q, Kp, Vp, bt = pop.gen_data()
    out = pop(Q, Kp, Vp, bt)
    cop = PrefillAttnOp(B, 32, 8, 128, S, q_lens, past, backend="hip")
    K, V = paged_to_contiguous(Kp, bt).contiguous(), paged_to_contiguous(Vp, bt).contiguous()
    assert torch.equal(out, cop(Q, K, V))



@pytest.mark.parametrize("paged", [False, True])
def test_prefill_attn_nonfinite_cache_tail(paged):
    """Cache rows past each sequence's last key (past + q_len) are never
    weighted: NaN / Inf there leave the output bit-identical.  The lengths
    end inside a 64-key tile, so the last tile straddles the written rows."""
    torch.manual_seed(31)
    q_lens, past = [100, 37], [5, 190]
    B, S, ps = 2, 512, 64
    kw = dict(page_size=ps, num_pages=B * S // ps) if paged else {}
    op = PrefillAttnOp(B, 32, 8, 128, S, q_lens, past, backend="hip", **kw)
    data = list(op.gen_data())
    ref = op(*data)
    K, V = data[1], data[2]
    if paged:  # block_table[b, p] is the page holding rows p*ps .. p*ps + ps - 1 of sequence b
        bt = data[3]
        for b in range(B):
            end = past[b] + q_lens[b]
            for p in range(S // ps):
                lo = max(end - p * ps, 0)
                if lo < ps:
                    pg = int(bt[b, p])
                    K[pg, :, lo:] = float("nan")
                    V[pg, :, lo:] = float("inf")
    else:
        for b in range(B):
            end = past[b] + q_lens[b]
            K[b, :, end:] = float("nan")
            V[b, :, end:] = float("inf")
    out = op(*data)
    assert torch.isfinite(out.float()).all()
    assert torch.equal(out, ref)


# ---- prefill layer and its GEMM
from ezops import Qwen3DenseDecodeOp, Qwen3PrefillOp, _hip  # noqa: E402

QWEN3_8B = dict(hidden_size=4096, intermediate_size=12288, num_heads=32, head_dim=128)


@pytest.mark.parametrize("M,N,K,resid", [
    (512, 6144, 4096, False), (77, 4096, 12288, True), (1, 200, 64, True),  # the MFMA kernel
    (300, 520, 128, False), (256, 256, 64, True), (4096, 768, 4096, "alias"),  # tile tails, one tile, R = Y
    (33, 100, 72, False), (5, 64, 72, True), (300, 520, 1000, "alias"), (257, 4100, 4104, True),
    (1024, 1024, 3000, False),  # K % 64 != 0: the MFMA kernel's masked last K-step
    (33, 100, 100, False), (70, 40, 9, True),  # K % 8 != 0: the linear-layer kernels
])
def test_gemm_vs_oracle(M, N, K, resid):
    rng = np.random.default_rng(M + N)
    X = oracle.bf16(rng.standard_normal((M, K)).astype(np.float32))
    W = oracle.bf16(rng.standard_normal((N, K)).astype(np.float32) * K ** -0.5)
    R = oracle.bf16(rng.standard_normal((M, N)).astype(np.float32))
    g = lambda a: torch.from_numpy(a).to(torch.bfloat16).cuda()  # noqa: E731
    Xg, Wg, Rg = g(X), g(W), g(R)
    Y = Rg.clone() if resid == "alias" else torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    Rp = Y.data_ptr() if resid == "alias" else (Rg.data_ptr() if resid else None)
    ws = torch.empty(_hip.size("ezops_gemm_workspace_size"), dtype=torch.uint8, device="cuda")
    _hip.call("ezops_gemm_bf16", Xg.data_ptr(), K, Wg.data_ptr(), Y.data_ptr(), N, Rp, M, N, K, ws.data_ptr(),
              ws.numel(), _hip.stream())
    ref = oracle.linear_bf16(X, W) + (R if resid else 0)
    np.testing.assert_allclose(n(Y), ref, **BF_TOL)
    if resid != "alias":  # fixed accumulation order: a second call is bit-identical
        Y2 = torch.empty_like(Y)
        _hip.call("ezops_gemm_bf16", Xg.data_ptr(), K, Wg.data_ptr(), Y2.data_ptr(), N,
                  Rg.data_ptr() if resid else None, M, N, K, ws.data_ptr(), ws.numel(), _hip.stream())
        assert torch.equal(Y, Y2)


def test_gemm_tile_widths_bit_identical():
    """256- and 128-column tiles accumulate every output over K in the same
    order: the same rows computed in a launch of wide tiles (4096 x 4096:
    256 tiles, one round) and of narrow tiles (2048 x 4096: 128 wide tiles
    would fill half the CUs, so it runs 256 narrow ones) are bit-identical."""
    torch.manual_seed(5)
    K = N = 4096
    X = torch.randn(4096, K, device="cuda").to(torch.bfloat16)
    W = (torch.randn(N, K, device="cuda") * K ** -0.5).to(torch.bfloat16)
    ws = torch.empty(_hip.size("ezops_gemm_workspace_size"), dtype=torch.uint8, device="cuda")
    out = {}
    for M in (4096, 2048):
        Y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        _hip.call("ezops_gemm_bf16", X.data_ptr(), K, W.data_ptr(), Y.data_ptr(), N, None, M, N, K, ws.data_ptr(),
                  ws.numel(), _hip.stream())
        out[M] = Y
    assert torch.equal(out[4096][:2048], out[2048])


@pytest.mark.parametrize("M,N,K,res", [(4096, 6144, 4096, False), (4096, 4096, 4096, True), (4000, 6000, 4032, True),
                                        (3000, 4100, 1088, False)])
def test_gemm_full_and_partial_grid_bit_identical(M, N, K, res):
    """A GEMM filling every CU and a 256-row launch of the same rows (narrow
    tiles) agree bit for bit (each output accumulates over K in the same
    order), with partial last tiles in M and N included; the whole output is
    within the bf16 bar of torch's fp32 product."""
    torch.manual_seed(M + N + K)
    X = torch.randn(M, K, device="cuda").to(torch.bfloat16)
    W = (torch.randn(N, K, device="cuda") * K ** -0.5).to(torch.bfloat16)
    R = torch.randn(M, N, device="cuda").to(torch.bfloat16) if res else None
    ws = torch.empty(_hip.size("ezops_gemm_workspace_size"), dtype=torch.uint8, device="cuda")
    out = {}
    for m in (M, 256):
        Y = torch.empty(m, N, dtype=torch.bfloat16, device="cuda")
        _hip.call("ezops_gemm_bf16", X.data_ptr(), K, W.data_ptr(), Y.data_ptr(), N,
                  None if R is None else R.data_ptr(), m, N, K, ws.data_ptr(), ws.numel(), _hip.stream())
        out[m] = Y
    assert torch.equal(out[M][:256], out[256])
    ref = X.float() @ W.float().T + (R.float() if res else 0)
    torch.testing.assert_close(out[M].float(), ref, rtol=1e-2, atol=2e-2)


def test_gemm_swiglu_full_and_partial_grid_bit_identical():
    """The fused gate/up + SwiGLU GEMM over 4096 rows (512 tiles) and over
    their first 256 rows (32 tiles) agree bit for bit on those rows, and
    match torch's fp32 gate/up with SwiGLU."""
    torch.manual_seed(9)
    M, IS, K = 4096, 4096, 4096
    X = torch.randn(M, K, device="cuda").to(torch.bfloat16)
    W = (torch.randn(2 * IS, K, device="cuda") * K ** -0.5).to(torch.bfloat16)
    out = {}
    for m in (M, 256):
        Y = torch.empty(m, IS, dtype=torch.bfloat16, device="cuda")
        _hip.call("ezops_gemm_swiglu_bf16", X.data_ptr(), K, W.data_ptr(), Y.data_ptr(), IS, m, IS, K, _hip.stream())
        out[m] = Y
    assert torch.equal(out[M][:256], out[256])
    # the reference's staging: gate and up rounded to bf16, silu(gate) rounded, the product rounded
    gu = (X[:512].float() @ W.float().T).to(torch.bfloat16).float()
    g, u = gu[:, :IS], gu[:, IS:]
    ref = (torch.nn.functional.silu(g).to(torch.bfloat16).float() * u).to(torch.bfloat16).float()
    torch.testing.assert_close(out[M][:512].float(), ref, rtol=1e-2, atol=2e-2)


@pytest.mark.parametrize("M,IS,K", [(300, 384, 256), (512, 1024, 512), (257, 128, 64), (300, 384, 200),
                                    (129, 256, 1096)])
def test_gemm_swiglu_vs_unfused(M, IS, K):
    """The fused gate/up + SwiGLU GEMM against the plain GEMM into [M, 2 IS]
    followed by SwiGLU on the host (bf16 gate/up, bf16 activation, bf16
    product): equal up to the device exp (1 bf16 ulp), bitwise repeatable."""
    rng = np.random.default_rng(M + IS)
    X = oracle.bf16(rng.standard_normal((M, K)).astype(np.float32))
    W = oracle.bf16(rng.standard_normal((2 * IS, K)).astype(np.float32) * K ** -0.5)
    g = lambda a: torch.from_numpy(a).to(torch.bfloat16).cuda()  # noqa: E731
    Xg, Wg = g(X), g(W)
    gu = torch.empty(M, 2 * IS, dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(_hip.size("ezops_gemm_workspace_size"), dtype=torch.uint8, device="cuda")
    _hip.call("ezops_gemm_bf16", Xg.data_ptr(), K, Wg.data_ptr(), gu.data_ptr(), 2 * IS, None, M, 2 * IS, K,
              ws.data_ptr(), ws.numel(), _hip.stream())
    Y = torch.empty(M, IS, dtype=torch.bfloat16, device="cuda")
    _hip.call("ezops_gemm_swiglu_bf16", Xg.data_ptr(), K, Wg.data_ptr(), Y.data_ptr(), IS, M, IS, K, _hip.stream())
    gh = n(gu)
    act = oracle.bf16(gh[:, :IS] / (1.0 + np.exp(-gh[:, :IS])))
    ref = oracle.bf16(act * gh[:, IS:])
    np.testing.assert_allclose(n(Y), ref, rtol=1e-2, atol=1e-2)
    assert np.mean(n(Y) == ref) > 0.99  # all but exp-rounding ties are bit-equal
    Y2 = torch.empty_like(Y)
    _hip.call("ezops_gemm_swiglu_bf16", Xg.data_ptr(), K, Wg.data_ptr(), Y2.data_ptr(), IS, M, IS, K, _hip.stream())
    assert torch.equal(Y, Y2)


def test_gemm_swiglu_rejects_unsupported():
    X = torch.zeros(16, 64, dtype=torch.bfloat16, device="cuda")
    W = torch.zeros(2 * 96, 64, dtype=torch.bfloat16, device="cuda")
    Y = torch.zeros(16, 96, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="-22"):  # IS = 96 is not a multiple of 128: EINVAL
        _hip.call("ezops_gemm_swiglu_bf16", X.data_ptr(), 64, W.data_ptr(), Y.data_ptr(), 96, 16, 96, 64,
                  _hip.stream())


def _prefill_ref(op, data, paged):
    npy = [n(x) for x in data]
    K0, V0 = npy[1], npy[2]
    if paged:
        bt = data[-1].cpu().numpy()
        K0, V0 = oracle.paged_to_contiguous(K0, bt, op.page_size), oracle.paged_to_contiguous(V0, bt, op.page_size)
    return oracle.qwen3_prefill(npy[0], K0, V0, *npy[3:7], op.num_heads, op.num_kv_heads, op.head_dim, op.q_lens,
                                op.past_lens, in_norm_w=npy[7], q_norm_w=npy[8], k_norm_w=npy[9],
                                post_norm_w=npy[10], cos=npy[11], sin=npy[12])


@pytest.mark.parametrize("q_lens,past,S", [([512], [0], 1024), ([100, 1, 257], [0, 600, 300], 1024)])
def test_qwen3_prefill_vs_oracle(q_lens, past, S):
    torch.manual_seed(len(q_lens))
    op = Qwen3PrefillOp(len(q_lens), S, q_lens=q_lens, past_lens=past, backend="hip", num_kv_heads=8,
                        norm_weights=True, rope_theta=1e6, **QWEN3_8B)
    data = op.gen_data()
    K0, V0 = data[1].clone(), data[2].clone()
    ref, Kc, Vc = _prefill_ref(op, (data[0], K0, V0, *data[3:]), False)
    out = op(*data)
    ref_t = torch.from_numpy(ref).cuda()
    assert op.check(out, ref_t), (out.float() - ref_t).norm().item() / ref_t.norm().item()
    np.testing.assert_allclose(n(data[1]), Kc, **BF_TOL)
    np.testing.assert_allclose(n(data[2]), Vc, **BF_TOL)  # V rows are QKV GEMM outputs


@pytest.mark.parametrize("norm_weights,rope_theta", [(False, None), (True, None), (False, 1e6)])
def test_qwen3_prefill_without_weights_or_rope(norm_weights, rope_theta):
    """Unit norm weights and / or no RoPE (the attention's q transform with
    its weight or tables absent) against the package's torch ref path."""
    q_lens, past, S = [200, 57], [0, 300], 512
    torch.manual_seed(7)
    kw = dict(q_lens=q_lens, past_lens=past, num_kv_heads=8, norm_weights=norm_weights, rope_theta=rope_theta,
              **QWEN3_8B)
    op = Qwen3PrefillOp(2, S, backend="hip", **kw)
    ref_op = Qwen3PrefillOp(2, S, backend="ref", **kw)
    data = op.gen_data()
    ref_data = [x.clone() for x in data]
    out = op(*data)
    ref = ref_op(*ref_data)
    assert op.check(out, ref), (out.float() - ref.float()).norm().item() / ref.float().norm().item()
    np.testing.assert_allclose(n(data[1]), n(ref_data[1]), **BF_TOL)  # cache rows written alike


def test_qwen3_prefill_paged_equals_contiguous_then_decode():
    """Paged prefill equals contiguous prefill bit-for-bit (output and cache);
    the decode layer then continues from the prefilled cache."""
    q_lens, past, S, P = [300, 45], [0, 100], 1024, 64
    torch.manual_seed(3)
    pop = Qwen3PrefillOp(2, S, q_lens=q_lens, past_lens=past, backend="hip", num_kv_heads=8, norm_weights=True,
                         rope_theta=1e6, page_size=P, **QWEN3_8B)
    data = list(pop.gen_data())
    bt = data[-1]
    Kc = paged_to_contiguous(data[1], bt).contiguous()
    Vc = paged_to_contiguous(data[2], bt).contiguous()
    out = pop(*data)
    cop = Qwen3PrefillOp(2, S, q_lens=q_lens, past_lens=past, backend="hip", num_kv_heads=8, norm_weights=True,
                         rope_theta=1e6, **QWEN3_8B)
    cout = cop(data[0], Kc, Vc, *data[3:-1])
    assert torch.equal(out, cout)
    assert torch.equal(paged_to_contiguous(data[1], bt), Kc) and torch.equal(paged_to_contiguous(data[2], bt), Vc)
    # one decode step on top of the prefilled (paged) cache vs the oracle
    lens = [p + q + 1 for p, q in zip(past, q_lens)]
    dop = Qwen3DenseDecodeOp(2, S, backend="hip", num_kv_heads=8, kv_lens=lens, norm_weights=True, rope_theta=1e6,
                             page_size=P, **QWEN3_8B)
    hid = torch.randn(2, 4096, device="cuda").to(torch.bfloat16)
    K_before = paged_to_contiguous(data[1], bt).cpu().float().numpy()
    V_before = paged_to_contiguous(data[2], bt).cpu().float().numpy()
    dout = dop(hid, data[1], data[2], *data[3:])
    npw = [n(x) for x in data[3:13]]
    ref, _, _ = oracle.qwen3_layer(n(hid), K_before, V_before, *npw[:4], 32, 8, 128, kv_lens=lens, in_norm_w=npw[4],
                                   q_norm_w=npw[5], k_norm_w=npw[6], post_norm_w=npw[7], cos=npw[8], sin=npw[9])
    assert dop.check(dout, torch.from_numpy(ref).cuda())


def test_prefill_attn_clamps_device_lengths():
    """cu_seqlens / past_lens live in device memory and are clamped there: a
    negative past length acts as 0 and offsets past T end the sequence."""
    torch.manual_seed(12)
    op = PrefillAttnOp(2, 32, 8, 128, 512, [100, 50], [0, 0], backend="hip")
    Q, K, V = op.gen_data()
    ref = op(Q, K, V)
    cu = torch.tensor([0, 100, 150], dtype=torch.int32, device="cuda")
    past = torch.tensor([-3, 0], dtype=torch.int32, device="cuda")
    out = torch.zeros_like(ref)
    _hip.call("ezops_prefill_attn_bf16", Q.data_ptr(), K.data_ptr(), V.data_ptr(), out.data_ptr(), cu.data_ptr(),
              past.data_ptr(), 2, 150, 32, 8, 512, 128, 100, None, 0, 0, 0.0, _hip.stream())
    assert torch.equal(out, ref)
    cu_over = torch.tensor([0, 100, 4000], dtype=torch.int32, device="cuda")  # second sequence runs past T = 150
    out2 = torch.zeros_like(ref)
    _hip.call("ezops_prefill_attn_bf16", Q.data_ptr(), K.data_ptr(), V.data_ptr(), out2.data_ptr(),
              cu_over.data_ptr(), None, 2, 150, 32, 8, 512, 128, 100, None, 0, 0, 0.0, _hip.stream())
    assert torch.equal(out2, ref)


def test_prefill_deterministic_and_writes_only_chunk_rows():
    """Prefill attention leaves its inputs untouched and repeats bit-for-bit;
    the prefill layer writes exactly the chunk's cache rows and repeats
    bit-for-bit from the same starting cache."""
    torch.manual_seed(33)
    at = PrefillAttnOp(2, 32, 8, 128, 1024, [200, 77], [100, 0], backend="hip")
    data = at.gen_data()
    before = [t.clone() for t in data]
    x, y = at(*data), at(*data)
    assert torch.equal(x, y) and all(torch.equal(u, v) for u, v in zip(data, before))

    q_lens, past = [130, 20], [0, 500]
    op = Qwen3PrefillOp(2, 1024, q_lens=q_lens, past_lens=past, backend="hip", num_kv_heads=8, norm_weights=True,
                        rope_theta=1e6, **QWEN3_8B)
    d = list(op.gen_data())
    K0, V0 = d[1].clone(), d[2].clone()
    out1 = op(*d)
    K1, V1 = d[1].clone(), d[2].clone()
    d[1].copy_(K0)
    d[2].copy_(V0)
    out2 = op(*d)
    assert torch.equal(out1, out2) and torch.equal(d[1], K1) and torch.equal(d[2], V1)
    touched = torch.zeros(2, 1024, dtype=torch.bool, device="cuda")
    for b_, (n_, p_) in enumerate(zip(q_lens, past)):
        touched[b_, p_:p_ + n_] = True
    rows = lambda t: t.transpose(1, 2)[~touched]  # noqa: E731
    assert torch.equal(rows(K1), rows(K0)) and torch.equal(rows(V1), rows(V0))
