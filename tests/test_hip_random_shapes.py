"""Seeded random shapes through the linear-stage and prefill-GEMM entry
points against the numpy oracle (GPU).

Each case draws its sizes from a fixed seed, so a failure names a
reproducible shape.  Linear stages: batch 1-64 (row-block GEMV, wave-per-row
GEMV, X-stationary and DMA-ring MFMA kernels), widths with and without a
masked last chunk, every epilogue, RMSNorm on and off, padded X rows.
GEMM: M, N up to ~2K, K % 8 == 0 (the MFMA kernel, masked last K-step) and
K % 8 != 0 (the linear-layer kernels), padded rows, residual on and off.
Decode attention: batch, group size, head_dim, capacity, ragged lengths and
length bounds.  The whole decode layer: batch 1-64, group sizes 1-16,
head_dim 64 / 128, widths, contiguous or paged caches.  Prefill attention:
chunk lengths (empty ones included), cached prefixes, groups, paging; the
prefill layer likewise, with widths that take the separate SwiGLU pass.
QK-norm + RoPE: batch, heads, head_dim 16-256 (both kernels), positions.
Row ops: RMSNorm fp32 / bf16, softmax and the full sum over random widths.
Bar: bf16 allclose(atol 2e-2, rtol 1e-2) against the fp32-accumulated
oracle (the layer: that bar with the oracle's own accumulation-order slack).
"""

import numpy as np
import pytest
import torch

import oracle
from ezops import _hip

pytestmark = pytest.mark.gpu
BF_TOL = dict(rtol=1e-2, atol=2e-2)
DEV = "cuda"


def n(x):
    return x.detach().float().cpu().numpy()


def g(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).to(DEV)


def _stage_ref(X, W, W2, R, w, norm, epi):
    Xn = oracle.rmsnorm_bf16(X, w) if norm else X
    g_ = oracle.linear_bf16(Xn, W)
    if epi == 0:
        return g_
    if epi == 1:
        return oracle.bf16(R + g_)
    u = oracle.linear_bf16(Xn, W2)
    return oracle.bf16(oracle.bf16(g_ / (1 + np.exp(-g_.astype(np.float64)))) * u)


@pytest.mark.parametrize("seed", list(range(40)) + [100 + i for i in range(10)])
def test_linear_stage_random(seed):
    rng = np.random.default_rng(1000 + seed)
    M = int(rng.integers(1, 21)) if seed < 100 else int(rng.integers(21, 65))  # 100+: batch 21-64
    N = int(rng.integers(1, 700))
    K = int(rng.choice([8 * int(rng.integers(1, 260)), 4096, 1024, 2048 + 8, int(rng.integers(1, 600))]))
    epi = int(rng.integers(0, 3))
    norm = int(rng.integers(0, 2))
    pad = int(rng.choice([0, 0, 8, 3]))  # X row padding (3: unaligned rows, the scalar kernel)
    if norm and M > 4:
        pad = 0  # the staged batched prologue takes contiguous rows
    ldx = K + pad
    X = oracle.bf16(rng.standard_normal((M, ldx)).astype(np.float32))
    W = oracle.bf16(rng.standard_normal((N, K)).astype(np.float32) * K ** -0.5)
    W2 = oracle.bf16(rng.standard_normal((N, K)).astype(np.float32) * K ** -0.5)
    R = oracle.bf16(rng.standard_normal((M, N)).astype(np.float32))
    w = oracle.bf16(rng.standard_normal(K).astype(np.float32) * 0.1 + 1)
    ref = _stage_ref(X[:, :K], W, W2, R, w, norm, epi)
    tX, tW, tW2, tR, tw = g(X), g(W), g(W2), g(R), g(w)
    Y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
    ws = torch.zeros(max(256, _hip.size("ezops_linear_stage_workspace_size", M, K, norm)), dtype=torch.uint8,
                     device=DEV)
    _hip.call("ezops_linear_stage_bf16", tX.data_ptr(), ldx, tW.data_ptr(), tW2.data_ptr(), Y.data_ptr(), N,
              tR.data_ptr(), N, tw.data_ptr(), norm, 1e-6, epi, M, N, K, ws.data_ptr(), ws.numel(), _hip.stream())
    np.testing.assert_allclose(n(Y), ref, **BF_TOL, err_msg=f"M={M} N={N} K={K} ldx={ldx} epi={epi} norm={norm}")


@pytest.mark.parametrize("seed", range(24))
def test_gemm_random(seed):
    rng = np.random.default_rng(2000 + seed)
    M = int(rng.integers(1, 1500))
    N = int(rng.integers(1, 1300))
    K = int(rng.choice([8 * int(rng.integers(1, 300)), 64 * int(rng.integers(1, 40)), int(rng.integers(1, 400))]))
    pad = int(rng.choice([0, 8, 1]))
    resid = bool(rng.integers(0, 2))
    ldx = K + pad
    X = oracle.bf16(rng.standard_normal((M, ldx)).astype(np.float32))
    W = oracle.bf16(rng.standard_normal((N, K)).astype(np.float32) * K ** -0.5)
    R = oracle.bf16(rng.standard_normal((M, N)).astype(np.float32))
    tX, tW, tR = g(X), g(W), g(R)
    Y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
    _hip.call("ezops_gemm_bf16", tX.data_ptr(), ldx, tW.data_ptr(), Y.data_ptr(), N, tR.data_ptr() if resid else None,
              M, N, K, None, 0, _hip.stream())
    ref = oracle.linear_bf16(X[:, :K], W)
    if resid:
        ref = oracle.bf16(R + ref)
    np.testing.assert_allclose(n(Y), ref, **BF_TOL, err_msg=f"M={M} N={N} K={K} ldx={ldx} resid={resid}")


@pytest.mark.parametrize("seed", range(24))
def test_attn_decode_random(seed):
    """Decode attention over random batch, group size, head_dim, capacity,
    ragged lengths and length bound (none, exact, loose): the interleaved,
    contiguous-run and ragged split plans."""
    rng = np.random.default_rng(3000 + seed)
    B = int(rng.integers(1, 9))
    G = int(rng.choice([1, 2, 4, 8, 16]))
    Hkv = int(rng.choice([1, 2, 8])) if G < 16 else 1
    H, D = G * Hkv, int(rng.choice([64, 128]))
    S = int(rng.integers(1, 3000))
    lens = rng.integers(1, S + 1, size=B).astype(np.int32)
    hint = int(rng.choice([0, lens.max(), min(S, lens.max() + 97)]))
    gen = torch.Generator(device=DEV).manual_seed(seed)
    Q = torch.randn(B, H, D, generator=gen, device=DEV).to(torch.bfloat16)
    K = torch.randn(B, Hkv, S, D, generator=gen, device=DEV).to(torch.bfloat16)
    V = torch.randn(B, Hkv, S, D, generator=gen, device=DEV).to(torch.bfloat16)
    tl = torch.from_numpy(lens).to(DEV)
    out = torch.full((B, H, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    ws = torch.zeros(max(256, _hip.size("ezops_attn_decode_workspace_size", B, H, Hkv, S, D)), dtype=torch.uint8,
                     device=DEV)
    _hip.call("ezops_attn_decode_bf16", Q.data_ptr(), K.data_ptr(), V.data_ptr(), out.data_ptr(), B, H, Hkv, S, D,
              tl.data_ptr(), hint, 0.0, ws.data_ptr(), ws.numel(), _hip.stream())
    ref = oracle.attn_decode(n(Q), n(K), n(V), kv_lens=lens)
    np.testing.assert_allclose(n(out), ref, **BF_TOL, err_msg=f"B={B} H={H} Hkv={Hkv} S={S} D={D} hint={hint}")


# ---- whole decode layer and prefill attention
from ezops import PrefillAttnOp, Qwen3DenseDecodeOp  # noqa: E402


def _layer_bar(out, ref, msg):
    """The layer's bar: the elementwise bf16 bar on all but at most
    max(2, 1e-4 n) elements and every element within twice it (fp32
    accumulation orders of the oracle itself differ past the bar on single
    elements of a layer; tests/test_oracle.py::test_layer_bar_order_sensitivity)."""
    d = np.abs(out - ref)
    bar = BF_TOL["atol"] + BF_TOL["rtol"] * np.abs(ref)
    assert (d <= 2 * bar).all(), (msg, float((d - 2 * bar).max()))
    assert int((d > bar).sum()) <= max(2, int(1e-4 * d.size)), (msg, int((d > bar).sum()))


@pytest.mark.parametrize("seed", list(range(16)) + [100 + i for i in range(6)])
def test_qwen3_layer_random(seed):
    """The decode layer over random batch (1-20: row-block GEMV, MFMA and
    X-stationary stages; seeds 100+: 21-64, the ragged-batch limit of the
    length-sorted attention plan), group size, head_dim, widths, capacity and ragged
    lengths, contiguous or paged, with weighted norms and RoPE, against the
    oracle layer; the decoded token's k / v land in their cache rows."""
    rng = np.random.default_rng(5000 + seed)
    B = int(rng.integers(1, 21)) if seed < 100 else int(rng.integers(21, 65))  # 100+: up to the ragged-batch limit
    G = int(rng.choice([1, 2, 4, 8, 16]))
    Hkv = int(rng.choice([1, 2, 4])) if G < 16 else int(rng.choice([1, 2]))
    H, D = G * Hkv, int(rng.choice([64, 128]))
    HS = int(rng.choice([256, 512, 1024, 2048]))
    IS = int(rng.choice([512, 1024, 1536, 3072]))
    paged = bool(rng.integers(0, 2))
    ps = int(rng.choice([32, 64])) if paged else None
    S = int(rng.integers(2, 33)) * (ps or 64)
    lens = rng.integers(1, S + 1, size=B).tolist()
    msg = f"B={B} H={H} Hkv={Hkv} D={D} HS={HS} IS={IS} S={S} page={ps}"
    torch.manual_seed(seed)
    kw = dict(page_size=ps, num_pages=B * (S // ps) + 3) if paged else {}
    op = Qwen3DenseDecodeOp(B, S, HS, IS, H, D, backend="hip", num_kv_heads=Hkv, kv_lens=lens, norm_weights=True,
                            rope_theta=1e6, **kw)
    data = list(op.gen_data(DEV))
    K0, V0 = n(data[1]), n(data[2])
    out = op(*data)
    npy = [n(x) for x in data[:13]]
    if paged:
        bt = data[13].cpu().numpy()
        K0, V0 = oracle.paged_to_contiguous(K0, bt, ps), oracle.paged_to_contiguous(V0, bt, ps)
        Kw = oracle.paged_to_contiguous(n(data[1]), bt, ps)
    else:
        Kw = n(data[1])
    ref, rK, _ = oracle.qwen3_layer(npy[0], K0, V0, *npy[3:7], H, Hkv, D, kv_lens=lens, in_norm_w=npy[7],
                                    q_norm_w=npy[8], k_norm_w=npy[9], post_norm_w=npy[10], cos=npy[11], sin=npy[12])
    _layer_bar(n(out), ref, msg)
    for b, L in enumerate(lens):
        np.testing.assert_allclose(Kw[b, :, L - 1], rK[b, :, L - 1], **BF_TOL, err_msg=msg)


@pytest.mark.parametrize("seed", range(16))
def test_prefill_attn_random(seed):
    """Prefill attention over random sequence counts, chunk lengths (empty
    chunks included), cached prefixes, group sizes and capacities, contiguous
    or paged, against the oracle."""
    rng = np.random.default_rng(6000 + seed)
    B = int(rng.integers(1, 5))
    G = int(rng.choice([1, 2, 4, 8]))
    Hkv = int(rng.choice([1, 2, 4]))
    paged = bool(rng.integers(0, 2))
    ps = int(rng.choice([32, 64, 128])) if paged else None
    S = int(rng.integers(2, 25)) * (ps or 64)
    q_lens = [int(rng.integers(0, min(S, 300) + 1)) for _ in range(B)]
    past = [int(rng.integers(0, S - q + 1)) for q in q_lens]
    if sum(q_lens) == 0:
        q_lens[0] = 1
        past[0] = min(past[0], S - 1)
    msg = f"B={B} G={G} Hkv={Hkv} S={S} q={q_lens} past={past} page={ps}"
    torch.manual_seed(seed)
    kw = dict(page_size=ps, num_pages=B * (S // ps) + 2) if paged else {}
    op = PrefillAttnOp(B, G * Hkv, Hkv, 128, S, q_lens, past, backend="hip", **kw)
    data = list(op.gen_data(DEV))
    out = op(*data)
    K, V = n(data[1]), n(data[2])
    if paged:
        bt = data[3].cpu().numpy()
        K, V = oracle.paged_to_contiguous(K, bt, ps), oracle.paged_to_contiguous(V, bt, ps)
    ref = oracle.prefill_attn(n(data[0]), K, V, q_lens, past)
    np.testing.assert_allclose(n(out), ref, **BF_TOL, err_msg=msg)


@pytest.mark.parametrize("seed", range(10))
def test_qwen3_prefill_random(seed):
    """The prefill layer over random sequence counts, chunk lengths (empty
    chunks included), cached prefixes, group sizes, widths (IS % 128 != 0:
    the separate SwiGLU pass) and paging, against the oracle: the output and
    every cache row the chunk writes."""
    from ezops import Qwen3PrefillOp

    rng = np.random.default_rng(7000 + seed)
    B = int(rng.integers(1, 4))
    G = int(rng.choice([1, 2, 4, 8]))
    Hkv = int(rng.choice([1, 2, 4]))
    HS = int(rng.choice([256, 512, 1024]))
    IS = int(rng.choice([512, 768, 1000, 1536]))
    paged = bool(rng.integers(0, 2))
    ps = int(rng.choice([32, 64])) if paged else None
    S = int(rng.integers(4, 17)) * (ps or 64)
    q_lens = [int(rng.integers(0, min(S, 200) + 1)) for _ in range(B)]
    if sum(q_lens) == 0:
        q_lens[0] = 1
    past = [int(rng.integers(0, S - q + 1)) for q in q_lens]
    msg = f"B={B} G={G} Hkv={Hkv} HS={HS} IS={IS} S={S} q={q_lens} past={past} page={ps}"
    torch.manual_seed(seed)
    kw = dict(page_size=ps, num_pages=B * (S // ps) + 2) if paged else {}
    op = Qwen3PrefillOp(B, S, HS, IS, G * Hkv, 128, q_lens, past, backend="hip", num_kv_heads=Hkv, norm_weights=True,
                        rope_theta=1e6, **kw)
    data = list(op.gen_data(DEV))
    K0, V0 = n(data[1]), n(data[2])
    out = op(*data)
    Kw, Vw = n(data[1]), n(data[2])
    if paged:
        bt = data[13].cpu().numpy()
        K0, V0 = oracle.paged_to_contiguous(K0, bt, ps), oracle.paged_to_contiguous(V0, bt, ps)
        Kw, Vw = oracle.paged_to_contiguous(Kw, bt, ps), oracle.paged_to_contiguous(Vw, bt, ps)
    npy = [n(x) for x in data[:13]]
    ref, rK, rV = oracle.qwen3_prefill(npy[0], K0, V0, *npy[3:7], G * Hkv, Hkv, 128, q_lens, past, in_norm_w=npy[7],
                                       q_norm_w=npy[8], k_norm_w=npy[9], post_norm_w=npy[10], cos=npy[11],
                                       sin=npy[12])
    _layer_bar(n(out), ref, msg)
    for b, (q, p) in enumerate(zip(q_lens, past)):
        np.testing.assert_allclose(Kw[b, :, p:p + q], rK[b, :, p:p + q], **BF_TOL, err_msg=msg)
        np.testing.assert_allclose(Vw[b, :, p:p + q], rV[b, :, p:p + q], **BF_TOL, err_msg=msg)


@pytest.mark.parametrize("seed", range(12))
def test_qk_norm_rope_random(seed):
    """Fused QK-norm + RoPE over random batch, head counts, head_dim (the
    16-byte-lane kernel at 64 / 128 / 256, the pair-per-lane kernel below),
    capacity and positions (one for the batch or one per sequence): q / k
    against the oracle, the written cache slot, every other slot untouched."""
    from ezops import FusedQkNormRopeOp

    rng = np.random.default_rng(8000 + seed)
    B = int(rng.integers(1, 17))
    Hkv = int(rng.choice([1, 2, 4, 8]))
    H = Hkv * int(rng.choice([1, 2, 4, 8]))
    D = int(rng.choice([16, 32, 64, 128, 256]))
    S = int(rng.integers(1, 4097))
    per_seq = bool(rng.integers(0, 2))
    pos = rng.integers(0, S, size=B).tolist() if per_seq else int(rng.integers(0, S))
    msg = f"B={B} H={H} Hkv={Hkv} D={D} S={S} pos={pos}"
    torch.manual_seed(seed)
    op = FusedQkNormRopeOp(B, H, D, S, pos, backend="hip", num_kv_heads=Hkv)
    data = list(op.gen_data(DEV))
    K0, V0 = data[7].clone(), data[8].clone()
    q_out, k_out = op(*data)
    p = np.broadcast_to(np.asarray(pos), (B,))
    rq, rk, _, _ = oracle.qk_norm_rope(*[n(x) for x in data[:7]], n(K0), n(V0), p)
    np.testing.assert_allclose(n(q_out), rq, **BF_TOL, err_msg=msg)
    np.testing.assert_allclose(n(k_out), rk, **BF_TOL, err_msg=msg)
    Kc, Vc = data[7], data[8]
    for b in range(B):
        np.testing.assert_allclose(n(Kc[b, :, p[b]]), rk[b], **BF_TOL, err_msg=msg)
        assert torch.equal(Vc[b, :, p[b]], data[2][b]), msg
        keep = torch.ones(S, dtype=torch.bool, device=DEV)
        keep[int(p[b])] = False
        assert torch.equal(Kc[b][:, keep], K0[b][:, keep]) and torch.equal(Vc[b][:, keep], V0[b][:, keep]), msg


@pytest.mark.parametrize("seed", range(12))
def test_row_ops_random(seed):
    """RMSNorm (fp32, and bf16 with a weight), row softmax and the full sum over
    random row counts and widths (every kernel choice: register-resident rows
    up to 32768, the looping kernel above, widths that are not a multiple of
    4 and so take the scalar path) against the oracle with the ops' own checks."""
    from ezops import ReduceOp, RmsNormOp, SoftmaxOp

    rng = np.random.default_rng(9000 + seed)
    rows = int(rng.integers(1, 300))
    dim = int(rng.choice([int(rng.integers(1, 64)), int(rng.integers(64, 4097)), int(rng.integers(4097, 40000))]))
    msg = f"rows={rows} dim={dim}"
    torch.manual_seed(seed)
    op = RmsNormOp(rows, dim, backend="hip")
    X, Out = op.gen_data(DEV)
    op(X, Out)
    assert op.check(Out, torch.from_numpy(oracle.rmsnorm_f32(n(X))).to(DEV)), msg
    opb = RmsNormOp(rows, dim, backend="hip", dtype=torch.bfloat16, weighted=True)
    Xb, Wb, Ob = opb.gen_data(DEV)
    opb(Xb, Wb, Ob)
    np.testing.assert_allclose(n(Ob), oracle.rmsnorm_bf16(n(Xb), n(Wb)), **BF_TOL, err_msg=msg)
    ops = SoftmaxOp(rows, dim, backend="hip")
    Xs, Os = ops.gen_data(DEV)
    Xs.mul_(4)
    ops(Xs, Os)
    assert ops.check(Os, torch.from_numpy(oracle.softmax(n(Xs))).to(DEV)), msg
    size = int(rng.integers(1, 1 << 22))
    opr = ReduceOp(size, backend="hip")
    A, Or = opr.gen_data(DEV)
    opr(A, Or)
    assert opr.check(Or, torch.from_numpy(oracle.reduce_sum(n(A))).to(DEV)), (size, Or.item())
