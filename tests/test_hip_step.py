"""Multi-layer decode step (GPU): the chained C entry equals the single-layer
HIP kernel applied layer by layer (bit-exact: same kernels, same bf16
hand-offs), its logits equal the RMSNorm + LM-head stage, the oracle agrees
within the fused-op bar, and a graph-captured step replays exactly."""

import numpy as np
import pytest
import torch

import oracle
from ezops import Qwen3DecodeStepOp, Qwen3DenseDecodeOp
from ezops import _hip

pytestmark = pytest.mark.gpu
DEV = "cuda"
QWEN3_8B = dict(hidden_size=4096, intermediate_size=12288, num_heads=32, head_dim=128)


def n(x):
    return x.detach().float().cpu().numpy()


def norm_linear(X, W, w):
    """bf16 rmsnorm(X) * w @ W.T through the linear-stage entry (store epilogue)."""
    M, K = X.shape
    N = W.shape[0]
    Y = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    ws = torch.zeros(max(256, _hip.size("ezops_linear_stage_workspace_size", M, K, 1)), dtype=torch.uint8,
                     device=DEV)
    _hip.call("ezops_linear_stage_bf16", X.data_ptr(), K, W.data_ptr(), None, Y.data_ptr(), N, None, 0,
              w.data_ptr(), 1, 1e-6, 0, M, N, K, ws.data_ptr(), ws.numel(), _hip.stream())
    return Y


def _step(batch, seq_len, n_layers, vocab, paged=False, small=False):
    shapes = dict(hidden_size=256, intermediate_size=512, num_heads=8, head_dim=64) if small else QWEN3_8B
    rng = np.random.default_rng(batch * 7 + n_layers)
    lens = rng.integers(min(1024, seq_len // 2), seq_len + 1, size=batch).tolist()
    kw = dict(kv_lens=lens, norm_weights=True, rope_theta=1e6)
    if paged:
        kw.update(page_size=64)
    op = Qwen3DecodeStepOp(batch, seq_len, num_layers=n_layers, backend="hip", num_kv_heads=shapes["num_heads"] // 4,
                           vocab_size=vocab, **shapes, **kw)
    torch.manual_seed(batch)
    return op, op.gen_data(), lens, shapes, kw


@pytest.mark.parametrize("batch,seq_len,n_layers,vocab,paged", [
    (1, 16384, 3, 151936, False),   # Qwen3-8B shapes, full vocabulary
    (16, 4096, 2, 5000, False),
    (4, 4096, 3, 0, True),          # paged cache shared across layers, no LM head
])
def test_step_equals_layer_chain(batch, seq_len, n_layers, vocab, paged):
    op, data, lens, shapes, kw = _step(batch, seq_len, n_layers, vocab, paged)
    hidden, layers, cos, sin, fw, lm, bt = data
    caches0 = [(L[0].clone(), L[1].clone()) for L in layers]
    h, logits = op(*data)
    # single-layer kernel chain on the original caches
    lop = Qwen3DenseDecodeOp(batch, seq_len, backend="hip", num_kv_heads=shapes["num_heads"] // 4, **shapes, **kw)
    x = hidden
    for L, (K0, V0) in zip(layers, caches0):
        extra = [bt] if paged else []
        x = lop(x, K0, V0, *L[2:], cos, sin, *extra)
        assert torch.equal(L[0], K0) and torch.equal(L[1], V0)  # same slot writes
    assert torch.equal(h, x)
    if vocab:
        ref = norm_linear(x, lm, fw)
        assert torch.equal(logits, ref)
        ro = oracle.linear_bf16(oracle.rmsnorm_bf16(n(x), n(fw)), n(lm))
        assert op.check(logits, torch.from_numpy(ro).to(DEV))
    else:
        assert logits is None


def test_step_small_vs_oracle():
    op, data, lens, shapes, kw = _step(3, 512, 4, 300, small=True)
    hidden, layers, cos, sin, fw, lm, bt = data
    npl = [[n(t) for t in L] for L in layers]
    h, logits = op(*data)
    x = n(hidden)
    for L in npl:
        x, _, _ = oracle.qwen3_layer(x, L[0], L[1], *L[2:6], 8, 2, 64, kv_lens=lens, in_norm_w=L[6],
                                     q_norm_w=L[7], k_norm_w=L[8], post_norm_w=L[9], cos=n(cos), sin=n(sin))
    assert op.check(h, torch.from_numpy(x).to(DEV))
    ro = oracle.linear_bf16(oracle.rmsnorm_bf16(x, n(fw)), n(lm))
    assert op.check(logits, torch.from_numpy(ro).to(DEV))


def test_step_graph_replays():
    op, data, lens, shapes, kw = _step(2, 4096, 4, 1000)
    eager_h, eager_l = (t.clone() for t in op(*data))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        op(*data)
        g_ = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_, stream=s):
            h, logits = op(*data)
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(3):
        g_.replay()
        torch.cuda.synchronize()
        assert torch.equal(h, eager_h) and torch.equal(logits, eager_l)
        op(*data)  # eager work between replays
