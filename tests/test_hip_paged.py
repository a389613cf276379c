"""Paged-KV decode attention (GPU): bit-exact against the contiguous HIP
kernel on the gathered cache, and within the bf16 bar of the oracle.

Both kernels run the same split plan for the same (B, H, Hkv, S, max_kv_len),
so the paged path must reproduce the contiguous one bit-for-bit; only the
address of each 32-row tile differs.
"""

import numpy as np
import pytest
import torch

import oracle
from ezops import AttnDecodeOp, PagedAttnDecodeOp, Qwen3DenseDecodeOp
from ezops.ops.paged_attn_decode import paged_to_contiguous

pytestmark = pytest.mark.gpu
BF_TOL = dict(rtol=1e-2, atol=2e-2)
DEV = "cuda"


def n(x):
    return x.detach().float().cpu().numpy()


@pytest.mark.parametrize("B,H,Hkv,D,P,M,NP", [
    (1, 32, 8, 128, 64, 256, 300),   # Qwen3-8B heads, 16K capacity, spare pool pages
    (4, 32, 8, 128, 32, 40, 200),
    (3, 16, 8, 64, 128, 9, 27),
    (16, 32, 8, 128, 256, 16, 256),  # B=16 at 4K capacity
    (2, 32, 4, 128, 1024, 3, 8),     # group 8, pages larger than a split chunk
    (2, 16, 1, 128, 64, 40, 100),    # group 16
])
def test_paged_equals_contiguous(B, H, Hkv, D, P, M, NP):
    torch.manual_seed(B * 100 + P)
    op = PagedAttnDecodeOp(B, H, Hkv, D, page_size=P, max_pages=M, num_pages=NP, backend="hip")
    Q, Kp, Vp, bt, lens = op.gen_data()
    lens[0] = M * P
    if B > 2:
        lens[1] = 1
    bound = int(lens.max())
    out = op(Q, Kp, Vp, bt, lens, max_kv_len=bound)
    K, V = paged_to_contiguous(Kp, bt).contiguous(), paged_to_contiguous(Vp, bt).contiguous()
    cop = AttnDecodeOp(B, H, M * P, D, backend="hip", num_kv_heads=Hkv)
    cout = cop._kernel(Q, K, V, lens, max_kv_len=bound)
    assert torch.equal(out, cout)
    ref = oracle.paged_attn_decode(n(Q)[:, :, 0], n(Kp), n(Vp), bt.cpu().numpy(), n(lens).astype(np.int64), P)
    np.testing.assert_allclose(n(out)[:, :, 0], ref, **BF_TOL)


def test_paged_unused_table_entries_and_shared_pages():
    """Entries past a sequence's last page may hold anything (here -1 and
    huge ids): they are never dereferenced outside the pool and do not change
    the result.  Two sequences sharing prefix pages read the same pool pages."""
    B, H, Hkv, D, P, M, NP = 3, 32, 8, 128, 64, 32, 70
    torch.manual_seed(9)
    op = PagedAttnDecodeOp(B, H, Hkv, D, page_size=P, max_pages=M, num_pages=NP, backend="hip")
    Q, Kp, Vp, bt, _ = op.gen_data()
    lens = torch.tensor([M * P, 700, 65], dtype=torch.int32, device=DEV)
    bt[1, :4] = bt[0, :4]  # shared prefix
    ref_bt = bt.clone()
    for b in range(B):
        used = (int(lens[b]) + P - 1) // P
        bt[b, used:] = torch.tensor([-1, 1 << 30], dtype=torch.int32, device=DEV).repeat(M)[: M - used]
        ref_bt[b, used:] = 0
    # max_kv_len = 0 (capacity): the first tiles of short sequences are
    # requested at the capacity bound, i.e. through the garbage entries.
    out = op(Q, Kp, Vp, bt, lens)
    ref = oracle.paged_attn_decode(n(Q)[:, :, 0], n(Kp), n(Vp), ref_bt.cpu().numpy(), n(lens).astype(np.int64), P)
    np.testing.assert_allclose(n(out)[:, :, 0], ref, **BF_TOL)
    assert torch.equal(out, op(Q, Kp, Vp, ref_bt, lens))


def test_paged_graph_replays():
    B, H, Hkv, D, P, M = 4, 32, 8, 128, 64, 64
    torch.manual_seed(4)
    op = PagedAttnDecodeOp(B, H, Hkv, D, page_size=P, max_pages=M, backend="hip")
    Q, Kp, Vp, bt, lens = op.gen_data()
    eager = op(Q, Kp, Vp, bt, lens, max_kv_len=M * P)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        g_ = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_, stream=s):
            out = op(Q, Kp, Vp, bt, lens, max_kv_len=M * P)
    for _ in range(3):
        g_.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        op(Q, Kp, Vp, bt, lens)  # eager work between replays


QWEN3_8B = dict(hidden_size=4096, intermediate_size=12288, num_heads=32, head_dim=128)


@pytest.mark.parametrize("batch,seq_len,page_size", [(1, 16384, 64), (4, 4096, 32), (16, 4096, 256)])
def test_paged_layer_equals_contiguous(batch, seq_len, page_size):
    """The Qwen3-8B layer over a paged cache: output bit-identical to the
    contiguous layer on the gathered cache, the decoded rows land in the
    right pool pages and nothing else in the pools changes."""
    torch.manual_seed(batch)
    rng = np.random.default_rng(batch)
    lens = rng.integers(min(1024, seq_len), seq_len + 1, size=batch).tolist()
    mode = dict(kv_lens=lens, norm_weights=True, rope_theta=1e6)
    pop = Qwen3DenseDecodeOp(batch, seq_len, backend="hip", num_kv_heads=8, page_size=page_size,
                             num_pages=batch * seq_len // page_size + 3, **QWEN3_8B, **mode)
    data = list(pop.gen_data())
    bt = data[-1]
    Kc = paged_to_contiguous(data[1], bt).contiguous()
    Vc = paged_to_contiguous(data[2], bt).contiguous()
    K0, V0 = data[1].clone(), data[2].clone()
    out = pop(*data)
    cop = Qwen3DenseDecodeOp(batch, seq_len, backend="hip", num_kv_heads=8, **QWEN3_8B, **mode)
    cout = cop(data[0], Kc, Vc, *data[3:-1])
    assert torch.equal(out, cout)
    assert torch.equal(paged_to_contiguous(data[1], bt), Kc)
    assert torch.equal(paged_to_contiguous(data[2], bt), Vc)
    touched = torch.zeros(K0.shape[0], page_size, dtype=torch.bool, device=DEV)
    for b, L in enumerate(lens):
        touched[int(bt[b, (L - 1) // page_size]), (L - 1) % page_size] = True
    rows = lambda t: t.transpose(1, 2)[~touched]  # noqa: E731  (page, row) pairs not written
    assert torch.equal(rows(data[1]), rows(K0)) and torch.equal(rows(data[2]), rows(V0))


def test_paged_attn_deterministic_and_inputs_read_only():
    op = PagedAttnDecodeOp(4, 32, 8, 128, page_size=64, max_pages=32, num_pages=160, backend="hip")
    torch.manual_seed(31)
    data = op.gen_data()
    before = [t.clone() for t in data]
    a = op(*data, max_kv_len=2048)
    b = op(*data, max_kv_len=2048)
    assert torch.equal(a, b)
    assert all(torch.equal(x, y) for x, y in zip(data, before))


def test_paged_nonfinite_rows_past_lengths():
    """Pool rows that hold no live position (past a sequence's length, or
    pages no table entry reaches) may hold NaN / Inf: they are never read."""
    B, H, Hkv, D, P, M, NP = 4, 32, 8, 128, 32, 8, 40
    torch.manual_seed(17)
    op = PagedAttnDecodeOp(B, H, Hkv, D, page_size=P, max_pages=M, num_pages=NP, backend="hip")
    Q, Kp, Vp, bt, _ = op.gen_data()
    lens = torch.tensor([M * P, 33, 1, 95], dtype=torch.int32, device=DEV)
    ref = oracle.paged_attn_decode(n(Q)[:, :, 0], n(Kp), n(Vp), bt.cpu().numpy(), n(lens).astype(np.int64), P)
    live = torch.zeros(NP, P, dtype=torch.bool, device=DEV)
    for b, L in enumerate(lens.tolist()):
        for t in range(L):
            live[int(bt[b, t // P]), t % P] = True
    Kg, Vg = Kp.clone(), Vp.clone()
    Kg.transpose(1, 2)[~live] = float("nan")
    Vg.transpose(1, 2)[~live] = float("inf")
    out = op(Q, Kg, Vg, bt, lens)
    assert torch.isfinite(out).all()
    np.testing.assert_allclose(n(out)[:, :, 0], ref, **BF_TOL)
