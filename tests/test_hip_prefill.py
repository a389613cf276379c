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
