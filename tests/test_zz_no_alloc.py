"""The allocation-free decode attention entry point against the workspace one (GPU).

Both run the same kernels and the same split plan, so the outputs must be
bit-identical.  Two calls in a row, the second on a smaller input (fewer
sequences, shorter cache, ragged lengths), check that the shared device
scratch of the first call never leaks into the second.  Oversized shapes are
rejected before any launch.
"""

import pytest
import torch

from ezops import _hip

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(B, H, Hkv, S, D, seed, ragged):
    g = torch.Generator(device=DEV).manual_seed(seed)
    Q = torch.randn(B, H, D, generator=g, device=DEV).to(torch.bfloat16)
    K = torch.randn(B, Hkv, S, D, generator=g, device=DEV).to(torch.bfloat16)
    V = torch.randn(B, Hkv, S, D, generator=g, device=DEV).to(torch.bfloat16)
    lens = None
    if ragged:
        lens = torch.randint(1, S + 1, (B,), generator=g, device=DEV, dtype=torch.int32)
    return Q, K, V, lens


def _run(name, Q, K, V, lens, ws=None):
    B, H, D = Q.shape
    Hkv, S = K.shape[1], K.shape[2]
    out = torch.full((B, H, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    lp = lens.data_ptr() if lens is not None else None
    mx = int(lens.max()) if lens is not None else 0
    args = [Q.data_ptr(), K.data_ptr(), V.data_ptr(), out.data_ptr(), B, H, Hkv, S, D, lp, mx, 0.0]
    if ws is not None:
        args += [ws.data_ptr(), ws.numel()]
    _hip.call(name, *args, _hip.stream())
    return out


def _reference(Q, K, V, lens):
    B, H, D = Q.shape
    nbytes = _hip.size("ezops_attn_decode_workspace_size", B, H, K.shape[1], K.shape[2], D)
    ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=DEV)  # zero-filled, as the ABI asks
    return _run("ezops_attn_decode_bf16", Q, K, V, lens, ws)


@pytest.mark.parametrize("first,second", [
    ((8, 32, 8, 8192, 128, False), (2, 32, 8, 1000, 128, True)),   # Qwen3-8B heads, then a smaller ragged batch
    ((1, 32, 8, 16384, 128, False), (1, 16, 16, 300, 64, False)),  # B=1 long context (32 splits), then MHA D=64
])
def test_noalloc_matches_workspace_entry(first, second):
    for i, shape in enumerate((first, second)):
        Q, K, V, lens = _inputs(*shape[:5], seed=10 + i, ragged=shape[5])
        got = _run("ezops_attn_decode_noalloc_bf16", Q, K, V, lens)
        ref = _reference(Q, K, V, lens)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, ref), (shape, (got.float() - ref.float()).abs().max().item())


def test_noalloc_rejects_oversized_partials():
    cap = _hip.lib().ezops_attn_decode_noalloc_max_scratch()
    assert cap == 8 << 20
    # 2 sequences x 64 kv heads at group 8, head_dim 128: 8.1 MiB of split partials
    B, H, Hkv, S, D = 2, 512, 64, 1 << 16, 128
    need = _hip.size("ezops_attn_decode_workspace_size", B, H, Hkv, S, D)
    assert need > cap
    d = 64  # never dereferenced: the size check comes first
    rc = _hip.lib().ezops_attn_decode_noalloc_bf16(d, d, d, d, B, H, Hkv, S, D, None, 0, 0.0, None)
    assert rc == _hip.EINVAL and b"scratch" in _hip.lib().ezops_hip_last_error()
