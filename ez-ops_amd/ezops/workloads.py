"""Seeded synthetic inputs for the benchmark configurations of the decode path.

Each function draws its tensors from one ``torch.Generator`` seeded with the
configuration's seed, in the order its docstring lists, then moves them to
``device``.  The generator lives on ``gen_device`` (default: ``device``):
drawing on the GPU is fast for the 1 GiB inputs; ``gen_device="cpu"`` gives
values that do not depend on the GPU's generator (the two differ for the
same seed).  A CPU baseline copies the GPU's tensors, so both sides always
see the same values.  All values are synthetic: random-init weights, no
checkpoint.

Configurations (names used by tests/ and bench.py):
  G   bf16 GEMV, W [4096, 4096] ~ N(0, 0.02), x [4096] ~ N(0, 1), seed 0
  N   RMSNorm bf16 [64, 4096] with weight ~ N(1, 0.1); softmax fp32
      [4096, 32768] ~ N(0, 3); sum of 2^28 fp32 ~ U(-1, 1); seed 1
  A   GQA decode B=32, H=32, Hkv=8, S=8192, D=128, q/K/V ~ N(0, 1), seed 2
  F1  QK-norm + RoPE at Qwen3-8B heads (32 / 8 x 128), positions ~ U[0, 32768)
      over a 32768-row cache, theta 1e6, seed 3
  F2  o_proj + SwiGLU FFN at Qwen3-8B (4096 / 12288), weights ~ N(0, 0.02), seed 3
  L   Qwen3-8B dense decode layer, kv_lens ~ U[1024, 16384], seed 4 (the
      layer op's own ``gen_data`` under ``torch.manual_seed(4)``)
"""

from __future__ import annotations

import torch

SEQ_MAX_L = 16384
QWEN3_8B = dict(hidden_size=4096, intermediate_size=12288, num_heads=32, head_dim=128, num_kv_heads=8)


class _Gen:
    def __init__(self, seed: int, device, gen_device: str):
        self.device = torch.device(device)
        self.gdev = torch.device(device if gen_device is None else gen_device)
        self.g = torch.Generator(device=self.gdev).manual_seed(seed)

    def normal(self, *shape, dtype=torch.bfloat16, std=1.0, mean=0.0):
        t = torch.randn(*shape, generator=self.g, device=self.gdev)
        if std != 1.0:
            t.mul_(std)
        if mean != 0.0:
            t.add_(mean)
        return t.to(dtype).to(self.device)

    def uniform(self, *shape, lo=-1.0, hi=1.0):
        t = torch.rand(*shape, generator=self.g, device=self.gdev)
        return t.mul_(hi - lo).add_(lo).to(self.device)

    def randint(self, lo, hi, n):
        return torch.randint(lo, hi, (n,), generator=self.g, device=self.gdev).tolist()


def config_g(device="cuda", gen_device=None):
    """G: W [4096, 4096] then x [4096]; returns (x, W), y = W x."""
    r = _Gen(0, device, gen_device)
    W = r.normal(4096, 4096, std=0.02)
    x = r.normal(4096)
    return x, W


def config_n(device="cuda", gen_device=None, parts=("rmsnorm", "softmax", "sum")):
    """N: rmsnorm (X [64, 4096], w [4096]), softmax X [4096, 32768], sum A [2^28],
    drawn in that order from one stream.  ``parts`` selects which are moved to
    ``device`` and returned; every part is drawn, so each keeps its values."""
    r = _Gen(1, device, gen_device)
    keep = {}
    r.device = r.gdev  # draw everything on the generator's device, move what is asked for
    keep["rmsnorm"] = (r.normal(64, 4096), r.normal(4096, std=0.1, mean=1.0))
    keep["softmax"] = r.normal(4096, 32768, dtype=torch.float32, std=3.0)
    keep["sum"] = r.uniform(1 << 28)
    dev = torch.device(device)
    out = {}
    for k in parts:
        v = keep[k]
        out[k] = tuple(t.to(dev) for t in v) if isinstance(v, tuple) else v.to(dev)
    return out


def config_a(device="cuda", gen_device=None, B=32, H=32, Hkv=8, S=8192, D=128):
    """A: Q [B, H, 1, D], K [B, Hkv, S, D], V [B, Hkv, S, D], in that order."""
    r = _Gen(2, device, gen_device)
    return r.normal(B, H, 1, D), r.normal(B, Hkv, S, D), r.normal(B, Hkv, S, D)


def config_f1(B: int, device="cuda", gen_device=None, S=32768):
    """F1: positions [B] ~ U[0, S), q [B, 32, 128], k, v [B, 8, 128],
    q_norm_w, k_norm_w [128] ~ N(1, 0.1), K_cache, V_cache [B, 8, S, 128];
    returns (positions, q, k, v, q_norm_w, k_norm_w, cos, sin, K_cache, V_cache)
    with the HF bf16 RoPE tables at theta 1e6."""
    from .ops.fused_qk_norm_rope import rope_tables

    r = _Gen(3, device, gen_device)
    pos = r.randint(0, S, B)
    q, k, v = r.normal(B, 32, 128), r.normal(B, 8, 128), r.normal(B, 8, 128)
    qw, kw = r.normal(128, std=0.1, mean=1.0), r.normal(128, std=0.1, mean=1.0)
    cos, sin = rope_tables(S, 128, 1e6, device)
    K, V = r.normal(B, 8, S, 128), r.normal(B, 8, S, 128)
    return pos, q, k, v, qw, kw, cos, sin, K, V


def config_f1_positions(B: int, device="cuda", gen_device=None, S=32768) -> list[int]:
    """F1's positions alone (the configuration's first draw, same values as ``config_f1``)."""
    return _Gen(3, device, gen_device).randint(0, S, B)


def config_f2(B: int, device="cuda", gen_device=None):
    """F2: attn [B, 4096], residual [B, 4096], Wo [4096, 4096], post_norm_w [4096]
    ~ N(1, 0.1), Wg, Wu [12288, 4096], Wd [4096, 12288] (weights ~ N(0, 0.02)),
    in that order: the FusedOProjFfnOp forward arguments."""
    r = _Gen(3, device, gen_device)
    return (r.normal(B, 4096), r.normal(B, 4096), r.normal(4096, 4096, std=0.02), r.normal(4096, std=0.1, mean=1.0),
            r.normal(12288, 4096, std=0.02), r.normal(12288, 4096, std=0.02), r.normal(4096, 12288, std=0.02))


def config_l_lens(B: int) -> list[int]:
    """L: the per-sequence KV lengths, U[1024, 16384] from a CPU generator seeded 4."""
    g = torch.Generator().manual_seed(4)
    return torch.randint(1024, SEQ_MAX_L + 1, (B,), generator=g).tolist()


def layer_bytes(batch: int, lens, hidden: int = 4096, inter: int = 12288, heads: int = 32, kv_heads: int = 8,
                head_dim: int = 128) -> int:
    """Algorithmic bytes of one Qwen3 decode-layer step (Qwen3-8B by default):
    every weight once, K and V over ``lens``, the hidden row in and out and the
    decoded token's k/v written."""
    qkv = (heads + 2 * kv_heads) * head_dim
    weights = (qkv * hidden + hidden * heads * head_dim + 3 * inter * hidden) * 2  # 385,875,968 at 8B
    kv = 2 * kv_heads * head_dim * 2 * sum(lens)
    act = batch * hidden * 2 * 2 + batch * 2 * kv_heads * head_dim * 2
    return weights + kv + act


def layer_op(B: int, backend="hip", **op_kw):
    """L's layer op: Qwen3-8B, weighted norms, RoPE theta 1e6, 16384-row cache,
    kv_lens from ``config_l_lens``."""
    from .ops.qwen3_dense_decode import Qwen3DenseDecodeOp

    return Qwen3DenseDecodeOp(B, SEQ_MAX_L, backend=backend, kv_lens=config_l_lens(B), norm_weights=True,
                              rope_theta=1e6, **QWEN3_8B, **op_kw)


def config_l(B: int, device="cuda", gen_device=None, backend="hip", **op_kw):
    """L: (op, data, lens) -- the Qwen3-8B layer op (weighted norms, RoPE theta
    1e6, 16384-row cache, kv_lens from ``config_l_lens``) and its forward
    inputs, drawn in this order: hidden [B, 4096] ~ N(0, 1), K_cache, V_cache
    [B, 8, 16384, 128] ~ N(0, 1), Wqkv [6144, 4096], Wo [4096, 4096], Wgu
    [24576, 4096], Wd [4096, 12288] ~ N(0, 0.02), then the input, q, k and
    post-attention norm weights ~ N(1, 0.1); the RoPE tables follow."""
    from .ops.fused_qk_norm_rope import rope_tables

    lens = config_l_lens(B)
    op = layer_op(B, backend, **op_kw)
    r = _Gen(4, device, gen_device)
    HS, IS, D = 4096, 12288, 128
    data = [r.normal(B, HS), r.normal(B, 8, SEQ_MAX_L, D), r.normal(B, 8, SEQ_MAX_L, D),
            r.normal(6144, HS, std=0.02), r.normal(HS, 4096, std=0.02), r.normal(2 * IS, HS, std=0.02),
            r.normal(HS, IS, std=0.02)]
    for n in (HS, D, D, HS):
        data.append(r.normal(n, std=0.1, mean=1.0))
    data += list(rope_tables(SEQ_MAX_L, D, 1e6, device))
    return op, tuple(data), lens
