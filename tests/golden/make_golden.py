"""Write tests/golden/golden.npz: tiny known-answer vectors for every op.

The expected outputs are computed by straightforward pure-Python loops over
Python floats (fp64), with bf16 rounding done bit-by-bit through ``struct``;
no numpy or torch arithmetic is involved, so the vectors are an independent
check of the numpy oracle and of the HIP kernels.  Inputs are seeded numpy
draws rounded to bf16.  Semantics follow the reference ops:
ezops/ops/gemv.py:37-38, rmsnorm.py:34-36, fused_o_proj_ffn.py:107-125,
softmax.py:33-34, reduce.py:30-31, attn_decode.py:64-67,
fused_qk_norm_rope.py:119-169, qwen3_dense_decode.py:142-176.

Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

import math
import struct
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "golden.npz"


def f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def bf(x: float) -> float:
    """Round a Python float to fp32, then to bf16 (nearest, ties to even)."""
    (u,) = struct.unpack("<I", struct.pack("<f", x))
    if (u & 0x7FFFFFFF) > 0x7F800000:
        return x
    lsb = (u >> 16) & 1
    u = ((u + 0x7FFF + lsb) & 0xFFFF0000) & 0xFFFFFFFF
    return struct.unpack("<f", struct.pack("<I", u))[0]


def draw(rng, shape, scale=1.0, mean=0.0):
    a = (rng.standard_normal(shape) * scale + mean).astype(np.float32)
    return np.vectorize(bf, otypes=[np.float32])(a)


def dot(a, b):
    return sum(float(x) * float(y) for x, y in zip(a, b))


def rms_inv(row, eps):
    return 1.0 / math.sqrt(sum(float(x) * float(x) for x in row) / len(row) + eps)


def gemv(x, W):
    return [bf(dot(W[n], x)) for n in range(len(W))]


def linear(X, W):
    return [[bf(dot(W[n], X[m])) for n in range(len(W))] for m in range(len(X))]


def rmsnorm_f32(X, eps):
    return [[f32(float(v) * rms_inv(r, eps)) for v in r] for r in X]


def rmsnorm_bf16(X, w, eps):
    out = []
    for r in X:
        s = rms_inv(r, eps)
        out.append([bf(float(v) * s * (1.0 if w is None else float(w[i]))) for i, v in enumerate(r)])
    return out


def softmax(X):
    out = []
    for r in X:
        m = max(float(v) for v in r)
        e = [math.exp(float(v) - m) for v in r]
        t = sum(e)
        out.append([f32(v / t) for v in e])
    return out


def attn(Q, K, V, lens):
    B, H, D = Q.shape
    Hkv = K.shape[1]
    G = H // Hkv
    out = np.zeros((B, H, D), np.float32)
    for b in range(B):
        for h in range(H):
            kv = h // G
            s = [dot(Q[b, h], K[b, kv, p]) / math.sqrt(D) for p in range(lens[b])]
            m = max(s)
            e = [math.exp(x - m) for x in s]
            t = sum(e)
            for d in range(D):
                out[b, h, d] = bf(sum(e[p] * float(V[b, kv, p, d]) for p in range(lens[b])) / t)
    return out


def rope_tables(S, D, theta):
    cos = np.zeros((S, D), np.float32)
    sin = np.zeros((S, D), np.float32)
    for p in range(S):
        for i in range(D // 2):
            inv = f32(1.0 / f32(f32(theta) ** f32(f32(2 * i) / D)))
            ang = f32(f32(p) * inv)
            cos[p, i] = cos[p, i + D // 2] = bf(math.cos(ang))
            sin[p, i] = sin[p, i + D // 2] = bf(math.sin(ang))
    return cos, sin


def norm_rope_head(x, w, c, s, eps):
    D = len(x)
    r = rms_inv(x, eps)
    y = [float(x[i]) * r * float(w[i]) for i in range(D)]
    if c is None:
        return [bf(v) for v in y]
    h = D // 2
    out = []
    for i in range(D):
        rot = -y[i + h] if i < h else y[i - h]
        out.append(bf(y[i] * float(c[i]) + rot * float(s[i])))
    return out


def silu(x):
    return x / (1.0 + math.exp(-x))


def ffn(attn_in, res, Wo, w, Wg, Wu, Wd, eps):
    B = len(attn_in)
    o = linear(attn_in, Wo)
    x2 = [[bf(float(res[m][n]) + o[m][n]) for n in range(len(Wo))] for m in range(B)]
    xn = rmsnorm_bf16(x2, w, eps)
    g, u = linear(xn, Wg), linear(xn, Wu)
    h = [[bf(bf(silu(g[m][i])) * u[m][i]) for i in range(len(Wg))] for m in range(B)]
    d = linear(h, Wd)
    return [[bf(x2[m][n] + d[m][n]) for n in range(len(Wd))] for m in range(B)]


def main():
    rng = np.random.default_rng(20261201)
    eps = 1e-6
    g = {}

    # gemv
    x, W = draw(rng, (16,)), draw(rng, (8, 16), 0.5)
    g.update(gemv_x=x, gemv_W=W, gemv_y=np.array(gemv(x, W), np.float32))

    # rmsnorm fp32 (unweighted) and bf16 weighted
    X = rng.standard_normal((3, 10)).astype(np.float32)
    g.update(rms32_X=X, rms32_out=np.array(rmsnorm_f32(X, eps), np.float32))
    X, w = draw(rng, (2, 16)), draw(rng, (16,), 0.1, 1.0)
    g.update(rmsbf_X=X, rmsbf_w=w, rmsbf_out=np.array(rmsnorm_bf16(X, w, eps), np.float32))

    # softmax, reduce
    X = (rng.standard_normal((3, 10)) * 3).astype(np.float32)
    g.update(softmax_X=X, softmax_out=np.array(softmax(X), np.float32))
    A = rng.uniform(-1, 1, 37).astype(np.float32)
    g.update(reduce_A=A, reduce_out=np.array([f32(math.fsum(float(a) for a in A))], np.float32))

    # attention B=2, H=4, Hkv=2, S=5, D=8, ragged lengths
    Q, K, V = draw(rng, (2, 4, 8)), draw(rng, (2, 2, 5, 8)), draw(rng, (2, 2, 5, 8))
    lens = np.array([5, 3], np.int32)
    g.update(attn_Q=Q, attn_K=K, attn_V=V, attn_lens=lens, attn_out=attn(Q, K, V, lens))

    # qk-norm + rope
    B, H, Hkv, D, S = 2, 4, 2, 8, 6
    q, k, v = draw(rng, (B, H, D)), draw(rng, (B, Hkv, D)), draw(rng, (B, Hkv, D))
    qw, kw = draw(rng, (D,), 0.1, 1.0), draw(rng, (D,), 0.1, 1.0)
    cos, sin = rope_tables(S, D, 1e4)
    pos = np.array([1, 4], np.int32)
    Kc, Vc = draw(rng, (B, Hkv, S, D)), draw(rng, (B, Hkv, S, D))
    qo = np.array([[norm_rope_head(q[b, h], qw, cos[pos[b]], sin[pos[b]], eps) for h in range(H)] for b in range(B)], np.float32)
    ko = np.array([[norm_rope_head(k[b, h], kw, cos[pos[b]], sin[pos[b]], eps) for h in range(Hkv)] for b in range(B)], np.float32)
    g.update(rope_q=q, rope_k=k, rope_v=v, rope_qw=qw, rope_kw=kw, rope_cos=cos, rope_sin=sin,
             rope_pos=pos, rope_Kc=Kc, rope_Vc=Vc, rope_qout=qo, rope_kout=ko)

    # o_proj + ffn: B=2, HS=8, IS=12, QR=8
    a_in, res = draw(rng, (2, 8)), draw(rng, (2, 8))
    Wo, pw = draw(rng, (8, 8), 8 ** -0.5), draw(rng, (8,), 0.1, 1.0)
    Wg, Wu, Wd = draw(rng, (12, 8), 8 ** -0.5), draw(rng, (12, 8), 8 ** -0.5), draw(rng, (8, 12), 12 ** -0.5)
    g.update(ffn_attn=a_in, ffn_res=res, ffn_Wo=Wo, ffn_w=pw, ffn_Wg=Wg, ffn_Wu=Wu, ffn_Wd=Wd,
             ffn_out=np.array(ffn(a_in, res, Wo, pw, Wg, Wu, Wd, eps), np.float32))

    # full layer, Qwen3 mode: B=2, HS=16, IS=24, H=4, Hkv=2, D=8, S=6, lens [6, 3]
    B, HS, IS, H, Hkv, D, S = 2, 16, 24, 4, 2, 8, 6
    QR, KVR = H * D, Hkv * D
    hid = draw(rng, (B, HS))
    Kc, Vc = draw(rng, (B, Hkv, S, D)), draw(rng, (B, Hkv, S, D))
    Wqkv = draw(rng, (QR + 2 * KVR, HS), HS ** -0.5)
    Wo = draw(rng, (HS, QR), QR ** -0.5)
    Wgu = draw(rng, (2 * IS, HS), HS ** -0.5)
    Wd = draw(rng, (HS, IS), IS ** -0.5)
    inw, qw, kw, pw = (draw(rng, (n,), 0.1, 1.0) for n in (HS, D, D, HS))
    cos, sin = rope_tables(S, D, 1e4)
    lens = np.array([6, 3], np.int32)
    xn = rmsnorm_bf16(hid, inw, eps)
    qkv = linear(xn, Wqkv)
    Kn, Vn = Kc.copy(), Vc.copy()
    qn = np.zeros((B, H, D), np.float32)
    for b in range(B):
        p = lens[b] - 1
        for h in range(H):
            qn[b, h] = norm_rope_head(qkv[b][h * D:(h + 1) * D], qw, cos[p], sin[p], eps)
        for h in range(Hkv):
            Kn[b, h, p] = norm_rope_head(qkv[b][QR + h * D:QR + (h + 1) * D], kw, cos[p], sin[p], eps)
            Vn[b, h, p] = qkv[b][QR + KVR + h * D:QR + KVR + (h + 1) * D]
    att = attn(qn, Kn, Vn, lens).reshape(B, QR)
    out = ffn(att, hid, Wo, pw, Wgu[:IS], Wgu[IS:], Wd, eps)
    g.update(layer_hidden=hid, layer_Kc=Kc, layer_Vc=Vc, layer_Wqkv=Wqkv, layer_Wo=Wo, layer_Wgu=Wgu,
             layer_Wd=Wd, layer_inw=inw, layer_qw=qw, layer_kw=kw, layer_pw=pw, layer_cos=cos,
             layer_sin=sin, layer_lens=lens, layer_out=np.array(out, np.float32), layer_Kc_out=Kn,
             layer_Vc_out=Vn)

    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT} ({len(g)} arrays)")


if __name__ == "__main__":
    main()
