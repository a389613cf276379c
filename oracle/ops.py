"""numpy restatement of the reference's ``_ref_forward`` semantics.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Every function cites the
reference file:line it restates.  Arrays are float32 numpy arrays; bf16
tensors are represented by float32 arrays whose values are exactly
bf16-representable, and ``bf16()`` performs the round-to-nearest-even
conversion the reference's ``.to(torch.bfloat16)`` and bf16 tensor
arithmetic perform.  Matrix products accumulate in fp32 (BLAS), matching
the fp32-accumulated bf16 matmuls of the reference; statistics that the
reference keeps in fp32 are evaluated in fp64 and rounded to fp32.

How each function is pinned (tests/test_oracle.py):
  bf16             torch .to(bfloat16) on random and special values
  gemv             pure-Python loops; torch.mv (fp64)
  rmsnorm_f32      torch.nn.functional.rms_norm; unit-RMS invariant
  rmsnorm_bf16     pure-Python loops; torch rms_norm with weight
  softmax          torch.softmax; rows sum to one
  reduce_sum       math.fsum
  attn_decode      torch SDPA (MATH backend, enable_gqa); S=1 returns V;
                   output inside [min V, max V]; G=1 equals MHA; kv_lens
                   equals truncating the cache
  prefill_attn     each token equals attn_decode with kv_len = past + i + 1;
                   torch SDPA is_causal on a fresh prompt
  paged_attn_decode  gather map: scatter/gather identity over a random page
                   permutation, one-page reshape, shared pages; equals
                   attn_decode bit-for-bit on the scattered cache
  qk_norm_rope     pure-Python loops; position 0 is identity; RoPE keeps
                   each (i, i+D/2) pair's norm; cache slot isolation
  o_proj_ffn       pure-Python loops (committed golden vectors)
  qwen3_layer      composition of the pinned functions above; pure-Python
                   loops on a tiny layer (committed golden vectors)
  qwen3_prefill    one token per sequence equals qwen3_layer; a prompt
                   prefilled in two chunks equals it in one
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "bf16", "gemv", "linear_bf16", "rmsnorm_f32", "rmsnorm_bf16", "softmax", "reduce_sum", "attn_decode",
    "paged_to_contiguous", "paged_attn_decode", "prefill_attn", "rope_tables", "qk_norm_rope", "o_proj_ffn",
    "qwen3_layer", "qwen3_prefill",
]


def bf16(x) -> np.ndarray:
    """fp32 -> bf16 (round to nearest, ties to even), returned as fp32 values."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) & np.uint32(0xFFFF0000)
    r = np.where(nan, (u | np.uint32(0x00400000)) & np.uint32(0xFFFF0000), r).astype(np.uint32)
    return r.view(np.float32)


def _f32(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32)


def gemv(x, W) -> np.ndarray:
    """``C = A @ B`` with bf16 output (ezops/ops/gemv.py:37-38); W is [N, K] here."""
    return bf16(_f32(W) @ _f32(x))


def linear_bf16(X, W) -> np.ndarray:
    """bf16 ``X @ W.T`` with fp32 accumulation and one bf16 rounding."""
    return bf16(_f32(X) @ _f32(W).T)


def _rsqrt_mean_sq(x, eps) -> np.ndarray:
    x64 = np.asarray(x, dtype=np.float64)
    ms = np.mean(x64 * x64, axis=-1, keepdims=True)
    return (1.0 / np.sqrt(ms + eps)).astype(np.float32)


def rmsnorm_f32(X, eps=1e-6) -> np.ndarray:
    """``X * rsqrt(mean(X^2) + eps)`` (ezops/ops/rmsnorm.py:34-36)."""
    x64 = np.asarray(X, dtype=np.float64)
    return (x64 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + eps)).astype(np.float32)


def rmsnorm_bf16(X, W=None, eps=1e-6) -> np.ndarray:
    """``(x * rsqrt(var + eps) * w).to(bf16)`` with fp32 statistics.

    ezops/ops/fused_o_proj_ffn.py:107-110 (weighted) and
    ezops/ops/qwen3_dense_decode.py:137-140 (W None = unit weight).
    """
    x = _f32(X)
    y = x * _rsqrt_mean_sq(x, eps)
    if W is not None:
        y = y * _f32(W)
    return bf16(y)


def softmax(X) -> np.ndarray:
    """``torch.softmax(X, -1)`` (ezops/ops/softmax.py:33-34), evaluated in fp64."""
    x = np.asarray(X, dtype=np.float64)
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)


def reduce_sum(A) -> np.ndarray:
    """``Out.copy_(A.sum())`` (ezops/ops/reduce.py:30-31), fp64 accumulation."""
    return np.array([np.sum(np.asarray(A, dtype=np.float64))], dtype=np.float32)


def attn_decode(Q, K, V, kv_lens=None, scale=None) -> np.ndarray:
    """GQA decode SDPA (ezops/ops/attn_decode.py:64-67): Q [B,H,D], K/V [B,Hkv,S,D].

    Query head h attends kv head h // (H/Hkv) (``enable_gqa``); scores,
    softmax and the value sum in fp32; output rounded to bf16.  ``kv_lens``
    restricts sequence b to slots [0, kv_lens[b]).
    """
    Q, K, V = _f32(Q), _f32(K), _f32(V)
    B, H, D = Q.shape
    Hkv, S = K.shape[1], K.shape[2]
    G = H // Hkv
    scale = D ** -0.5 if scale is None else scale
    q = Q.reshape(B, Hkv, G, D)
    s = np.matmul(q, np.swapaxes(K, -1, -2)) * np.float32(scale)  # [B,Hkv,G,S]
    if kv_lens is not None:
        mask = np.arange(S)[None, :] >= np.asarray(kv_lens)[:, None]
        s = np.where(mask[:, None, None, :], -np.inf, s)
    s64 = s.astype(np.float64)
    p = np.exp(s64 - s64.max(axis=-1, keepdims=True))
    p = (p / p.sum(axis=-1, keepdims=True)).astype(np.float32)
    o = np.matmul(p, V)  # [B,Hkv,G,D]
    return bf16(o.reshape(B, H, D))


def paged_to_contiguous(pages, block_table, page_size):
    """Gather a page pool [P, Hkv, page_size, D] through block_table [B, M] into
    the contiguous cache [B, Hkv, M*page_size, D] (row t of sequence b is row
    t % page_size of pool page block_table[b, t // page_size]).  The
    reference has no paged cache (ezops/ops/attn_decode.py:60-61 takes one
    contiguous [B, Hkv, S, D] tensor); this is the layout map alone."""
    pages = np.asarray(pages)
    bt = np.asarray(block_table)
    g = pages[bt]  # [B, M, Hkv, page_size, D]
    B, M, Hkv, P, D = g.shape
    return np.ascontiguousarray(g.transpose(0, 2, 1, 3, 4).reshape(B, Hkv, M * P, D))


def paged_attn_decode(Q, K_pages, V_pages, block_table, kv_lens, page_size, scale=None) -> np.ndarray:
    """GQA decode SDPA over a paged cache: ``attn_decode`` on the gathered cache."""
    K = paged_to_contiguous(K_pages, block_table, page_size)
    V = paged_to_contiguous(V_pages, block_table, page_size)
    return attn_decode(Q, K, V, kv_lens, scale)


def prefill_attn(Q, K, V, q_lens, past_lens=None, scale=None) -> np.ndarray:
    """Causal GQA attention of new tokens over the cache.  Q [T, H, D] holds
    the sequences' new tokens back to back (q_lens[b] rows each); token i of
    sequence b sits at cache row past_lens[b] + i of K/V [B, Hkv, S, D] and
    attends rows [0, past_lens[b] + i] — per token, the decode formula of
    ezops/ops/attn_decode.py:64-67 with kv_len = past + i + 1.  fp32 scores,
    fp64 softmax, output rounded to bf16."""
    Q, K, V = _f32(Q), _f32(K), _f32(V)
    T, H, D = Q.shape
    Hkv = K.shape[1]
    G = H // Hkv
    scale = D ** -0.5 if scale is None else scale
    past_lens = [0] * len(q_lens) if past_lens is None else past_lens
    out = np.zeros((T, H, D), dtype=np.float32)
    t0 = 0
    for b, (n, p) in enumerate(zip(q_lens, past_lens)):
        L = p + n
        q = Q[t0:t0 + n].reshape(n, Hkv, G, D).transpose(1, 2, 0, 3)  # [Hkv, G, n, D]
        s = np.matmul(q, np.swapaxes(K[b, :, :L], -1, -2)[:, None]) * np.float32(scale)  # [Hkv, G, n, L]
        mask = np.arange(L)[None, :] > (p + np.arange(n))[:, None]
        s = np.where(mask, -np.inf, s).astype(np.float64)
        w = np.exp(s - s.max(axis=-1, keepdims=True))
        w = (w / w.sum(axis=-1, keepdims=True)).astype(np.float32)
        o = np.matmul(w, V[b, :, :L][:, None])  # [Hkv, G, n, D]
        out[t0:t0 + n] = o.transpose(2, 0, 1, 3).reshape(n, H, D)
        t0 += n
    return bf16(out)


def rope_tables(max_seq_len, head_dim, theta=1e6):
    """HF bf16 cos/sin tables (ezops/ops/fused_qk_norm_rope.py:119-125), fp32 angles."""
    inv_freq = (1.0 / (np.float32(theta) ** (np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim)))).astype(np.float32)
    ang = np.arange(max_seq_len, dtype=np.float32)[:, None] * inv_freq[None, :]
    cos = np.cos(ang.astype(np.float64)).astype(np.float32)
    sin = np.sin(ang.astype(np.float64)).astype(np.float32)
    return bf16(np.concatenate([cos, cos], -1)), bf16(np.concatenate([sin, sin], -1))


def _head_norm_rope(x, w, cos_p, sin_p, eps):
    """fp32 RMSNorm*w then rotate_half RoPE, one bf16 rounding (:138-147)."""
    x = _f32(x)
    y = (x * _rsqrt_mean_sq(x, eps)) * _f32(w)
    if cos_p is None:
        return bf16(y)
    half = y.shape[-1] // 2
    rot = np.concatenate([-y[..., half:], y[..., :half]], axis=-1)
    return bf16(y * cos_p + rot * sin_p)


def qk_norm_rope(q, k, v, q_norm_w, k_norm_w, cos, sin, K_cache, V_cache, positions, eps=1e-6):
    """Fused QK-norm + RoPE + cache write (ezops/ops/fused_qk_norm_rope.py:149-169).

    q [B,H,D], k/v [B,Hkv,D]; ``positions`` is an int or one int per sequence.
    cos/sin None skips RoPE.  Returns (q_out, k_out, K_cache', V_cache') with
    new cache arrays (inputs are not modified).
    """
    B = q.shape[0]
    pos = np.broadcast_to(np.asarray(positions, dtype=np.int64), (B,))
    cp = None if cos is None else _f32(cos)[pos][:, None, :]
    sp = None if sin is None else _f32(sin)[pos][:, None, :]
    q_out = _head_norm_rope(q, q_norm_w, cp, sp, eps)
    k_out = _head_norm_rope(k, k_norm_w, cp, sp, eps)
    Kc, Vc = _f32(K_cache).copy(), _f32(V_cache).copy()
    for b in range(B):
        Kc[b, :, pos[b], :] = k_out[b]
        Vc[b, :, pos[b], :] = _f32(v)[b]
    return q_out, k_out, Kc, Vc


def _silu(x):
    x64 = np.asarray(x, dtype=np.float64)
    return (x64 / (1.0 + np.exp(-x64))).astype(np.float32)


def o_proj_ffn(attn, residual, Wo, post_norm_w, Wg, Wu, Wd, eps=1e-6) -> np.ndarray:
    """bf16-staged o_proj + RMSNorm + SwiGLU (ezops/ops/fused_o_proj_ffn.py:112-125)."""
    x2 = bf16(_f32(residual) + linear_bf16(attn, Wo))
    xn = rmsnorm_bf16(x2, post_norm_w, eps)
    gate, up = linear_bf16(xn, Wg), linear_bf16(xn, Wu)
    h = bf16(bf16(_silu(gate)) * up)
    return bf16(x2 + linear_bf16(h, Wd))


def qwen3_layer(hidden, K_cache, V_cache, Wqkv, Wo, Wgu, Wd, num_heads, num_kv_heads, head_dim,
                kv_lens=None, in_norm_w=None, q_norm_w=None, k_norm_w=None, post_norm_w=None,
                cos=None, sin=None, eps=1e-6):
    """One Qwen3 dense decode step (ezops/ops/qwen3_dense_decode.py:142-176).

    Reference mode: kv_lens None (new token in slot S-1, attend all S), unit
    norm weights, no RoPE.  Qwen3 mode: per-sequence kv_lens (token at
    kv_len-1), norm weights, and RoPE at the token position with q/k norm +
    RoPE as in the fused QK-norm+RoPE op.  Returns (out, K_cache', V_cache').
    """
    hidden = _f32(hidden)
    B, HS = hidden.shape
    S = K_cache.shape[2]
    D = head_dim
    QR, KVR = num_heads * D, num_kv_heads * D
    IS = Wd.shape[1]
    lens = np.full(B, S, dtype=np.int64) if kv_lens is None else np.asarray(kv_lens, dtype=np.int64)

    x = rmsnorm_bf16(hidden, in_norm_w, eps)
    qkv = linear_bf16(x, Wqkv)
    q = qkv[:, :QR].reshape(B, num_heads, D)
    k = qkv[:, QR:QR + KVR].reshape(B, num_kv_heads, D)
    v = qkv[:, QR + KVR:].reshape(B, num_kv_heads, D)
    ones = np.ones(D, dtype=np.float32)
    qn, _, Kc, Vc = qk_norm_rope(q, k, v, ones if q_norm_w is None else q_norm_w,
                                 ones if k_norm_w is None else k_norm_w, cos, sin, K_cache, V_cache,
                                 lens - 1, eps)
    att = attn_decode(qn, Kc, Vc, None if kv_lens is None else lens)
    Wgu = _f32(Wgu)
    out = o_proj_ffn(att.reshape(B, QR), hidden, Wo, post_norm_w if post_norm_w is not None else np.ones(HS, np.float32),
                     Wgu[:IS], Wgu[IS:], Wd, eps)
    return out, Kc, Vc


def qwen3_prefill(hidden, K_cache, V_cache, Wqkv, Wo, Wgu, Wd, num_heads, num_kv_heads, head_dim, q_lens,
                  past_lens=None, in_norm_w=None, q_norm_w=None, k_norm_w=None, post_norm_w=None, cos=None,
                  sin=None, eps=1e-6):
    """Prefill of a chunk of new tokens through one Qwen3 dense layer: the
    decode layer's stages (ezops/ops/qwen3_dense_decode.py:142-176) applied to
    every token, each token's k/v written at cache row past + i of its
    sequence and its query attending rows [0, past + i] (``prefill_attn``).
    hidden [T, HS] holds the sequences' tokens back to back.  Returns
    (out [T, HS], K_cache', V_cache')."""
    hidden = _f32(hidden)
    T, HS = hidden.shape
    D = head_dim
    QR, KVR = num_heads * D, num_kv_heads * D
    IS = Wd.shape[1]
    past_lens = [0] * len(q_lens) if past_lens is None else list(past_lens)
    seq = np.repeat(np.arange(len(q_lens)), q_lens)
    pos = np.concatenate([p + np.arange(n) for n, p in zip(q_lens, past_lens)]).astype(np.int64) if T else \
        np.zeros(0, np.int64)
    x = rmsnorm_bf16(hidden, in_norm_w, eps)
    qkv = linear_bf16(x, Wqkv)
    q = qkv[:, :QR].reshape(T, num_heads, D)
    k = qkv[:, QR:QR + KVR].reshape(T, num_kv_heads, D)
    v = qkv[:, QR + KVR:].reshape(T, num_kv_heads, D)
    ones = np.ones(D, dtype=np.float32)
    cp = None if cos is None else _f32(cos)[pos][:, None, :]
    sp = None if sin is None else _f32(sin)[pos][:, None, :]
    qn = _head_norm_rope(q, ones if q_norm_w is None else q_norm_w, cp, sp, eps)
    kn = _head_norm_rope(k, ones if k_norm_w is None else k_norm_w, cp, sp, eps)
    Kc, Vc = _f32(K_cache).copy(), _f32(V_cache).copy()
    Kc[seq, :, pos, :] = kn
    Vc[seq, :, pos, :] = _f32(v)
    att = prefill_attn(qn, Kc, Vc, q_lens, past_lens)
    Wgu = _f32(Wgu)
    out = o_proj_ffn(att.reshape(T, QR), hidden, Wo, post_norm_w if post_norm_w is not None else np.ones(HS, np.float32),
                     Wgu[:IS], Wgu[IS:], Wd, eps)
    return out, Kc, Vc
