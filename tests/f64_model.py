"""Independent double-precision statement of the attention cores.

Written from the mathematics of the Qwen3.5 hybrid attention (not from the
C restatement): vectorised numpy in float64.  It pins the oracle: the oracle
computes in float32 with the reference's operation order, so the two must
agree to float32 rounding; a dropped term, a wrong sign, a swapped head
mapping, interleaved instead of half-split RoPE or an eps in the wrong place
shows up as an O(1e-2..1) difference instead.
"""
from __future__ import annotations

import numpy as np


def bf(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def rmsnorm(x, w=None, eps=1e-6):
    x = np.asarray(x, np.float64)
    y = x / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    return y if w is None else y * w


def rope(x, pos, rd, theta=1e7):
    """Half-split rotary on the first rd dims: pairs (i, i + rd/2)."""
    x = np.array(x, np.float64)
    half = rd // 2
    inv = 1.0 / theta ** (2.0 * np.arange(half) / rd)
    ang = pos * inv
    c, s = np.cos(ang), np.sin(ang)
    a, b = x[..., :half].copy(), x[..., half:rd].copy()
    x[..., :half] = a * c - b * s
    x[..., half:rd] = a * s + b * c
    return x


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))


def gqa_step(kc, vc, q_gate, k, v, qn_w, kn_w, token):
    """kc, vc: [token][kvh][d] past rows (already normed/rotated).
    Returns (out [H][d], k_new [kvh][d])."""
    H, d2 = q_gate.shape
    d = d2 // 2
    kvh = k.shape[0]
    rd = int(d * 0.25)
    q = rope(rmsnorm(q_gate[:, :d], bf(qn_w)), token, rd)
    kn = rope(rmsnorm(k, bf(kn_w)), token, rd)
    K = np.concatenate([np.asarray(kc, np.float64), kn[None]], 0)
    V = np.concatenate([np.asarray(vc, np.float64), np.asarray(v, np.float64)[None]], 0)
    out = np.zeros((H, d))
    for h in range(H):
        g = h // (H // kvh)
        s = K[:, g] @ q[h] / np.sqrt(d)
        w = np.exp(s - s.max())
        out[h] = (w / w.sum()) @ V[:, g]
    return out * sigmoid(q_gate[:, d:]), kn


def gqa_prefill(q_gate, k, v, qn_w, kn_w, t0=0, kc=None, vc=None):
    """Causal prefill over T tokens starting at position t0 (past rows kc/vc)."""
    T, H, d2 = q_gate.shape
    d = d2 // 2
    rd = int(d * 0.25)
    pos = t0 + np.arange(T)
    q = np.stack([rope(rmsnorm(q_gate[t, :, :d], bf(qn_w)), pos[t], rd) for t in range(T)])
    kn = np.stack([rope(rmsnorm(k[t], bf(kn_w)), pos[t], rd) for t in range(T)])
    K = kn if kc is None else np.concatenate([kc, kn], 0)
    V = np.asarray(v, np.float64) if vc is None else np.concatenate([vc, v], 0)
    kvh = k.shape[1]
    out = np.zeros((T, H, d))
    for h in range(H):
        g = h // (H // kvh)
        s = q[:, h] @ K[:, g].T / np.sqrt(d)                  # [T][t0+T]
        mask = np.arange(K.shape[0])[None, :] <= pos[:, None]
        s = np.where(mask, s, -np.inf)
        w = np.exp(s - s.max(1, keepdims=True))
        out[:, h] = (w / w.sum(1, keepdims=True)) @ V[:, g]
    return out * sigmoid(q_gate[:, :, d:]), kn


def lin_step(ring_hist, S, qkv, z, a, b, conv_w, A_log, dt_bias, norm_w, kh, vh, kd, vd):
    """ring_hist: [3][rows] raw rows of tokens t-3..t-1 (zeros where absent).
    S: [vh][kd][vd].  Returns (out [vh*vd], S_new, qkv_post)."""
    rows = qkv.shape[0]
    W = bf(conv_w).reshape(rows, 4)
    X = np.concatenate([np.asarray(ring_hist, np.float64), np.asarray(qkv, np.float64)[None]], 0)
    acc = (X.T * W).sum(1)
    post = acc * sigmoid(acc)
    q = rmsnorm(post[:kh * kd].reshape(kh, kd)) / kd
    k = rmsnorm(post[kh * kd:2 * kh * kd].reshape(kh, kd)) / np.sqrt(kd)
    v = post[2 * kh * kd:].reshape(vh, vd)
    x = np.asarray(a, np.float64) + bf(dt_bias)
    g = -np.exp(np.asarray(A_log, np.float64)) * np.logaddexp(0.0, x)
    beta = sigmoid(b)
    Sn = np.array(S, np.float64) * np.exp(g)[:, None, None]
    kk = np.repeat(k, 2, axis=0)                 # value head h <- key head h // 2
    qq = np.repeat(q, 2, axis=0)
    mem = np.einsum("hij,hi->hj", Sn, kk)
    delta = (v - mem) * beta[:, None]
    Sn = Sn + kk[:, :, None] * delta[:, None, :]
    o = np.einsum("hij,hi->hj", Sn, qq)
    zz = np.asarray(z, np.float64).reshape(vh, vd)
    out = rmsnorm(o, bf(norm_w)) * (zz * sigmoid(zz))
    qkv_post = np.concatenate([q.reshape(-1), k.reshape(-1), v.reshape(-1)])
    return out.reshape(-1), Sn, qkv_post


def mlx4_dense(w):
    """Dense float64 [rows][cols] of an MLX 4-bit weight (attributes vals,
    scales, biases, rows, cols), decoded from the format's definition:
    element k = r*cols + c is nibble k % 8 (low first) of word k / 8, and
    w = q * scale + bias with the BF16 scale / bias of group k / 64."""
    n = w.rows * w.cols
    k = np.arange(n, dtype=np.int64)
    vals = np.asarray(w.vals, np.uint32)
    q = ((vals[k >> 3] >> (4 * (k & 7)).astype(np.uint32)) & 0xF).astype(np.float64)
    dense = q * bf(w.scales)[k // 64]
    if w.biases is not None:
        dense += bf(w.biases)[k // 64]
    return dense.reshape(w.rows, w.cols)


def gqa_block(kc, vc, state, w, token, heads, kv_heads, d):
    """A full-GQA layer on the residual stream: state + o_proj(attn(
    input_layernorm(state))).  Returns (new state, k_new normed + rotated)."""
    xin = rmsnorm(state, bf(w.in_norm))
    qg = (mlx4_dense(w.q) @ xin).reshape(heads, 2 * d)
    k = (mlx4_dense(w.k) @ xin).reshape(kv_heads, d)
    v = (mlx4_dense(w.v) @ xin).reshape(kv_heads, d)
    out, kn = gqa_step(kc, vc, qg, k, v, w.qn, w.kn, token)
    return np.asarray(state, np.float64) + mlx4_dense(w.o) @ out.reshape(-1), kn, v


def lin_block(ring_hist, S, state, w, kh, vh, kd, vd):
    """A gated delta-rule layer on the residual stream: state +
    out_proj(core(input_layernorm(state))).  Returns (new state, S_new,
    raw qkv of this token)."""
    xin = rmsnorm(state, bf(w.in_norm))
    qkv = mlx4_dense(w.qkv) @ xin
    z = mlx4_dense(w.z) @ xin
    a = mlx4_dense(w.a) @ xin
    b = mlx4_dense(w.b) @ xin
    c = w.core
    out, Sn, _ = lin_step(ring_hist, S, qkv, z, a, b, c.conv_w, c.A_log, c.dt_bias, c.norm_w,
                          kh, vh, kd, vd)
    return np.asarray(state, np.float64) + mlx4_dense(w.out) @ out, Sn, qkv
