"""Synthetic workloads of the hybrid-attention hot path.

Shapes and distributions follow the five workloads the path is measured on:

* GQA decode step: 16 q / 2 kv heads, head_dim 256, bf16 KV cache of
  ``n_past`` tokens drawn N(0,1) (taken as already normed and rotated),
  q|gate, k, v fp32 N(0,1), q_norm / k_norm weights bf16(1 + 0.1 N).
* Gated delta-rule decode step: 16 key / 32 value heads of 128, conv1d over
  8192 channels, k = 4, weights N(0, 0.1) bf16, 3 past conv rows N(0,1),
  a, b N(0,1), A_log U(0, 2.7), dt_bias N(0, 0.1) bf16, state N(0, 0.05).
* GQA prefill and delta-rule prefill over T tokens (per-token tensors are
  the decode tensors at step = token index).
* The 40-layer stack (GQA at layer % 4 == 3) decoding consecutive steps.
* Whole attention layers (input RMSNorm, MLX 4-bit projections, the core,
  the output projection and the residual) on a hidden state of 2048: the
  projection weights are synthetic MLX 4-bit matrices (``mlx4_matrix``).

All arrays are numpy; bf16 tensors are returned as uint16 bits (weights) or
as float32 holding bf16 values (caches), matching what each side consumes.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import synth as S


@dataclass(frozen=True)
class GqaGeom:
    heads: int = 16
    kv_heads: int = 2
    head_dim: int = 256

    @property
    def rd(self) -> int:  # rotary dims, src/attn_qwen.c:298
        return int(self.head_dim * 0.25)


@dataclass(frozen=True)
class LinGeom:
    k_heads: int = 16
    v_heads: int = 32
    kd: int = 128
    vd: int = 128

    @property
    def rows(self) -> int:  # qkv channels, src/attn_qwen.c:866
        return 2 * self.k_heads * self.kd + self.v_heads * self.vd


def gqa_weights(g: GqaGeom, seed: int = 0, layer: int = 0):
    qn = S.bf16_bits(S.normal(seed, S.tid(S.GQA_QNW, layer), g.head_dim, 1.0, 0.1))
    kn = S.bf16_bits(S.normal(seed, S.tid(S.GQA_KNW, layer), g.head_dim, 1.0, 0.1))
    return qn, kn


def gqa_token(g: GqaGeom, seed: int = 0, layer: int = 0, step: int = 0, bf16_inputs=False):
    """q|gate [heads][2*d], k, v [kv_heads][d] of one token (fp32)."""
    q = S.normal(seed, S.tid(S.GQA_QGATE, layer, step), g.heads * 2 * g.head_dim)
    k = S.normal(seed, S.tid(S.GQA_K, layer, step), g.kv_heads * g.head_dim)
    v = S.normal(seed, S.tid(S.GQA_V, layer, step), g.kv_heads * g.head_dim)
    if bf16_inputs:
        q, k, v = S.bf16_round(q), S.bf16_round(k), S.bf16_round(v)
    return (q.reshape(g.heads, 2 * g.head_dim), k.reshape(g.kv_heads, g.head_dim),
            v.reshape(g.kv_heads, g.head_dim))


def gqa_cache(g: GqaGeom, n_past: int, seed: int = 0, layer: int = 0):
    """Past K and V rows [n_past][kv_heads][d], bf16 values held in float32."""
    n = n_past * g.kv_heads * g.head_dim
    kc = S.bf16_round(S.normal(seed, S.tid(S.GQA_KCACHE, layer), n))
    vc = S.bf16_round(S.normal(seed, S.tid(S.GQA_VCACHE, layer), n))
    shp = (n_past, g.kv_heads, g.head_dim)
    return kc.reshape(shp), vc.reshape(shp)


def gqa_prefill_tokens(g: GqaGeom, T: int, seed: int = 0, layer: int = 0):
    """bf16-valued q|gate [T][heads][2d], k, v [T][kv_heads][d]."""
    q = np.empty((T, g.heads, 2 * g.head_dim), np.float32)
    k = np.empty((T, g.kv_heads, g.head_dim), np.float32)
    v = np.empty((T, g.kv_heads, g.head_dim), np.float32)
    for t in range(T):
        q[t], k[t], v[t] = gqa_token(g, seed, layer, t, bf16_inputs=True)
    return q, k, v


@dataclass
class LinWeights:
    conv_w: np.ndarray   # uint16 [rows][4]
    A_log: np.ndarray    # float32 [v_heads]
    dt_bias: np.ndarray  # uint16 [v_heads]
    norm_w: np.ndarray   # uint16 [vd]


def lin_weights(g: LinGeom, seed: int = 0, layer: int = 0) -> LinWeights:
    cw = S.bf16_bits(S.normal(seed, S.tid(S.LIN_CONVW, layer), g.rows * 4, 0.0, 0.1))
    al = S.uniform(seed, S.tid(S.LIN_ALOG, layer), g.v_heads, 0.0, 2.7)
    dt = S.bf16_bits(S.normal(seed, S.tid(S.LIN_DTB, layer), g.v_heads, 0.0, 0.1))
    nw = S.bf16_bits(S.normal(seed, S.tid(S.LIN_NORMW, layer), g.vd, 1.0, 0.1))
    return LinWeights(cw.reshape(g.rows, 4), al, dt, nw)


def lin_state(g: LinGeom, seed: int = 0, layer: int = 0, sigma: float = 0.05):
    """Initial recurrent state [v_heads][kd][vd] (row = key dim)."""
    return S.normal(seed, S.tid(S.LIN_STATE, layer), g.v_heads * g.kd * g.vd, 0.0,
                    sigma).reshape(g.v_heads, g.kd, g.vd)


def lin_conv_history(g: LinGeom, seed: int = 0, layer: int = 0):
    """Three past raw qkv rows (tokens t-3, t-2, t-1), [3][rows]."""
    return S.normal(seed, S.tid(S.LIN_CONVSTATE, layer), 3 * g.rows).reshape(3, g.rows)


def lin_token(g: LinGeom, seed: int = 0, layer: int = 0, step: int = 0):
    """qkv [rows], z [v_heads*vd], a, b [v_heads] of one token (fp32)."""
    qkv = S.normal(seed, S.tid(S.LIN_QKV, layer, step), g.rows)
    z = S.normal(seed, S.tid(S.LIN_Z, layer, step), g.v_heads * g.vd)
    a = S.normal(seed, S.tid(S.LIN_A, layer, step), g.v_heads)
    b = S.normal(seed, S.tid(S.LIN_B, layer, step), g.v_heads)
    return qkv, z, a, b


def lin_tokens(g: LinGeom, T: int, seed: int = 0, layer: int = 0, step0: int = 0):
    qkv = np.empty((T, g.rows), np.float32)
    z = np.empty((T, g.v_heads * g.vd), np.float32)
    a = np.empty((T, g.v_heads), np.float32)
    b = np.empty((T, g.v_heads), np.float32)
    for t in range(T):
        qkv[t], z[t], a[t], b[t] = lin_token(g, seed, layer, step0 + t)
    return qkv, z, a, b


def ring_from_history(g: LinGeom, hist: np.ndarray, token: int) -> np.ndarray:
    """Conv ring [4][rows] holding hist[0..2] as tokens token-3..token-1
    (ring slot = position % 4, src/attn_qwen.c:479)."""
    ring = np.zeros((4, g.rows), np.float32)
    for j in range(3):
        p = token - 3 + j
        if p >= 0:
            ring[p % 4] = hist[j]
    return ring


def stack_kinds(n_layers: int = 40, interval: int = 4):
    """Per-layer kind: 2 = full GQA (layer % interval == interval-1), 1 = linear."""
    return [2 if (L + 1) % interval == 0 else 1 for L in range(n_layers)]


def mlx4_pack(q: np.ndarray) -> np.ndarray:
    """Pack 4-bit values (flattened, row-major) into U32 words of 8 nibbles,
    low nibble first (src/kernels.c:104-113); the tail word is zero-padded."""
    q = np.asarray(q, np.uint32).reshape(-1)
    n = q.size
    qq = np.zeros((n + 7) // 8 * 8, np.uint32)
    qq[:n] = q & 0xF
    qq = qq.reshape(-1, 8)
    return (qq << (4 * np.arange(8, dtype=np.uint32))).sum(axis=1, dtype=np.uint64).astype(np.uint32)


def mlx4_matrix(R: int, C: int, seed: int = 0, layer: int = 0, bias: bool = True,
                scale=(0.002, 0.02)):
    """A synthetic MLX 4-bit affine [R x C] matrix: (vals U32, scales BF16,
    biases BF16 or None).  q uniform in 0..15; per 64-element group a scale
    in U(*scale) and a bias of -scale * U(6, 9), the shape an affine
    quantiser gives a zero-centred weight group (w = q * scale + bias)."""
    n, ng = R * C, (R * C + 63) // 64
    q = (S.draws(seed, S.tid(S.MLX4_Q, layer), 0, n) >> np.uint64(60)).astype(np.uint32)
    sc = S.uniform(seed, S.tid(S.MLX4_SCALE, layer), ng, scale[0], scale[1])
    scales = S.bf16_bits(sc)
    biases = None
    if bias:
        biases = S.bf16_bits(-S.bits_to_f32(scales) * S.uniform(seed, S.tid(S.MLX4_BIAS, layer), ng, 6.0, 9.0))
    return mlx4_pack(q), scales, biases


def mlx4_x(C: int, seed: int = 0, layer: int = 0, step: int = 0) -> np.ndarray:
    """An input vector N(0, 1) of the matvec (fp32)."""
    return S.normal(seed, S.tid(S.MLX4_X, layer, step), C)


@dataclass
class Mlx4W:
    """One MLX 4-bit weight: U32 nibble words, BF16 scales / biases per 64
    elements, decoded shape rows x cols."""
    vals: np.ndarray
    scales: np.ndarray
    biases: np.ndarray | None
    rows: int
    cols: int


# Scales of the layers' projection weights: an affine 4-bit quantiser's
# per-group step for weights of std about 0.02-0.03 (the scale of a 2048-wide
# transformer's projections), so activations stay O(1) through the layer.
PROJ_SCALE = (0.003, 0.010)


def mlx4_weight(R: int, C: int, seed: int = 0, layer: int = 0, j: int = 0) -> Mlx4W:
    """Projection j (0..7) of layer `layer`: its own streams."""
    vals, scales, biases = mlx4_matrix(R, C, seed, 8 * layer + j, scale=PROJ_SCALE)
    return Mlx4W(vals, scales, biases, R, C)


def norm_weight(n: int, seed: int = 0, layer: int = 0) -> np.ndarray:
    """input_layernorm weight bf16(1 + 0.1 N) [n] (uint16 bits)."""
    return S.bf16_bits(S.normal(seed, S.tid(S.BLK_INNORM, layer), n, 1.0, 0.1))


def hidden_state(hidden: int = 2048, seed: int = 0, step: int = 0) -> np.ndarray:
    """A residual-stream vector N(0, 1) [hidden] (fp32)."""
    return S.normal(seed, S.tid(S.BLK_STATE, 0, step), hidden)


@dataclass
class GqaLayerW:
    """Weights of a full-GQA layer step (src/attn_qwen.c:87-225)."""
    in_norm: np.ndarray   # uint16 [hidden]
    q: Mlx4W              # [heads*2*d x hidden] (q | gate per head)
    k: Mlx4W              # [kv_heads*d x hidden]
    v: Mlx4W              # [kv_heads*d x hidden]
    o: Mlx4W              # [hidden x heads*d]
    qn: np.ndarray        # uint16 [d]
    kn: np.ndarray        # uint16 [d]


def gqa_layer_weights(g: GqaGeom, hidden: int = 2048, seed: int = 0, layer: int = 0) -> GqaLayerW:
    qn, kn = gqa_weights(g, seed, layer)
    return GqaLayerW(norm_weight(hidden, seed, layer),
                     mlx4_weight(g.heads * 2 * g.head_dim, hidden, seed, layer, 0),
                     mlx4_weight(g.kv_heads * g.head_dim, hidden, seed, layer, 1),
                     mlx4_weight(g.kv_heads * g.head_dim, hidden, seed, layer, 2),
                     mlx4_weight(hidden, g.heads * g.head_dim, seed, layer, 3), qn, kn)


@dataclass
class LinLayerW:
    """Weights of a gated delta-rule layer step (src/attn_qwen.c:837-968)."""
    in_norm: np.ndarray   # uint16 [hidden]
    qkv: Mlx4W            # [rows x hidden]
    z: Mlx4W              # [v_heads*vd x hidden]
    a: Mlx4W              # [v_heads x hidden]
    b: Mlx4W              # [v_heads x hidden]
    out: Mlx4W            # [hidden x v_heads*vd]
    core: LinWeights


def lin_layer_weights(g: LinGeom, hidden: int = 2048, seed: int = 0, layer: int = 0) -> LinLayerW:
    return LinLayerW(norm_weight(hidden, seed, layer),
                     mlx4_weight(g.rows, hidden, seed, layer, 0),
                     mlx4_weight(g.v_heads * g.vd, hidden, seed, layer, 1),
                     mlx4_weight(g.v_heads, hidden, seed, layer, 2),
                     mlx4_weight(g.v_heads, hidden, seed, layer, 3),
                     mlx4_weight(hidden, g.v_heads * g.vd, seed, layer, 4),
                     lin_weights(g, seed, layer))

