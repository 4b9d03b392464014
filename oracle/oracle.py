"""ctypes binding of the CPU restatement (liborc_q35.so).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, by __graft_entry__.smoke() and
by bench.py's cpu_baseline leg, always as the checker or the timed CPU
baseline, never as a path that produces product results.  The C sources it
binds (q35_oracle.c) restate src/attn_qwen.c gqa_body (:235-397) and
lin_body (:434-764) with the projections removed, and the MLX 4-bit matvec
of src/kernels.c (:118-219) that the projections and the output head use.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liborc_q35.so")

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_lib = None


def build() -> str:
    """Compile liborc_q35.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-B", "-C", HERE, "liborc_q35.so"], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        i = ctypes.c_int
        L.orc_gqa_body.argtypes = [i, i, i, i, _f32p, i, _f32p, _f32p, _f32p, _u16p, _u16p, _f32p]
        L.orc_gqa_body.restype = i
        L.orc_lin_body.argtypes = [i, i, i, i, i, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                                   _u16p, _f32p, _u16p, _u16p, _f32p]
        L.orc_lin_body.restype = i
        L.orc_gqa_prefill.argtypes = [i, i, i, i, _f32p, i, i, _f32p, _f32p, _f32p, _u16p, _u16p,
                                      _f32p]
        L.orc_gqa_prefill.restype = i
        L.orc_lin_prefill.argtypes = [i, i, i, i, i, i, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                                      _u16p, _f32p, _u16p, _u16p, _f32p]
        L.orc_lin_prefill.restype = i
        L.orc_gqa_cache_row.argtypes = [i, i, i, _f32p, _f32p, _u16p, _f32p]
        L.orc_gqa_cache_row.restype = None
        L.orc_rope_table.argtypes = [i, i, ctypes.c_double, _f32p, _f32p]
        L.orc_rope_table.restype = None
        L.orc_rmsnorm.argtypes = [_u16p, i, _f32p]
        L.orc_rmsnorm.restype = None
        vp = ctypes.c_void_p
        L.orc_mlx4_decode.argtypes = [vp, vp, vp, i, vp]
        L.orc_mlx4_decode.restype = None
        L.orc_mlx4_matvec.argtypes = [vp, vp, vp, i, i, vp, vp]
        L.orc_mlx4_matvec.restype = None
        mp = ctypes.POINTER(_Mlx4)
        L.orc_gqa_step.argtypes = [i, i, i, i, _f32p, i, i, _f32p, vp, mp, mp, mp, mp, _u16p, _u16p]
        L.orc_gqa_step.restype = i
        L.orc_lin_step.argtypes = [i, i, i, i, i, i, i, _f32p, _f32p, _f32p, vp, mp, mp, mp, mp, mp,
                                   _u16p, _f32p, _u16p, _u16p]
        L.orc_lin_step.restype = i
        L.orc_gqa_chunk.argtypes = [i, i, i, i, _f32p, i, i, i, _f32p, vp, mp, mp, mp, mp, _u16p,
                                    _u16p]
        L.orc_gqa_chunk.restype = i
        L.orc_lin_chunk.argtypes = [i, i, i, i, i, i, i, i, _f32p, _f32p, _f32p, vp, mp, mp, mp,
                                    mp, mp, _u16p, _f32p, _u16p, _u16p]
        L.orc_lin_chunk.restype = i
        _lib = L
    return _lib


class _Mlx4(ctypes.Structure):
    """OrcMlx4: one MLX 4-bit weight (q35_oracle.h)."""
    _fields_ = [("vals", ctypes.c_void_p), ("scales", ctypes.c_void_p),
                ("biases", ctypes.c_void_p), ("rows", ctypes.c_int), ("cols", ctypes.c_int)]


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def gqa_body(kv_layer, token, q, k, v, qn_w, kn_w, heads, kv_heads, head_dim):
    """One decode token.  kv_layer [max_tokens][2*kv_heads*head_dim] fp32 is
    updated in place; returns (attn_out [heads*head_dim], k after norm+RoPE)."""
    assert kv_layer.dtype == np.float32 and kv_layer.flags["C_CONTIGUOUS"]
    k = _c(k, np.float32).reshape(-1).copy()
    out = np.zeros(heads * head_dim, np.float32)
    rc = lib().orc_gqa_body(heads, kv_heads, head_dim, kv_layer.shape[0], kv_layer, token,
                            _c(q, np.float32), k, _c(v, np.float32), _c(qn_w, np.uint16),
                            _c(kn_w, np.uint16), out)
    if rc != 0:
        raise RuntimeError("orc_gqa_body failed")
    return out, k


def gqa_prefill(kv_layer, t0, q, k, v, qn_w, kn_w, heads, kv_heads, head_dim):
    B = q.shape[0]
    k = _c(k, np.float32).reshape(B, -1).copy()
    out = np.zeros((B, heads * head_dim), np.float32)
    rc = lib().orc_gqa_prefill(heads, kv_heads, head_dim, kv_layer.shape[0], kv_layer, t0, B,
                               _c(q, np.float32), k, _c(v, np.float32), _c(qn_w, np.uint16),
                               _c(kn_w, np.uint16), out)
    if rc != 0:
        raise RuntimeError("orc_gqa_prefill failed")
    return out, k


def lin_body(conv_ring, S, token, qkv, z, a, b, conv_w, A_log, dt_bias, norm_w,
             k_heads, v_heads, kd, vd):
    """One decode token.  conv_ring [4][rows] and S [v_heads][kd][vd] are
    updated in place; returns (out [v_heads*vd], qkv after conv + norm)."""
    assert conv_ring.dtype == np.float32 and conv_ring.flags["C_CONTIGUOUS"]
    assert S.dtype == np.float32 and S.flags["C_CONTIGUOUS"]
    qkv = _c(qkv, np.float32).reshape(-1).copy()
    out = np.zeros(v_heads * vd, np.float32)
    rc = lib().orc_lin_body(k_heads, v_heads, kd, vd, token, conv_ring, S, qkv,
                            _c(z, np.float32), _c(a, np.float32), _c(b, np.float32),
                            _c(conv_w, np.uint16), _c(A_log, np.float32), _c(dt_bias, np.uint16),
                            _c(norm_w, np.uint16), out)
    if rc != 0:
        raise RuntimeError("orc_lin_body failed")
    return out, qkv


def lin_prefill(conv_ring, S, t0, qkv, z, a, b, conv_w, A_log, dt_bias, norm_w,
                k_heads, v_heads, kd, vd):
    B = qkv.shape[0]
    qkv = _c(qkv, np.float32).copy()
    out = np.zeros((B, v_heads * vd), np.float32)
    rc = lib().orc_lin_prefill(k_heads, v_heads, kd, vd, t0, B, conv_ring, S, qkv,
                               _c(z, np.float32), _c(a, np.float32), _c(b, np.float32),
                               _c(conv_w, np.uint16), _c(A_log, np.float32),
                               _c(dt_bias, np.uint16), _c(norm_w, np.uint16), out)
    if rc != 0:
        raise RuntimeError("orc_lin_prefill failed")
    return out, qkv


def gqa_cache_rows(k, v, kn_w, t0, kv_heads, head_dim):
    """fp32 cache rows of tokens t0.. (k normed + rotated, v raw), [B][2*kvh*d]."""
    B = k.shape[0]
    rows = np.zeros((B, 2 * kv_heads * head_dim), np.float32)
    kk = _c(k, np.float32).reshape(B, -1).copy()
    vv = _c(v, np.float32).reshape(B, -1)
    knw = _c(kn_w, np.uint16)
    for b in range(B):
        kb = kk[b].copy()
        out = np.zeros(2 * kv_heads * head_dim, np.float32)
        lib().orc_gqa_cache_row(kv_heads, head_dim, t0 + b, kb, np.ascontiguousarray(vv[b]), knw,
                                out)
        rows[b] = out
    return rows


def rope_table(token, rd=64, theta=1e7):
    c = np.zeros(rd // 2, np.float32)
    s = np.zeros(rd // 2, np.float32)
    lib().orc_rope_table(token, rd, theta, c, s)
    return c, s


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def mlx4_decode(vals, scales, biases, n):
    """Dequantised elements 0..n-1 of an MLX 4-bit matrix (flattened)."""
    vals, scales = _c(vals, np.uint32), _c(scales, np.uint16)
    biases = None if biases is None else _c(biases, np.uint16)
    out = np.empty(n, np.float32)
    lib().orc_mlx4_decode(_ptr(vals), _ptr(scales), _ptr(biases), n, _ptr(out))
    return out


def mlx4_matvec(vals, scales, biases, R, C, x):
    """y = W x for the MLX 4-bit [R x C] matrix (vals, scales, biases)."""
    vals, scales, x = _c(vals, np.uint32), _c(scales, np.uint16), _c(x, np.float32)
    biases = None if biases is None else _c(biases, np.uint16)
    assert vals.size >= (R * C + 7) // 8 and scales.size >= (R * C + 63) // 64 and x.size >= C
    y = np.empty(R, np.float32)
    lib().orc_mlx4_matvec(_ptr(vals), _ptr(scales), _ptr(biases), R, C, _ptr(x), _ptr(y))
    return y


def _mlx4(w, keep):
    """OrcMlx4 of a weight with attributes vals, scales, biases, rows, cols;
    the contiguous arrays are appended to `keep` to outlive the call."""
    vals, scales = _c(w.vals, np.uint32), _c(w.scales, np.uint16)
    biases = None if w.biases is None else _c(w.biases, np.uint16)
    keep += [vals, scales, biases]
    return ctypes.byref(_Mlx4(_ptr(vals), _ptr(scales), _ptr(biases), w.rows, w.cols))


def gqa_step(kv_layer, token, state, w, heads, kv_heads, head_dim):
    """One full-GQA layer step (orc_gqa_step) on the hidden state.  w has
    in_norm, q, k, v, o, qn, kn (MLX 4-bit weights as in _mlx4).  kv_layer
    is updated in place; returns the new state."""
    st = _c(state, np.float32).copy()
    keep = []
    innorm = None if w.in_norm is None else _c(w.in_norm, np.uint16)
    rc = lib().orc_gqa_step(heads, kv_heads, head_dim, kv_layer.shape[0], kv_layer, token,
                            st.size, st, _ptr(innorm), _mlx4(w.q, keep), _mlx4(w.k, keep),
                            _mlx4(w.v, keep), _mlx4(w.o, keep), _c(w.qn, np.uint16),
                            _c(w.kn, np.uint16))
    if rc != 0:
        raise RuntimeError("orc_gqa_step failed")
    return st


def lin_step(conv_ring, S, token, state, w, k_heads, v_heads, kd, vd, max_tokens=1 << 30):
    """One gated delta-rule layer step (orc_lin_step).  w has in_norm, qkv,
    z, a, b, out and core (conv_w, A_log, dt_bias, norm_w).  conv_ring and S
    are updated in place; returns the new state."""
    st = _c(state, np.float32).copy()
    keep = []
    innorm = None if w.in_norm is None else _c(w.in_norm, np.uint16)
    c = w.core
    rc = lib().orc_lin_step(k_heads, v_heads, kd, vd, max_tokens, token, st.size, conv_ring, S,
                            st, _ptr(innorm), _mlx4(w.qkv, keep), _mlx4(w.z, keep),
                            _mlx4(w.a, keep), _mlx4(w.b, keep), _mlx4(w.out, keep),
                            _c(c.conv_w, np.uint16), _c(c.A_log, np.float32),
                            _c(c.dt_bias, np.uint16), _c(c.norm_w, np.uint16))
    if rc != 0:
        raise RuntimeError("orc_lin_step failed")
    return st


def gqa_chunk(kv_layer, t0, states, w, heads, kv_heads, head_dim):
    """A GQA prefill chunk on states [B][hidden] (orc_gqa_chunk); kv_layer
    is updated in place; returns the new states."""
    st = np.array(states, dtype=np.float32, order="C", copy=True)
    keep = []
    innorm = None if w.in_norm is None else _c(w.in_norm, np.uint16)
    rc = lib().orc_gqa_chunk(heads, kv_heads, head_dim, kv_layer.shape[0], kv_layer, t0,
                             st.shape[0], st.shape[1], st, _ptr(innorm), _mlx4(w.q, keep),
                             _mlx4(w.k, keep), _mlx4(w.v, keep), _mlx4(w.o, keep),
                             _c(w.qn, np.uint16), _c(w.kn, np.uint16))
    if rc != 0:
        raise RuntimeError("orc_gqa_chunk failed")
    return st


def lin_chunk(conv_ring, S, t0, states, w, k_heads, v_heads, kd, vd, max_tokens=1 << 30):
    """A delta-rule prefill chunk on states [B][hidden] (orc_lin_chunk);
    conv_ring and S are updated in place; returns the new states."""
    st = np.array(states, dtype=np.float32, order="C", copy=True)
    keep = []
    innorm = None if w.in_norm is None else _c(w.in_norm, np.uint16)
    c = w.core
    rc = lib().orc_lin_chunk(k_heads, v_heads, kd, vd, max_tokens, t0, st.shape[0], st.shape[1],
                             conv_ring, S, st, _ptr(innorm), _mlx4(w.qkv, keep), _mlx4(w.z, keep),
                             _mlx4(w.a, keep), _mlx4(w.b, keep), _mlx4(w.out, keep),
                             _c(c.conv_w, np.uint16), _c(c.A_log, np.float32),
                             _c(c.dt_bias, np.uint16), _c(c.norm_w, np.uint16))
    if rc != 0:
        raise RuntimeError("orc_lin_chunk failed")
    return st

