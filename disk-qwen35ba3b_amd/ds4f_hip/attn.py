"""Host-side mirror of the engine's attention interface over the HIP plugin.

``KvCache`` is the engine's state container (include/ds4f/attn.h:26-42,
allocated as src/attn.c:27-91 does) held in numpy; ``GpuAttention`` binds it
to the plugin and exposes the entry points of include/ds4f_gpu_attn.h with
the argument meaning and error behaviour of the reference bodies they
replace (src/attn_qwen.c gqa_body :235-397, lin_body :434-764): inputs
mutated in place where the reference mutates them, silent skip for tokens
outside the cache, -1 (raised here as RuntimeError) for unusable state.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import lib as _L
from .workloads import GqaGeom, GqaLayerW, LinGeom, LinLayerW, LinWeights


def _p(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a


def _u16(a):
    return np.ascontiguousarray(a, dtype=np.uint16)


class KvCache:
    """Ds4fKvCache: kv [n_layers][max_tokens][kvlat], lin [n_layers][vh][kd][vd],
    conv [n_layers][4][conv_rows], all fp32 and zero-initialised (calloc)."""

    def __init__(self, n_layers: int, max_tokens: int, gq: GqaGeom = GqaGeom(),
                 lg: LinGeom = LinGeom(), with_kv: bool = True):
        self.n_layers, self.max_tokens = n_layers, max_tokens
        self.kvlat = 2 * gq.kv_heads * gq.head_dim
        self.kv = np.zeros((n_layers, max_tokens, self.kvlat), np.float32) if with_kv else None
        self.lin = np.zeros((n_layers, lg.v_heads, lg.kd, lg.vd), np.float32)
        self.conv = np.zeros((n_layers, 4, lg.rows), np.float32)


class GpuAttention:
    """The plugin bound to one KvCache (or to device-only state)."""

    def __init__(self, kinds, max_tokens: int, cache: KvCache | None = None,
                 gq: GqaGeom = GqaGeom(), lg: LinGeom = LinGeom(), n_kv_tokens: int = 0):
        self.lib = _L.load()
        _L.check(self.lib.ds4f_gpu_init(), "ds4f_gpu_init")
        self.gq, self.lg = gq, lg
        self.kinds = np.ascontiguousarray(kinds, dtype=np.int32)
        self.geom = _L.Geom(len(kinds), max_tokens, gq.heads, gq.kv_heads, gq.head_dim, lg.kd,
                            lg.vd)
        self.cache = cache
        kv = cache.kv if cache is not None else None
        lin = cache.lin if cache is not None else None
        conv = cache.conv if cache is not None else None
        rc = self.lib.ds4f_gpu_attn_bind(ctypes.byref(self.geom), _p(self.kinds), _p(kv), _p(lin),
                                         _p(conv), n_kv_tokens)
        _L.check(rc, "ds4f_gpu_attn_bind")

    def close(self):
        self.lib.ds4f_gpu_attn_unbind()

    def sync(self, L: int = -1, to_host: bool = True, n_kv_tokens: int = 0):
        d = _L.SYNC_TO_HOST if to_host else _L.SYNC_TO_DEVICE
        _L.check(self.lib.ds4f_gpu_attn_sync(L, d, n_kv_tokens), "ds4f_gpu_attn_sync")

    # ---- host-pointer entry points ----
    def gqa_decode(self, L, token, q_gate, k, v, qn_w, kn_w):
        """Returns (attn_out [H*D], k normed+rotated)."""
        g = self.gq
        q_gate, v = _f32(q_gate), _f32(v)
        k = _f32(k).reshape(-1).copy()
        out = np.zeros(g.heads * g.head_dim, np.float32)
        rc = self.lib.ds4f_gpu_gqa_decode(L, token, _p(q_gate), _p(k), _p(v), _p(_u16(qn_w)),
                                          _p(_u16(kn_w)), _p(out))
        _L.check(rc, "ds4f_gpu_gqa_decode")
        return out, k

    def lin_decode(self, L, token, qkv, z, a, b, w: LinWeights):
        """Returns (out [vh*vd], qkv after conv + norm)."""
        g = self.lg
        qkv = _f32(qkv).reshape(-1).copy()
        out = np.zeros(g.v_heads * g.vd, np.float32)
        rc = self.lib.ds4f_gpu_lin_decode(L, token, _p(qkv), _p(_f32(z)), _p(_f32(a)),
                                          _p(_f32(b)), _p(_u16(w.conv_w)), _p(_f32(w.A_log)),
                                          _p(_u16(w.dt_bias)), _p(_u16(w.norm_w)), _p(out))
        _L.check(rc, "ds4f_gpu_lin_decode")
        return out, qkv

    def gqa_prefill(self, L, t0, q_gate, k, v, qn_w, kn_w):
        g = self.gq
        B = q_gate.shape[0]
        q_gate, v = _f32(q_gate), _f32(v)
        k = _f32(k).reshape(B, -1).copy()
        out = np.zeros((B, g.heads * g.head_dim), np.float32)
        rc = self.lib.ds4f_gpu_gqa_prefill(L, t0, B, _p(q_gate), _p(k), _p(v), _p(_u16(qn_w)),
                                           _p(_u16(kn_w)), _p(out))
        _L.check(rc, "ds4f_gpu_gqa_prefill")
        return out, k

    def lin_prefill(self, L, t0, qkv, z, a, b, w: LinWeights):
        g = self.lg
        B = qkv.shape[0]
        qkv = _f32(qkv).reshape(B, -1).copy()
        out = np.zeros((B, g.v_heads * g.vd), np.float32)
        rc = self.lib.ds4f_gpu_lin_prefill(L, t0, B, _p(qkv), _p(_f32(z)), _p(_f32(a)),
                                           _p(_f32(b)), _p(_u16(w.conv_w)), _p(_f32(w.A_log)),
                                           _p(_u16(w.dt_bias)), _p(_u16(w.norm_w)), _p(out))
        _L.check(rc, "ds4f_gpu_lin_prefill")
        return out, qkv


    # ---- whole layer steps (src/attn_qwen.c:87-225, :837-968) ----
    def set_layer_weights(self, L: int, w: GqaLayerW | LinLayerW):
        """Upload layer L's weights (ds4f_gpu_attn_weights)."""
        keep = []

        def arr(a, dt):
            if a is None:
                return None
            a = np.ascontiguousarray(a, dtype=dt)
            keep.append(a)
            return a.ctypes.data

        def m4(m):
            return _L.Mlx4W(arr(m.vals, np.uint32), arr(m.scales, np.uint16),
                            arr(m.biases, np.uint16), m.rows, m.cols)

        lw = _L.LayerW()
        lw.in_norm = arr(w.in_norm, np.uint16)
        if isinstance(w, GqaLayerW):
            lw.q, lw.k, lw.v, lw.o = m4(w.q), m4(w.k), m4(w.v), m4(w.o)
            lw.q_norm, lw.k_norm = arr(w.qn, np.uint16), arr(w.kn, np.uint16)
        else:
            lw.qkv, lw.z, lw.a, lw.b, lw.out = m4(w.qkv), m4(w.z), m4(w.a), m4(w.b), m4(w.out)
            c = w.core
            lw.conv_w, lw.dt_bias = arr(c.conv_w, np.uint16), arr(c.dt_bias, np.uint16)
            lw.norm_w, lw.A_log = arr(c.norm_w, np.uint16), arr(c.A_log, np.float32)
        _L.check(self.lib.ds4f_gpu_attn_weights(L, ctypes.byref(lw)), "ds4f_gpu_attn_weights")

    def attn_step(self, L: int, token: int, state):
        """One decode token of layer L on the residual stream; returns the
        new state (ds4f_gpu_attn_step)."""
        st = _f32(state).reshape(-1).copy()
        _L.check(self.lib.ds4f_gpu_attn_step(L, token, _p(st)), "ds4f_gpu_attn_step")
        return st


    def attn_chunk(self, L: int, t0: int, states):
        """A prefill chunk of the tokens t0.. of layer L on their hidden
        states [B][hidden]; returns the new states (ds4f_gpu_attn_chunk)."""
        st = np.array(states, dtype=np.float32, order="C", copy=True)
        B = st.shape[0]
        ptrs = (ctypes.c_void_p * B)(*[st[b].ctypes.data for b in range(B)])
        _L.check(self.lib.ds4f_gpu_attn_chunk(L, t0, B, ptrs), "ds4f_gpu_attn_chunk")
        return st


def dptr(t) -> ctypes.c_void_p | None:
    """Device pointer of a torch tensor (None passes NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())
