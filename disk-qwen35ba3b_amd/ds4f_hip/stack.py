"""The hybrid attention stack decoding consecutive tokens on the device.

One decode step is one token through every layer in order, the way the
engine's token loop calls ``ds4f_attn_qwen_step`` per layer
(src/main.c:924-957 -> src/attn_qwen.c:1255-1264): full GQA at
layer % 4 == 3, the gated delta rule elsewhere.  Attention cores only: the
post-projection activations of every (layer, step) are synthetic tensors
drawn on the device from the workload streams before any step runs.

``StackDecode`` owns the binding, the device state (KV caches of the GQA
layers, delta-rule states and conv rings) and the activations, and
``launch_step`` enqueues one step's layer calls through the device-pointer
entry points (``ds4f_hip_gqa_decode_async`` / ``ds4f_hip_lin_decode_async``)
on a stream, so a step can be captured as one HIP graph.  ``bench.py`` times
this sequence and ``tests/test_gpu_stack.py`` checks it against the oracle,
so both run the same launches.
"""
from __future__ import annotations

import ctypes

from . import lib as _L
from . import synth as S
from . import workloads as W
from .attn import GpuAttention, KvCache, dptr


class StackDecode:
    """`steps` decode steps of an `n_layers` stack at context `ctx`: step s
    is the token at position ctx + s attending ctx + s cached rows.

    host_cache: bind a host KvCache (kv / lin / conv arrays) so the state can
    be synced to the host; its kv array is a lazily zero-filled allocation of
    n_layers rows, of which only the GQA layers' pages are ever touched."""

    def __init__(self, ctx: int, steps: int, seed: int = 0, n_layers: int = 40,
                 host_cache: bool = False):
        import torch

        self.lib = _L.load()
        torch.cuda.init()
        dev = torch.device("cuda:0")
        self.gq, self.lg = W.GqaGeom(), W.LinGeom()
        self.kinds = W.stack_kinds(n_layers)
        self.ctx, self.steps, self.seed = ctx, steps, seed
        self.max_tokens = ctx + steps + 64
        self.cache = KvCache(n_layers, self.max_tokens) if host_cache else None
        self.ga = GpuAttention(self.kinds, self.max_tokens, self.cache)
        lib, gq, lg = self.lib, self.gq, self.lg
        self.synth_state()

        def synth(n, dtype, dist, p0, p1, tid, t=None):
            if t is None:
                t = torch.empty(n, dtype=torch.float32 if dtype == 0 else torch.int16, device=dev)
            _L.check(lib.ds4f_hip_synth(dptr(t), n, dtype, dist, p0, p1, seed, tid, None),
                     "synth")
            return t

        T = steps
        self.layers = []
        for Lr, kd in enumerate(self.kinds):
            d = {"kind": kd}
            if kd == _L.LAYER_GQA:
                d["qn"] = synth(gq.head_dim, 1, 0, 1.0, 0.1, S.tid(S.GQA_QNW, Lr))
                d["kn"] = synth(gq.head_dim, 1, 0, 1.0, 0.1, S.tid(S.GQA_KNW, Lr))
                nq, nk = gq.heads * 2 * gq.head_dim, gq.kv_heads * gq.head_dim
                d["q"] = torch.empty((T, nq), dtype=torch.float32, device=dev)
                d["k"] = torch.empty((T, nk), dtype=torch.float32, device=dev)
                d["v"] = torch.empty((T, nk), dtype=torch.float32, device=dev)
                for s in range(T):
                    pos = ctx + s
                    synth(nq, 0, 0, 0.0, 1.0, S.tid(S.GQA_QGATE, Lr, pos), d["q"][s])
                    synth(nk, 0, 0, 0.0, 1.0, S.tid(S.GQA_K, Lr, pos), d["k"][s])
                    synth(nk, 0, 0, 0.0, 1.0, S.tid(S.GQA_V, Lr, pos), d["v"][s])
                d["out"] = torch.empty((T, gq.heads * gq.head_dim), dtype=torch.float32,
                                       device=dev)
            else:
                d["cw"] = synth(lg.rows * 4, 1, 0, 0.0, 0.1, S.tid(S.LIN_CONVW, Lr))
                d["al"] = synth(lg.v_heads, 0, 1, 0.0, 2.7, S.tid(S.LIN_ALOG, Lr))
                d["dt"] = synth(lg.v_heads, 1, 0, 0.0, 0.1, S.tid(S.LIN_DTB, Lr))
                d["nw"] = synth(lg.vd, 1, 0, 1.0, 0.1, S.tid(S.LIN_NORMW, Lr))
                nz = lg.v_heads * lg.vd
                d["qkv"] = torch.empty((T, lg.rows), dtype=torch.float32, device=dev)
                d["z"] = torch.empty((T, nz), dtype=torch.float32, device=dev)
                d["a"] = torch.empty((T, lg.v_heads), dtype=torch.float32, device=dev)
                d["b"] = torch.empty((T, lg.v_heads), dtype=torch.float32, device=dev)
                for s in range(T):
                    synth(lg.rows, 0, 0, 0.0, 1.0, S.tid(S.LIN_QKV, Lr, s), d["qkv"][s])
                    synth(nz, 0, 0, 0.0, 1.0, S.tid(S.LIN_Z, Lr, s), d["z"][s])
                    synth(lg.v_heads, 0, 0, 0.0, 1.0, S.tid(S.LIN_A, Lr, s), d["a"][s])
                    synth(lg.v_heads, 0, 0, 0.0, 1.0, S.tid(S.LIN_B, Lr, s), d["b"][s])
                d["out"] = torch.empty((T, nz), dtype=torch.float32, device=dev)
            self.layers.append(d)
        torch.cuda.synchronize()

    def synth_state(self) -> None:
        """The layers' starting state on the device, generated in place from
        the seed: the GQA caches' ctx rows, the delta-rule states and conv
        rings (the same values every call, so a run can put it back)."""
        lib, ctx, seed = self.lib, self.ctx, self.seed
        for Lr, kd in enumerate(self.kinds):
            if kd == _L.LAYER_GQA:
                _L.check(lib.ds4f_hip_synth_gqa_cache(Lr, ctx, seed, S.tid(S.GQA_KCACHE, Lr),
                                                      S.tid(S.GQA_VCACHE, Lr), None), "synth kv")
            else:
                _L.check(lib.ds4f_hip_synth_lin_state(Lr, 0.05, seed, S.tid(S.LIN_STATE, Lr),
                                                      None), "synth state")
                _L.check(lib.ds4f_hip_synth_conv_history(Lr, ctx, seed,
                                                         S.tid(S.LIN_CONVSTATE, Lr), None),
                         "synth conv")

    def launch_layer(self, Lr: int, s: int, stream) -> None:
        """Enqueue layer Lr of step s on `stream` (a ctypes void pointer)."""
        lib, d, pos = self.lib, self.layers[Lr], self.ctx + s
        if d["kind"] == _L.LAYER_GQA:
            rc = lib.ds4f_hip_gqa_decode_async(Lr, pos, dptr(d["q"][s]), dptr(d["k"][s]),
                                               dptr(d["v"][s]), dptr(d["qn"]), dptr(d["kn"]),
                                               dptr(d["out"][s]), None, stream)
        else:
            rc = lib.ds4f_hip_lin_decode_async(Lr, pos, dptr(d["qkv"][s]), dptr(d["z"][s]),
                                               dptr(d["a"][s]), dptr(d["b"][s]), dptr(d["cw"]),
                                               dptr(d["al"]), dptr(d["dt"]), dptr(d["nw"]),
                                               dptr(d["out"][s]), None, stream)
        _L.check(rc, f"layer {Lr} step {s}")

    def launch_step(self, s: int, stream) -> None:
        """Enqueue step s: every layer in order."""
        for Lr in range(len(self.layers)):
            self.launch_layer(Lr, s, stream)

    def capture(self, steps):
        """One HIP graph per step (torch CUDAGraph on a side stream)."""
        import torch

        graphs = []
        side = torch.cuda.Stream()
        for s in steps:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                self.launch_step(s, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            graphs.append(g)
        return graphs

    def close(self) -> None:
        self.ga.close()
