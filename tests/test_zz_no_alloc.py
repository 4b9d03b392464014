"""The delta-rule prefill entry that allocates nothing
(ds4f_hip_lin_prefill_noalloc: its workspace is the library's static device
array) against the allocating entry (ds4f_hip_lin_prefill_async) through the
C ABI.  Both run the same kernels, so two layers starting from the same
state must agree bit for bit: outputs, post-conv rows, delta states and conv
rings, over two calls in a row, the second smaller than the first.  A chunk
longer than the entry's maximum of 128 tokens is refused with an error and
launches nothing.
"""
import numpy as np
import pytest

from ds4f_hip import workloads as W
from ds4f_hip.attn import GpuAttention, KvCache, dptr

pytestmark = pytest.mark.gpu

LG = W.LinGeom()


def test_noalloc_lin_prefill_matches_allocating_entry():
    import torch

    from ds4f_hip.lib import last_error, load
    lib = load()
    seed, max_tokens = 21, 1024
    cache = KvCache(2, max_tokens, with_kv=False)
    t0 = 5
    for L in (0, 1):
        cache.lin[L] = W.lin_state(LG, seed, 0)
        cache.conv[L] = W.ring_from_history(LG, W.lin_conv_history(LG, seed, 0), t0)
    ga = GpuAttention([1, 1], max_tokens, cache)
    w = W.lin_weights(LG, seed, 0)
    dev = torch.device("cuda:0")

    def d(a, dt=torch.float32):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev) if dt is None else \
            torch.from_numpy(np.ascontiguousarray(a)).to(dev, dt)

    cw = d(w.conv_w.view(np.int16), None)
    al = d(w.A_log)
    dt_b = d(w.dt_bias.view(np.int16), None)
    nw = d(w.norm_w.view(np.int16), None)

    # (t0, B, qkv_post given): the largest chunk without a post buffer, then
    # a smaller one continuing it with one
    for call, (tt, B, with_post) in enumerate([(t0, 128, False), (t0 + 128, 37, True)]):
        qkv, z, a, b = (d(x) for x in W.lin_tokens(LG, B, seed, 0, tt))
        outs, posts = [], []
        for L, fn in ((0, lib.ds4f_hip_lin_prefill_async), (1, lib.ds4f_hip_lin_prefill_noalloc)):
            out = torch.full((B, LG.v_heads * LG.vd), float("nan"), device=dev)
            post = torch.full((B, LG.rows), float("nan"), device=dev) if with_post else None
            rc = fn(L, tt, B, dptr(qkv), dptr(z), dptr(a), dptr(b), dptr(cw), dptr(al),
                    dptr(dt_b), dptr(nw), dptr(out), dptr(post), None)
            assert rc == 0, last_error()
            outs.append(out)
            posts.append(post)
        torch.cuda.synchronize()
        o0, o1 = outs[0].cpu().numpy(), outs[1].cpu().numpy()
        assert np.isfinite(o0).all()
        assert np.array_equal(o0, o1), f"call {call}: outputs differ"
        if with_post:
            assert np.array_equal(posts[0].cpu().numpy(), posts[1].cpu().numpy())
        ga.sync(-1, to_host=True)
        assert np.array_equal(cache.lin[0], cache.lin[1]), f"call {call}: states differ"
        assert np.array_equal(cache.conv[0], cache.conv[1]), f"call {call}: rings differ"
        print(f"call {call}: t0 {tt} B {B} post {with_post}: identical", flush=True)

    # beyond the static workspace: refused, nothing launched
    snap = cache.lin[1].copy(), cache.conv[1].copy()
    B = 129
    qkv, z, a, b = (d(x) for x in W.lin_tokens(LG, B, seed, 0, 200))
    out = torch.empty((B, LG.v_heads * LG.vd), device=dev)
    rc = lib.ds4f_hip_lin_prefill_noalloc(1, 200, B, dptr(qkv), dptr(z), dptr(a), dptr(b),
                                          dptr(cw), dptr(al), dptr(dt_b), dptr(nw), dptr(out),
                                          None, None)
    assert rc == -1
    assert "maximum of 128" in last_error()
    torch.cuda.synchronize()
    ga.sync(1, to_host=True)
    assert np.array_equal(cache.lin[1], snap[0]) and np.array_equal(cache.conv[1], snap[1])
    ga.close()
