"""GPU parity of the prefill kernels against the oracle (needs an MI355X).

GQA prefill runs fp16 MFMA flash attention; the bar is max |gpu - oracle|
<= 2e-3 on the attention outputs.  At T = 4096 the oracle's serial loop is
split into its cache-row helper (the rows the loop writes) and the body at
each token over those rows, run on a thread pool: the same computations as
the serial loop, every token checked.
"""
import sys

import numpy as np
import pytest

import oracle as O
from ds4f_hip import synth as S
from ds4f_hip import workloads as W
from ds4f_hip.attn import GpuAttention, KvCache

pytestmark = pytest.mark.gpu

GQ = W.GqaGeom()
ATOL = 2e-3


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _err(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    mx = float(np.abs(got - ref).max())
    rr = float(np.sqrt(((got - ref) ** 2).sum() / max((ref ** 2).sum(), 1e-300)))
    return mx, rr


@pytest.mark.parametrize("T", [1, 17, 64, 200])
def test_gqa_prefill_small_full_check(T):
    qn, kn = W.gqa_weights(GQ)
    q, k, v = W.gqa_prefill_tokens(GQ, T)
    cache = KvCache(1, T + 16)
    ref_kv = cache.kv[0].copy()
    ga = GpuAttention([2], T + 16, cache)
    out, kp = ga.gqa_prefill(0, 0, q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1), qn, kn)
    ref, rk = O.gqa_prefill(ref_kv, 0, q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1), qn,
                            kn, GQ.heads, GQ.kv_heads, GQ.head_dim)
    mx, rr = _err(out, ref)
    _say(f"gqa prefill T={T}: max abs {mx:.3e} rel-rms {rr:.3e}")
    assert mx <= ATOL
    assert _err(kp, rk)[0] < 1e-5
    ga.sync(0, to_host=True, n_kv_tokens=T)
    half = GQ.kv_heads * GQ.head_dim
    assert np.array_equal(cache.kv[0, :T, :half], S.bf16_round(rk))
    assert np.array_equal(cache.kv[0, :T, half:], S.bf16_round(v.reshape(T, -1)))
    ga.close()


def test_gqa_prefill_4096_every_token():
    """The 4096-token prefill checked at every token against the oracle's
    body over the oracle's own cache rows (the rows of a serial prefill,
    made by its cache-row helper; each body call is the serial loop's call
    at that token).  The calls are independent given the rows, so they run
    on a thread pool, each thread on its own copy of the rows."""
    from concurrent.futures import ThreadPoolExecutor

    T = 4096
    _say("gqa prefill T=4096")
    qn, kn = W.gqa_weights(GQ)
    q, k, v = W.gqa_prefill_tokens(GQ, T)
    ga = GpuAttention([2], T + 64, None)
    out, kp = ga.gqa_prefill(0, 0, q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1), qn, kn)
    rows = O.gqa_cache_rows(k, v, kn, 0, GQ.kv_heads, GQ.head_dim)
    half = GQ.kv_heads * GQ.head_dim
    assert np.abs(kp - rows[:, :half]).max() < 1e-5

    def worst_of(part):
        kv = rows.copy()      # the body rewrites row t with the helper's values
        w = 0.0
        for b in part:
            o, _ = O.gqa_body(kv, b, q[b].reshape(-1), k[b].reshape(-1), v[b].reshape(-1), qn, kn,
                              GQ.heads, GQ.kv_heads, GQ.head_dim)
            w = max(w, _err(out[b], o)[0])
        return w

    nthr = 16
    parts = [list(range(i, T, nthr)) for i in range(nthr)]      # interleaved: equal work
    with ThreadPoolExecutor(max_workers=nthr) as pool:
        worst = max(pool.map(worst_of, parts))
    _say(f"  all {T} tokens: worst max abs {worst:.3e}")
    assert worst <= ATOL
    ga.close()


@pytest.mark.parametrize("t0,B", [(32704, 64), (32749, 37)])
def test_gqa_prefill_chunk_on_long_cache(t0, B):
    """A prefill chunk on top of a long cache, as the engine's chunked prompt
    reaches it at 32K context (aligned and unaligned t0).  The device draws
    the t0 prefix rows into its bf16 cache (ds4f_hip_synth_gqa_cache) and the
    chunk attends to all of them and causally to its own rows.  Every token
    is checked against the oracle's body over the same prefix rows and the
    oracle's own rows for the chunk, on a thread pool as in the 4096-token
    test; the prefix rows stay untouched and the chunk's rows are the
    oracle's in bf16."""
    from concurrent.futures import ThreadPoolExecutor

    from ds4f_hip.lib import check, load

    _say(f"gqa prefill chunk t0={t0} B={B} over a drawn cache")
    max_tokens = t0 + B + 8
    cache = KvCache(1, max_tokens)
    ga = GpuAttention([2], max_tokens, cache)
    try:
        check(load().ds4f_hip_synth_gqa_cache(0, t0, 0, S.tid(S.GQA_KCACHE, 0),
                                              S.tid(S.GQA_VCACHE, 0), None), "synth kv")
        ga.sync(0, to_host=True, n_kv_tokens=t0)
        kv = cache.kv[0].copy()
        assert np.abs(kv[:t0]).max() > 0
        qn, kn = W.gqa_weights(GQ)
        q, k, v = W.gqa_prefill_tokens(GQ, B)
        out, kp = ga.gqa_prefill(0, t0, q.reshape(B, -1), k.reshape(B, -1), v.reshape(B, -1), qn, kn)
        kv[t0:t0 + B] = O.gqa_cache_rows(k, v, kn, t0, GQ.kv_heads, GQ.head_dim)
        half = GQ.kv_heads * GQ.head_dim
        assert np.abs(kp - kv[t0:t0 + B, :half]).max() < 1e-5

        def worst_of(part):
            kvc = kv.copy()      # the body rewrites row t0 + b with the helper's values
            w = 0.0
            for b in part:
                o, _ = O.gqa_body(kvc, t0 + b, q[b].reshape(-1), k[b].reshape(-1), v[b].reshape(-1),
                                  qn, kn, GQ.heads, GQ.kv_heads, GQ.head_dim)
                w = max(w, _err(out[b], o)[0])
            return w

        nthr = 16
        parts = [list(range(i, B, nthr)) for i in range(nthr)]
        with ThreadPoolExecutor(max_workers=nthr) as pool:
            worst = max(pool.map(worst_of, parts))
        _say(f"  all {B} tokens: worst max abs {worst:.3e}")
        assert worst <= ATOL

        prefix = kv[:t0].copy()
        ga.sync(0, to_host=True, n_kv_tokens=t0 + B)
        assert np.array_equal(cache.kv[0, :t0], prefix)
        ref = kv[t0:t0 + B]
        dev = cache.kv[0, t0:t0 + B]
        assert (np.abs(dev - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-5).all()   # bf16 of the rows
    finally:
        ga.close()


def test_gqa_prefill_second_4096_chunk():
    """The second 4096-token chunk of an 8192-token prompt (t0 = 4096 over
    4096 cached rows): every workgroup's pair of q blocks then also covers
    the 128 prefix key tiles of 32.  About 190 tokens are checked against the
    oracle's body over the prefix rows and the oracle's own rows for the
    chunk: the block edges, the last token of every 32-key tile and random
    ones, on a thread pool as in the 4096-token test."""
    from concurrent.futures import ThreadPoolExecutor

    t0, B = 4096, 4096
    _say(f"gqa prefill chunk t0={t0} B={B}")
    kc, vc = W.gqa_cache(GQ, t0, 2, 0)
    half = GQ.kv_heads * GQ.head_dim
    cache = KvCache(1, t0 + B + 64)
    cache.kv[0, :t0, :half] = kc.reshape(t0, half)
    cache.kv[0, :t0, half:] = vc.reshape(t0, half)
    kv = cache.kv[0].copy()
    ga = GpuAttention([2], t0 + B + 64, cache, n_kv_tokens=t0)
    try:
        qn, kn = W.gqa_weights(GQ)
        q, k, v = W.gqa_prefill_tokens(GQ, B)
        out, kp = ga.gqa_prefill(0, t0, q.reshape(B, -1), k.reshape(B, -1), v.reshape(B, -1), qn, kn)
        assert np.isfinite(out).all()
        kv[t0:t0 + B] = O.gqa_cache_rows(k, v, kn, t0, GQ.kv_heads, GQ.head_dim)
        assert np.abs(kp - kv[t0:t0 + B, :half]).max() < 1e-5
        rng = np.random.default_rng(5)
        samples = sorted(set([0, 1, 15, 16, 17, 31, 32, 63, 64, 2047, 2048, 4095] +
                             list(range(31, B, 32)) +
                             [int(x) for x in rng.integers(0, B, 48)]))

        def worst_of(part):
            kvc = kv.copy()      # the body rewrites row t0 + b with the helper's values
            w = 0.0
            for b in part:
                o, _ = O.gqa_body(kvc, t0 + b, q[b].reshape(-1), k[b].reshape(-1), v[b].reshape(-1),
                                  qn, kn, GQ.heads, GQ.kv_heads, GQ.head_dim)
                w = max(w, _err(out[b], o)[0])
            return w

        nthr = 16
        parts = [samples[i::nthr] for i in range(nthr)]
        with ThreadPoolExecutor(max_workers=nthr) as pool:
            worst = max(pool.map(worst_of, parts))
        _say(f"  {len(samples)} sampled tokens: worst max abs {worst:.3e}")
        assert worst <= ATOL
    finally:
        ga.close()


def test_gqa_prefill_continues_a_cache():
    """Chunked prefill: 100 tokens, then 77 more at t0 = 100 (unaligned),
    then one decode step; all against the oracle's serial body."""
    qn, kn = W.gqa_weights(GQ)
    q, k, v = W.gqa_prefill_tokens(GQ, 178)
    cache = KvCache(1, 256)
    ref_kv = cache.kv[0].copy()
    ga = GpuAttention([2], 256, cache)
    worst = 0.0
    for t0, B in ((0, 100), (100, 77)):
        sl = slice(t0, t0 + B)
        out, _ = ga.gqa_prefill(0, t0, q[sl].reshape(B, -1), k[sl].reshape(B, -1),
                                v[sl].reshape(B, -1), qn, kn)
        ref, _ = O.gqa_prefill(ref_kv, t0, q[sl].reshape(B, -1), k[sl].reshape(B, -1),
                               v[sl].reshape(B, -1), qn, kn, GQ.heads, GQ.kv_heads, GQ.head_dim)
        # the device cache holds bf16 rows: give the oracle the same rows
        ref_kv[sl] = S.bf16_round(ref_kv[sl])
        worst = max(worst, _err(out, ref)[0])
    out, _ = ga.gqa_decode(0, 177, q[177], k[177], v[177], qn, kn)
    ref, _ = O.gqa_body(ref_kv, 177, q[177].reshape(-1), k[177].reshape(-1), v[177].reshape(-1),
                        qn, kn, GQ.heads, GQ.kv_heads, GQ.head_dim)
    worst = max(worst, _err(out, ref)[0])
    _say(f"chunked prefill + decode: worst max abs {worst:.3e}")
    assert worst <= ATOL
    ga.close()


@pytest.mark.parametrize("t0,B", [(37, 100), (45, 200), (13, 33), (3, 250)])
def test_gqa_prefill_unaligned_start(t0, B):
    """Prefill at t0 not a multiple of 16 over a cache of t0 past rows.
    These (t0, B) give the workgroup that pairs q blocks so that its second
    wave group starts the long block at a key tile lying wholly after the
    first positions of that block (tile 4 of t0 = 37, B = 100 starts at key
    128 for q positions 117..132): those columns see no valid key in the
    tile and must contribute nothing, not a NaN."""
    qn, kn = W.gqa_weights(GQ)
    q, k, v = W.gqa_prefill_tokens(GQ, t0 + B)
    cache = KvCache(1, t0 + B + 16)
    ref_kv = cache.kv[0].copy()
    ga = GpuAttention([2], t0 + B + 16, cache)
    try:
        past = slice(0, t0)
        ga.gqa_prefill(0, 0, q[past].reshape(t0, -1), k[past].reshape(t0, -1),
                       v[past].reshape(t0, -1), qn, kn)
        O.gqa_prefill(ref_kv, 0, q[past].reshape(t0, -1), k[past].reshape(t0, -1),
                      v[past].reshape(t0, -1), qn, kn, GQ.heads, GQ.kv_heads, GQ.head_dim)
        ref_kv[past] = S.bf16_round(ref_kv[past])
        sl = slice(t0, t0 + B)
        out, _ = ga.gqa_prefill(0, t0, q[sl].reshape(B, -1), k[sl].reshape(B, -1),
                                v[sl].reshape(B, -1), qn, kn)
        ref, _ = O.gqa_prefill(ref_kv, t0, q[sl].reshape(B, -1), k[sl].reshape(B, -1),
                               v[sl].reshape(B, -1), qn, kn, GQ.heads, GQ.kv_heads, GQ.head_dim)
        mx, rr = _err(out, ref)
        _say(f"gqa prefill t0={t0} B={B}: max abs {mx:.3e} rel-rms {rr:.3e}")
        assert np.isfinite(out).all()
        assert mx <= ATOL
    finally:
        ga.close()


# ------------------------------------------------------------------ delta rule
LG = W.LinGeom()
STATE_RTOL = 1e-4


def _lin_binding(max_tokens, t0, seed, zero_state):
    cache = KvCache(1, max_tokens, with_kv=False)
    if not zero_state:
        cache.lin[0] = W.lin_state(LG, seed, 0)
        cache.conv[0] = W.ring_from_history(LG, W.lin_conv_history(LG, seed, 0), t0)
    ring, S0 = cache.conv[0].copy(), cache.lin[0].copy()
    return GpuAttention([1], max_tokens, cache), cache, ring, S0, W.lin_weights(LG, seed, 0)


def _lin_check(ga, cache, ring, S0, w, t0, qkv, z, a, b, what):
    out, post = ga.lin_prefill(0, t0, qkv, z, a, b, w)
    ref, rpost = O.lin_prefill(ring, S0, t0, qkv, z, a, b, w.conv_w, w.A_log, w.dt_bias,
                               w.norm_w, LG.k_heads, LG.v_heads, LG.kd, LG.vd)
    ga.sync(0, to_host=True)
    mx, rr = _err(out, ref)
    pmx = _err(post, rpost)[0]
    smx, srr = _err(cache.lin[0], S0)
    _say(f"{what}: out max abs {mx:.3e} rel-rms {rr:.3e}; post {pmx:.3e}; "
         f"state rel {srr:.3e} max abs {smx:.3e}")
    assert mx <= ATOL
    assert pmx <= 1e-5
    assert srr <= STATE_RTOL
    assert np.array_equal(cache.conv[0], ring)       # raw rows: exact
    return out


@pytest.mark.parametrize("T,t0", [(1, 0), (3, 0), (5, 0), (64, 0), (65, 0), (200, 0),
                                  (1, 9), (2, 9), (130, 7), (2100, 5)])
def test_lin_prefill_chunked_vs_serial(T, t0):
    """Chunk boundaries (64), ragged last chunks, B < 4 (ring keeps older
    rows), a prefill continuing at an unaligned position with a past state
    and conv history; at 2100 tokens the chunk kernel's 528 (chunk, key
    head) items exceed its 512 workgroups, so 16 of them take a second,
    ragged item."""
    ga, cache, ring, S0, w = _lin_binding(t0 + T + 8, t0, 11, zero_state=(t0 == 0))
    qkv, z, a, b = W.lin_tokens(LG, T, 11)
    _lin_check(ga, cache, ring, S0, w, t0, qkv, z, a, b, f"lin prefill T={T} t0={t0}")
    ga.close()


def test_lin_prefill_4096_zero_state():
    """The 4096-token prefill from a zero state and zero conv ring (the
    benchmark's delta prefill), against 4096 serial oracle bodies."""
    T = 4096
    _say("lin prefill T=4096 (oracle serial loop takes a while)")
    ga, cache, ring, S0, w = _lin_binding(T + 8, 0, 0, zero_state=True)
    qkv, z, a, b = W.lin_tokens(LG, T, 0)
    _lin_check(ga, cache, ring, S0, w, 0, qkv, z, a, b, "lin prefill T=4096")
    ga.close()


def test_lin_prefill_then_decode():
    """Prefill 100 tokens, then 37 more, then three decode steps, all against
    the oracle's serial body on the same state."""
    ga, cache, ring, S0, w = _lin_binding(256, 0, 13, zero_state=True)
    qkv, z, a, b = W.lin_tokens(LG, 140, 13)
    for t0, B in ((0, 100), (100, 37)):
        sl = slice(t0, t0 + B)
        _lin_check(ga, cache, ring, S0, w, t0, qkv[sl], z[sl], a[sl], b[sl],
                   f"lin prefill t0={t0} B={B}")
    worst = 0.0
    for tok in range(137, 140):
        out, _ = ga.lin_decode(0, tok, qkv[tok], z[tok], a[tok], b[tok], w)
        ref, _ = O.lin_body(ring, S0, tok, qkv[tok], z[tok], a[tok], b[tok], w.conv_w, w.A_log,
                            w.dt_bias, w.norm_w, LG.k_heads, LG.v_heads, LG.kd, LG.vd)
        worst = max(worst, _err(out, ref)[0])
    _say(f"decode after chunked prefill: worst max abs {worst:.3e}")
    assert worst <= ATOL
    ga.close()


def test_gqa_prefill_fp16_range_falls_back():
    """A value beyond fp16 range (2^17, exact in bf16) planted in one token's
    v: the prefill's fp16 operand conversion flags it (status bit 1) and the
    host entry recomputes the tokens on the decode kernels.  The outputs are
    bit for bit those of B ds4f_gpu_gqa_decode calls on a fresh binding, and
    match the oracle's serial body with bf16 cache rows (the decode path's
    row format) relative to their magnitude, which the planted value raises
    to about 1e5.  Without the plant the fp16 path matches the oracle as
    usual.  The host entry flags into a status word of its own, so the
    device-pointer callers' word reads 0 after it either way; the
    device-pointer prefill of the planted tokens sets bit 1 there."""
    import torch

    from ds4f_hip.attn import dptr
    from ds4f_hip.lib import check, load
    lib = load()
    T = 40
    qn, kn = W.gqa_weights(GQ)
    q, k, v = W.gqa_prefill_tokens(GQ, T)
    for plant in (False, True):
        vv = v.copy()
        if plant:
            vv[3, 0, 7] = 2.0 ** 17
        cache = KvCache(1, T + 16)
        ref_kv = cache.kv[0].copy()
        ga = GpuAttention([2], T + 16, cache)
        assert lib.ds4f_hip_f16_status(None, 1) >= 0
        out, _ = ga.gqa_prefill(0, 0, q.reshape(T, -1), k.reshape(T, -1), vv.reshape(T, -1), qn,
                                kn)
        bits = lib.ds4f_hip_f16_status(None, 1)
        ga.close()
        assert bits == 0
        if plant:
            ga = GpuAttention([2], T + 16, KvCache(1, T + 16))
            dec = np.stack([ga.gqa_decode(0, b, q[b], k[b], vv[b], qn, kn)[0] for b in range(T)])
            # the same tokens through the device-pointer prefill: flagged in word 0
            dev = torch.device("cuda:0")
            tq, tk, tv = (torch.tensor(np.ascontiguousarray(a.reshape(T, -1)), device=dev)
                          for a in (q, k, vv))
            tqn = torch.tensor(qn.view(np.int16), device=dev)
            tkn = torch.tensor(kn.view(np.int16), device=dev)
            tout = torch.empty((T, GQ.heads * GQ.head_dim), dtype=torch.float32, device=dev)
            torch.cuda.synchronize()
            check(lib.ds4f_hip_gqa_prefill_async(0, 0, T, dptr(tq), dptr(tk), dptr(tv), dptr(tqn),
                                                 dptr(tkn), dptr(tout), None, None), "prefill async")
            bits = lib.ds4f_hip_f16_status(None, 1)
            del tq, tk, tv, tqn, tkn, tout
            ga.close()
            assert np.array_equal(out, dec)
            ref = np.empty_like(out)
            for b in range(T):
                ref[b], _ = O.gqa_body(ref_kv, b, q[b].reshape(-1), k[b].reshape(-1),
                                       vv[b].reshape(-1), qn, kn, GQ.heads, GQ.kv_heads,
                                       GQ.head_dim)
                ref_kv[b] = S.bf16_round(ref_kv[b])
        else:
            ref, _ = O.gqa_prefill(ref_kv, 0, q.reshape(T, -1), k.reshape(T, -1),
                                   vv.reshape(T, -1), qn, kn, GQ.heads, GQ.kv_heads, GQ.head_dim)
        assert np.isfinite(out).all()
        scaled = float((np.abs(out - ref) / np.maximum(1.0, np.abs(ref))).max())
        _say(f"fp16 range plant={plant}: status {bits}, |ref| max {np.abs(ref).max():.3e}, "
             f"max scaled err {scaled:.3e}")
        assert bits == (1 if plant else 0)
        assert scaled <= ATOL
