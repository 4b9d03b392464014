"""GPU parity of the decode kernels against the oracle (needs an MI355X).

Tolerances (stated by the path's parity bar): max |gpu - oracle| <= 2e-3 on
attention outputs, fp32 state relative error (Frobenius) <= 1e-4 after 4096
steps.  Relative RMS is printed beside every max-abs check.
"""
import os
import sys

import numpy as np
import pytest

import oracle as O
from ds4f_hip import synth as S
from ds4f_hip import workloads as W
from ds4f_hip.attn import GpuAttention, KvCache

pytestmark = pytest.mark.gpu

GQ = W.GqaGeom()
LG = W.LinGeom()
ATOL = 2e-3
STATE_RTOL = 1e-4


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _err(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    mx = float(np.abs(got - ref).max()) if got.size else 0.0
    rr = float(np.sqrt(((got - ref) ** 2).sum() / max((ref ** 2).sum(), 1e-300)))
    return mx, rr


# ------------------------------------------------------------------ helpers
def _gqa_setup(n_past, max_tokens, seed=0, layer=0):
    """A one-GQA-layer binding whose cache holds n_past bf16 rows; returns
    (plugin, oracle kv block, weights).  Up to 8192 rows the host draws them
    and binds; beyond, the device draws them (ds4f_hip_synth_gqa_cache, the
    same streams) and the rows are synced to the host for the oracle."""
    cache = KvCache(1, max_tokens)
    if n_past <= 8192:
        kc, vc = W.gqa_cache(GQ, n_past, seed, layer)
        half = GQ.kv_heads * GQ.head_dim
        cache.kv[0, :n_past, :half] = kc.reshape(n_past, half)
        cache.kv[0, :n_past, half:] = vc.reshape(n_past, half)
        ga = GpuAttention([2], max_tokens, cache, n_kv_tokens=n_past)
    else:
        from ds4f_hip.lib import check, load
        ga = GpuAttention([2], max_tokens, cache)
        check(load().ds4f_hip_synth_gqa_cache(0, n_past, seed, S.tid(S.GQA_KCACHE, layer),
                                              S.tid(S.GQA_VCACHE, layer), None), "synth kv")
        ga.sync(0, to_host=True, n_kv_tokens=n_past)
    ref_kv = cache.kv[0].copy()
    return ga, cache, ref_kv, W.gqa_weights(GQ, seed, layer)


def _lin_setup(token, seed=0, layer=0, max_tokens=8192):
    cache = KvCache(1, max_tokens, with_kv=False)
    cache.lin[0] = W.lin_state(LG, seed, layer)
    cache.conv[0] = W.ring_from_history(LG, W.lin_conv_history(LG, seed, layer), token)
    ref_ring, ref_S = cache.conv[0].copy(), cache.lin[0].copy()
    ga = GpuAttention([1], max_tokens, cache)
    return ga, cache, ref_ring, ref_S, W.lin_weights(LG, seed, layer)


# ------------------------------------------------------------------ synth
def test_device_generator_matches_numpy():
    import torch
    from ds4f_hip.lib import load
    from ds4f_hip.attn import dptr
    lib = load()
    assert lib.ds4f_gpu_init() == 0
    n = 1 << 20
    f = torch.empty(n, dtype=torch.float32, device="cuda")
    h = torch.empty(n, dtype=torch.int16, device="cuda")
    u = torch.empty(n, dtype=torch.float32, device="cuda")
    assert lib.ds4f_hip_synth(dptr(f), n, 0, 0, 0.0, 0.05, 0, 77, None) == 0
    assert lib.ds4f_hip_synth(dptr(h), n, 1, 0, 1.0, 0.1, 0, 78, None) == 0
    assert lib.ds4f_hip_synth(dptr(u), n, 0, 1, 0.0, 2.7, 0, 79, None) == 0
    torch.cuda.synchronize()
    f_ref = S.normal(0, 77, n, 0.0, 0.05)
    h_ref = S.bf16_bits(S.normal(0, 78, n, 1.0, 0.1))
    u_ref = S.uniform(0, 79, n, 0.0, 2.7)
    fg = f.cpu().numpy()
    ulp = np.abs(fg.view(np.int32).astype(np.int64) - f_ref.view(np.int32).astype(np.int64))
    _say(f"synth normal: {int((ulp > 0).sum())} of {n} differ, max {int(ulp.max())} ulp")
    assert ulp.max() <= 1
    assert np.array_equal(h.cpu().numpy().view(np.uint16), h_ref)
    assert np.array_equal(u.cpu().numpy(), u_ref)


def test_device_state_generator_matches_numpy():
    """ds4f_hip_synth_lin_state writes the value-major device state of a
    bound layer; synced back it is workloads.lin_state (row = key dim) to 1
    ulp, and exactly zero for sigma 0."""
    from ds4f_hip.lib import load
    lib = load()
    cache = KvCache(1, 64, with_kv=False)
    ga = GpuAttention([1], 64, cache)
    tid = S.tid(S.LIN_STATE, 0)
    assert lib.ds4f_hip_synth_lin_state(0, 0.05, 5, tid, None) == 0
    ga.sync(0, to_host=True)
    ref = W.lin_state(LG, 5, 0)
    ulp = np.abs(cache.lin[0].astype(np.float32).view(np.int32).astype(np.int64)
                 - ref.astype(np.float32).view(np.int32).astype(np.int64))
    _say(f"synth lin state: {int((ulp > 0).sum())} of {ulp.size} differ, max {int(ulp.max())} ulp")
    assert ulp.max() <= 1
    assert lib.ds4f_hip_synth_lin_state(0, 0.0, 5, tid, None) == 0
    ga.sync(0, to_host=True)
    assert not np.any(cache.lin[0])


# ------------------------------------------------------------------ delta rule
def test_lin_decode_single_step_full_shape():
    token = 3
    ga, cache, ring, S0, w = _lin_setup(token)
    qkv, z, a, b = W.lin_token(LG, 0, 0, 0)
    out, post = ga.lin_decode(0, token, qkv, z, a, b, w)
    ref, rpost = O.lin_body(ring, S0, token, qkv, z, a, b, w.conv_w, w.A_log, w.dt_bias,
                            w.norm_w, LG.k_heads, LG.v_heads, LG.kd, LG.vd)
    ga.sync(0, to_host=True)
    mx, rr = _err(out, ref)
    _say(f"lin decode out: max abs {mx:.3e} rel-rms {rr:.3e} (|ref| max {np.abs(ref).max():.3f})")
    assert mx <= ATOL and rr < 1e-5
    assert _err(post, rpost)[0] < 1e-5
    smx, srr = _err(cache.lin[0], S0)
    _say(f"lin decode state: max abs {smx:.3e} rel {srr:.3e}")
    assert srr <= STATE_RTOL / 100
    assert np.array_equal(cache.conv[0], ring)           # ring slot token%4 = raw row
    ga.close()


@pytest.mark.parametrize("token", [0, 1, 2, 5])
def test_lin_decode_early_tokens_skip_taps(token):
    ga, cache, ring, S0, w = _lin_setup(token, seed=3)
    # junk in slots of negative positions must not be read
    cache.conv[0][:] = np.where(cache.conv[0] == 0, 7.0, cache.conv[0])
    ring[:] = cache.conv[0]
    ga.sync(0, to_host=False)
    qkv, z, a, b = W.lin_token(LG, 3, 0, token)
    out, post = ga.lin_decode(0, token, qkv, z, a, b, w)
    ref, rpost = O.lin_body(ring, S0, token, qkv, z, a, b, w.conv_w, w.A_log, w.dt_bias,
                            w.norm_w, LG.k_heads, LG.v_heads, LG.kd, LG.vd)
    assert _err(out, ref)[0] <= ATOL and _err(post, rpost)[0] < 1e-5
    ga.close()


def test_lin_decode_4096_steps_state():
    T = 4096
    ga, cache, ring, S0, w = _lin_setup(3, seed=5)
    worst = 0.0
    for s in range(T):
        tok = 3 + s
        qkv, z, a, b = W.lin_token(LG, 5, 0, s)
        out, _ = ga.lin_decode(0, tok, qkv, z, a, b, w)
        ref, _ = O.lin_body(ring, S0, tok, qkv, z, a, b, w.conv_w, w.A_log, w.dt_bias, w.norm_w,
                            LG.k_heads, LG.v_heads, LG.kd, LG.vd)
        worst = max(worst, _err(out, ref)[0])
        if s % 1024 == 1023:
            _say(f"step {s + 1}: worst out err so far {worst:.3e}")
    ga.sync(0, to_host=True)
    smx, srr = _err(cache.lin[0], S0)
    _say(f"state after {T} steps: rel {srr:.3e} max abs {smx:.3e}; worst out err {worst:.3e}")
    assert srr <= STATE_RTOL
    assert worst <= ATOL
    assert np.array_equal(cache.conv[0], ring)
    ga.close()


# ------------------------------------------------------------------ GQA
# 8193: 65 split-K chunks of 128 positions, the last holding one;
# 16383 / 16384 / 16385: the split goes from 128 chunks of 128 positions to
# 86 chunks of 192, the last one ragged (65)
@pytest.mark.parametrize("n_past", [4096, 0, 1, 15, 16, 17, 63, 64, 65, 1000, 8191, 8193, 16383,
                                    16384, 16385, 32768, 131072, 262143])
def test_gqa_decode_step(n_past):
    max_tokens = max(n_past + 8, 64)
    _say(f"gqa decode n_past={n_past}")
    ga, cache, ref_kv, (qn, kn) = _gqa_setup(n_past, max_tokens)
    q, k, v = W.gqa_token(GQ, 0, 0, n_past)
    out, kpost = ga.gqa_decode(0, n_past, q, k, v, qn, kn)
    ref, rk = O.gqa_body(ref_kv, n_past, q, k, v, qn, kn, GQ.heads, GQ.kv_heads, GQ.head_dim)
    mx, rr = _err(out, ref)
    _say(f"  out max abs {mx:.3e} rel-rms {rr:.3e} (|ref| max {np.abs(ref).max():.3f})")
    assert mx <= ATOL and rr < 1e-4
    assert _err(kpost, rk)[0] < 1e-5
    ga.sync(0, to_host=True, n_kv_tokens=n_past + 1)
    row = cache.kv[0, n_past]
    half = GQ.kv_heads * GQ.head_dim
    assert np.array_equal(row[:half], S.bf16_round(rk))
    assert np.array_equal(row[half:], S.bf16_round(v.reshape(-1)))
    assert np.array_equal(cache.kv[0, :n_past], ref_kv[:n_past])   # past rows untouched
    ga.close()


def test_gqa_decode_consecutive_steps():
    """64 steps from 500 past rows.  The device cache holds bf16 rows, so the
    oracle's cache gets each new row bf16-rounded too (same inputs); the
    distance to the all-fp32 cache is reported."""
    n0, steps = 500, 64
    ga, cache, ref_kv, (qn, kn) = _gqa_setup(n0, n0 + steps + 8)
    fp32_kv = ref_kv.copy()
    worst = worst32 = 0.0
    half = GQ.kv_heads * GQ.head_dim
    for s in range(steps):
        tok = n0 + s
        q, k, v = W.gqa_token(GQ, 0, 0, tok)
        out, _ = ga.gqa_decode(0, tok, q, k, v, qn, kn)
        ref, rk = O.gqa_body(ref_kv, tok, q, k, v, qn, kn, GQ.heads, GQ.kv_heads, GQ.head_dim)
        ref_kv[tok] = S.bf16_round(ref_kv[tok])
        ref32, _ = O.gqa_body(fp32_kv, tok, q, k, v, qn, kn, GQ.heads, GQ.kv_heads, GQ.head_dim)
        worst = max(worst, _err(out, ref)[0])
        worst32 = max(worst32, _err(out, ref32)[0])
    _say(f"64 steps: worst vs bf16-row oracle {worst:.3e}, vs fp32-cache oracle {worst32:.3e}")
    assert worst <= ATOL
    ga.close()


# ------------------------------------------------------------------ plumbing
def test_bind_sync_roundtrip():
    rng = np.random.default_rng(0)
    cache = KvCache(4, 100)
    cache.kv[:] = S.bf16_round(rng.standard_normal(cache.kv.shape).astype(np.float32))
    cache.lin[:] = rng.standard_normal(cache.lin.shape).astype(np.float32)
    cache.conv[:] = rng.standard_normal(cache.conv.shape).astype(np.float32)
    kinds = [1, 1, 1, 2]
    snap = (cache.kv.copy(), cache.lin.copy(), cache.conv.copy())
    ga = GpuAttention(kinds, 100, cache, n_kv_tokens=100)
    cache.kv[:] = 0
    cache.lin[:] = 0
    cache.conv[:] = 0
    ga.sync(-1, to_host=True, n_kv_tokens=100)
    assert np.array_equal(cache.kv[3], snap[0][3])        # GQA layer only
    assert not cache.kv[:3].any()
    for L in range(3):
        assert np.array_equal(cache.lin[L], snap[1][L]) and np.array_equal(cache.conv[L], snap[2][L])
    ga.close()


def test_prefill_entry_points_serial_semantics():
    T = 40
    # delta rule
    ga, cache, ring, S0, w = _lin_setup(0, seed=9)
    ring[:] = 0
    cache.conv[0][:] = 0
    ga.sync(0, to_host=False)
    qkv, z, a, b = W.lin_tokens(LG, T, 9)
    out, post = ga.lin_prefill(0, 0, qkv, z, a, b, w)
    ref, rpost = O.lin_prefill(ring, S0, 0, qkv, z, a, b, w.conv_w, w.A_log, w.dt_bias,
                               w.norm_w, LG.k_heads, LG.v_heads, LG.kd, LG.vd)
    assert _err(out, ref)[0] <= ATOL
    ga.close()
    # GQA
    ga, cache, ref_kv, (qn, kn) = _gqa_setup(0, 64)
    q, k, v = W.gqa_prefill_tokens(GQ, T)
    out, kp = ga.gqa_prefill(0, 0, q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1), qn, kn)
    ref, rk = O.gqa_prefill(ref_kv, 0, q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1), qn,
                            kn, GQ.heads, GQ.kv_heads, GQ.head_dim)
    mx, rr = _err(out, ref)
    _say(f"gqa prefill (serial decode path) T={T}: max abs {mx:.3e} rel-rms {rr:.3e}")
    assert mx <= ATOL
    assert _err(kp, rk)[0] < 1e-5
    ga.close()


def test_forced_failure_falls_back_with_state_written_back():
    """DS4F_GPU_FAIL_AFTER=n: the (n+1)-th call fails before launching; the
    device state lands in the bound host arrays and the plugin stays off."""
    from ds4f_hip.lib import load
    lib = load()
    lib.ds4f_gpu_free()
    os.environ["DS4F_GPU_FAIL_AFTER"] = "3"
    try:
        ga, cache, ring, S0, w = _lin_setup(3, seed=11)
        for s in range(3):
            qkv, z, a, b = W.lin_token(LG, 11, 0, s)
            ga.lin_decode(0, 3 + s, qkv, z, a, b, w)
            O.lin_body(ring, S0, 3 + s, qkv, z, a, b, w.conv_w, w.A_log, w.dt_bias, w.norm_w,
                       LG.k_heads, LG.v_heads, LG.kd, LG.vd)
        cache.lin[:] = 0
        cache.conv[:] = 0
        qkv, z, a, b = W.lin_token(LG, 11, 0, 3)
        with pytest.raises(RuntimeError, match="forced failure"):
            ga.lin_decode(0, 6, qkv, z, a, b, w)
        # written back: the state after 3 steps, ring included
        assert _err(cache.lin[0], S0)[1] < 1e-5
        assert np.array_equal(cache.conv[0], ring)
        # the CPU continues from there
        O.lin_body(cache.conv[0], cache.lin[0], 6, qkv, z, a, b, w.conv_w, w.A_log, w.dt_bias,
                   w.norm_w, LG.k_heads, LG.v_heads, LG.kd, LG.vd)
        # sticky: the next call is refused too
        with pytest.raises(RuntimeError):
            ga.lin_decode(0, 7, qkv, z, a, b, w)
    finally:
        os.environ.pop("DS4F_GPU_FAIL_AFTER", None)
        lib.ds4f_gpu_free()
