"""Pins of the CPU oracle (no GPU).

The reference path has no test or golden vector of its own for these cores,
and it does not compile in this image, so the oracle is pinned by:
  * the double-precision model in f64_model.py (independent statement),
  * closed forms and invariants the mathematics fixes,
  * known-answer vectors of the input generator,
  * the reference's own known answers for the MLX 4-bit format and matvec
    (tests/test_kernels.c:357-446 of the reference, restated as values in
    the MLX 4-bit tests below).
"""
import numpy as np
import pytest

import oracle as O
import f64_model as F
from ds4f_hip import synth as S
from ds4f_hip import workloads as W

SMALL_GQA = W.GqaGeom(heads=4, kv_heads=2, head_dim=64)
FULL_GQA = W.GqaGeom()
SMALL_LIN = W.LinGeom(k_heads=2, v_heads=4, kd=32, vd=32)
FULL_LIN = W.LinGeom()


# ---------------------------------------------------------------- generator
def test_splitmix64_known_answer():
    # splitmix64 seeded with 0: the published first outputs of the algorithm.
    d = S.draws(0, 0, 0, 3)
    assert [int(x) for x in d] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_generator_offsets_and_moments():
    a = S.draws(0, 7, 0, 100)
    b = S.draws(0, 7, 40, 60)
    assert np.array_equal(a[40:], b)
    z = S.normal(0, 123, 200000)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01
    u = S.uniform(0, 5, 100000, 0.0, 2.7)
    assert u.min() >= 0 and u.max() < 2.7 and abs(u.mean() - 1.35) < 0.02


def test_bf16_round_known_values():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 1.0 + 2 ** -9], np.float32)
    bits = S.bf16_bits(x)
    # 1+2^-8 is a tie -> even (0x3F80); 1+3*2^-8 tie -> even (0x3F82)
    assert [hex(int(v)) for v in bits] == ["0x3f80", "0x3f80", "0x3f82", "0xc020", "0x3f80"]


# ---------------------------------------------------------------- GQA
def _gqa_case(g, n_past, seed=0):
    qn, kn = W.gqa_weights(g, seed)
    kc, vc = W.gqa_cache(g, n_past, seed)
    q, k, v = W.gqa_token(g, seed)
    return qn, kn, kc, vc, q, k, v


def _kv_layer(g, kc, vc, max_tokens):
    row = 2 * g.kv_heads * g.head_dim
    kv = np.zeros((max_tokens, row), np.float32)
    n = kc.shape[0]
    kv[:n, : g.kv_heads * g.head_dim] = kc.reshape(n, -1)
    kv[:n, g.kv_heads * g.head_dim:] = vc.reshape(n, -1)
    return kv


@pytest.mark.parametrize("g,n_past", [(SMALL_GQA, 37), (FULL_GQA, 300)])
def test_gqa_oracle_matches_f64(g, n_past):
    qn, kn, kc, vc, q, k, v = _gqa_case(g, n_past)
    kv = _kv_layer(g, kc, vc, n_past + 5)
    out, k_post = O.gqa_body(kv, n_past, q, k, v, qn, kn, g.heads, g.kv_heads, g.head_dim)
    ref, kref = F.gqa_step(kc, vc, q, k, v, qn, kn, n_past)
    assert np.abs(out - ref.reshape(-1)).max() < 2e-6
    assert np.abs(k_post - kref.reshape(-1)).max() < 2e-6
    # the cache row at `token` holds the normed, rotated k and the raw v
    half = g.kv_heads * g.head_dim
    assert np.array_equal(kv[n_past, :half], k_post)
    assert np.array_equal(kv[n_past, half:], v.reshape(-1))
    assert not kv[n_past + 1:].any()


def test_gqa_first_token_is_gated_v():
    g = FULL_GQA
    qn, kn, _, _, q, k, v = _gqa_case(g, 0)
    kv = np.zeros((4, 2 * g.kv_heads * g.head_dim), np.float32)
    out, _ = O.gqa_body(kv, 0, q, k, v, qn, kn, g.heads, g.kv_heads, g.head_dim)
    gate = q[:, g.head_dim:]
    want = v[np.arange(g.heads) // 8] * (1 / (1 + np.exp(-gate.astype(np.float64))))
    assert np.abs(out.reshape(g.heads, -1) - want).max() < 1e-6


def test_gqa_identical_keys_average_values():
    g = SMALL_GQA
    qn, kn, kc, vc, q, k, v = _gqa_case(g, 20)
    # every past key equals the new key after norm+RoPE at this position, so
    # all scores tie and the output is the mean of V times the gate
    _, kpost = O.gqa_body(np.zeros((32, 2 * g.kv_heads * g.head_dim), np.float32), 20, q, k, v,
                          qn, kn, g.heads, g.kv_heads, g.head_dim)
    kc[:] = kpost.reshape(g.kv_heads, g.head_dim)[None]
    kv = _kv_layer(g, kc, vc, 32)
    out, _ = O.gqa_body(kv, 20, q, k, v, qn, kn, g.heads, g.kv_heads, g.head_dim)
    V = np.concatenate([vc, v[None]], 0).astype(np.float64)
    grp = g.heads // g.kv_heads
    want = V.mean(0)[np.arange(g.heads) // grp] * F.sigmoid(q[:, g.head_dim:])
    assert np.abs(out.reshape(g.heads, -1) - want).max() < 1e-5


def test_rope_table_and_half_split():
    c0, s0 = O.rope_table(0)
    assert np.all(c0 == 1) and np.all(s0 == 0)          # position 0 = identity
    c, s = O.rope_table(1000)
    inv = 1.0 / 1e7 ** (np.arange(32) * 2 / 64.0)
    assert np.array_equal(c, np.cos(1000 * inv).astype(np.float32))
    assert np.array_equal(s, np.sin(1000 * inv).astype(np.float32))
    # half-split detector: energy in dim 0 moves to dim 32, not dim 1
    g = W.GqaGeom(heads=1, kv_heads=1, head_dim=256)
    q = np.zeros((1, 512), np.float32)
    q[0, 0] = 1.0
    k = np.zeros((1, 256), np.float32)
    k[0, 0] = 1.0
    v = np.ones((1, 256), np.float32)
    w1 = S.bf16_bits(np.ones(256, np.float32))
    kv = np.zeros((8, 512), np.float32)
    _, kp = O.gqa_body(kv, 5, q, k, v, w1, w1, 1, 1, 256)
    r = np.sqrt(1.0 / 256 + 1e-6)
    assert abs(kp[0] - np.float32(1 / r) * np.cos(5.0)) < 1e-4
    assert abs(kp[32] - np.float32(1 / r) * np.sin(5.0)) < 1e-4
    assert kp[1] == 0 and np.all(kp[64:] == 0)


def test_rope_relative_position():
    g = W.GqaGeom(heads=1, kv_heads=1, head_dim=256)
    rng = np.random.default_rng(1)
    x = rng.standard_normal(256)
    y = rng.standard_normal(256)
    d1 = F.rope(x, 100, 64) @ F.rope(y, 90, 64)
    d2 = F.rope(x, 2010, 64) @ F.rope(y, 2000, 64)
    assert abs(d1 - d2) < 1e-9
    # the oracle's rotation preserves each pair's norm
    q = np.zeros((1, 512), np.float32)
    q[0, :256] = x
    k = y.astype(np.float32)[None]
    w1 = S.bf16_bits(np.ones(256, np.float32))
    kv = np.zeros((3000, 512), np.float32)
    _, kp = O.gqa_body(kv, 2000, q, k, np.ones((1, 256), np.float32), w1, w1, 1, 1, 256)
    kn = F.rmsnorm(y)
    assert np.allclose(kp[:32] ** 2 + kp[32:64] ** 2, kn[:32] ** 2 + kn[32:64] ** 2, atol=1e-5)


def test_gqa_token_out_of_range_is_silent_skip():
    g = SMALL_GQA
    qn, kn, kc, vc, q, k, v = _gqa_case(g, 4)
    kv = _kv_layer(g, kc, vc, 4)
    before = kv.copy()
    out, kp = O.gqa_body(kv, 4, q, k, v, qn, kn, g.heads, g.kv_heads, g.head_dim)
    assert np.array_equal(kv, before) and not out.any() and np.array_equal(kp, k.reshape(-1))


def test_gqa_prefill_matches_f64_causal():
    g = SMALL_GQA
    T = 40
    qn, kn = W.gqa_weights(g)
    q, k, v = W.gqa_prefill_tokens(g, T)
    kv = np.zeros((T, 2 * g.kv_heads * g.head_dim), np.float32)
    out, kp = O.gqa_prefill(kv, 0, q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1), qn, kn,
                            g.heads, g.kv_heads, g.head_dim)
    ref, kref = F.gqa_prefill(q, k, v, qn, kn)
    assert np.abs(out - ref.reshape(T, -1)).max() < 2e-6
    assert np.abs(kp - kref.reshape(T, -1)).max() < 2e-6


# ---------------------------------------------------------------- linear
def _lin_case(g, token=3, seed=0, layer=0, step=0):
    w = W.lin_weights(g, seed, layer)
    S0 = W.lin_state(g, seed, layer)
    hist = W.lin_conv_history(g, seed, layer)
    qkv, z, a, b = W.lin_token(g, seed, layer, step)
    return w, S0, hist, qkv, z, a, b


def _hist_for(hist, token):
    h = hist.copy()
    for j in range(3):
        if token - 3 + j < 0:
            h[j] = 0
    return h


@pytest.mark.parametrize("g,token", [(SMALL_LIN, 3), (SMALL_LIN, 1), (FULL_LIN, 3), (FULL_LIN, 9)])
def test_lin_oracle_matches_f64(g, token):
    w, S0, hist, qkv, z, a, b = _lin_case(g, token)
    ring = W.ring_from_history(g, hist, token)
    St = S0.copy()
    out, post = O.lin_body(ring, St, token, qkv, z, a, b, w.conv_w, w.A_log, w.dt_bias, w.norm_w,
                           g.k_heads, g.v_heads, g.kd, g.vd)
    ref, Sref, pref = F.lin_step(_hist_for(hist, token), S0, qkv, z, a, b, w.conv_w, w.A_log,
                                 w.dt_bias, w.norm_w, g.k_heads, g.v_heads, g.kd, g.vd)
    assert np.abs(St - Sref).max() / np.abs(Sref).max() < 1e-5
    assert np.abs(post - pref).max() < 1e-5
    assert np.abs(out - ref).max() < 1e-4 * max(1.0, np.abs(ref).max())
    assert np.array_equal(ring[token % 4], qkv)           # raw row written to slot t%4


def test_conv_taps_and_zero_padding():
    g = SMALL_LIN
    rows = g.rows
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, rows)).astype(np.float32)
    ones = S.bf16_bits(np.ones((rows, 4), np.float32))
    w0 = W.lin_weights(g)
    zeros_vh = np.zeros(g.v_heads, np.float32)
    for tap in range(4):
        cw = np.zeros((rows, 4), np.float32)
        cw[:, tap] = 1.0
        ring = np.zeros((4, rows), np.float32)
        for p in range(3):
            ring[p] = x[p]
        S0 = np.zeros((g.v_heads, g.kd, g.vd), np.float32)
        _, post = O.lin_body(ring, S0, 3, x[3], np.ones(g.v_heads * g.vd, np.float32), zeros_vh,
                             zeros_vh, S.bf16_bits(cw), w0.A_log, w0.dt_bias, w0.norm_w,
                             g.k_heads, g.v_heads, g.kd, g.vd)
        src = x[tap].astype(np.float64)                    # tap 0 = oldest (t-3)
        silu = src * F.sigmoid(src)
        vpart = post[2 * g.k_heads * g.kd:]
        assert np.abs(vpart - silu[2 * g.k_heads * g.kd:]).max() < 1e-6
    # token 0: taps before position 0 are skipped even if the ring holds junk
    ring = np.full((4, rows), 123.0, np.float32)
    S0 = np.zeros((g.v_heads, g.kd, g.vd), np.float32)
    _, post = O.lin_body(ring, S0, 0, x[0], np.ones(g.v_heads * g.vd, np.float32), zeros_vh,
                         zeros_vh, ones, w0.A_log, w0.dt_bias, w0.norm_w,
                         g.k_heads, g.v_heads, g.kd, g.vd)
    src = x[0].astype(np.float64)
    assert np.abs(post[2 * g.k_heads * g.kd:] - (src * F.sigmoid(src))[2 * g.k_heads * g.kd:]).max() < 1e-6


def _gate_inputs(g, a_val, b_val, alog_val):
    w = W.lin_weights(g)
    return (np.full(g.v_heads, a_val, np.float32), np.full(g.v_heads, b_val, np.float32),
            np.full(g.v_heads, alog_val, np.float32), w)


def test_delta_beta_zero_is_pure_decay():
    g = SMALL_LIN
    w, S0, hist, qkv, z, a, b = _lin_case(g)
    b = np.full(g.v_heads, -200.0, np.float32)             # sigmoid -> 0 exactly
    ring = W.ring_from_history(g, hist, 3)
    St = S0.copy()
    _, post = O.lin_body(ring, St, 3, qkv, z, a, b, w.conv_w, w.A_log, w.dt_bias, w.norm_w,
                         g.k_heads, g.v_heads, g.kd, g.vd)
    x = a.astype(np.float64) + F.bf(w.dt_bias)
    dec = np.exp(-np.exp(w.A_log.astype(np.float64)) * np.logaddexp(0, x))
    want = S0 * dec[:, None, None]
    assert np.abs(St - want).max() < 1e-6 * np.abs(S0).max() + 1e-12


def test_delta_write_property():
    # decay 1 (A_log -> -inf), beta 1, ||k|| ~ 1: after the update S^T k = v
    g = SMALL_LIN
    w, S0, hist, qkv, z, a, b = _lin_case(g)
    A_log = np.full(g.v_heads, -200.0, np.float32)
    b = np.full(g.v_heads, 200.0, np.float32)
    ring = W.ring_from_history(g, hist, 3)
    St = S0.copy()
    _, post = O.lin_body(ring, St, 3, qkv, z, a, b, w.conv_w, A_log, w.dt_bias, w.norm_w,
                         g.k_heads, g.v_heads, g.kd, g.vd)
    kk = post[g.k_heads * g.kd:2 * g.k_heads * g.kd].reshape(g.k_heads, g.kd)
    vv = post[2 * g.k_heads * g.kd:].reshape(g.v_heads, g.vd)
    for h in range(g.v_heads):
        k = kk[h // 2].astype(np.float64)
        nk = k @ k                                          # 1 up to eps/mean(k^2)
        got = St[h].T.astype(np.float64) @ k
        want = vv[h] * nk + S0[h].T.astype(np.float64) @ k * (1 - nk)
        assert np.abs(got - want).max() < 1e-4


def test_delta_from_zero_state_closed_form():
    g = SMALL_LIN
    w, _, hist, qkv, z, a, b = _lin_case(g)
    ring = W.ring_from_history(g, hist, 3)
    St = np.zeros((g.v_heads, g.kd, g.vd), np.float32)
    out, post = O.lin_body(ring, St, 3, qkv, z, a, b, w.conv_w, w.A_log, w.dt_bias, w.norm_w,
                           g.k_heads, g.v_heads, g.kd, g.vd)
    q = post[:g.k_heads * g.kd].reshape(g.k_heads, g.kd).astype(np.float64)
    kk = post[g.k_heads * g.kd:2 * g.k_heads * g.kd].reshape(g.k_heads, g.kd).astype(np.float64)
    vv = post[2 * g.k_heads * g.kd:].reshape(g.v_heads, g.vd).astype(np.float64)
    beta = F.sigmoid(b)
    zz = z.reshape(g.v_heads, g.vd).astype(np.float64)
    for h in range(g.v_heads):
        assert np.abs(St[h] - beta[h] * np.outer(kk[h // 2], vv[h])).max() < 1e-6
        o = beta[h] * (kk[h // 2] @ q[h // 2]) * vv[h]          # S^T q
        want = F.rmsnorm(o, F.bf(w.norm_w)) * zz[h] * F.sigmoid(zz[h])
        assert np.abs(out[h * g.vd:(h + 1) * g.vd] - want).max() < 1e-4


def test_softplus_branch_and_gated_norm_zero():
    g = SMALL_LIN
    w, S0, hist, qkv, z, a, b = _lin_case(g)
    z0 = np.zeros_like(z)
    ring = W.ring_from_history(g, hist, 3)
    out, _ = O.lin_body(ring, S0.copy(), 3, qkv, z0, a, b, w.conv_w, w.A_log, w.dt_bias,
                        w.norm_w, g.k_heads, g.v_heads, g.kd, g.vd)
    assert not out.any()                                   # silu(0) = 0 gates to 0
    # both softplus branches give log1p(exp(x)) to float precision
    for aval in (-30.0, -3.0, 0.0, 3.0, 30.0):
        a1 = np.full(g.v_heads, aval, np.float32)
        St = S0.copy()
        bneg = np.full(g.v_heads, -200.0, np.float32)
        O.lin_body(W.ring_from_history(g, hist, 3), St, 3, qkv, z, a1, bneg, w.conv_w, w.A_log,
                   w.dt_bias, w.norm_w, g.k_heads, g.v_heads, g.kd, g.vd)
        x = a1.astype(np.float64) + F.bf(w.dt_bias)
        dec = np.exp(-np.exp(w.A_log.astype(np.float64)) * np.logaddexp(0, x))
        ratio = St[:, 0, 0] / S0[:, 0, 0]
        assert np.allclose(ratio, dec, rtol=2e-5, atol=1e-30)


def test_qk_norm_eps_on_mean():
    # tiny-norm q/k: eps sits on mean(x^2), not on sum(x^2) (an l2norm with
    # eps on the sum would give a visibly different scale)
    g = SMALL_LIN
    w, S0, hist, qkv, z, a, b = _lin_case(g)
    ones = np.zeros((g.rows, 4), np.float32)
    ones[:, 3] = 1.0
    small = qkv * 1e-3
    ring = np.zeros((4, g.rows), np.float32)
    _, post = O.lin_body(ring, S0.copy(), 0, small, z, a, b, S.bf16_bits(ones), w.A_log,
                         w.dt_bias, w.norm_w, g.k_heads, g.v_heads, g.kd, g.vd)
    x = small.astype(np.float64)
    act = x * F.sigmoid(x)
    q0 = act[:g.kd]
    want = q0 / np.sqrt((q0 ** 2).mean() + 1e-6) / g.kd
    assert np.abs(post[:g.kd] - want).max() < 1e-6 * np.abs(want).max() + 1e-9
    l2 = q0 / np.sqrt((q0 ** 2).sum() + 1e-6) / np.sqrt(g.kd)
    assert np.abs(post[:g.kd] - l2).max() > 1e-3 * np.abs(want).max()


def test_lin_prefill_equals_serial_and_f64():
    g = SMALL_LIN
    T = 24
    w = W.lin_weights(g)
    qkv, z, a, b = W.lin_tokens(g, T)
    ring = np.zeros((4, g.rows), np.float32)
    S0 = np.zeros((g.v_heads, g.kd, g.vd), np.float32)
    out, _ = O.lin_prefill(ring, S0, 0, qkv, z, a, b, w.conv_w, w.A_log, w.dt_bias, w.norm_w,
                           g.k_heads, g.v_heads, g.kd, g.vd)
    hist = np.zeros((3, g.rows))
    Sf = np.zeros((g.v_heads, g.kd, g.vd))
    for t in range(T):
        ref, Sf, _ = F.lin_step(hist, Sf, qkv[t], z[t], a[t], b[t], w.conv_w, w.A_log, w.dt_bias,
                                w.norm_w, g.k_heads, g.v_heads, g.kd, g.vd)
        hist = np.concatenate([hist[1:], qkv[t][None].astype(np.float64)], 0)
        assert np.abs(out[t] - ref).max() < 2e-4 * max(1.0, np.abs(ref).max())
    assert np.abs(S0 - Sf).max() / np.abs(Sf).max() < 1e-5


def test_gqa_cache_row_helper_equals_body_rows():
    # the cheap cache-row helper writes exactly the rows the serial body writes
    g = FULL_GQA
    T = 40
    qn, kn = W.gqa_weights(g)
    q, k, v = W.gqa_prefill_tokens(g, T)
    rows = O.gqa_cache_rows(k, v, kn, 0, g.kv_heads, g.head_dim)
    kv = np.zeros((T, 2 * g.kv_heads * g.head_dim), np.float32)
    O.gqa_prefill(kv, 0, q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1), qn, kn,
                  g.heads, g.kv_heads, g.head_dim)
    assert np.array_equal(kv, rows)


# ---------------------------------------------------------------- MLX 4-bit
def _mlx4_dense(vals, scales, biases, R, C, offset=0):
    """Independent float64 dequantisation of an MLX 4-bit [R x C] matrix:
    element k = r*C + c is nibble k%8 of word k/8, group k/64."""
    k = np.arange(R * C)
    q = ((vals[k >> 3] >> (4 * (k & 7)).astype(np.uint32)) & 0xF).astype(np.float64) - offset
    g = k // 64
    s = S.bits_to_f32(scales[g]).astype(np.float64)
    b = 0.0 if biases is None else S.bits_to_f32(biases[g]).astype(np.float64)
    return (q * s + b).reshape(R, C)


def test_mlx4_decode_known_vector():
    # The reference's known answers (tests/test_kernels.c:357-391): nibbles
    # (i*8+j) % 16 with scale 1.0, bias 0 decode to k % 16; element 64 of a
    # second group (scale 2.0, nibble 5) decodes to 10.
    vals = np.zeros(8, np.uint32)
    for i in range(8):
        for j in range(8):
            vals[i] |= np.uint32(((i * 8 + j) % 16) << (4 * j))
    out = O.mlx4_decode(vals, np.array([0x3F80], np.uint16), np.array([0], np.uint16), 64)
    assert np.array_equal(out, (np.arange(64) % 16).astype(np.float32))
    v2 = np.zeros(9, np.uint32)
    v2[8] = 5
    out2 = O.mlx4_decode(v2, np.array([0x3F80, 0x4000], np.uint16), np.zeros(2, np.uint16), 72)
    assert out2[64] == 10.0 and not np.any(out2[:64]) and not np.any(out2[65:])


@pytest.mark.parametrize("R,C", [(8, 200), (3, 64), (5, 96), (16, 2048), (7, 4096)])
def test_mlx4_matvec_against_dense(R, C):
    # The reference's test 13 (tests/test_kernels.c:394-446) restated, with
    # shapes whose 64-element groups straddle rows (C = 200, 96).
    vals, scales, biases = W.mlx4_matrix(R, C, 3, R)
    x = W.mlx4_x(C, 3, R)
    y = O.mlx4_matvec(vals, scales, biases, R, C, x)
    dense = _mlx4_dense(vals, scales, biases, R, C)
    ref = dense @ x.astype(np.float64)
    assert np.all(np.abs(y - ref) <= 1e-3 * (1 + np.abs(ref)))       # the reference's bound
    bound = 1e-6 * (np.abs(dense) @ np.abs(x.astype(np.float64)))     # fp32 accumulation, C <= 4096
    assert np.all(np.abs(y - ref) <= bound)


def test_mlx4_matvec_linearity_and_absent_bias():
    R, C = 6, 320
    vals, scales, _ = W.mlx4_matrix(R, C, 4, 0)
    x1, x2 = W.mlx4_x(C, 4, 0, 0), W.mlx4_x(C, 4, 0, 1)
    y1 = O.mlx4_matvec(vals, scales, None, R, C, x1)
    y2 = O.mlx4_matvec(vals, scales, None, R, C, x2)
    y12 = O.mlx4_matvec(vals, scales, None, R, C, 2.0 * x1 - 0.5 * x2)
    assert np.allclose(y12, 2.0 * y1 - 0.5 * y2, rtol=1e-5, atol=1e-5)
    yz = O.mlx4_matvec(vals, scales, np.zeros(scales.size, np.uint16), R, C, x1)
    assert np.array_equal(y1, yz)


def test_mlx4_offset_mistake_is_caught():
    # A planted mistake: the q - 8 offset of a stale comment in the reference
    # header (include/ds4f/kernels.h:111) instead of the code's raw q
    # (src/kernels.c:127-130).  The dense check above must reject it.
    R, C = 8, 200
    vals, scales, biases = W.mlx4_matrix(R, C, 3, R)
    x = W.mlx4_x(C, 3, R)
    y = O.mlx4_matvec(vals, scales, biases, R, C, x)
    wrong = _mlx4_dense(vals, scales, biases, R, C, offset=8) @ x.astype(np.float64)
    assert not np.all(np.abs(y - wrong) <= 1e-3 * (1 + np.abs(wrong)))


# ---- whole layer steps (gqa_step :87-225, linear_step :837-968) ----------

def _gqa_step_case(n_past=23, layer=3, scale=3.0):
    g = W.GqaGeom()
    w = W.gqa_layer_weights(g, 2048, 0, layer)
    kc, vc = W.gqa_cache(g, n_past, layer=layer)
    kv = np.zeros((64, 2 * g.kv_heads * g.head_dim), np.float32)
    half = g.kv_heads * g.head_dim
    kv[:n_past, :half] = kc.reshape(n_past, -1)
    kv[:n_past, half:] = vc.reshape(n_past, -1)
    # rms 3: the input norm changes the projections' input by 3x, so feeding
    # them the raw state is an O(1) mistake
    state = (scale * W.hidden_state(2048, 0, layer)).astype(np.float32)
    return g, w, kc, vc, kv, state


def test_gqa_step_matches_f64_block():
    g, w, kc, vc, kv, state = _gqa_step_case()
    n_past = kc.shape[0]
    new = O.gqa_step(kv, n_past, state, w, g.heads, g.kv_heads, g.head_dim)
    ref, kn, v = F.gqa_block(kc, vc, state, w, n_past, g.heads, g.kv_heads, g.head_dim)
    tol = 2e-5 * (1.0 + np.abs(ref))
    assert np.all(np.abs(new - ref) <= tol)
    half = g.kv_heads * g.head_dim
    assert np.allclose(kv[n_past, :half], kn.reshape(-1), rtol=1e-5, atol=1e-5)
    assert np.allclose(kv[n_past, half:], v.reshape(-1), rtol=1e-5, atol=1e-5)
    # planted wiring mistakes the comparison must reject: the residual added
    # to the normed copy, and the projections fed the raw state
    xin = F.rmsnorm(state, F.bf(w.in_norm))
    wrong1 = ref - state + xin
    assert np.abs(new - wrong1).max() > 100 * tol.max()
    xr = np.asarray(state, np.float64)
    qg = (F.mlx4_dense(w.q) @ xr).reshape(g.heads, -1)
    k = (F.mlx4_dense(w.k) @ xr).reshape(g.kv_heads, -1)
    vv = (F.mlx4_dense(w.v) @ xr).reshape(g.kv_heads, -1)
    out, _ = F.gqa_step(kc, vc, qg, k, vv, w.qn, w.kn, n_past)
    wrong2 = state + F.mlx4_dense(w.o) @ out.reshape(-1)
    assert np.abs(new - wrong2).max() > 100 * tol.max()


def test_gqa_step_silent_skip_and_no_norm():
    g, w, kc, vc, kv, state = _gqa_step_case(n_past=5)
    before = kv.copy()
    out = O.gqa_step(kv, 64, state, w, g.heads, g.kv_heads, g.head_dim)   # token = max_tokens
    assert np.array_equal(out, state) and np.array_equal(kv, before)
    # without an input norm weight the projections read the state itself
    w0 = W.GqaLayerW(None, w.q, w.k, w.v, w.o, w.qn, w.kn)
    new = O.gqa_step(kv, 5, state, w0, g.heads, g.kv_heads, g.head_dim)
    xr = np.asarray(state, np.float64)
    qg = (F.mlx4_dense(w.q) @ xr).reshape(g.heads, -1)
    k = (F.mlx4_dense(w.k) @ xr).reshape(g.kv_heads, -1)
    v = (F.mlx4_dense(w.v) @ xr).reshape(g.kv_heads, -1)
    out, _ = F.gqa_step(kc, vc, qg, k, v, w.qn, w.kn, 5)
    ref = xr + F.mlx4_dense(w.o) @ out.reshape(-1)
    assert np.all(np.abs(new - ref) <= 2e-5 * (1.0 + np.abs(ref)))


def test_lin_step_matches_f64_block():
    lg = W.LinGeom()
    layer, token = 1, 5
    w = W.lin_layer_weights(lg, 2048, 0, layer)
    hist = W.lin_conv_history(lg, layer=layer)
    ring = W.ring_from_history(lg, hist, token)
    S0 = W.lin_state(lg, layer=layer).astype(np.float32)
    S = S0.copy()
    state = (3.0 * W.hidden_state(2048, 0, 40 + layer)).astype(np.float32)
    new = O.lin_step(ring, S, token, state, w, lg.k_heads, lg.v_heads, lg.kd, lg.vd)
    ref, Sn, qkv = F.lin_block(hist, S0, state, w, lg.k_heads, lg.v_heads, lg.kd, lg.vd)
    tol = 2e-5 * (1.0 + np.abs(ref))
    assert np.all(np.abs(new - ref) <= tol)
    assert np.abs(S - Sn).max() <= 1e-5 * np.abs(Sn).max()
    assert np.allclose(ring[token % 4], qkv, rtol=1e-5, atol=1e-5)    # raw row into the ring
    xin = F.rmsnorm(state, F.bf(w.in_norm))
    assert np.abs(new - (ref - state + xin)).max() > 100 * tol.max()
    # the silent skip of :882 leaves everything untouched
    ring2, S2 = ring.copy(), S.copy()
    out = O.lin_step(ring2, S2, 70, state, w, lg.k_heads, lg.v_heads, lg.kd, lg.vd, max_tokens=64)
    assert np.array_equal(out, state) and np.array_equal(ring2, ring) and np.array_equal(S2, S)


def test_chunks_equal_serial_layer_steps():
    # ds4f_attn_*_chunk (:1145-1252, :977-1135) equals the per-token layer
    # steps in order: the chunk restatement is pinned to the pinned steps
    g, w, kc, vc, kv, _ = _gqa_step_case(n_past=9)
    states = np.stack([W.hidden_state(2048, 0, 500 + b) for b in range(5)])
    kv2 = kv.copy()
    got = O.gqa_chunk(kv, 9, states, w, g.heads, g.kv_heads, g.head_dim)
    for b in range(5):
        ref = O.gqa_step(kv2, 9 + b, states[b], w, g.heads, g.kv_heads, g.head_dim)
        assert np.array_equal(got[b], ref)
    assert np.array_equal(kv, kv2)
    lg = W.LinGeom()
    wl = W.lin_layer_weights(lg, 2048, 0, 2)
    ring = W.ring_from_history(lg, W.lin_conv_history(lg, layer=2), 6)
    S = W.lin_state(lg, layer=2).astype(np.float32)
    ring2, S2 = ring.copy(), S.copy()
    got = O.lin_chunk(ring, S, 6, states, wl, lg.k_heads, lg.v_heads, lg.kd, lg.vd)
    for b in range(5):
        ref = O.lin_step(ring2, S2, 6 + b, states[b], wl, lg.k_heads, lg.v_heads, lg.kd, lg.vd)
        assert np.array_equal(got[b], ref)
    assert np.array_equal(S, S2) and np.array_equal(ring, ring2)
