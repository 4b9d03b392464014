"""GPU parity of the MLX 4-bit matvecs (ds4f_gpu_mlx4_matvec / _batch and
the device-resident async form) against the oracle's restatement of
ds4f_mlx4_matvec (src/kernels.c:196-219).

Tolerance: the GPU sums in a different order (gpu.h:13-18), so each output
is held to the fp32 accumulation bound |y - y_oracle| <= 1e-5 * sum_c
|w_rc x_c| (+1e-30), and to the reference's own matvec bound
1e-3 * (1 + |y|) (tests/test_kernels.c:435).
"""
import ctypes
import sys

import numpy as np
import pytest

import oracle as O
from ds4f_hip import workloads as W

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _lib():
    from ds4f_hip.lib import load
    lib = load()
    assert lib.ds4f_gpu_init() == 0
    return lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _absdot(vals, scales, biases, R, C, x):
    """sum_c |w_rc x_c| in float64 (the accumulation bound's scale)."""
    k = np.arange(R * C)
    q = ((vals[k >> 3] >> (4 * (k & 7)).astype(np.uint32)) & 0xF).astype(np.float64)
    g = k // 64
    s = (scales[g].astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    b = 0.0 if biases is None else (biases[g].astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return (np.abs(q * s + b).reshape(R, C)) @ np.abs(x.astype(np.float64))


def _check(y, ref, scale, what):
    d = np.abs(y.astype(np.float64) - ref)
    _say(f"{what}: max |d| {d.max():.3e}, max |d|/bound {(d / (1e-5 * scale + 1e-30)).max():.3f}")
    assert np.all(d <= 1e-5 * scale + 1e-30)
    assert np.all(d <= 1e-3 * (1 + np.abs(ref)))


@pytest.mark.parametrize("R,C,bias", [(3, 64, True), (5, 96, True), (16, 2048, True),
                                      (16, 2048, False), (7, 4096, True), (33, 8192, True),
                                      (2049, 512, False), (1, 32, True)])
def test_mlx4_matvec_matches_oracle(R, C, bias):
    lib = _lib()
    vals, scales, biases = W.mlx4_matrix(R, C, 11, R, bias)
    x = W.mlx4_x(C, 11, R)
    y = np.full(R, np.nan, np.float32)
    assert lib.ds4f_gpu_mlx4_matvec(_p(vals), _p(scales), _p(biases), R, C, _p(x), _p(y)) == 0
    ref = O.mlx4_matvec(vals, scales, biases, R, C, x).astype(np.float64)
    _check(y, ref, _absdot(vals, scales, biases, R, C, x), f"mlx4 {R}x{C} bias={bias}")


def test_mlx4_output_head_shape():
    # the engine's largest matvec: the 248320 x 2048 output head (gpu.h:11-14)
    lib = _lib()
    R, C = 248320, 2048
    rng = np.random.default_rng(7)
    q = rng.integers(0, 16, R * C, dtype=np.uint8)
    vals = W.mlx4_pack(q)
    del q
    ng = R * C // 64
    sc = rng.uniform(0.002, 0.02, ng).astype(np.float32)
    scales = (sc.view(np.uint32) >> 16).astype(np.uint16)
    biases = ((-sc * rng.uniform(6, 9, ng).astype(np.float32)).view(np.uint32) >> 16).astype(np.uint16)
    x = rng.standard_normal(C).astype(np.float32)
    y = np.empty(R, np.float32)
    assert lib.ds4f_gpu_mlx4_matvec(_p(vals), _p(scales), _p(biases), R, C, _p(x), _p(y)) == 0
    ref = O.mlx4_matvec(vals, scales, biases, R, C, x).astype(np.float64)
    # second call: x changes, the cached weight is reused
    x2 = rng.standard_normal(C).astype(np.float32)
    y2 = np.empty(R, np.float32)
    assert lib.ds4f_gpu_mlx4_matvec(_p(vals), _p(scales), _p(biases), R, C, _p(x2), _p(y2)) == 0
    ref2 = O.mlx4_matvec(vals, scales, biases, R, C, x2).astype(np.float64)
    rows = np.arange(0, R, 97)        # the bound's scale on a row sample
    d = np.abs(y.astype(np.float64) - ref)
    d2 = np.abs(y2.astype(np.float64) - ref2)
    _say(f"mlx4 head {R}x{C}: max |d| {d.max():.3e} / {d2.max():.3e}, max |y| {np.abs(ref).max():.3f}")
    assert np.all(d <= 1e-3 * (1 + np.abs(ref))) and np.all(d2 <= 1e-3 * (1 + np.abs(ref2)))
    k = (rows[:, None] * C + np.arange(C)[None, :]).reshape(-1)
    qq = ((vals[k >> 3] >> (4 * (k & 7)).astype(np.uint32)) & 0xF).astype(np.float64)
    g = k // 64
    w = qq * (scales[g].astype(np.uint32) << 16).view(np.float32) + (biases[g].astype(np.uint32) << 16).view(np.float32)
    scale = np.abs(w.reshape(len(rows), C)) @ np.abs(x.astype(np.float64))
    assert np.all(d[rows] <= 1e-5 * scale)


def test_mlx4_unsupported_shape_returns_minus_one():
    # C = 200 (the reference's own test shape) is not a multiple of 32: the
    # call declines and leaves y alone, so the caller's CPU matvec runs.
    lib = _lib()
    R, C = 8, 200
    vals, scales, biases = W.mlx4_matrix(R, C, 1, 0)
    x = W.mlx4_x(C, 1, 0)
    y = np.full(R, 123.0, np.float32)
    assert lib.ds4f_gpu_mlx4_matvec(_p(vals), _p(scales), _p(biases), R, C, _p(x), _p(y)) == -1
    assert np.all(y == 123.0)


def test_mlx4_matvec_replaces_cached_weight():
    # a new weight at a new pointer (same shape) must not reuse the old copy
    lib = _lib()
    R, C = 64, 1024
    a = W.mlx4_matrix(R, C, 21, 0)
    b = W.mlx4_matrix(R, C, 22, 0)
    x = W.mlx4_x(C, 21, 0)
    for m in (a, b, a):
        y = np.empty(R, np.float32)
        assert lib.ds4f_gpu_mlx4_matvec(_p(m[0]), _p(m[1]), _p(m[2]), R, C, _p(x), _p(y)) == 0
        ref = O.mlx4_matvec(m[0], m[1], m[2], R, C, x).astype(np.float64)
        _check(y, ref, _absdot(m[0], m[1], m[2], R, C, x), "mlx4 cache switch")


def test_mlx4_batch_matches_oracle():
    lib = _lib()
    R, C, nexp = 512, 2048, 6
    mats = [W.mlx4_matrix(R, C, 31, e) for e in range(nexp)]
    ids = [ctypes.c_void_p(0x1000 + e) for e in range(nexp)]
    for call, order in enumerate(([0, 1, 2, 3], [2, 4, 0, 5, 1], [5])):
        n = len(order)
        xs = [W.mlx4_x(C, 31, e, call) for e in order]
        ys = [np.empty(R, np.float32) for _ in order]
        arr = lambda seq: (ctypes.c_void_p * n)(*[_p(a) for a in seq])
        vals = arr([mats[e][0] for e in order])
        scs = arr([mats[e][1] for e in order])
        bis = arr([mats[e][2] for e in order])
        idp = (ctypes.c_void_p * n)(*[ids[e] for e in order])
        assert lib.ds4f_gpu_mlx4_batch(vals, scs, bis, arr(xs), arr(ys), idp, R, C, n) == 0
        for e, x, y in zip(order, xs, ys):
            v, s, b = mats[e]
            ref = O.mlx4_matvec(v, s, b, R, C, x).astype(np.float64)
            _check(y, ref, _absdot(v, s, b, R, C, x), f"mlx4 batch call {call} expert {e}")


def test_mlx4_async_device_pointers():
    import torch
    from ds4f_hip.attn import dptr
    lib = _lib()
    R, C = 3000, 2048
    vals, scales, biases = W.mlx4_matrix(R, C, 41, 0)
    x = W.mlx4_x(C, 41, 0)
    dv = torch.from_numpy(vals.view(np.int32)).cuda()
    ds = torch.from_numpy(scales.view(np.int16)).cuda()
    db = torch.from_numpy(biases.view(np.int16)).cuda()
    dx = torch.from_numpy(x).cuda()
    dy = torch.full((R,), float("nan"), device="cuda")
    # enqueued on torch's stream, after the copies that filled the inputs
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.ds4f_hip_mlx4_matvec_async(dptr(dv), dptr(ds), dptr(db), R, C, dptr(dx), dptr(dy),
                                          st) == 0
    torch.cuda.synchronize()
    y = dy.cpu().numpy()
    ref = O.mlx4_matvec(vals, scales, biases, R, C, x).astype(np.float64)
    _check(y, ref, _absdot(vals, scales, biases, R, C, x), "mlx4 async")
