"""ctypes binding of the HIP attention plugin (libds4f_attn_hip.so).

The signatures mirror include/ds4f_gpu_attn.h one to one.  Loading fails
loudly when the library has not been built: there is no CPU fallback in
this package -- the CPU path belongs to the engine (and, for checking, to
the oracle under oracle/).
"""
from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
# DS4F_HIP_LIB names another build of the plugin to load (comparing builds)
LIB_PATH = os.environ.get("DS4F_HIP_LIB") or os.path.join(HERE, "libds4f_attn_hip.so")
HEADER = os.path.join(os.path.dirname(os.path.dirname(HERE)), "include", "ds4f_gpu_attn.h")

LAYER_NONE, LAYER_LINEAR, LAYER_GQA = 0, 1, 2
SYNC_TO_HOST, SYNC_TO_DEVICE = 0, 1


class Geom(ctypes.Structure):
    """Ds4fGpuAttnGeom."""
    _fields_ = [(n, ctypes.c_int) for n in
                ("n_layers", "max_tokens", "n_heads", "n_kv_heads", "head_dim", "lin_kd",
                 "lin_vd")]


class Mlx4W(ctypes.Structure):
    """Ds4fGpuMlx4W."""
    _fields_ = [("vals", ctypes.c_void_p), ("scales", ctypes.c_void_p),
                ("biases", ctypes.c_void_p), ("rows", ctypes.c_int), ("cols", ctypes.c_int)]


class LayerW(ctypes.Structure):
    """Ds4fGpuLayerW."""
    _fields_ = ([("in_norm", ctypes.c_void_p)] +
                [(n, Mlx4W) for n in ("q", "k", "v", "o")] +
                [("q_norm", ctypes.c_void_p), ("k_norm", ctypes.c_void_p)] +
                [(n, Mlx4W) for n in ("qkv", "z", "a", "b", "out")] +
                [(n, ctypes.c_void_p) for n in ("conv_w", "dt_bias", "norm_w", "A_log")])


_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_d = ctypes.c_double

_SIGS = {
    "ds4f_gpu_init": ([], _i),
    "ds4f_gpu_free": ([], None),
    "ds4f_gpu_attn_bind": ([ctypes.POINTER(Geom), _vp, _vp, _vp, _vp, _i], _i),
    "ds4f_gpu_attn_unbind": ([], _i),
    "ds4f_gpu_attn_sync": ([_i, _i, _i], _i),
    "ds4f_gpu_gqa_decode": ([_i, _i, _vp, _vp, _vp, _vp, _vp, _vp], _i),
    "ds4f_gpu_lin_decode": ([_i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp], _i),
    "ds4f_gpu_gqa_prefill": ([_i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp], _i),
    "ds4f_gpu_lin_prefill": ([_i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp], _i),
    "ds4f_hip_gqa_decode_async": ([_i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp], _i),
    "ds4f_hip_gqa_prefill_async": ([_i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp], _i),
    "ds4f_hip_lin_prefill_async": ([_i, _i, _i] + [_vp] * 11, _i),
    "ds4f_hip_lin_prefill_noalloc": ([_i, _i, _i] + [_vp] * 11, _i),
    "ds4f_hip_lin_decode_async": ([_i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                   _vp], _i),
    "ds4f_hip_synth": ([_vp, _i64, _i, _i, _d, _d, _u64, _u64, _vp], _i),
    "ds4f_hip_launch_floor": ([_i, _i, _i, _vp], _i),
    "ds4f_hip_synth_gqa_cache": ([_i, _i, _u64, _u64, _u64, _vp], _i),
    "ds4f_hip_synth_lin_state": ([_i, _d, _u64, _u64, _vp], _i),
    "ds4f_hip_synth_conv_history": ([_i, _i, _u64, _u64, _vp], _i),
    "ds4f_gpu_last_error": ([], ctypes.c_char_p),
    "ds4f_hip_f16_status": ([_vp, _i], _i),
    "ds4f_gpu_attn_weights": ([_i, ctypes.POINTER(LayerW)], _i),
    "ds4f_gpu_attn_step": ([_i, _i, _vp], _i),
    "ds4f_hip_attn_step_async": ([_i, _i, _vp, _vp], _i),
    "ds4f_gpu_attn_chunk": ([_i, _i, _i, ctypes.POINTER(ctypes.c_void_p)], _i),
    "ds4f_hip_attn_chunk_async": ([_i, _i, _i, _vp, _vp], _i),
    "ds4f_gpu_mlx4_matvec": ([_vp, _vp, _vp, _i, _i, _vp, _vp], _i),
    "ds4f_gpu_mlx4_batch": ([_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i], _i),
    "ds4f_hip_mlx4_matvec_async": ([_vp, _vp, _vp, _i, _i, _vp, _vp, _vp], _i),
    "ds4f_gpu_trunk_roles": ([_vp, _i, _vp], _i),
    "ds4f_gpu_attn_weights_trunk": ([_i, _vp, _i, _vp], _i),
}

_lib = None


def header_functions(path: str = HEADER) -> list[str]:
    """Names of the functions include/ds4f_gpu_attn.h declares."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ds4f_\w+)\s*\(", text)))


def load():
    """Load the plugin, attaching the header's signatures."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"HIP attention plugin not built: {LIB_PATH} is missing "
                               "(run __graft_entry__.build())")
        # torch's wheel ships its own HIP runtime under the same soname
        # (libamdhip64.so.7).  Importing torch first makes the plugin bind to
        # that copy, so the process holds ONE runtime and torch tensors,
        # streams and the plugin's kernels share it; loading the plugin first
        # would pull in /opt/rocm's copy beside torch's and the second
        # runtime to initialise finds no devices.
        import torch  # noqa: F401
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGS.items():
            if os.environ.get("DS4F_HIP_LIB") and not hasattr(L, name):
                continue          # another build, without this entry
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def last_error() -> str:
    e = load().ds4f_gpu_last_error()
    return e.decode() if e else ""


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed: {last_error()}")
