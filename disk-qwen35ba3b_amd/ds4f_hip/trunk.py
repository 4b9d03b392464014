"""The engine's packed trunk on disk: trunk.bin, trunk.offsets, trunk.json.

The layout is the one tools/build-trunk-mlx.py:95-160 writes and the engine
reads (src/trunk.c:14-45 for trunk.offsets, ds4f_trunk_layout_load in
src/moe.c:162-300 for trunk.json):

* trunk.bin      the layers' payloads back to back; inside a layer its
                 tensors sorted by name, each at an 8-byte aligned offset;
* trunk.offsets  little-endian u64s: n, then (offset, size) of each layer's
                 payload in trunk.bin;
* trunk.json     {"n_layers": n, "layers": [{"layer": L, "tensors":
                 [{"n", "dtype", "shape", "off", "nbytes"}, ...]}, ...]},
                 "off" relative to the layer's payload.

``write_trunk`` lays synthetic layers out that way (checkpoint tensor names,
MLX 4-bit projections as U32 [rows, cols / 8] words with BF16 scales and
biases); ``read_trunk`` reads a trunk back into per-layer tensor lists in the
engine's Ds4fTrunkTensor layout plus the layer payloads, which is what
``ds4f_gpu_attn_weights_trunk`` takes.
"""
from __future__ import annotations

import ctypes
import json
import os
import struct

import numpy as np

from .workloads import GqaLayerW, LinLayerW, Mlx4W

# dtype codes of the engine's trunk parser (src/moe.c:36-42)
DTYPE_CODE = {"F32": 0, "I8": 1, "F8_E4M3": 2, "BF16": 4, "U32": 5}
PREFIX = "language_model.model.layers"


class TrunkTensor(ctypes.Structure):
    """Ds4fGpuTrunkTensor (= the engine's Ds4fTrunkTensor)."""
    _fields_ = [("name", ctypes.c_char * 96), ("dtype", ctypes.c_int),
                ("dims", ctypes.c_long * 4), ("rank", ctypes.c_int), ("off", ctypes.c_long),
                ("nbytes", ctypes.c_long)]


class TrunkRoles(ctypes.Structure):
    """Ds4fGpuTrunkRoles."""
    _fields_ = ([("in_norm", ctypes.c_int)] +
                [(n, ctypes.c_int * 3) for n in ("q", "k", "v", "o")] +
                [(n, ctypes.c_int) for n in ("q_norm", "k_norm", "conv", "A_log", "dt_bias")] +
                [(n, ctypes.c_int * 3) for n in ("qkv", "z", "a", "b", "out")] +
                [("norm", ctypes.c_int)])


def _mlx4_entries(base: str, m: Mlx4W):
    """The triplet of one MLX 4-bit projection: U32 words [rows, cols/8],
    BF16 scales and biases [rows, cols/64]."""
    g = m.cols // 64
    out = [(base + ".weight", "U32", [m.rows, m.cols // 8], np.ascontiguousarray(m.vals, np.uint32)),
           (base + ".scales", "BF16", [m.rows, g], np.ascontiguousarray(m.scales, np.uint16))]
    if m.biases is not None:
        out.append((base + ".biases", "BF16", [m.rows, g], np.ascontiguousarray(m.biases, np.uint16)))
    return out


def layer_entries(L: int, w: GqaLayerW | LinLayerW, extra: bool = True):
    """Checkpoint-named tensors of one attention layer (and, with extra,
    tensors of the layer's other parts, which the role resolution ignores)."""
    p = f"{PREFIX}.{L}"
    ent = [(f"{p}.input_layernorm.weight", "BF16", [w.in_norm.size],
            np.ascontiguousarray(w.in_norm, np.uint16))]
    if isinstance(w, GqaLayerW):
        for n, m in (("q_proj", w.q), ("k_proj", w.k), ("v_proj", w.v), ("o_proj", w.o)):
            ent += _mlx4_entries(f"{p}.self_attn.{n}", m)
        ent += [(f"{p}.self_attn.q_norm.weight", "BF16", [w.qn.size], np.ascontiguousarray(w.qn, np.uint16)),
                (f"{p}.self_attn.k_norm.weight", "BF16", [w.kn.size], np.ascontiguousarray(w.kn, np.uint16))]
    else:
        c = w.core
        for n, m in (("in_proj_qkv", w.qkv), ("in_proj_z", w.z), ("in_proj_a", w.a),
                     ("in_proj_b", w.b), ("out_proj", w.out)):
            ent += _mlx4_entries(f"{p}.linear_attn.{n}", m)
        rows = c.conv_w.shape[0]
        ent += [(f"{p}.linear_attn.conv1d.weight", "BF16", [rows, 4, 1],
                 np.ascontiguousarray(c.conv_w, np.uint16)),
                (f"{p}.linear_attn.A_log", "F32", [c.A_log.size], np.ascontiguousarray(c.A_log, np.float32)),
                (f"{p}.linear_attn.dt_bias", "BF16", [c.dt_bias.size],
                 np.ascontiguousarray(c.dt_bias, np.uint16)),
                (f"{p}.linear_attn.norm.weight", "BF16", [c.norm_w.size],
                 np.ascontiguousarray(c.norm_w, np.uint16))]
    if extra:
        hid = w.in_norm.size
        ent += [(f"{p}.post_attention_layernorm.weight", "BF16", [hid], np.ones(hid, np.uint16)),
                (f"{p}.mlp.gate.weight", "BF16", [8, hid], np.zeros((8, hid), np.uint16))]
    return ent


def write_trunk(out_dir: str, layers: dict) -> None:
    """layers: {L: [(name, dtype, shape, array), ...]}.  Writes trunk.bin,
    trunk.offsets and trunk.json as tools/build-trunk-mlx.py:95-160 does:
    per layer the tensors sorted by name at 8-byte aligned offsets, the
    payloads back to back with 8-byte padding between them."""
    os.makedirs(out_dir, exist_ok=True)
    align = 8
    meta = {"n_layers": len(layers), "layers": []}
    at = 0
    with open(os.path.join(out_dir, "trunk.bin"), "wb") as tb, \
            open(os.path.join(out_dir, "trunk.offsets"), "wb") as to:
        to.write(struct.pack("<Q", len(layers)))
        for L in sorted(layers):
            to.write(struct.pack("<Q", at))
            lay = 0
            tens = []
            for name, dt, shape, arr in sorted(layers[L], key=lambda e: e[0]):
                pad = (-lay) % align
                tb.write(b"\0" * pad)
                lay += pad
                raw = np.ascontiguousarray(arr).tobytes()
                tb.write(raw)
                tens.append({"n": name, "dtype": dt, "shape": list(shape), "off": lay,
                             "nbytes": len(raw)})
                lay += len(raw)
            to.write(struct.pack("<Q", lay))
            meta["layers"].append({"layer": L, "tensors": tens})
            at += lay
            pad = (-at) % align
            tb.write(b"\0" * pad)
            at += pad
    with open(os.path.join(out_dir, "trunk.json"), "w") as f:
        json.dump(meta, f)


def read_trunk(trunk_dir: str):
    """Returns {L: (tensors, payload)}: the layer's tensor list as a ctypes
    array of TrunkTensor (the engine's Ds4fTrunkTensor fields) and its
    payload, the layer's bytes of trunk.bin (uint8 array)."""
    with open(os.path.join(trunk_dir, "trunk.offsets"), "rb") as f:
        raw = f.read()
    n = struct.unpack_from("<Q", raw, 0)[0]
    spans = [struct.unpack_from("<QQ", raw, 8 + 16 * i) for i in range(n)]
    with open(os.path.join(trunk_dir, "trunk.json")) as f:
        meta = json.load(f)
    bin_ = np.memmap(os.path.join(trunk_dir, "trunk.bin"), dtype=np.uint8, mode="r")
    out = {}
    for i, ly in enumerate(meta["layers"]):
        off, nb = spans[i]
        payload = np.array(bin_[off:off + nb])
        tens = (TrunkTensor * len(ly["tensors"]))()
        for j, e in enumerate(ly["tensors"]):
            t = tens[j]
            t.name = e["n"].encode()[:95]
            t.dtype = DTYPE_CODE.get(e["dtype"], 3)
            shp = e["shape"][:4]
            t.rank = len(shp)
            for d, v in enumerate(shp):
                t.dims[d] = int(v)
            t.off = int(e["off"])
            t.nbytes = int(e["nbytes"])
        out[int(ly["layer"])] = (tens, payload)
    return out
