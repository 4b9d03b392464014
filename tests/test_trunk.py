"""The packed trunk (no GPU): the on-disk layout of tools/build-trunk-mlx.py
and the role resolution of ds4f_trunk_layout_load (src/moe.c:372-373,
:425-490) done by the plugin's ds4f_gpu_trunk_roles.

A synthetic 4-layer trunk (three delta-rule layers and a GQA layer with the
checkpoint's tensor names, plus tensors of the layers' other parts) is
written, read back, and resolved: every payload round-trips byte for byte,
the tensors of a layer are sorted by name at 8-byte aligned offsets, the
kinds follow the reference's dispatch, and each role points at the tensor
of that name.
"""
import ctypes

import numpy as np

from ds4f_hip import lib as L
from ds4f_hip import trunk as T
from ds4f_hip import workloads as W

GQ, LG = W.GqaGeom(), W.LinGeom()
HID = 256       # a small hidden size keeps the synthetic weights small


def _small_layers():
    gq = W.GqaGeom(heads=2, kv_heads=1, head_dim=256)
    lg = W.LinGeom(k_heads=2, v_heads=4, kd=128, vd=128)
    ws = {L_: W.lin_layer_weights(lg, HID, 0, L_) for L_ in range(3)}
    ws[3] = W.gqa_layer_weights(gq, HID, 0, 3)
    return ws


def test_trunk_roundtrip_and_roles(tmp_path):
    ws = _small_layers()
    ent = {L_: T.layer_entries(L_, w) for L_, w in ws.items()}
    T.write_trunk(str(tmp_path), ent)
    got = T.read_trunk(str(tmp_path))
    lib = L.load()
    assert sorted(got) == [0, 1, 2, 3]
    for L_, (tens, payload) in got.items():
        names = [t.name.decode() for t in tens]
        assert names == sorted(names)                       # sorted by name
        src = {e[0]: e for e in ent[L_]}
        for t in tens:
            assert t.off % 8 == 0                          # 8-byte aligned
            name, dt, shape, arr = src[t.name.decode()]
            assert T.DTYPE_CODE[dt] == t.dtype and list(t.dims[:t.rank]) == list(shape)
            raw = np.ascontiguousarray(arr).tobytes()
            assert t.nbytes == len(raw)
            assert payload[t.off:t.off + t.nbytes].tobytes() == raw
        roles = T.TrunkRoles()
        kind = lib.ds4f_gpu_trunk_roles(ctypes.cast(tens, ctypes.c_void_p), len(tens),
                                        ctypes.byref(roles))
        assert kind == (2 if L_ == 3 else 1)

        def nm(i):
            return names[i] if i >= 0 else None
        assert nm(roles.in_norm).endswith(".input_layernorm.weight")
        if kind == 2:
            for r, n in ((roles.q, "q_proj"), (roles.k, "k_proj"), (roles.v, "v_proj"),
                         (roles.o, "o_proj")):
                assert [nm(i).rsplit(".", 2)[-2:] for i in r] == [[n, "weight"], [n, "scales"],
                                                                   [n, "biases"]]
            assert nm(roles.q_norm).endswith("q_norm.weight")
            assert nm(roles.k_norm).endswith("k_norm.weight")
            assert roles.conv == -1 and roles.qkv[0] == -1
        else:
            for r, n in ((roles.qkv, "in_proj_qkv"), (roles.z, "in_proj_z"), (roles.a, "in_proj_a"),
                         (roles.b, "in_proj_b"), (roles.out, "out_proj")):
                assert [nm(i).rsplit(".", 2)[-2:] for i in r] == [[n, "weight"], [n, "scales"],
                                                                   [n, "biases"]]
            assert nm(roles.conv).endswith("conv1d.weight")
            assert nm(roles.A_log).endswith("A_log") and nm(roles.dt_bias).endswith("dt_bias")
            assert nm(roles.norm).endswith("linear_attn.norm.weight")
            assert roles.q[0] == -1


def test_roles_dispatch_and_first_match():
    """A list without attention roles is kind NONE; the first of two tensors
    with the same role wins (src/moe.c:426, `if (... < 0)`)."""
    lib = L.load()
    tens = (T.TrunkTensor * 3)()
    for i, n in enumerate(["model.layers.0.mlp.gate.weight",
                           "model.layers.0.linear_attn.conv1d.weight",
                           "x.linear_attn.conv1d.weight"]):
        tens[i].name = n.encode()
    roles = T.TrunkRoles()
    assert lib.ds4f_gpu_trunk_roles(ctypes.cast(tens, ctypes.c_void_p), 1, ctypes.byref(roles)) == 0
    assert lib.ds4f_gpu_trunk_roles(ctypes.cast(tens, ctypes.c_void_p), 3, ctypes.byref(roles)) == 1
    assert roles.conv == 1


def test_input_norm_names():
    """The input norm is found under either name the reference maps to
    attn_norm (src/moe.c:371-373), the first tensor in list order winning;
    a linear layer's own norm (linear_attn.norm.weight) is not taken for it."""
    lib = L.load()
    for names, want in ((["model.layers.0.attn_norm.weight",
                          "model.layers.0.linear_attn.conv1d.weight"], 0),
                        (["model.layers.0.input_layernorm.weight",
                          "model.layers.0.linear_attn.conv1d.weight"], 0),
                        (["model.layers.0.linear_attn.norm.weight",
                          "model.layers.0.attn_norm.weight",
                          "model.layers.0.input_layernorm.weight",
                          "model.layers.0.linear_attn.conv1d.weight"], 1),
                        (["model.layers.0.linear_attn.norm.weight",
                          "model.layers.0.post_attention_layernorm.weight",
                          "model.layers.0.linear_attn.conv1d.weight"], -1)):
        tens = (T.TrunkTensor * len(names))()
        for i, n in enumerate(names):
            tens[i].name = n.encode()
        roles = T.TrunkRoles()
        assert lib.ds4f_gpu_trunk_roles(ctypes.cast(tens, ctypes.c_void_p), len(names),
                                        ctypes.byref(roles)) == 1
        assert roles.in_norm == want, names
