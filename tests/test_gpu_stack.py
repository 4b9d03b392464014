"""GPU parity of the whole attention stack decode: 40 layers (GQA at
layer % 4 == 3, the gated delta rule elsewhere) at 32768 cached positions
for 256 consecutive steps (the full decode run of the stack workload) and
at 131072 for three, each step one HIP graph of the 40 layer launches --
the sequence bench.py times (ds4f_hip.stack.StackDecode), in the engine's
order (src/main.c:924-957 calling ds4f_attn_qwen_step per layer,
src/attn_qwen.c:1255-1264).

Every layer's output of every step is checked against the oracle's
gqa_body / lin_body (src/attn_qwen.c:235-397, :434-764) run on the same
state and the same activations (copied back from the device), each layer's
steps in order; afterwards the device's delta-rule states, conv rings and
the GQA cache rows the steps wrote are checked against the oracle's.  The
GQA layers attend over the whole cache (no window, :346-386).  A layer's
steps depend only on its own state and activations, so the oracle runs
the layers side by side on host threads (ctypes releases the GIL), each
layer's steps in order.

Tolerances: max |gpu - oracle| <= 2e-3 and relative RMS <= 1e-4 on every
layer's output (the relative RMS is the telling one for the GQA outputs,
which average tens of thousands of value rows); delta state
relative error (Frobenius, per layer) <= 1e-4; conv rings bit-exact; the
device's cache rows are the bf16 rounding of the oracle's fp32 rows.  The
device keeps bf16 cache rows, so the oracle's new rows are rounded to bf16
after each step, as the device stores them.
"""
import sys
import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import oracle as O
from ds4f_hip import synth as S
from ds4f_hip import workloads as W

pytestmark = pytest.mark.gpu

ATOL = 2e-3
RRMS = 1e-4
STATE_RTOL = 1e-4
STEPS = {32768: 256, 131072: 3}


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _err(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    mx = float(np.abs(got - ref).max()) if got.size else 0.0
    rr = float(np.sqrt(((got - ref) ** 2).sum() / max((ref ** 2).sum(), 1e-300)))
    return mx, rr


@pytest.mark.parametrize("ctx", [32768, 131072])
def test_stack_decode_graph_steps_match_oracle(ctx):
    import torch

    from ds4f_hip.stack import StackDecode

    steps = STEPS[ctx]
    t_start = time.time()
    _say(f"stack decode: 40 layers, ctx {ctx}, {steps} graph steps")
    sd = StackDecode(ctx, steps, seed=0, host_cache=True)
    cache, kinds, gq, lg = sd.cache, sd.kinds, sd.gq, sd.lg
    sd.ga.sync(-1, to_host=True, n_kv_tokens=ctx)       # the oracle's starting state
    _say(f"  state synced to the host ({time.time() - t_start:.1f} s)")

    # the activations exactly as the device holds them
    acts = []
    for d in sd.layers:
        if d["kind"] == 2:
            acts.append({k: d[k].cpu().numpy() for k in ("q", "k", "v", "qn", "kn")})
        else:
            acts.append({k: d[k].cpu().numpy() for k in ("qkv", "z", "a", "b", "cw", "al", "dt",
                                                          "nw")})

    graphs = sd.capture(range(steps))
    torch.cuda.synchronize()
    for s in range(steps):
        graphs[s].replay()
        # eager work and a synchronisation between the replays
        torch.zeros(1024, device="cuda").add_(1.0)
        torch.cuda.synchronize()
    outs = [d["out"].cpu().numpy() for d in sd.layers]
    del graphs
    _say(f"  {steps} steps replayed ({time.time() - t_start:.1f} s)")

    def oracle_layer(Lr):
        """Layer Lr's steps in order; returns (layer, worst max abs, worst
        rel-rms, the step of the worst max abs)."""
        a = acts[Lr]
        w_mx, w_rr, w_s = 0.0, 0.0, -1
        for s in range(steps):
            pos = ctx + s
            if kinds[Lr] == 2:
                ref, _ = O.gqa_body(cache.kv[Lr], pos, a["q"][s], a["k"][s], a["v"][s],
                                    a["qn"].view(np.uint16), a["kn"].view(np.uint16), gq.heads,
                                    gq.kv_heads, gq.head_dim)
                cache.kv[Lr, pos] = S.bf16_round(cache.kv[Lr, pos])   # the device's row format
            else:
                ref, _ = O.lin_body(cache.conv[Lr], cache.lin[Lr], pos, a["qkv"][s], a["z"][s],
                                    a["a"][s], a["b"][s], a["cw"].view(np.uint16), a["al"],
                                    a["dt"].view(np.uint16), a["nw"].view(np.uint16), lg.k_heads,
                                    lg.v_heads, lg.kd, lg.vd)
            mx, rr = _err(outs[Lr][s], ref)
            # the GQA outputs average ~ctx value rows (|out| ~ 1e-2), so the
            # relative RMS is checked beside the absolute bar
            assert mx <= ATOL and rr <= RRMS, \
                f"step {s} layer {Lr}: max abs {mx:.3e} rel-rms {rr:.3e}"
            if mx > w_mx:
                w_mx, w_s = mx, s
            w_rr = max(w_rr, rr)
        return Lr, w_mx, w_rr, w_s

    worst = {1: 0.0, 2: 0.0}
    worst_rr = {1: 0.0, 2: 0.0}
    # the GQA layers (the long ones) first; 12 host threads at most
    order = sorted(range(len(kinds)), key=lambda L: kinds[L] != 2)
    with ThreadPoolExecutor(max_workers=12) as pool:
        for Lr, mx, rr, ws in pool.map(oracle_layer, order):
            worst[kinds[Lr]] = max(worst[kinds[Lr]], mx)
            worst_rr[kinds[Lr]] = max(worst_rr[kinds[Lr]], rr)
            _say(f"  layer {Lr} ({'GQA' if kinds[Lr] == 2 else 'delta'}): {steps} steps, worst "
                 f"max abs {mx:.3e} (step {ws}), worst rel-rms {rr:.3e} "
                 f"({time.time() - t_start:.1f} s)")

    # the oracle's state after the steps, then the device's
    ref_lin = cache.lin.copy()
    ref_conv = cache.conv.copy()
    ref_rows = {Lr: cache.kv[Lr, ctx:ctx + steps].copy() for Lr in range(len(kinds))
                if kinds[Lr] == 2}
    sd.ga.sync(-1, to_host=True, n_kv_tokens=ctx + steps)
    worst_state = 0.0
    for Lr, kd in enumerate(kinds):
        if kd == 2:
            assert np.array_equal(cache.kv[Lr, ctx:ctx + steps], ref_rows[Lr]), f"layer {Lr} rows"
        else:
            srr = _err(cache.lin[Lr], ref_lin[Lr])[1]
            worst_state = max(worst_state, srr)
            assert srr <= STATE_RTOL, f"layer {Lr}: state rel {srr:.3e}"
            assert np.array_equal(cache.conv[Lr], ref_conv[Lr]), f"layer {Lr} conv ring"
    _say(f"  ctx {ctx}, {steps} steps: worst output err GQA {worst[2]:.3e} (rel-rms "
         f"{worst_rr[2]:.3e}) delta {worst[1]:.3e} (rel-rms {worst_rr[1]:.3e}); worst state "
         f"rel {worst_state:.3e}; {time.time() - t_start:.1f} s")
    sd.close()


def test_stack_start_state_regenerates():
    """bench.py hands the CPU baseline the stack's starting state after the
    timed steps, regenerated in place (StackDecode.synth_state): that state
    must equal the one the steps started from -- the GQA cache rows below
    ctx, the delta-rule states and the conv ring slots of positions
    ctx - 3 .. ctx - 1, bit for bit.  (The fourth slot is the one the step
    at ctx writes before anything reads it, src/attn_qwen.c:480-500.)"""
    import torch

    from ds4f_hip.stack import StackDecode

    ctx, steps = 4096, 3
    sd = StackDecode(ctx, steps, seed=0, host_cache=True)
    cache, kinds = sd.cache, sd.kinds
    sd.ga.sync(-1, to_host=True, n_kv_tokens=ctx)
    kv0 = {Lr: cache.kv[Lr, :ctx].copy() for Lr in range(len(kinds)) if kinds[Lr] == 2}
    lin0, conv0 = cache.lin.copy(), cache.conv.copy()
    graphs = sd.capture(range(steps))
    for g in graphs:
        g.replay()
    torch.cuda.synchronize()
    del graphs
    sd.ga.sync(-1, to_host=True, n_kv_tokens=ctx)
    moved = any(not np.array_equal(cache.lin[Lr], lin0[Lr]) for Lr in range(len(kinds))
                if kinds[Lr] != 2)
    assert moved, "the steps did not advance the delta-rule states"
    sd.synth_state()
    sd.ga.sync(-1, to_host=True, n_kv_tokens=ctx)
    for Lr, kd in enumerate(kinds):
        if kd == 2:
            assert np.array_equal(cache.kv[Lr, :ctx], kv0[Lr]), f"layer {Lr} cache rows"
        else:
            assert np.array_equal(cache.lin[Lr], lin0[Lr]), f"layer {Lr} state"
            taps = [(ctx - j) % 4 for j in (3, 2, 1)]
            assert np.array_equal(cache.conv[Lr][taps], conv0[Lr][taps]), f"layer {Lr} conv ring"
    sd.close()
