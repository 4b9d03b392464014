#!/usr/bin/env python3
"""Benchmark of the Qwen3.5 hybrid-attention hot path on one MI355X.

Default workload (--workload stack_decode, the path's headline
configuration): 40 layers, full GQA at
layer % 4 == 3 (10 layers: 16 q / 2 kv heads, head_dim 256, bf16 KV cache of
`--ctx` past tokens drawn N(0,1)), gated delta rule elsewhere (30 layers:
16 key / 32 value heads of 128, fp32 state N(0, 0.05), conv ring with 3 past
rows).  Attention cores only: the post-projection activations of every
(layer, step) are synthetic N(0,1) tensors, generated on the device before
the timed region.  One step = one token through all 40 layers at position
ctx + s; every step is one HIP graph of the 40 layer launches.

Prints one JSON line: tokens/s (value), the whole stack's algorithmic HBM
rate, the roofline of the dominant kernel (the GQA decode: split-K kernel
plus merge kernel, its 10 x K launches of the same steps replayed as one
HIP graph between two hipEvents) and the CPU baseline (the C oracle on the
host, one thread, on a bounded sample of the same steps).

Other workloads (one JSON line each, same fields):
  gqa_prefill   causal GQA prefill of --tokens (4096) tokens, one layer,
                bf16-valued q|gate/k/v N(0,1); MFMA roofline.
  gqa_decode    one GQA decode call at n_past = --npast (4096), rotated over
                --rotate (128) bound layers so the KV read (1.08 GB in all)
                comes from HBM, not the 256 MB MALL; HBM roofline.
  lin_decode    one delta-rule decode call, rotated over --rotate (256)
                bound layers (0.5 GB of state); HBM roofline.
  hbm_copy      an elementwise copy (dst = src * 1) of a 1 GiB fp32 buffer:
                the measured HBM ceiling, and the known-size kernel that
                scales the FETCH_SIZE / WRITE_SIZE counters of the traffic
                profiles.
  lin_prefill   gated delta-rule prefill of --tokens (4096) tokens, one
                layer, zero state and conv ring, fp32 qkv/z/a/b N(0,1);
                chunked form on fp32 MFMA, roofline against the dense
                bf16 / fp16 MFMA peak (the prefill bar's basis), the fp32
                MFMA peak's fraction beside it.
  launch_floor  an empty kernel launched 200 times in one HIP graph: the
                fixed cost of a kernel boundary.
  mlx4_head     the MLX 4-bit affine matvec of the output head (248320 x
                2048, 287 MB of nibbles, scales and biases: more than the
                256 MB MALL, so the weight streams from HBM every call),
                device-resident; HBM roofline.
  block_decode  the same 40-layer stack at --ctx, whole attention layers on
                the residual stream (input RMSNorm, MLX 4-bit q/k/v or
                qkv/z/a/b projections, the core, the output projection and
                the residual add: ds4f_hip_attn_step_async), 697 MB of
                synthetic 4-bit weights; one HIP graph per step; HBM
                roofline over the whole step's algorithmic bytes.
  block_prefill a prefill of --tokens (4096) tokens from position 0 through
                the same 40 whole layers, one chunk per layer
                (ds4f_hip_attn_chunk_async: 4-bit projections as dequant
                MFMA GEMMs); one HIP graph per pass; MFMA roofline over the
                pass's algorithmic flops.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "disk-qwen35ba3b_amd"))

HBM_PEAK_GBPS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0     # dense bf16 / fp16
MFMA_F32_PEAK_TFLOPS = 157.3  # dense fp32
METRIC = "GQA+delta-rule attn tokens/s and HBM GB/s %peak, decode @32K ctx, 1 GPU"


def gqa_split_bytes(n_past: int) -> int:
    """Algorithmic HBM bytes of one GQA split-K launch: the bf16 K and V rows
    of n_past positions (2 kv heads x 256 x 2 B x 2), the new bf16 row, the q
    half of q|gate (16 x 256 fp32), new k/v fp32, norm weights, cos/sin."""
    return 2048 * n_past + 2048 + 16384 + 4096 + 1024 + 256


def gqa_layer_bytes(n_past: int) -> int:
    """Algorithmic bytes of one GQA decode step (KV + 48,384 B of q|gate,
    k/v, output, norms, cos/sin)."""
    return 2048 * n_past + 48384


LIN_LAYER_BYTES = 4448960   # state r+w 4 MiB, conv rows/weights, qkv, z, gates, output


def host_cpu() -> dict:
    """The host the CPU baseline ran on: logical CPUs (os.cpu_count and the
    process's affinity set) and the CPU model from /proc/cpuinfo."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        aff = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        aff = None
    return {"nproc": os.cpu_count(), "affinity_cpus": aff, "cpu_model": model}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--ctx", type=int, default=32768)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="CPU-baseline sample budget (whole steps: at least 5 after a warm-up, "
                         "more while within this budget)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", default="stack_decode", choices=["stack_decode", "gqa_prefill",
                                                                    "lin_prefill", "hbm_copy",
                                                                    "gqa_decode", "lin_decode",
                                                                    "mlx4_head",
                                                                    "block_decode", "block_prefill",
                                                                    "launch_floor"])
    ap.add_argument("--tokens", type=int, default=4096, help="prefill length (prefill workloads)")
    ap.add_argument("--npast", type=int, default=4096, help="cached positions (gqa_decode)")
    ap.add_argument("--rotate", type=int, default=0,
                    help="bound layers cycled through (single-layer decode workloads)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (--gpus 1); the multi-GPU sharding "
              "of the path is a design note, not an implementation", file=sys.stderr)
        return 2
    if args.workload == "gqa_prefill":
        return run_gqa_prefill(args)
    if args.workload == "lin_prefill":
        return run_lin_prefill(args)
    if args.workload == "hbm_copy":
        return run_hbm_copy(args)
    if args.workload in ("gqa_decode", "lin_decode"):
        return run_layer_decode(args)
    if args.workload == "mlx4_head":
        return run_mlx4_head(args)
    if args.workload == "block_decode":
        return run_block_decode(args)
    if args.workload == "block_prefill":
        return run_block_prefill(args)
    if args.workload == "launch_floor":
        return run_launch_floor(args)
    return run_stack_decode(args)


def run_launch_floor(args) -> int:
    """The fixed cost of a kernel boundary: n launches of an empty kernel
    captured as one HIP graph, replayed between two events, for the launch
    shapes of the decode step (the delta-rule layer's 32 x 1024, the GQA
    split's 256 x 512 and merge's 256 x 256) and a single wave."""
    import torch

    from ds4f_hip import lib as L

    lib = L.load()
    L.check(lib.ds4f_gpu_init(), "init")
    torch.cuda.init()
    n = 200
    shapes = [(32, 1024), (256, 512), (256, 256), (1, 64)]
    res = []
    for grid, block in shapes:
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        with torch.cuda.graph(g, stream=side):
            st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            L.check(lib.ds4f_hip_launch_floor(n, grid, block, st), "launch floor")
        for _ in range(3):
            g.replay()
        torch.cuda.synchronize()
        best = None
        for _ in range(max(3, args.steps // 10)):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            g.replay()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / n
            best = us if best is None else min(best, us)
        res.append({"grid": grid, "block": block, "us_per_launch": round(best, 3)})
        del g
    line = {"metric": "empty-kernel launch floor in a HIP graph", "value": res[0]["us_per_launch"],
            "unit": "us/launch", "n_gpus": 1, "steps": n, "warmup": 3, "higher_is_better": False,
            "config": {"workload": "launch_floor", "launches_per_graph": n},
            "shapes": res}
    print(json.dumps(line), flush=True)
    return 0


def run_stack_decode(args) -> int:
    import torch

    from ds4f_hip.stack import StackDecode

    N, K, WU, seed = args.ctx, args.steps, args.warmup, args.seed
    T = WU + K
    want_cpu = not args.no_cpu_baseline

    # device state and per-(layer, step) activations, resident in HBM; the
    # host arrays are bound only when the CPU baseline needs the state
    sd = StackDecode(N, T, seed, host_cache=want_cpu)
    lib, ga, cache, layers, kinds = sd.lib, sd.ga, sd.cache, sd.layers, sd.kinds
    gq, lg = sd.gq, sd.lg

    graphs = sd.capture(range(T))
    torch.cuda.synchronize()
    for s in range(WU):
        graphs[s].replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(WU, T):
        graphs[s].replay()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    sec = t1 - t0
    ms_step = sec / K * 1e3
    tok_s = K / sec
    alg_bytes = sum(10 * gqa_layer_bytes(N + s) + 30 * LIN_LAYER_BYTES for s in range(WU, T))
    stack_gbps = alg_bytes / sec / 1e9

    # ---- dominant kernel: the GQA decode (split-K kernel + merge kernel) of
    # the same K steps, all 10 x K launches captured in one HIP graph and
    # timed with hipEvents around its replay on the launch stream
    del graphs
    gq_graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    with torch.cuda.graph(gq_graph, stream=side):
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for s in range(WU, T):
            for Lr, d in enumerate(layers):
                if d["kind"] == 2:
                    sd.launch_layer(Lr, s, st)
    n_gqa_launch = 10 * K
    gq_graph.replay()                      # warm
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    gq_graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    gqa_us = ev0.elapsed_time(ev1) * 1e3 / n_gqa_launch
    del gq_graph
    gqa_bytes = sum(gqa_layer_bytes(N + s) for s in range(WU, T)) / K
    achieved = gqa_bytes / (gqa_us * 1e-6) / 1e9
    traffic = load_traffic(f"gqa_decode_ctx{N}")
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                "kernel": "gqa decode = gqa_split_kernel + gqa_merge_kernel",
                "launches": n_gqa_launch, "us_per_launch": round(gqa_us, 3),
                "bytes_per_launch": int(gqa_bytes)}
    # the committed kernel trace of this command (same launches, traced):
    # the split and merge durations of the GQA graph's ops and the fraction
    # they give; tracing lengthens each dispatch, so it sits below `frac`
    traced = load_traced(f"gqa_decode_ctx{N}")
    if traced:
        roofline["rocprof_traced"] = {
            "us_per_launch": traced["sum_of_means_us"],
            "frac": round(gqa_bytes / (traced["sum_of_means_us"] * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
            "traced_run_event_us_per_launch": traced.get("traced_run_event_us_per_launch"),
            "source": f"profiles/gqa_decode_ctx{N}_rocprof.json"}

    # ---- CPU baseline: the oracle, one thread, same state and streams.  The
    # starting state goes to the host only now, regenerated in place on the
    # device: a device -> host sync of the caches before the timed steps left
    # them about 3 % slower (20-step runs, with or without 200 ms of other GPU
    # work or 50 warm-up steps in between)
    cpu = None
    if want_cpu:
        sd.synth_state()
        ga.sync(-1, to_host=True, n_kv_tokens=N)
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import numpy as np
        import oracle as O
        from ds4f_hip import workloads as W
        O.lib()
        wts = {}
        for Lr, kd in enumerate(kinds):
            wts[Lr] = W.gqa_weights(gq, seed, Lr) if kd == 2 else W.lin_weights(lg, seed, Lr)
        def cpu_step(s):
            """One decode step of the 40 layers on the oracle; returns the
            seconds spent inside the oracle's bodies (activations drawn
            outside the timed calls)."""
            pos, spent = N + s, 0.0
            for Lr, kd in enumerate(kinds):
                if kd == 2:
                    q, k, v = W.gqa_token(gq, seed, Lr, pos)
                    c0 = time.perf_counter()
                    O.gqa_body(cache.kv[Lr], pos, q, k, v, wts[Lr][0], wts[Lr][1], gq.heads,
                               gq.kv_heads, gq.head_dim)
                    spent += time.perf_counter() - c0
                else:
                    qkv, z, a, b = W.lin_token(lg, seed, Lr, s)
                    w = wts[Lr]
                    c0 = time.perf_counter()
                    O.lin_body(cache.conv[Lr], cache.lin[Lr], pos, qkv, z, a, b, w.conv_w,
                               w.A_log, w.dt_bias, w.norm_w, lg.k_heads, lg.v_heads, lg.kd,
                               lg.vd)
                    spent += time.perf_counter() - c0
            return spent

        # one untimed warm-up step, then whole steps (at least 5, within the
        # --cpu-seconds budget, at most 16): the median step time
        cpu_step(0)
        times = []
        while len(times) < 16 and (len(times) < 5 or sum(times) < args.cpu_seconds):
            times.append(cpu_step(len(times) + 1))
        med = float(np.median(times))
        cpu = {"value": round(1.0 / med, 4), "unit": "tokens/s", "cores": 1, "kind": "port",
               "sample": f"median of {len(times)} decode steps of the same 40-layer stack at {N} "
                         f"context (positions {N + 1}..{N + len(times)}, after a warm-up step at "
                         f"{N}), C oracle gcc -O2, 1 thread; step times {min(times):.2f}-"
                         f"{max(times):.2f} s", "host": host_cpu()}

    sd.close()
    # the headline metric names the 32K context; another --ctx says its own
    metric = METRIC if N == 32768 else METRIC.replace("@32K ctx", f"@{N} ctx")
    line = {"metric": metric, "value": round(tok_s, 2), "unit": "tokens/s", "n_gpus": 1,
            "steps": K, "warmup": WU, "ms_per_step": round(ms_step, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "bf16-kv/fp32",
            "data": "synthetic (splitmix64 streams, seed 0: KV bf16 N(0,1), state N(0,0.05), "
                    "activations N(0,1))",
            "config": {"workload": "qwen3.5-35b-a3b attention stack decode: 40 layers "
                                   "(30 gated delta-rule + 10 GQA 16q/2kv d256), attention "
                                   "cores only",
                       "context": N, "layers": 40, "gqa_layers": 10, "delta_layers": 30,
                       "batch": 1, "graph_per_step": True},
            "hbm_gbps": round(stack_gbps, 1), "hbm_frac": round(stack_gbps / HBM_PEAK_GBPS, 4),
            "roofline": roofline, "cpu_baseline": cpu}
    print(json.dumps(line), flush=True)
    return 0


def run_gqa_prefill(args) -> int:
    """One causal GQA prefill of T tokens (one layer, t0 = 0) per step."""
    import torch

    from ds4f_hip import lib as L
    from ds4f_hip import synth as S
    from ds4f_hip import workloads as W
    from ds4f_hip.attn import GpuAttention, dptr

    lib = L.load()
    torch.cuda.init()
    dev = torch.device("cuda:0")
    gq = W.GqaGeom()
    T, K, WU, seed = args.tokens, max(1, min(args.steps, 50)), max(1, min(args.warmup, 5)), args.seed
    ga = GpuAttention([2], T + 64, None)
    nq, nk = gq.heads * 2 * gq.head_dim, gq.kv_heads * gq.head_dim
    q = torch.empty((T, nq), dtype=torch.float32, device=dev)
    k = torch.empty((T, nk), dtype=torch.float32, device=dev)
    v = torch.empty((T, nk), dtype=torch.float32, device=dev)
    for t in range(T):     # bf16-valued N(0,1) inputs, per-token streams
        L.check(lib.ds4f_hip_synth(dptr(q[t]), nq, 2, 0, 0.0, 1.0, seed,
                                   S.tid(S.GQA_QGATE, 0, t), None), "synth")
        L.check(lib.ds4f_hip_synth(dptr(k[t]), nk, 2, 0, 0.0, 1.0, seed, S.tid(S.GQA_K, 0, t),
                                   None), "synth")
        L.check(lib.ds4f_hip_synth(dptr(v[t]), nk, 2, 0, 0.0, 1.0, seed, S.tid(S.GQA_V, 0, t),
                                   None), "synth")
    qn = torch.empty(gq.head_dim, dtype=torch.int16, device=dev)
    kn = torch.empty(gq.head_dim, dtype=torch.int16, device=dev)
    L.check(lib.ds4f_hip_synth(dptr(qn), gq.head_dim, 1, 0, 1.0, 0.1, seed, S.tid(S.GQA_QNW, 0),
                               None), "synth")
    L.check(lib.ds4f_hip_synth(dptr(kn), gq.head_dim, 1, 0, 1.0, 0.1, seed, S.tid(S.GQA_KNW, 0),
                               None), "synth")
    out = torch.empty((T, gq.heads * gq.head_dim), dtype=torch.float32, device=dev)
    stream = torch.cuda.Stream()          # a real stream: events and launches share it
    torch.cuda.set_stream(stream)
    st = ctypes.c_void_p(stream.cuda_stream)

    def step():
        L.check(lib.ds4f_hip_gqa_prefill_async(0, 0, T, dptr(q), dptr(k), dptr(v), dptr(qn),
                                               dptr(kn), dptr(out), None, st), "gqa prefill")

    # first call eagerly (it sizes the workspace), then the op's kernels as
    # one HIP graph, replayed per step like the other workloads
    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step()
    torch.cuda.synchronize()
    for _ in range(WU):
        graph.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(K):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    sec = time.perf_counter() - t0
    op_us = ev0.elapsed_time(ev1) * 1e3 / K
    flops = 4.0 * gq.heads * gq.head_dim * T * (T + 1) / 2
    tflops = flops / (op_us * 1e-6) / 1e12
    roofline = {"bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(tflops / MFMA_PEAK_TFLOPS, 4),
                "traffic": load_traffic(f"gqa_prefill_t{T}"),
                "kernel": "gqa prefill = prep_kernel (k rows, v blocks, prefix rows) + attn_kernel (fp16 MFMA)",
                "launches": K, "us_per_launch": round(op_us, 2), "flops_per_launch": flops}

    cpu = None
    if not args.no_cpu_baseline:
        # the reference prefill is T serial gqa_body calls; time the body at
        # sampled positions on the same inputs and integrate the linear fit
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import numpy as np
        import oracle as O
        qn_h, kn_h = W.gqa_weights(gq, seed, 0)
        pos = np.linspace(0, T - 1, 9).astype(int)
        hq, hk, hv = W.gqa_prefill_tokens(gq, int(pos.max()) + 1, seed, 0)
        rows = O.gqa_cache_rows(hk, hv, kn_h, 0, gq.kv_heads, gq.head_dim)
        kv = np.zeros((T, 2 * gq.kv_heads * gq.head_dim), np.float32)
        kv[:rows.shape[0]] = rows
        secs = []
        for t in pos:    # each position: the median of 5 calls after a warm-up call
            secs.append(med_time(lambda: O.gqa_body(kv, int(t), hq[t].reshape(-1), hk[t].reshape(-1),
                                                    hv[t].reshape(-1), qn_h, kn_h, gq.heads,
                                                    gq.kv_heads, gq.head_dim))[0])
        a, b = np.polyfit(pos.astype(float), np.array(secs), 1)
        est = float(sum(a * t + b for t in range(T)))
        cpu = {"value": round(T / est, 3), "unit": "tokens/s", "cores": 1, "kind": "port",
               "sample": f"oracle gqa_body at {len(pos)} positions 0..{T - 1} of the same "
                         f"prefill, each the median of 5 calls after a warm-up, linear fit "
                         f"integrated over the {T} serial calls the reference makes "
                         f"(est. {est:.1f} s)", "host": host_cpu()}
    ga.close()
    line = {"metric": f"GQA causal prefill tokens/s ({T} tokens, 16q/2kv d256, 1 layer)",
            "value": round(T / (op_us * 1e-6), 1), "unit": "tokens/s", "n_gpus": 1, "steps": K,
            "warmup": WU, "ms_per_step": round(op_us / 1e3, 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "fp16-mfma/fp32",
            "data": "synthetic (splitmix64 streams, seed 0: bf16-valued q|gate, k, v N(0,1))",
            "config": {"workload": "gqa causal prefill", "tokens": T, "t0": 0, "layers": 1, "graph_per_step": True},
            "wall_ms_per_step": round(sec / K * 1e3, 4),
            "roofline": roofline, "cpu_baseline": cpu}
    print(json.dumps(line), flush=True)
    return 0


def med_time(fn, reps: int = 5, warm: int = 1):
    """Median wall time (s) of `reps` calls of fn() after `warm` untimed
    calls, and the list of times."""
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        c0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - c0)
    return sorted(ts)[len(ts) // 2], ts


def load_traced(name: str):
    """The GQA graph's ops in the committed kernel trace of the stack
    workload (profiles/<name>_rocprof.json, written from a rocprofv3 kernel
    trace by ds4f_hip.trace; None when absent)."""
    tpath = os.path.join(ROOT, "profiles", f"{name}_rocprof.json")
    if os.path.exists(tpath):
        return json.load(open(tpath))
    return None


def load_traffic(name: str):
    """HBM bytes per launch measured by the FETCH_SIZE / WRITE_SIZE counter
    runs summarised in profiles/<name>_traffic.json (null when absent)."""
    tpath = os.path.join(ROOT, "profiles", f"{name}_traffic.json")
    if os.path.exists(tpath):
        return json.load(open(tpath)).get("bytes_per_launch")
    return None


def run_hbm_copy(args) -> int:
    """dst = src * 1 over a 1 GiB fp32 buffer: 1 GiB read + 1 GiB written
    per launch."""
    import torch

    torch.cuda.init()
    dev = torch.device("cuda:0")
    n = (1 << 30) // 4
    src = torch.ones(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    K, WU = max(1, min(args.steps, 50)), max(1, min(args.warmup, 5))
    for _ in range(WU):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(K):
        torch.mul(src, 1.0, out=dst)
    ev1.record()
    torch.cuda.synchronize()
    us = ev0.elapsed_time(ev1) * 1e3 / K
    gbps = 2.0 * n * 4 / (us * 1e-6) / 1e9
    line = {"metric": "HBM copy GB/s (1 GiB fp32, read + write)", "value": round(gbps, 1),
            "unit": "GB/s", "n_gpus": 1, "steps": K, "warmup": WU,
            "ms_per_step": round(us / 1e3, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f32", "data": "synthetic (ones)",
            "config": {"workload": "hbm copy", "bytes_read": n * 4, "bytes_written": n * 4},
            "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS,
                         "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
                         "traffic": None, "kernel": "torch elementwise mul (copy)",
                         "launches": K, "us_per_launch": round(us, 2)},
            "cpu_baseline": None}
    print(json.dumps(line), flush=True)
    return 0


def run_layer_decode(args) -> int:
    """One decode call of one layer per unit of work, cycled over R bound
    layers of the same kind inside one HIP graph; every call does the same
    work (a GQA call at position n_past rewrites the same cache row)."""
    import numpy as np
    import torch

    from ds4f_hip import lib as L
    from ds4f_hip import synth as S
    from ds4f_hip import workloads as W
    from ds4f_hip.attn import GpuAttention, dptr

    lib = L.load()
    torch.cuda.init()
    dev = torch.device("cuda:0")
    gq, lg = W.GqaGeom(), W.LinGeom()
    gqa = args.workload == "gqa_decode"
    R = args.rotate or (128 if gqa else 256)
    N, seed = args.npast, args.seed
    pos = N if gqa else 3
    ga = GpuAttention([2 if gqa else 1] * R, (N + 64) if gqa else 64, None)

    def synth(n, dtype, dist, p0, p1, tid):
        t = torch.empty(n, dtype=torch.float32 if dtype == 0 else torch.int16, device=dev)
        L.check(lib.ds4f_hip_synth(dptr(t), n, dtype, dist, p0, p1, seed, tid, None), "synth")
        return t

    layers = []
    for Lr in range(R):
        d = {}
        if gqa:
            L.check(lib.ds4f_hip_synth_gqa_cache(Lr, N, seed, S.tid(S.GQA_KCACHE, Lr),
                                                 S.tid(S.GQA_VCACHE, Lr), None), "synth kv")
            d["qn"] = synth(gq.head_dim, 1, 0, 1.0, 0.1, S.tid(S.GQA_QNW, Lr))
            d["kn"] = synth(gq.head_dim, 1, 0, 1.0, 0.1, S.tid(S.GQA_KNW, Lr))
            d["q"] = synth(gq.heads * 2 * gq.head_dim, 0, 0, 0.0, 1.0, S.tid(S.GQA_QGATE, Lr, N))
            d["k"] = synth(gq.kv_heads * gq.head_dim, 0, 0, 0.0, 1.0, S.tid(S.GQA_K, Lr, N))
            d["v"] = synth(gq.kv_heads * gq.head_dim, 0, 0, 0.0, 1.0, S.tid(S.GQA_V, Lr, N))
            d["out"] = torch.empty(gq.heads * gq.head_dim, dtype=torch.float32, device=dev)
        else:
            L.check(lib.ds4f_hip_synth_lin_state(Lr, 0.05, seed, S.tid(S.LIN_STATE, Lr), None),
                    "synth state")
            L.check(lib.ds4f_hip_synth_conv_history(Lr, pos, seed, S.tid(S.LIN_CONVSTATE, Lr),
                                                    None), "synth conv")
            d["cw"] = synth(lg.rows * 4, 1, 0, 0.0, 0.1, S.tid(S.LIN_CONVW, Lr))
            d["al"] = synth(lg.v_heads, 0, 1, 0.0, 2.7, S.tid(S.LIN_ALOG, Lr))
            d["dt"] = synth(lg.v_heads, 1, 0, 0.0, 0.1, S.tid(S.LIN_DTB, Lr))
            d["nw"] = synth(lg.vd, 1, 0, 1.0, 0.1, S.tid(S.LIN_NORMW, Lr))
            d["qkv"] = synth(lg.rows, 0, 0, 0.0, 1.0, S.tid(S.LIN_QKV, Lr, 0))
            d["z"] = synth(lg.v_heads * lg.vd, 0, 0, 0.0, 1.0, S.tid(S.LIN_Z, Lr, 0))
            d["a"] = synth(lg.v_heads, 0, 0, 0.0, 1.0, S.tid(S.LIN_A, Lr, 0))
            d["b"] = synth(lg.v_heads, 0, 0, 0.0, 1.0, S.tid(S.LIN_B, Lr, 0))
            d["out"] = torch.empty(lg.v_heads * lg.vd, dtype=torch.float32, device=dev)
        layers.append(d)
    torch.cuda.synchronize()

    def launch_all(stream):
        for Lr, d in enumerate(layers):
            if gqa:
                rc = lib.ds4f_hip_gqa_decode_async(Lr, pos, dptr(d["q"]), dptr(d["k"]), dptr(d["v"]),
                                                   dptr(d["qn"]), dptr(d["kn"]), dptr(d["out"]),
                                                   None, stream)
            else:
                rc = lib.ds4f_hip_lin_decode_async(Lr, pos, dptr(d["qkv"]), dptr(d["z"]),
                                                   dptr(d["a"]), dptr(d["b"]), dptr(d["cw"]),
                                                   dptr(d["al"]), dptr(d["dt"]), dptr(d["nw"]),
                                                   dptr(d["out"]), None, stream)
            L.check(rc, f"layer {Lr}")

    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        launch_all(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    reps = max(1, args.steps // R)
    for _ in range(max(1, args.warmup // R)):
        graph.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(reps):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    sec = time.perf_counter() - t0
    calls = reps * R
    us = ev0.elapsed_time(ev1) * 1e3 / calls
    nbytes = gqa_layer_bytes(N) if gqa else LIN_LAYER_BYTES
    gbps = nbytes / (us * 1e-6) / 1e9
    kname = ("gqa decode = gqa_split_kernel + gqa_merge_kernel" if gqa else "lin_decode_kernel")
    roofline = {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(gbps / HBM_PEAK_GBPS, 4),
                "traffic": load_traffic(f"gqa_decode_ctx{N}" if gqa else "lin_decode"),
                "kernel": kname, "launches": calls, "us_per_launch": round(us, 3),
                "bytes_per_launch": nbytes}

    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O
        times = []
        if gqa:
            kc, vc = W.gqa_cache(gq, N, seed, 0)
            half = gq.kv_heads * gq.head_dim
            kv = np.zeros((N + 1, 2 * half), np.float32)
            kv[:N, :half] = kc.reshape(N, half)
            kv[:N, half:] = vc.reshape(N, half)
            qn_h, kn_h = W.gqa_weights(gq, seed, 0)
            q, k, v = W.gqa_token(gq, seed, 0, N)
            O.gqa_body(kv, N, q.reshape(-1), k.reshape(-1).copy(), v.reshape(-1), qn_h, kn_h,
                       gq.heads, gq.kv_heads, gq.head_dim)                 # warm-up
            while len(times) < 5 or sum(times) < min(args.cpu_seconds, 5.0):
                c0 = time.perf_counter()
                O.gqa_body(kv, N, q.reshape(-1), k.reshape(-1).copy(), v.reshape(-1), qn_h, kn_h,
                           gq.heads, gq.kv_heads, gq.head_dim)
                times.append(time.perf_counter() - c0)
        else:
            wt = W.lin_weights(lg, seed, 0)
            S0 = W.lin_state(lg, seed, 0).astype(np.float32)
            ring = W.ring_from_history(lg, W.lin_conv_history(lg, seed, 0), pos)
            qkv, z, a, b = W.lin_token(lg, seed, 0, 0)
            O.lin_body(ring, S0, pos, qkv, z, a, b, wt.conv_w, wt.A_log, wt.dt_bias,
                       wt.norm_w, lg.k_heads, lg.v_heads, lg.kd, lg.vd)         # warm-up
            while len(times) < 5 or sum(times) < min(args.cpu_seconds, 5.0):
                c0 = time.perf_counter()
                O.lin_body(ring, S0, pos, qkv, z, a, b, wt.conv_w, wt.A_log, wt.dt_bias,
                           wt.norm_w, lg.k_heads, lg.v_heads, lg.kd, lg.vd)
                times.append(time.perf_counter() - c0)
        med = sorted(times)[len(times) // 2]
        cpu = {"value": round(1.0 / med, 3), "unit": "tokens/s", "cores": 1, "kind": "port",
               "sample": f"median of {len(times)} oracle {'gqa_body' if gqa else 'lin_body'} calls "
                         f"of the same layer shape after a warm-up call ({sum(times):.1f} s)",
               "host": host_cpu()}
    ga.close()
    what = (f"GQA decode tokens/s (1 layer, 16q/2kv d256, n_past {N})" if gqa
            else "gated delta-rule decode tokens/s (1 layer, 32 heads 128x128)")
    line = {"metric": what, "value": round(1e6 / us, 1), "unit": "tokens/s", "n_gpus": 1,
            "steps": calls, "warmup": max(1, args.warmup // R) * R, "ms_per_step": round(us / 1e3, 5),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "bf16-kv/fp32" if gqa else "f32",
            "data": "synthetic (splitmix64 streams, seed 0)",
            "config": {"workload": args.workload, "n_past": N if gqa else None, "position": pos,
                       "layers_rotated": R,
                       "rotated_state_bytes": R * (2048 * N if gqa else 2 * 1024 * 1024)},
            "wall_ms_per_step": round(sec / calls * 1e3, 5),
            "roofline": roofline, "cpu_baseline": cpu}
    print(json.dumps(line), flush=True)
    return 0


def lin_prefill_flops(T: int, C: int = 64, heads: int = 32, dk: int = 128, dv: int = 128) -> float:
    """Algorithmic flops of the chunked (WY) delta-rule prefill with every
    intra-chunk product counted as a full matrix, per (value head, chunk):
    2 C^2 (3 dk + 2 dv) for K K^T, Q K^T, the W / U products and their
    applications, 6 C dk dv for K S0, Q S0 and K^T Delta, 2 C^3 / 3 for the
    triangular inverse: 11,709,098.7 flop, 2.398e10 at 4096 tokens."""
    per = 2.0 * C * C * (3 * dk + 2 * dv) + 6.0 * C * dk * dv + 2.0 * C ** 3 / 3.0
    return per * heads * ((T + C - 1) // C)


def lin_prefill_flops_useful(T: int, C: int = 64, heads: int = 32, dk: int = 128,
                             dv: int = 128) -> float:
    """The flops this build's T-form kernels issue as useful work, per (value
    head, chunk): K K^T and Q K^T on their lower triangles, once per key head
    (C^2 dk a value head); T = (I + A)^-1 (C^3 / 3); K S0, Q S0 and the state
    update K^T Delta (6 C dk dv); T X and Pm Delta on their triangles
    (2 C^2 dv): 16.29 GFLOP at 4096 tokens."""
    per = 1.0 * C * C * dk + C ** 3 / 3.0 + 6.0 * C * dk * dv + 2.0 * C * C * dv
    return per * heads * ((T + C - 1) // C)


def run_lin_prefill(args) -> int:
    """One delta-rule prefill of T tokens (one layer, t0 = 0, zero state and
    conv ring) per step."""
    import torch

    from ds4f_hip import lib as L
    from ds4f_hip import synth as S
    from ds4f_hip import workloads as W
    from ds4f_hip.attn import GpuAttention, dptr

    lib = L.load()
    torch.cuda.init()
    dev = torch.device("cuda:0")
    lg = W.LinGeom()
    T, K, WU, seed = args.tokens, max(1, min(args.steps, 50)), max(1, min(args.warmup, 5)), args.seed
    ga = GpuAttention([1], T + 64, None)       # zero state, zero ring
    nz = lg.v_heads * lg.vd
    qkv = torch.empty((T, lg.rows), dtype=torch.float32, device=dev)
    z = torch.empty((T, nz), dtype=torch.float32, device=dev)
    a = torch.empty((T, lg.v_heads), dtype=torch.float32, device=dev)
    b = torch.empty((T, lg.v_heads), dtype=torch.float32, device=dev)
    for t in range(T):     # the per-token streams of workloads.lin_token
        for buf, n, tid in ((qkv, lg.rows, S.LIN_QKV), (z, nz, S.LIN_Z), (a, lg.v_heads, S.LIN_A),
                            (b, lg.v_heads, S.LIN_B)):
            L.check(lib.ds4f_hip_synth(dptr(buf[t]), n, 0, 0, 0.0, 1.0, seed, S.tid(tid, 0, t),
                                       None), "synth")
    wt = W.lin_weights(lg, seed, 0)
    cw = torch.from_numpy(wt.conv_w.view("int16").reshape(-1).copy()).to(dev)
    al = torch.from_numpy(wt.A_log.copy()).to(dev)
    dtb = torch.from_numpy(wt.dt_bias.view("int16").copy()).to(dev)
    nw = torch.from_numpy(wt.norm_w.view("int16").copy()).to(dev)
    out = torch.empty((T, nz), dtype=torch.float32, device=dev)
    post = torch.empty((T, lg.rows), dtype=torch.float32, device=dev)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    st = ctypes.c_void_p(stream.cuda_stream)

    def step():
        # every step starts from the zero state (2 MiB fill, inside the timing)
        L.check(lib.ds4f_hip_synth_lin_state(0, 0.0, seed, S.tid(S.LIN_STATE, 0), st), "reset")
        L.check(lib.ds4f_hip_lin_prefill_async(0, 0, T, dptr(qkv), dptr(z), dptr(a), dptr(b),
                                               dptr(cw), dptr(al), dptr(dtb), dptr(nw),
                                               dptr(out), dptr(post), st), "lin prefill")

    for _ in range(WU):
        step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(K):
        step()
    ev1.record()
    torch.cuda.synchronize()
    sec = time.perf_counter() - t0
    op_us = ev0.elapsed_time(ev1) * 1e3 / K
    flops = lin_prefill_flops(T)
    tflops = flops / (op_us * 1e-6) / 1e12
    # frac against the dense bf16 / fp16 MFMA peak the path's prefill bar
    # names; the kernels run their products on fp32 MFMA, whose peak is kept
    # beside it (frac_fp32_peak)
    roofline = {"bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(tflops / MFMA_PEAK_TFLOPS, 4),
                "fp32_peak": MFMA_F32_PEAK_TFLOPS,
                "frac_fp32_peak": round(tflops / MFMA_F32_PEAK_TFLOPS, 4),
                "traffic": load_traffic(f"lin_prefill_t{T}"),
                "kernel": "delta prefill = conv + chunk + scan + gnorm kernels "
                          "(fp32 MFMA), state reset included",
                "launches": K, "us_per_launch": round(op_us, 2), "flops_per_launch": flops,
                "useful_flops_per_launch": lin_prefill_flops_useful(T),
                "useful_frac_fp32_peak": round(lin_prefill_flops_useful(T) / (op_us * 1e-6) / 1e12
                                               / MFMA_F32_PEAK_TFLOPS, 4)}

    cpu = None
    if not args.no_cpu_baseline:
        # the reference prefill is T serial lin_body calls; its cost per
        # token does not depend on the position: time a prefix of the same
        # prefill, whole 64-token batches, within the sample budget
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import numpy as np
        import oracle as O
        hq, hz, ha, hb = W.lin_tokens(lg, min(T, 4096), seed, 0)
        ring = np.zeros((4, lg.rows), np.float32)
        Sh = np.zeros((lg.v_heads, lg.kd, lg.vd), np.float32)
        done, times = 0, []
        while done + 64 <= hq.shape[0] and (len(times) < 6 or sum(times) < args.cpu_seconds):
            sl = slice(done, done + 64)
            c0 = time.perf_counter()
            O.lin_prefill(ring, Sh, done, hq[sl], hz[sl], ha[sl], hb[sl], wt.conv_w, wt.A_log,
                          wt.dt_bias, wt.norm_w, lg.k_heads, lg.v_heads, lg.kd, lg.vd)
            times.append(time.perf_counter() - c0)
            done += 64
        timed = times[1:]        # the first batch is the warm-up
        med = sorted(timed)[len(timed) // 2]
        cpu = {"value": round(64 / med, 3), "unit": "tokens/s", "cores": 1, "kind": "port",
               "sample": f"oracle serial lin_body over the first {done} tokens of the same prefill "
                         f"in 64-token batches: the median of {len(timed)} batches after a warm-up "
                         f"batch (per-token cost is position-independent)", "host": host_cpu()}
    ga.close()
    line = {"metric": f"gated delta-rule prefill tokens/s ({T} tokens, 32 heads 128x128, 1 layer)",
            "value": round(T / (op_us * 1e-6), 1), "unit": "tokens/s", "n_gpus": 1, "steps": K,
            "warmup": WU, "ms_per_step": round(op_us / 1e3, 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32",
            "data": "synthetic (splitmix64 streams, seed 0: qkv, z, a, b N(0,1) per token; "
                    "zero state and conv ring)",
            "config": {"workload": "delta-rule prefill", "tokens": T, "t0": 0, "chunk": 64,
                       "layers": 1},
            "wall_ms_per_step": round(sec / K * 1e3, 4),
            "roofline": roofline, "cpu_baseline": cpu}
    print(json.dumps(line), flush=True)
    return 0



def run_mlx4_head(args) -> int:
    """y = W x for the MLX 4-bit output head (R = 248320 vocabulary rows,
    C = 2048) through the device-resident entry; one launch per step."""
    import numpy as np
    import torch

    from ds4f_hip import lib as L
    from ds4f_hip.attn import dptr

    lib = L.load()
    torch.cuda.init()
    L.check(lib.ds4f_gpu_init(), "init")
    R, C, seed = 248320, 2048, args.seed
    rng = np.random.default_rng(seed)
    ng = R * C // 64
    vals = rng.integers(0, 1 << 32, R * C // 8, dtype=np.uint64).astype(np.uint32)
    sc = rng.uniform(0.002, 0.02, ng).astype(np.float32)
    scales = (sc.view(np.uint32) >> 16).astype(np.uint16)
    biases = ((-sc * rng.uniform(6, 9, ng).astype(np.float32)).view(np.uint32) >> 16).astype(np.uint16)
    x = rng.standard_normal(C).astype(np.float32)
    dev = torch.device("cuda:0")
    dv = torch.from_numpy(vals.view(np.int32)).to(dev)
    ds = torch.from_numpy(scales.view(np.int16)).to(dev)
    db = torch.from_numpy(biases.view(np.int16)).to(dev)
    dx = torch.from_numpy(x).to(dev)
    dy = torch.empty(R, dtype=torch.float32, device=dev)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    torch.cuda.set_stream(stream)
    st = ctypes.c_void_p(stream.cuda_stream)
    K, WU = max(1, min(args.steps, 200)), max(1, min(args.warmup, 20))

    def step():
        L.check(lib.ds4f_hip_mlx4_matvec_async(dptr(dv), dptr(ds), dptr(db), R, C, dptr(dx),
                                               dptr(dy), st), "mlx4")

    for _ in range(WU):
        step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(K):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    us = ev0.elapsed_time(ev1) * 1e3 / K
    nbytes = R * C // 2 + 2 * ng * 2 + C * 4 + R * 4
    gbps = nbytes / (us * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": load_traffic("mlx4_head"),
                "kernel": "mlx4_kernel (MLX 4-bit affine matvec)", "launches": K,
                "us_per_launch": round(us, 2), "bytes_per_launch": nbytes}
    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O
        rows = 8192          # a row sample of the same weight; the cost is linear in rows
        med, ts = med_time(lambda: O.mlx4_matvec(vals[:rows * C // 8], scales[:rows * C // 64],
                                                 biases[:rows * C // 64], rows, C, x), reps=9)
        cpu = {"value": round(rows / R / med, 3), "unit": "matvecs/s", "cores": 1,
               "kind": "port",
               "sample": f"oracle matvec of the first {rows} rows of the same weight, the median "
                         f"of {len(ts)} calls after a warm-up, scaled to {R} rows", "host": host_cpu()}
    line = {"metric": "MLX 4-bit output-head matvec (248320 x 2048) matvecs/s", "value": round(1e6 / us, 1),
            "unit": "matvecs/s", "n_gpus": 1, "steps": K, "warmup": WU,
            "ms_per_step": round(us / 1e3, 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "u4/bf16 weights, f32 x and accumulation",
            "data": f"synthetic (numpy default_rng({seed}): random nibble words, scales "
                    "U(0.002, 0.02), biases -scale * U(6, 9), x N(0, 1))",
            "config": {"workload": "mlx4_head", "rows": R, "cols": C, "weight_bytes": nbytes - C * 4 - R * 4},
            "roofline": roofline, "cpu_baseline": cpu}
    print(json.dumps(line), flush=True)
    return 0



def mlx4_bytes(R: int, C: int) -> int:
    """HBM bytes of one MLX 4-bit weight: nibbles, BF16 scales and biases."""
    return R * C // 2 + 2 * (R * C // 64) * 2


def register_block_weights(ga, kinds, H: int, seed: int, dev, keep: bool):
    """Synthetic MLX 4-bit layer weights for a stack: random nibbles,
    per-group scales in the projections' range and biases that centre each
    group, drawn on the device (torch generator seeded with seed) and
    registered per layer.  Returns (weights per layer if keep, total weight
    bytes, matrix MACs per token over the stack)."""
    import numpy as np
    import torch

    from ds4f_hip import workloads as W
    gq, lg = W.GqaGeom(), W.LinGeom()
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    lo, hi = W.PROJ_SCALE

    def m4(R, C):
        n, ng = R * C, R * C // 64
        vals = torch.randint(0, 256, (n // 2,), dtype=torch.uint8, device=dev, generator=gen)
        sc = torch.rand(ng, device=dev, generator=gen) * (hi - lo) + lo
        bi = -sc * (torch.rand(ng, device=dev, generator=gen) * 3.0 + 6.0)
        u16 = lambda t: t.to(torch.bfloat16).view(torch.int16).cpu().numpy().view(np.uint16)
        return W.Mlx4W(vals.cpu().numpy().view(np.uint32), u16(sc), u16(bi), R, C)

    weights, weight_bytes, macs = {}, 0, 0
    for Lr, kd in enumerate(kinds):
        in_norm = W.norm_weight(H, seed, Lr)
        if kd == 2:
            qn, kn = W.gqa_weights(gq, seed, Lr)
            w = W.GqaLayerW(in_norm, m4(gq.heads * 2 * gq.head_dim, H),
                            m4(gq.kv_heads * gq.head_dim, H), m4(gq.kv_heads * gq.head_dim, H),
                            m4(H, gq.heads * gq.head_dim), qn, kn)
            mats = (w.q, w.k, w.v, w.o)
        else:
            w = W.LinLayerW(in_norm, m4(lg.rows, H), m4(lg.v_heads * lg.vd, H), m4(lg.v_heads, H),
                            m4(lg.v_heads, H), m4(H, lg.v_heads * lg.vd), W.lin_weights(lg, seed, Lr))
            mats = (w.qkv, w.z, w.a, w.b, w.out)
        ga.set_layer_weights(Lr, w)
        weight_bytes += sum(mlx4_bytes(m.rows, m.cols) for m in mats)
        macs += sum(m.rows * m.cols for m in mats)
        if keep:
            weights[Lr] = w
    return weights, weight_bytes, macs


def run_block_decode(args) -> int:
    import numpy as np
    import torch

    from ds4f_hip import lib as L
    from ds4f_hip import synth as S
    from ds4f_hip import workloads as W
    from ds4f_hip.attn import GpuAttention, KvCache, dptr

    lib = L.load()
    torch.cuda.init()
    dev = torch.device("cuda:0")
    gq, lg = W.GqaGeom(), W.LinGeom()
    H = 2048
    kinds = W.stack_kinds(40)
    N, K, WU, seed = args.ctx, args.steps, args.warmup, args.seed
    T = WU + K
    max_tokens = N + T + 64
    want_cpu = not args.no_cpu_baseline

    cache = KvCache(40, max_tokens) if want_cpu else None
    ga = GpuAttention(kinds, max_tokens, cache)

    def synth_start():
        """The layers' caches and states and the per-step hidden states,
        generated in place from the seed (the same values every call)"""
        for Lr, kd in enumerate(kinds):
            if kd == 2:
                L.check(lib.ds4f_hip_synth_gqa_cache(Lr, N, seed, S.tid(S.GQA_KCACHE, Lr),
                                                     S.tid(S.GQA_VCACHE, Lr), None), "synth kv")
            else:
                L.check(lib.ds4f_hip_synth_lin_state(Lr, 0.05, seed, S.tid(S.LIN_STATE, Lr),
                                                     None), "synth state")
                L.check(lib.ds4f_hip_synth_conv_history(Lr, N, seed, S.tid(S.LIN_CONVSTATE, Lr),
                                                        None), "synth conv")
        for s in range(T):
            L.check(lib.ds4f_hip_synth(dptr(states[s]), H, 0, 0, 0.0, 1.0, seed,
                                       S.tid(S.BLK_STATE, 0, s), None), "synth state")

    weights, weight_bytes, _ = register_block_weights(ga, kinds, H, seed, dev, want_cpu)
    states = torch.empty((T, H), dtype=torch.float32, device=dev)
    synth_start()
    torch.cuda.synchronize()

    def launch_step(s, stream):
        for Lr in range(40):
            L.check(lib.ds4f_hip_attn_step_async(Lr, N + s, dptr(states[s]), stream),
                    f"layer {Lr} step {s}")

    graphs = []
    side = torch.cuda.Stream()
    for s in range(T):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            launch_step(s, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        graphs.append(g)
    torch.cuda.synchronize()
    for s in range(WU):
        graphs[s].replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for s in range(WU, T):
        graphs[s].replay()
    ev1.record()
    torch.cuda.synchronize()
    sec = time.perf_counter() - t0
    ev_sec = ev0.elapsed_time(ev1) * 1e-3
    del graphs
    if not bool(torch.isfinite(states).all()):
        raise RuntimeError("block_decode: non-finite hidden state")
    tok_s = K / sec
    act_bytes = 10 * (4 * (16 * 512 + 2 * 512 + 4096) + 2 * 2 * H * 4) + \
        30 * (4 * (8192 + 4096 + 64 + 4096) + 2 * 2 * H * 4)
    step_bytes = [weight_bytes + 10 * gqa_layer_bytes(N + s) + 30 * LIN_LAYER_BYTES + act_bytes
                  for s in range(WU, T)]
    achieved = sum(step_bytes) / ev_sec / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
                "kernel": "whole step: 40 x (mlx4 projections + core + mlx4 output/residual)",
                "launches": K, "us_per_launch": round(ev_sec / K * 1e6, 2),
                "bytes_per_launch": int(sum(step_bytes) / K)}

    cpu = None
    if want_cpu:
        # the starting caches, states and hidden rows go to the host only
        # now, regenerated in place (a device -> host sync before the timed
        # steps leaves them slower, as in the stack workload)
        synth_start()
        ga.sync(-1, to_host=True, n_kv_tokens=N)
        states0 = states.cpu().numpy()
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O
        O.lib()
        times = []
        # step 0 is the warm-up; then at least 5 timed steps (more within the budget)
        while len(times) < 16 and (len(times) < 6 or sum(times[1:]) < args.cpu_seconds):
            done = len(times)
            st = states0[done].copy()
            c0 = time.perf_counter()
            for Lr, kd in enumerate(kinds):
                if kd == 2:
                    st = O.gqa_step(cache.kv[Lr], N + done, st, weights[Lr], gq.heads,
                                    gq.kv_heads, gq.head_dim)
                else:
                    st = O.lin_step(cache.conv[Lr], cache.lin[Lr], N + done, st, weights[Lr],
                                    lg.k_heads, lg.v_heads, lg.kd, lg.vd)
            times.append(time.perf_counter() - c0)
        timed = times[1:]
        med = sorted(timed)[len(timed) // 2]
        cpu = {"value": round(1.0 / med, 4), "unit": "tokens/s", "cores": 1, "kind": "port",
               "sample": f"median of {len(timed)} decode steps of the same 40 whole layers at {N} "
                         f"context after a warm-up step, C oracle gcc -O2 (layer steps incl. the "
                         f"4-bit projections), 1 thread; step times {min(timed):.2f}-{max(timed):.2f} s",
               "host": host_cpu()}

    ga.close()
    line = {"metric": "attention-block decode tokens/s (40 layers, projections included), "
                      f"{N} ctx, 1 GPU",
            "value": round(tok_s, 2), "unit": "tokens/s", "n_gpus": 1, "steps": K,
            "warmup": WU, "ms_per_step": round(sec / K * 1e3, 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "mlx4-weights/bf16-kv/fp32",
            "data": "synthetic (MLX 4-bit weights from a seeded torch generator, KV bf16 N(0,1), "
                    "state N(0,0.05), hidden N(0,1))",
            "config": {"workload": "qwen3.5-35b-a3b attention layers on the residual stream: "
                                   "40 layers (30 gated delta-rule + 10 GQA), input norm, "
                                   "4-bit projections, core, output projection, residual",
                       "context": N, "layers": 40, "hidden": H, "weight_bytes": weight_bytes,
                       "batch": 1, "graph_per_step": True},
            "roofline": roofline, "cpu_baseline": cpu}
    print(json.dumps(line), flush=True)
    return 0

def run_block_prefill(args) -> int:
    """A prefill of --tokens tokens from position 0 through the 40 whole
    layers: per layer one chunk (ds4f_hip_attn_chunk_async: input norm and
    fp16 hi/lo split, the MLX 4-bit projections as one dequant MFMA GEMM,
    the prefill core, the output GEMM accumulating into the states).  One
    step = restore the input states (a 32 MB device copy) + the 40 chunks,
    replayed as one HIP graph."""
    import numpy as np
    import torch

    from ds4f_hip import lib as L
    from ds4f_hip import synth as S
    from ds4f_hip import workloads as W
    from ds4f_hip.attn import GpuAttention, KvCache, dptr

    lib = L.load()
    torch.cuda.init()
    dev = torch.device("cuda:0")
    gq, lg = W.GqaGeom(), W.LinGeom()
    H = 2048
    kinds = W.stack_kinds(40)
    T, K, WU, seed = args.tokens, args.steps, args.warmup, args.seed
    max_tokens = T + 64
    want_cpu = not args.no_cpu_baseline

    cache = KvCache(40, max_tokens) if want_cpu else None
    ga = GpuAttention(kinds, max_tokens, cache)
    weights, weight_bytes, macs = register_block_weights(ga, kinds, H, seed, dev, want_cpu)
    states0 = torch.empty((T, H), dtype=torch.float32, device=dev)
    L.check(lib.ds4f_hip_synth(dptr(states0), T * H, 0, 0, 0.0, 1.0, seed,
                               S.tid(S.BLK_STATE, 0, 0), None), "synth states")
    states = states0.clone()
    torch.cuda.synchronize()

    def launch_step(stream):
        states.copy_(states0)
        for Lr in range(40):
            L.check(lib.ds4f_hip_attn_chunk_async(Lr, 0, T, dptr(states), stream),
                    f"layer {Lr} chunk")

    # first pass eagerly: it sizes the workspaces, which the graph reuses
    launch_step(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        launch_step(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    for _ in range(WU):
        graph.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(K):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    sec = time.perf_counter() - t0
    ev_sec = ev0.elapsed_time(ev1) * 1e-3
    del graph
    if not bool(torch.isfinite(states).all()):
        raise RuntimeError("block_prefill: non-finite hidden state")

    # algorithmic flops of one pass: the 4-bit matrices at 2 flops per MAC
    # and token, the causal GQA attention, the chunked delta rule
    gemm_flops = 2.0 * macs * T
    gqa_flops = 10 * 4.0 * gq.heads * gq.head_dim * T * (T + 1) / 2
    lin_flops = 30 * lin_prefill_flops(T)
    flops = gemm_flops + gqa_flops + lin_flops
    tflops = flops / (ev_sec / K) / 1e12
    roofline = {"bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(tflops / MFMA_PEAK_TFLOPS, 4), "traffic": None,
                "kernel": "whole pass: 40 x (xprep + mlx4 dequant GEMM + prefill core + output "
                          "GEMM), the 10 GQA layers with an xprep before their output GEMM, the "
                          "30 delta-rule layers with the gated norm writing its X operand; peak "
                          "is the fp16 one, the delta-rule core runs on fp32 MFMA",
                "launches": K, "us_per_launch": round(ev_sec / K * 1e6, 2),
                "flops_per_launch": flops, "gemm_flops": gemm_flops, "gqa_flops": gqa_flops,
                "lin_flops": lin_flops}

    cpu = None
    if want_cpu:
        # the reference's chunk runs the layer steps of the tokens in order;
        # time all 40 layer steps at positions spread over the prefill (on
        # the caches the device pass left) and integrate the linear fit
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O
        O.lib()
        ga.sync(-1, to_host=True, n_kv_tokens=T)
        st_host = states0.cpu().numpy()
        pos = np.linspace(0, T - 1, 6).astype(int)
        def steps_at(t):
            st = st_host[t].copy()
            for Lr, kd in enumerate(kinds):
                if kd == 2:
                    st = O.gqa_step(cache.kv[Lr], int(t), st, weights[Lr], gq.heads, gq.kv_heads,
                                    gq.head_dim)
                else:
                    st = O.lin_step(cache.conv[Lr], cache.lin[Lr], int(t), st, weights[Lr],
                                    lg.k_heads, lg.v_heads, lg.kd, lg.vd)

        # each position: the median of 5 passes over the 40 layers after a
        # warm-up pass (a pass at t rewrites position t's rows and advances
        # the delta-rule states: the cost, not the values, is what is timed)
        secs = [med_time(lambda: steps_at(int(t)))[0] for t in pos]
        a, b = np.polyfit(pos.astype(float), np.array(secs), 1)
        est = float(sum(a * t + b for t in range(T)))
        cpu = {"value": round(T / est, 4), "unit": "tokens/s", "cores": 1, "kind": "port",
               "sample": f"C oracle (gcc -O2, 1 thread) 40 whole layer steps at {len(pos)} "
                         f"positions 0..{T - 1}, each the median of 5 passes after a warm-up, "
                         f"linear fit integrated over the {T} serial steps of the reference's "
                         f"chunk (est. {est:.0f} s)", "host": host_cpu()}

    ga.close()
    line = {"metric": f"attention-block prefill tokens/s ({T} tokens, 40 layers, projections "
                      "included), 1 GPU",
            "value": round(T * K / ev_sec, 1), "unit": "tokens/s", "n_gpus": 1, "steps": K,
            "warmup": WU, "ms_per_step": round(ev_sec / K * 1e3, 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "mlx4-weights/fp16-mfma/fp32",
            "data": "synthetic (MLX 4-bit weights from a seeded torch generator, hidden N(0,1))",
            "config": {"workload": "qwen3.5-35b-a3b attention layers on the residual stream, "
                                   "prefill: 40 layers (30 gated delta-rule + 10 GQA), input "
                                   "norm, 4-bit projections, core, output projection, residual",
                       "tokens": T, "t0": 0, "layers": 40, "hidden": H,
                       "weight_bytes": weight_bytes, "graph_per_step": True},
            "wall_ms_per_step": round(sec / K * 1e3, 4),
            "roofline": roofline, "cpu_baseline": cpu}
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
