#!/usr/bin/env python3
"""Decode throughput of the Mistral-7B-shaped input-adaptive model on one GPU.

Workload: 32 layers, dim 4096, FFN 14336, 32 query / 8 KV heads of 128,
vocabulary 32000 with a bucket-layout LM head, fp16 GQA KV cache of 4096
positions, RoPE theta 10000; random-init synthetic weights N(0, 0.02^2)
bucketized on the GPU; a 512-token random-id prompt fed token by token; then
greedy decode at effort 0.25.  A step is one decode token (captured once as a
HIP graph and replayed).  `value` is decode tokens per second, timed with
the library's walk counting switched off; the bytes per token come from
steps run with it on.

roofline: the bucket walk kernel (the dominant one) -- the selected weight
bytes it streams (2 * S * bucket_cols per matrix, counted on the device) per
launch over its average duration, timed with HIP events stamped by each
walk's own dispatch on the library's stream during eager steps, against the
8 TB/s HBM peak (and, as `frac_of_stream`, against the streaming-read
bandwidth measured in the same run: 16-byte loads over 2 GiB, reported as
`stream_read_GBs`).  `traffic` is the walk's measured HBM bytes per launch
(FETCH_SIZE + WRITE_SIZE, calibrated on a copy of known size) read from the
committed counter summary profiles/walk_attention_counters_mistral7b_effort025_ctx2048.md.
`walk_groups` splits the same steps by matrix group (q/k/v, o, w1/w3, w2, LM
head, and the attention kernel): bytes, microseconds and fraction per launch.

effort_sweep: the same decode continued at efforts 1.0, 0.5, 0.125 and
0.05 (graph-replayed steps, counting off): tok/s and the fraction of 8 TB/s
for the bytes touched per token at that effort, the selected bytes counted
over SWEEP_COUNT eager steps that follow (counting on, per-launch events).

The default run also measures the other workloads of the path:
  config1  one 4096x4096 bucketMul at effort 0.25 (rotating copies of W),
           fused (one launch) and as calcDispatch + mul (cutoff launch + walk)
  config2  one FFN block (RMSNorm, w1/w3 with SiLU gate, w2) at efforts 1.0,
           0.5, 0.25, 0.125: the standalone API on the model's layer
           matrices (rotating over the 32 layers), and the model's own FFN
           launches from the sweep's eager steps
  config3  one transformer layer at effort 0.25 with the KV cache filled with
           N(0,1) to 2048 positions
  config5  a short skew sample: KV cache N(0,1), 1% of hidden channels x20 at
           the embedding, 8 sequences near position 4095, efforts 0.05, 1.0
(`--config1` and `--skew` run longer versions of configs 1 and 5 alone.)

cpu_baseline: the C oracle on all host cores given to it (OpenMP threads),
timed on a bounded sample (about 12 s: decoder layers 0, 10, 21 and 31 of
the same model, each on its own input and KV cache, at the positions of the
timed GPU tokens and the same effort, and one LM head pass), scaled to
tokens per second of the 32-layer model.

Profiling modes (no JSON line): `--counter-probe` runs the workload the
rocprofv3 counter passes read; `--counter-summary` and `--trace-summary`
turn rocprofv3 output into the markdown kept under profiles/.
"""
import argparse
import csv
import importlib.util
import json
import os
import sqlite3
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "input-adaptive-matrix-inference-optimization_amd")

MISTRAL = dict(n_layers=32, dim=4096, ffn_dim=14336, n_heads=32, n_kv_heads=8, head_dim=128,
               vocab=32000, max_ctx=4096, rope_theta=10000.0, norm_eps=1e-5)
HBM_PEAK_GBS = 8000.0
SWEEP_EFFORTS = [1.0, 0.5, 0.25, 0.125, 0.05]   # the workloads' efforts
FFN_EFFORTS = [1.0, 0.5, 0.25, 0.125]
SWEEP_WARMUP = 4
SWEEP_COUNT = 4   # eager steps with walk counting on after each timed run: bytes per token
GROUPS = ("qkv", "o", "ffn13", "ffn2", "lm")
LAYER_CTX = 2048


def load_iam():
    spec = importlib.util.spec_from_file_location("iam", os.path.join(PKG, "iam.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def acc_dtype(args):
    return "f64" if args.acc == "fp64" else "f32"


def group_shapes(cfg):
    """(out_dim, in_dim) of the matrices of each walk group."""
    D, F, V = cfg["dim"], cfg["ffn_dim"], cfg["vocab"]
    KVD = cfg["n_kv_heads"] * cfg["head_dim"]
    return {"qkv": [(D, D), (KVD, D), (KVD, D)], "o": [(D, D)], "ffn13": [(F, D), (F, D)],
            "ffn2": [(D, F)], "lm": [(V, D)]}


def fixed_bytes(shapes):
    """Bytes a walk launch reads and writes besides the selected rows: one
    compact stats value per bucket row (2 * 16 * in), x (4 * in), the 4096
    fp16 probes, and the fp32 outputs (4 * out), per matrix."""
    return sum(2 * 16 * i + 4 * i + 2 * 4096 + 4 * o for o, i in shapes)


def kv_bytes(cfg, ctx_len):
    """fp16 K and V of ctx_len positions of one layer."""
    return 2 * 2 * cfg["n_kv_heads"] * cfg["head_dim"] * ctx_len


def per_token_fixed_bytes(cfg, ctx_len):
    """Bytes a decode token reads besides the selected weight rows: every
    walk's fixed part, the K and V of ctx_len positions per layer, and one
    fp16 embedding row."""
    sh = group_shapes(cfg)
    per_layer = sum(fixed_bytes(sh[g]) for g in ("qkv", "o", "ffn13", "ffn2")) + kv_bytes(cfg, ctx_len)
    return cfg["n_layers"] * per_layer + fixed_bytes(sh["lm"]) + 2 * cfg["dim"]


def group_table(ctx, cfg, ctx_len):
    """Per-launch bytes, time and roofline fraction of each walk group and of
    attention, from the kernel statistics and walk counters of the profiled
    steps since the last reset."""
    sh = group_shapes(cfg)
    out = {}
    for g in GROUPS:
        ms, calls = ctx.kernel_stat("bucket_walk." + g)
        wb, rows, _ = ctx.walk_group_counters(g)
        if not calls:
            continue
        b = wb / calls + fixed_bytes(sh[g])
        us = ms * 1e3 / calls
        out[g] = {"launches": calls, "weight_bytes": round(wb / calls), "bytes": round(b),
                  "us": round(us, 2), "GBs": round(b / us / 1e3, 1), "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}
        tries, hits = ctx.walk_group_hints(g)
        if tries:   # matrices whose cutoff search started from the previous step's cutoff, and held
            out[g]["hint_hits"] = round(hits / tries, 4)
    ms, calls = ctx.kernel_stat("attention")
    if calls:
        b = kv_bytes(cfg, ctx_len)
        us = ms * 1e3 / calls
        out["attention"] = {"launches": calls, "context": round(ctx_len), "bytes": round(b), "us": round(us, 2),
                            "GBs": round(b / us / 1e3, 1), "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}
    return out


def profiled_steps(ctx, model, n, effort):
    """n eager decode steps with walk counting and per-launch events on;
    returns the selected weight bytes they streamed."""
    ctx.set_walk_counting(True)
    ctx.walk_counters(reset=True)
    ctx.kernel_stats_reset()
    ctx.profiling(True)
    model.decode(n, effort, use_graph=False)
    ctx.sync()
    ctx.profiling(False)
    b, _, _ = ctx.walk_counters()
    return b


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "walk_attention_counters_mistral7b_effort025_ctx2048.md")


def walk_traffic():
    """HBM bytes per walk launch from the committed counter summary, or None."""
    try:
        for line in open(TRAFFIC_PROFILE):
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) >= 2 and cells[0] == "traffic_bytes_per_launch":
                return float(cells[1])
    except OSError:
        pass
    return None


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


CPU_LAYERS = (0, 10, 21, 31)


def cpu_baseline(model, cfg, positions, effort, budget_s=12.0):
    """Time the oracle on a bounded sample of the timed decode: layers 0, 10,
    21 and 31, each as a one-layer oracle over that layer's weights and its KV
    cache as the GPU filled it, fed that layer's input of the last GPU step,
    at the positions [lo, hi) of the timed GPU tokens in turn; then one
    final-norm + LM-head pass.  The per-layer median scaled to all layers,
    plus the head, is the time per token."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as O

    c1 = dict(cfg)
    c1["n_layers"] = 1
    kv = cfg["max_ctx"] * cfg["n_kv_heads"] * cfg["head_dim"]
    kc_all = model.read_tensor("kcache", np.uint16)
    vc_all = model.read_tensor("vcache", np.uint16)
    lo, hi = positions
    layers = [L for L in CPU_LAYERS if L < cfg["n_layers"]]
    t_layer, calls = [], []
    per_layer_s = budget_s * 0.85 / len(layers)
    for L in layers:
        def read(name, dtype, L=L):
            if name == "embed":
                return np.zeros(16, dtype)          # unused: the sample feeds hidden states
            if name.startswith("layer0."):
                name = f"layer{L}." + name[len("layer0."):]
            return model.read_tensor(name, dtype)

        orc = O.OracleModel(c1, read)
        orc.kc[:] = kc_all[L * kv:(L + 1) * kv]
        orc.vc[:] = vc_all[L * kv:(L + 1) * kv]
        h = model.read_tensor(f"layer{L}.h_in", np.float32)
        t0 = time.perf_counter()
        k = 0
        while time.perf_counter() - t0 < per_layer_s:
            t = time.perf_counter()
            orc.layer_forward(0, lo + k % (hi - lo), effort, h)
            t_layer.append(time.perf_counter() - t)
            k += 1
        calls.append(k)
    tl = float(np.median(t_layer))
    t = time.perf_counter()
    orc.forward(0, hi - 1, effort, hidden_in=model.read_tensor("hidden", np.float32))   # 1 layer + norm + LM head
    t_lm = max(time.perf_counter() - t - tl, 0.0)
    per_token = cfg["n_layers"] * tl + t_lm
    threads = O.threads()
    return {"value": round(1.0 / per_token, 4), "unit": "tok/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "host_cpus": len(os.sched_getaffinity(0)),
            "sample": f"C oracle, {threads} OpenMP threads: decoder layers {', '.join(map(str, layers))} "
                      f"({', '.join(map(str, calls))} calls) at the timed GPU tokens' positions {lo}..{hi - 1}, "
                      f"each layer fed its own input of the last GPU step (median {tl * 1e3:.1f} ms/layer), "
                      f"+ 1 final-norm/LM-head pass ({t_lm * 1e3:.1f} ms), effort {effort}, "
                      f"scaled to {cfg['n_layers']} layers"}


CONFIG1_COPIES = 40   # 40 x 32 MB of buckets: past the 256 MB Infinity Cache


def config1(iam, ctx, effort, reps):
    """One 4096x4096 bucketMul at the given effort, W ~ N(0, 0.02^2)
    bucketized on the GPU, x ~ N(0, 1), seed 0.  Timed as the decode step
    runs a matrix group (iam_bucketmul_fused: input, cutoff, selection and
    walk in one launch) and as the reference's calcDispatch + mul (multi: a
    cutoff launch, then the walk).  CONFIG1_COPIES copies of the bucketized
    matrix are used in turn, so none is in the Infinity Cache when it is
    read again; kernel durations come from per-dispatch events.  Bytes per
    call: 2*S*C + 2*R + 4*in + 2*4096 + 4*m (selected rows, one stats value
    per row, x, probes, y)."""
    n = out_dim = in_dim = 4096
    R, C = in_dim * 16, out_dim // 16
    u16 = np.uint16
    W = ctx.empty(n * n, u16)
    ctx.gen_f16(0, 1, n * n, 0.0, 0.02, W)
    x = ctx.empty(in_dim, np.float32)
    ctx.gen_f32(0, 2, in_dim, 0.0, 1.0, x)
    b0, s0, p0 = ctx.empty(R * C, u16), ctx.empty(R * 4, u16), ctx.empty(in_dim, u16)
    ctx.bucketize(W, out_dim, in_dim, b0, s0, p0)
    s3 = ctx.stats_compact(s0, R)
    mats, bufs = [], [W, b0, s0, p0, s3]
    for k in range(CONFIG1_COPIES):
        b, st, pr = ctx.empty(R * C, u16), ctx.empty(R, u16), ctx.empty(in_dim, u16)
        ctx.copy(b, b0, R * C * 2)
        ctx.copy(st, s3, R * 2)
        ctx.copy(pr, p0, in_dim * 2)
        bufs += [b, st, pr]
        mats.append(iam.BucketMatrix(b.ptr, st.ptr, pr.ptr, R, C, 1, 0))
    y = ctx.empty(out_dim, np.float32)
    res = {}
    for mode in ("fused", "cutoff_launch"):
        def call(m):
            if mode == "fused":
                ctx.fused([m], x, in_dim, [y], effort)
            else:
                ctx.multi([m], [x], [in_dim], [y], effort)
        for m in mats:
            call(m)
        ctx.sync()
        ctx.set_walk_counting(True)
        ctx.walk_counters(reset=True)
        ctx.kernel_stats_reset()
        ctx.profiling(True)
        for r in range(reps):
            call(mats[r % CONFIG1_COPIES])
        ctx.sync()
        ctx.profiling(False)
        _, rows, _ = ctx.walk_counters(reset=True)
        t_ms = 0.0
        parts = {}
        for name in ("bucket_cutoff", "bucket_walk"):
            ms, calls = ctx.kernel_stat(name)
            if calls:
                parts[name.split("_")[1] + "_us"] = round(ms / calls * 1e3, 2)
                t_ms += ms / reps
        S = rows / reps
        B = 2 * S * C + 2 * R + 4 * in_dim + 2 * 4096 + 4 * out_dim
        gbs = B / (t_ms * 1e-3) / 1e9
        res[mode] = dict(time_us=round(t_ms * 1e3, 2), **parts, selected_rows=round(S),
                         bytes_per_call=round(B), achieved_GBs=round(gbs, 1), frac=round(gbs / HBM_PEAK_GBS, 4))
        log(f"config 1, {mode}: {t_ms * 1e3:.2f} us per call ({parts}), S = {S:.0f}, "
            f"{B / 1e6:.2f} MB -> {gbs:.0f} GB/s")
    for d in bufs + [x, y]:
        d.free()
    return res


def config2(iam, ctx, model, cfg, efforts, reps):
    """One FFN block through the standalone API: x = RMSNorm(h) * ffn_gain
    fused into the w1/w3 launch, SiLU(w1 x) * (w3 x) by the silu_mul kernel,
    then w2, on the model's layer matrices (layer r mod 32 for block r, so
    the 352 MB of a block's matrices are not cache resident), h ~ N(0, 1).
    Kernel time summed over the three launches; bytes = the selected rows
    (counted on the device) + stats, x, probes and outputs of the three
    matrices + h and the fp16 gain."""
    D, F, L = cfg["dim"], cfg["ffn_dim"], cfg["n_layers"]
    f32 = np.float32
    h, x = ctx.empty(D, f32), ctx.empty(D, f32)
    g, u, s, y = ctx.empty(F, f32), ctx.empty(F, f32), ctx.empty(F, f32), ctx.empty(D, f32)
    ctx.gen_f32(0, 7001, D, 0.0, 1.0, h)
    layers = [(model.matrix(f"layer{i}.w1"), model.matrix(f"layer{i}.w3"), model.matrix(f"layer{i}.w2"),
               model.tensor(f"layer{i}.ffn_gain")[0]) for i in range(L)]
    sh = group_shapes(cfg)
    fixed = fixed_bytes(sh["ffn13"]) + fixed_bytes(sh["ffn2"]) + 4 * D + 2 * D

    def block(r, e):
        w1, w3, w2, gain = layers[r % L]
        ctx.fused([w1, w3], x, D, [g, u], e, h=h, gain=gain, eps=cfg["norm_eps"])
        ctx.silu_mul(g, u, F, s)
        ctx.fused([w2], s, F, [y], e)

    res = {}
    for e in efforts:
        for r in range(4):
            block(r, e)
        ctx.sync()
        ctx.set_walk_counting(True)
        ctx.walk_counters(reset=True)
        ctx.kernel_stats_reset()
        ctx.profiling(True)
        for r in range(reps):
            block(r, e)
        ctx.sync()
        ctx.profiling(False)
        wb, _, _ = ctx.walk_counters(reset=True)
        ms, _ = ctx.kernel_stat("*")
        walk_ms, _ = ctx.kernel_stat("bucket_walk")
        us = ms * 1e3 / reps
        b = wb / reps + fixed
        res[str(e)] = {"us": round(us, 2), "walk_us": round(walk_ms * 1e3 / reps, 2), "bytes": round(b),
                       "GBs": round(b / us / 1e3, 1), "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}
        log(f"config 2, effort {e}: {us:.1f} us per FFN block, {b / 1e6:.1f} MB -> {b / us / 1e3:.0f} GB/s")
    for d in (h, x, g, u, s, y):
        d.free()
    return res


def fill_kv_normal(ctx, model):
    """Every layer's K and V cache, all positions: fp16 N(0, 1)."""
    for name, tid in (("kcache", 9001), ("vcache", 9002)):
        ptr, nbytes = model.tensor(name)
        ctx.gen_f16(0, tid, nbytes // 2, 0.0, 1.0, ptr)


def config3(ctx, model, cfg, effort, steps=4, warmup=2):
    """One transformer layer at decode with the KV cache filled with N(0, 1)
    fp16 values: the model's decode steps at positions 2048.. (warm-up from
    2046), per-launch events; a layer is its q/k/v walk (attention norm and
    residual fused in), attention (RoPE and KV append fused in), o walk,
    w1/w3 walk (FFN norm, residual and SiLU fused in) and w2 walk."""
    fill_kv_normal(ctx, model)
    model.set_position(LAYER_CTX - warmup)
    model.write_tensor("token", np.array([1234], np.int32))
    ctx.set_walk_counting(True)
    model.decode(warmup, effort, use_graph=False)
    ctx.sync()
    profiled_steps(ctx, model, steps, effort)
    tab = group_table(ctx, cfg, LAYER_CTX + (steps + 1) / 2)
    parts = ("qkv", "attention", "o", "ffn13", "ffn2")
    us = sum(tab[p]["us"] for p in parts)
    b = sum(tab[p]["bytes"] for p in parts)
    all_ms, _ = ctx.kernel_stat("*")
    lm_ms, _ = ctx.kernel_stat("bucket_walk.lm")
    other = (all_ms - lm_ms) * 1e3 / steps - us * cfg["n_layers"]
    log(f"config 3: {us:.1f} us per layer, {b / 1e6:.1f} MB -> {b / us / 1e3:.0f} GB/s")
    return {"us": round(us, 2), "bytes": round(b), "GBs": round(b / us / 1e3, 1),
            "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4), "positions": f"{LAYER_CTX}..{LAYER_CTX + steps - 1}",
            "other_kernels_us_per_step": round(other, 2), "launches": {p: tab[p] for p in parts}}


SKEW_EFFORTS = [0.05, 1.0]
SKEW_SEQUENCES = 8


def skew(ctx, model, cfg, n, warmup, count, efforts=SKEW_EFFORTS, sequences=SKEW_SEQUENCES):
    """Skew stress: every layer's K and V filled with N(0,1) fp16 values for
    all 4096 positions, then `sequences` sequences decoded back-to-back near
    the end of the context, each with its own seeded 1% of hidden channels
    (41 of 4096) scaled 20x at the embedding (graph-replayed steps; `count`
    more steps per sequence with walk counting on give the bytes)."""
    fill_kv_normal(ctx, model)
    start = cfg["max_ctx"] - warmup - n - count - 1
    if n < 1 or start < 1:
        sys.exit(f"skew: {n} steps do not fit the context")
    rng = np.random.default_rng(5)
    res = {}
    for e in efforts:
        steps = counted = 0
        secs = 0.0
        wbytes = 0
        for sq in range(sequences):
            scale = np.ones(cfg["dim"], np.float32)
            scale[rng.choice(cfg["dim"], cfg["dim"] // 100, replace=False)] = 20.0
            model.set_embed_scale(scale)
            model.set_position(start)
            model.write_tensor("token", np.array([int(rng.integers(0, cfg["vocab"]))], np.int32))
            ctx.set_walk_counting(False)
            model.decode(warmup, e)
            ctx.sync()
            t0 = time.perf_counter()
            model.decode(n, e)
            ctx.sync()
            secs += time.perf_counter() - t0
            steps += n
            ctx.set_walk_counting(True)
            ctx.walk_counters(reset=True)
            model.decode(count, e)
            ctx.sync()
            b, _, _ = ctx.walk_counters(reset=True)
            wbytes += b
            counted += count
        bpt = wbytes / counted + per_token_fixed_bytes(cfg, start + warmup + n // 2)
        tps = steps / secs
        res[str(e)] = {"tok_s": round(tps, 2), "ms_per_token": round(secs / steps * 1e3, 4),
                       "bytes_per_token": round(bpt), "achieved_GBs": round(bpt * tps / 1e9, 1),
                       "frac": round(bpt * tps / 1e9 / HBM_PEAK_GBS, 4)}
        log(f"skew, effort {e}: {tps:.1f} tok/s over {steps} steps, {bpt / 1e9:.3f} GB/token")
    model.set_embed_scale(None)
    return res, start


def run_config1(args, iam, ctx):
    """`--config1`: config 1 alone, with more calls, as its own JSON line."""
    res = config1(iam, ctx, args.effort, args.config1_reps)
    stream_gbs = ctx.read_bandwidth(2 << 30, 10)
    f = res["fused"]
    out = {
        "metric": "config 1: one 4096x4096 bucketMul at effort 0.25 (cutoff, selection, walk), "
                  "achieved GB/s of the selected rows + stats + x + probes + y",
        "value": f["achieved_GBs"], "unit": "GB/s", "n_gpus": 1, "steps": args.config1_reps,
        "higher_is_better": True, "dtype": acc_dtype(args), "data": "synthetic (seed 0)",
        "config": {"workload": "W 4096x4096 fp16 N(0, 0.02^2) in bucket layout, x 4096 fp32 N(0,1), "
                               f"effort {args.effort}, {CONFIG1_COPIES} rotating copies of W"},
        "frac": f["frac"], "frac_of_stream": round(f["achieved_GBs"] / stream_gbs, 4),
        "stream_read_GBs": round(stream_gbs, 1), "fused": res["fused"], "cutoff_launch": res["cutoff_launch"],
    }
    print(json.dumps(out), flush=True)


def run_skew(args, iam, ctx):
    """`--skew`: the skew stress alone, 32 timed steps per sequence."""
    cfg = dict(MISTRAL)
    model = iam.Model(ctx, iam.ModelConfig(**cfg))
    model.synthesize(0)
    res, start = skew(ctx, model, cfg, args.skew_steps, SWEEP_WARMUP, SWEEP_COUNT)
    out = {
        "metric": "skew stress: decode tok/s at efforts 0.05 and 1.0, context 4096, 8 sequences",
        "value": res[str(SKEW_EFFORTS[0])]["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": args.skew_steps,
        "warmup": SWEEP_WARMUP, "higher_is_better": True, "vs_baseline": None, "dtype": acc_dtype(args),
        "dtype_detail": "fp16 weights, fp32 activations, %s products and accumulation" % args.acc,
        "data": "synthetic (random-init weights, N(0,1) KV cache, random token ids)",
        "config": {"workload": "Mistral-7B-shape decode, 1 percent of hidden channels x20 at the embedding, "
                               f"positions {start}..{start + SWEEP_WARMUP + args.skew_steps + SWEEP_COUNT - 1} "
                               "of 4096", "sequences": SKEW_SEQUENCES, "efforts": SKEW_EFFORTS},
        "efforts": res,
    }
    print(json.dumps(out), flush=True)
    model.close()


# ------------------------------------------------------------ profiling ---

PROBE_CFG = dict(MISTRAL)


def run_counter_probe(args, iam, ctx):
    """`--counter-probe`: the workload of the rocprofv3 counter passes.  The
    32-layer model, an 8-token prompt, then every layer's K and V cache
    filled with N(0,1) and the position set to `--probe-pos` (2048, the
    layer workload's context), and `--probe-steps` eager decode steps (the
    same launch mix as a decode step of the default run: per layer the
    q/k/v, o, w1/w3 and w2 walks and attention, then the LM head), then one
    device-to-device copy of 256 MiB that calibrates FETCH_SIZE and
    WRITE_SIZE.  Prints one JSON line with the decode steps' algorithmic
    bytes per launch of each walk group and of attention."""
    cfg = PROBE_CFG
    model = iam.Model(ctx, iam.ModelConfig(**cfg))
    model.synthesize(0)
    prompt = np.random.default_rng(0).integers(0, cfg["vocab"], 8).astype(np.int32)
    model.generate(prompt, 1, args.effort, use_graph=False)
    ctx.sync()
    pos0 = 8
    if args.probe_pos > 8:
        fill_kv_normal(ctx, model)
        model.set_position(args.probe_pos)
        pos0 = args.probe_pos
    n = args.probe_steps
    ctx.set_walk_counting(True)
    ctx.walk_counters(reset=True)
    model.decode(n, args.effort, use_graph=False)
    ctx.sync()
    sh = group_shapes(cfg)
    groups = {}
    for g in GROUPS:
        wb, _, _ = ctx.walk_group_counters(g)
        launches = n * (1 if g == "lm" else cfg["n_layers"])
        groups[g] = {"weight_bytes": wb / launches, "bytes": wb / launches + fixed_bytes(sh[g])}
    nbytes = 256 << 20
    a, b = ctx.alloc(nbytes), ctx.alloc(nbytes)
    ctx.copy(b, a, nbytes)
    ctx.sync()
    actx = pos0 + 1 + (n - 1) / 2
    print(json.dumps({"steps": n, "layers": cfg["n_layers"], "effort": args.effort, "position": pos0,
                      "attention_context": actx, "kv_bytes": kv_bytes(cfg, actx),
                      "groups": groups, "copy_bytes": nbytes}), flush=True)
    a.free()
    b.free()
    model.close()


def label_dispatches(rows, steps, layers):
    """The decode steps' dispatches of a counter or trace listing, labelled:
    rows = [(dispatch_id, kernel_name, value)] in dispatch order; the last
    steps * (4 * layers + 1) walk dispatches are q/k/v, o, w1/w3, w2 per
    layer and the LM head per step, and the last steps * layers attention
    dispatches are attention."""
    walks = [r for r in rows if "k_walk" in r[1]]
    attn = [r for r in rows if "k_attn" in r[1]]
    per_step = 4 * layers + 1
    walks = walks[-steps * per_step:]
    attn = attn[-steps * layers:]
    out = {g: [] for g in GROUPS + ("attention",)}
    for i, r in enumerate(walks):
        k = i % per_step
        out["lm" if k == 4 * layers else ("qkv", "o", "ffn13", "ffn2")[k % 4]].append(r)
    out["attention"] = attn
    return out


def read_counter_csv(path):
    """{counter: [(dispatch_id, kernel_name, value)]} of a rocprofv3
    counter_collection CSV (agent-level rows of one dispatch summed)."""
    vals = {}
    with open(path) as f:
        for row in csv.DictReader(f):
            key = (row["Counter_Name"], int(row["Dispatch_Id"]))
            v = float(row["Counter_Value"])
            name = row["Kernel_Name"]
            vals[key] = (name, vals[key][1] + v) if key in vals else (name, v)
    out = {}
    for (ctr, d), (name, v) in sorted(vals.items(), key=lambda kv: kv[0][1]):
        out.setdefault(ctr, []).append((d, name, v))
    return out


def run_counter_summary(args):
    """`--counter-summary CSV... --probe JSON`: markdown tables of the
    counters of each labelled launch kind, averaged per dispatch over the
    probe's decode steps; FETCH_SIZE and WRITE_SIZE (KiB) calibrated on the
    probe's copy and set beside the algorithmic bytes."""
    probe = json.loads(open(args.probe).read().strip().splitlines()[-1])
    steps, layers = probe["steps"], probe["layers"]
    kinds = GROUPS + ("attention",)
    algo = {g: probe["groups"][g]["bytes"] for g in GROUPS}
    algo["attention"] = probe["kv_bytes"]
    table = {}
    calib = {}
    for path in args.counter_summary:
        for ctr, rows in read_counter_csv(path).items():
            lab = label_dispatches(rows, steps, layers)
            table[ctr] = {k: (sum(v for _, _, v in lab[k]) / len(lab[k]) if lab[k] else float("nan"), len(lab[k]))
                          for k in kinds}
            if ctr in ("FETCH_SIZE", "WRITE_SIZE"):
                copy = [v for _, n, v in rows if "copy" in n.lower() and "walk" not in n]
                calib[ctr] = (max(copy), probe["copy_bytes"] / (max(copy) * 1024.0)) if copy else None
    if args.trace:
        c = sqlite3.connect(args.trace)
        disp = [(d, nm, dur) for d, nm, dur in c.execute("select dispatch_id, name, duration from kernels "
                                                         "order by dispatch_id")]
        lab = label_dispatches(disp, steps, layers)
        print("| kind | launches | algorithmic bytes | avg us | GB/s | fraction of 8 TB/s |")
        print("|---|---:|---:|---:|---:|---:|")
        for k in kinds:
            if not lab[k]:
                continue
            us = sum(x for _, _, x in lab[k]) / len(lab[k]) / 1e3
            print(f"| {k} | {len(lab[k])} | {algo[k]:.0f} | {us:.2f} | {algo[k] / us / 1e3:.0f} "
                  f"| {algo[k] / us / 1e3 / HBM_PEAK_GBS:.3f} |")
        print()
    print("| counter | " + " | ".join(kinds) + " |")
    print("|---|" + "---:|" * len(kinds))
    for ctr in sorted(table):
        print(f"| {ctr} | " + " | ".join(f"{table[ctr][k][0]:.4g}" for k in kinds) + " |")
    print(f"| dispatches averaged | " + " | ".join(str(next(iter(table.values()))[k][1]) for k in kinds) + " |")
    if "FETCH_SIZE" in table and "WRITE_SIZE" in table and calib.get("FETCH_SIZE") and calib.get("WRITE_SIZE"):
        fk, ff = calib["FETCH_SIZE"]
        wk, wf = calib["WRITE_SIZE"]
        print()
        print(f"Copy calibration: {probe['copy_bytes']} bytes copied; FETCH_SIZE {fk:.0f} KiB (factor {ff:.4f}), "
              f"WRITE_SIZE {wk:.0f} KiB (factor {wf:.4f}).")
        print()
        print("| kind | algorithmic bytes | HBM read (calibrated) | HBM written (calibrated) | traffic / algorithmic |")
        print("|---|---:|---:|---:|---:|")
        walk_t = walk_a = 0.0
        n_walk = 0
        for k in kinds:
            rd = table["FETCH_SIZE"][k][0] * 1024 * ff
            wr = table["WRITE_SIZE"][k][0] * 1024 * wf
            print(f"| {k} | {algo[k]:.0f} | {rd:.0f} | {wr:.0f} | {(rd + wr) / algo[k]:.3f} |")
            if k in GROUPS:
                c = table["FETCH_SIZE"][k][1]
                walk_t += (rd + wr) * c
                walk_a += algo[k] * c
                n_walk += c
        print()
        print("| quantity | value |")
        print("|---|---:|")
        print(f"| traffic_bytes_per_launch | {walk_t / n_walk:.0f} |")
        print(f"| algorithmic_bytes_per_launch | {walk_a / n_walk:.0f} |")
        print(f"| traffic / algorithmic (every walk launch) | {walk_t / walk_a:.3f} |")


def run_trace_summary(args):
    """`--trace-summary DB --trace-steps N --trace-layers L`: markdown of a
    rocprofv3 kernel trace (results .db): per-kernel totals, and the last N
    decode steps' walk and attention launches by kind."""
    c = sqlite3.connect(args.trace_summary)
    rows = list(c.execute(
        "select name, count(*), sum(duration), avg(duration), min(duration), max(duration) "
        "from kernels group by name order by sum(duration) desc"))
    total = sum(r[2] for r in rows)
    print("| kernel | calls | total ms | avg us | min us | max us | % |")
    print("|---|---:|---:|---:|---:|---:|---:|")
    for name, n, tot, avg, mn, mx in rows:
        print(f"| `{name[:70]}` | {n} | {tot / 1e6:.3f} | {avg / 1e3:.2f} | {mn / 1e3:.2f} | {mx / 1e3:.2f} "
              f"| {100.0 * tot / total:.1f} |")
    disp = [(d, n, dur) for d, n, dur in c.execute("select dispatch_id, name, duration from kernels "
                                                   "order by dispatch_id")]
    lab = label_dispatches(disp, args.trace_steps, args.trace_layers)
    print()
    print(f"Last {args.trace_steps} decode steps by launch kind:")
    print()
    print("| kind | launches | avg us | min us | max us | us per step |")
    print("|---|---:|---:|---:|---:|---:|")
    for k, v in lab.items():
        if not v:
            continue
        d = [x for _, _, x in v]
        print(f"| {k} | {len(d)} | {np.mean(d) / 1e3:.2f} | {min(d) / 1e3:.2f} | {max(d) / 1e3:.2f} "
              f"| {sum(d) / 1e3 / args.trace_steps:.1f} |")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--effort", type=float, default=0.25)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--profile-steps", type=int, default=8)
    ap.add_argument("--sweep-steps", type=int, default=32,
                    help="timed decode steps per effort of the effort sweep (0: no sweep)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the config 1/2/3/5 measurements of the default run")
    ap.add_argument("--acc", choices=["fp64", "fp32"], default="fp64",
                    help="walk/attention accumulation (fp64: results equal the correctly rounded sums)")
    ap.add_argument("--select-block", type=int, default=1,
                    help="block-structured selection: inputs per block (1: the reference's per-row selection)")
    ap.add_argument("--select-below", type=float, default=2.0,
                    help="with --select-block: apply it to efforts below this one")
    ap.add_argument("--eager", action="store_true",
                    help="launch every kernel from the host instead of replaying a captured graph")
    ap.add_argument("--skew", action="store_true",
                    help="run the skew stress (efforts 0.05 and 1.0 at context 4096, 8 sequences) instead")
    ap.add_argument("--skew-steps", type=int, default=32, help="timed decode steps per sequence and effort")
    ap.add_argument("--config1", action="store_true",
                    help="time config 1 instead (one 4096x4096 bucketMul, rotating copies of W)")
    ap.add_argument("--config1-reps", type=int, default=400, help="timed calls per mode of --config1")
    ap.add_argument("--counter-probe", action="store_true", help="run the counter passes' workload")
    ap.add_argument("--probe-steps", type=int, default=4)
    ap.add_argument("--probe-pos", type=int, default=LAYER_CTX,
                    help="position of the probe's decode steps (KV cache N(0,1) below it)")
    ap.add_argument("--counter-summary", nargs="+", metavar="CSV",
                    help="summarize rocprofv3 counter_collection CSVs of --counter-probe runs")
    ap.add_argument("--probe", help="the JSON line --counter-probe printed")
    ap.add_argument("--trace", metavar="DB", help="with --counter-summary: a kernel trace of the same probe command")
    ap.add_argument("--trace-summary", metavar="DB", help="summarize a rocprofv3 kernel trace")
    ap.add_argument("--trace-steps", type=int, default=8)
    ap.add_argument("--trace-layers", type=int, default=32)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        sys.exit(2)
    if args.counter_summary:
        if not args.probe:
            sys.exit("--counter-summary needs --probe")
        run_counter_summary(args)
        return
    if args.trace_summary:
        run_trace_summary(args)
        return
    if args.profile_steps < 1:
        sys.exit("--profile-steps must be at least 1 (they give the walk's bytes and launch times)")
    cfg = dict(MISTRAL)
    sweep_efforts = [e for e in SWEEP_EFFORTS if e != args.effort] if args.sweep_steps > 0 else []
    total = (args.prompt + args.warmup + args.steps + args.profile_steps + 1
             + len(sweep_efforts) * (SWEEP_WARMUP + args.sweep_steps + SWEEP_COUNT))
    limit = cfg["max_ctx"] if args.no_configs else LAYER_CTX - 2   # the layer measurement starts there
    if total > limit:
        sys.exit(f"prompt + warmup + steps + profile steps + sweep ({total}) exceed {limit} positions")

    iam = load_iam()
    ctx = iam.Ctx(0)
    ctx.set_accumulation(args.acc)
    if args.select_block != 1:
        ctx.set_selection_block(args.select_block, args.select_below)
    if args.counter_probe:
        run_counter_probe(args, iam, ctx)
        ctx.close()
        return
    if args.skew:
        run_skew(args, iam, ctx)
        ctx.close()
        return
    if args.config1:
        run_config1(args, iam, ctx)
        ctx.close()
        return
    use_graph = not args.eager
    name, cus, mem = ctx.device_info()
    log(f"device {name}, {cus} CUs, {mem / 2**30:.0f} GiB")
    t = time.perf_counter()
    model = iam.Model(ctx, iam.ModelConfig(**cfg))
    model.synthesize(0)
    log(f"model built and synthesized in {time.perf_counter() - t:.1f} s")

    prompt = np.random.default_rng(0).integers(0, cfg["vocab"], args.prompt).astype(np.int32)
    t = time.perf_counter()
    first = model.generate(prompt, 1, args.effort, use_graph=use_graph)
    ctx.sync()
    log(f"prefill of {args.prompt} tokens: {time.perf_counter() - t:.2f} s, first token {int(first[0])}")

    # the timed decode runs with the walk counting off (a captured graph of
    # that setting); the counted steps below give the bytes
    ctx.set_walk_counting(False)
    model.decode(args.warmup, args.effort, use_graph=use_graph)
    ctx.sync()
    t0 = time.perf_counter()
    model.decode(args.steps, args.effort, use_graph=use_graph)
    ctx.sync()
    t1 = time.perf_counter()
    dt = t1 - t0
    tok_s = args.steps / dt

    # per-kernel times: eager decode steps in which every kernel is launched
    # with a pair of HIP events stamped by its own dispatch on the library's
    # stream (hipExtLaunchKernelGGL), so each elapsed time is that kernel's
    # duration
    pos_prof = args.prompt + args.warmup + args.steps
    pbytes = profiled_steps(ctx, model, args.profile_steps, args.effort)
    walk_ms, walk_calls = ctx.kernel_stat("bucket_walk")
    log(ctx.kernel_stats())
    groups = group_table(ctx, cfg, pos_prof + 1 + (args.profile_steps - 1) / 2)
    per_launch = pbytes / walk_calls
    walk_avg_s = walk_ms / 1e3 / walk_calls
    achieved = per_launch / walk_avg_s / 1e9
    # bytes per token of the timed decode: the selected bytes of these
    # counted steps (the next positions of the same sequence) + the fixed part
    pos_mid = args.prompt + args.warmup + args.steps // 2
    bytes_per_token = pbytes / args.profile_steps + per_token_fixed_bytes(cfg, pos_mid)
    log(f"decode: {args.steps} tokens in {dt * 1e3:.1f} ms = {tok_s:.1f} tok/s; "
        f"{bytes_per_token / 1e9:.3f} GB/token -> {bytes_per_token * tok_s / 1e9:.0f} GB/s")
    # measured streaming-read peak (16-byte loads over 2 GiB, past the 256 MB
    # Infinity Cache), the second reference besides the published 8 TB/s
    stream_gbs = ctx.read_bandwidth(2 << 30, 10)
    log(f"streaming read: {stream_gbs:.0f} GB/s")

    # the same decode at the other efforts of the workloads, continuing the
    # sequence: tok/s and the roofline fraction of the bytes touched per
    # token; the counted eager steps also give the model's FFN launches
    sweep = {}
    ffn_model = {"0.25": None}
    pos_now = args.prompt + args.warmup + args.steps + args.profile_steps

    def ffn_of(tab):
        us = tab["ffn13"]["us"] + tab["ffn2"]["us"]
        b = tab["ffn13"]["bytes"] + tab["ffn2"]["bytes"]
        return {"us": round(us, 2), "bytes": round(b), "GBs": round(b / us / 1e3, 1),
                "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}

    if args.effort == 0.25:
        ffn_model["0.25"] = ffn_of(groups)
    for e in sweep_efforts:
        ctx.set_walk_counting(False)
        model.decode(SWEEP_WARMUP, e, use_graph=use_graph)
        ctx.sync()
        t0 = time.perf_counter()
        model.decode(args.sweep_steps, e, use_graph=use_graph)
        ctx.sync()
        dt_e = time.perf_counter() - t0
        eb = profiled_steps(ctx, model, SWEEP_COUNT, e)
        pos_e = pos_now + SWEEP_WARMUP + args.sweep_steps // 2
        tab = group_table(ctx, cfg, pos_now + SWEEP_WARMUP + args.sweep_steps + (SWEEP_COUNT + 1) / 2)
        if str(e) in map(str, FFN_EFFORTS):
            ffn_model[str(e)] = ffn_of(tab)
        bpt = eb / SWEEP_COUNT + per_token_fixed_bytes(cfg, pos_e)
        tps = args.sweep_steps / dt_e
        sweep[str(e)] = {"tok_s": round(tps, 2), "ms_per_token": round(dt_e / args.sweep_steps * 1e3, 4),
                         "bytes_per_token": round(bpt), "achieved_GBs": round(bpt * tps / 1e9, 1),
                         "frac": round(bpt * tps / 1e9 / HBM_PEAK_GBS, 4)}
        log(f"effort {e}: {tps:.1f} tok/s, {bpt / 1e9:.3f} GB/token -> {bpt * tps / 1e9:.0f} GB/s")
        pos_now += SWEEP_WARMUP + args.sweep_steps + SWEEP_COUNT
    ctx.set_walk_counting(True)
    cpu = None
    if not args.no_cpu_baseline:
        t = time.perf_counter()
        lo = args.prompt + args.warmup
        cpu = cpu_baseline(model, cfg, (lo, lo + args.steps), args.effort)
        log(f"cpu baseline: {cpu['value']} tok/s ({time.perf_counter() - t:.1f} s)")

    configs = None
    if not args.no_configs:
        t = time.perf_counter()
        c2 = config2(iam, ctx, model, cfg, FFN_EFFORTS, 64)
        c3 = config3(ctx, model, cfg, 0.25)
        c5, start5 = skew(ctx, model, cfg, n=8, warmup=2, count=1)
        c1 = config1(iam, ctx, 0.25, 200)
        configs = {
            "config1_bucketmul_4096": dict(c1, workload="W 4096x4096 fp16 N(0, 0.02^2), x N(0,1), seed 0, "
                                                        f"effort 0.25, {CONFIG1_COPIES} rotating copies of W"),
            "config2_ffn_block": {"standalone_api": c2, "model_decode": {k: v for k, v in ffn_model.items() if v},
                                  "workload": "RMSNorm + w1/w3 (SiLU gate) + w2, 14336x4096 / 4096x14336, "
                                              "layer matrices of the synthesized model"},
            "config3_layer_ctx2048": dict(c3, workload="one Mistral-7B layer at decode, effort 0.25, "
                                                       "KV cache N(0,1) fp16 to 2048 positions"),
            "config5_skew_sample": {"efforts": c5, "sequences": SKEW_SEQUENCES,
                                    "positions": f"{start5}..{start5 + 10}",
                                    "workload": "KV cache N(0,1), 1% of hidden channels x20, 2 warm-up + 8 "
                                                "timed graph steps + 1 counted step per sequence"},
        }
        log(f"configs 1, 2, 3, 5: {time.perf_counter() - t:.1f} s")

    out = {
        "metric": "decode tok/s @effort 0.25, Mistral-7B shape; bucketMul achieved HBM GB/s",
        "value": round(tok_s, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": acc_dtype(args),
        "dtype_detail": "fp16 weights, fp32 activations, %s products and accumulation" % args.acc,
        "data": "synthetic (random-init weights, random prompt ids)",
        "config": {"workload": "Mistral-7B-shape greedy decode, effort 0.25, 512-token prompt, "
                               "bucket-layout LM head, fp16 GQA KV cache (4096 positions)",
                   "effort": args.effort, "prompt_tokens": args.prompt, "layers": cfg["n_layers"],
                   "accumulation": args.acc, "graph_replay": use_graph,
                   "selection": "per row" if args.select_block == 1 else
                                f"blocks of {args.select_block} inputs below effort {args.select_below}",
                   "dim": cfg["dim"], "ffn_dim": cfg["ffn_dim"], "vocab": cfg["vocab"],
                   "global_batch": 1, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": "bucket_walk", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": walk_traffic(),
                     "bytes_per_launch": round(per_launch), "avg_launch_us": round(walk_avg_s * 1e6, 2),
                     "stream_read_GBs": round(stream_gbs, 1), "frac_of_stream": round(achieved / stream_gbs, 4)},
        "token_roofline": {"bytes_per_token": round(bytes_per_token), "achieved_GBs":
                           round(bytes_per_token * tok_s / 1e9, 1),
                           "frac": round(bytes_per_token * tok_s / 1e9 / HBM_PEAK_GBS, 4),
                           "frac_of_stream": round(bytes_per_token * tok_s / 1e9 / stream_gbs, 4)},
        "walk_groups": groups,
        "effort_sweep": sweep,
        "configs": configs,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    model.close()
    ctx.close()


if __name__ == "__main__":
    main()
