#!/usr/bin/env python3
"""Decode throughput of the Mistral-7B-shaped input-adaptive model on one GPU.

Workload: 32 layers, dim 4096, FFN 14336, 32 query / 8 KV heads of 128,
vocabulary 32000 with a bucket-layout LM head, fp16 GQA KV cache of 4096
positions, RoPE theta 10000; random-init synthetic weights N(0, 0.02^2)
bucketized on the GPU; a 512-token random-id prompt fed token by token; then
greedy decode at effort 0.25.  A step is one decode token (captured once as a
HIP graph and replayed).  `value` is decode tokens per second, timed with
the library's walk counting switched off (the reduce then skips adding up
the selected rows); the bytes per token come from steps run with it on.

roofline: the bucket walk kernel (the dominant one) -- the selected weight
bytes it streams (2 * S * bucket_cols per matrix, counted on the device) per
launch over its average duration, timed with HIP events stamped by each
walk's own dispatch on the library's stream during eager steps, against the
8 TB/s HBM peak (and, as `frac_of_stream`, against the streaming-read
bandwidth measured in the same run: 16-byte loads over 2 GiB, reported as
`stream_read_GBs`).  `traffic` is the walk's measured HBM bytes per launch
(FETCH_SIZE + WRITE_SIZE, calibrated on a copy of known size) read from the
committed counter summary profiles/walk_hbm_traffic_mistral7b_effort025.md.

effort_sweep: the same decode continued at efforts 1.0, 0.5, 0.125 and
0.05 (32 graph-replayed steps each, counting off): tok/s and the fraction of
8 TB/s for the bytes touched per token at that effort, the selected bytes
counted over the next SWEEP_COUNT steps (counting on).

cpu_baseline: the C oracle on one host core, timed on a bounded sample
(about 10 s: up to 256 decoder layers at consecutive positions, and one LM
head pass, of the same model at the same effort and context), scaled to
tokens per second of the 32-layer model.
"""
import argparse
import importlib.util
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "input-adaptive-matrix-inference-optimization_amd")

MISTRAL = dict(n_layers=32, dim=4096, ffn_dim=14336, n_heads=32, n_kv_heads=8, head_dim=128,
               vocab=32000, max_ctx=4096, rope_theta=10000.0, norm_eps=1e-5)
HBM_PEAK_GBS = 8000.0
SWEEP_EFFORTS = [1.0, 0.5, 0.25, 0.125, 0.05]   # the configs' efforts
SWEEP_WARMUP = 4
SWEEP_COUNT = 4   # steps with walk counting on after each timed run: bytes per token


def load_iam():
    spec = importlib.util.spec_from_file_location("iam", os.path.join(PKG, "iam.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def per_token_fixed_bytes(cfg, ctx_len):
    """Bytes a decode token reads besides the selected weight rows: compact
    stats (2 B per bucket row), probes, x, y of every sparse matmul, the fp16
    K and V of ctx_len positions per layer, and one embedding row."""
    D, F, V = cfg["dim"], cfg["ffn_dim"], cfg["vocab"]
    KVD = cfg["n_kv_heads"] * cfg["head_dim"]
    mats = [(D, D), (KVD, D), (KVD, D), (D, D), (F, D), (F, D), (D, F)]
    per_layer = 0
    for out_dim, in_dim in mats:
        per_layer += 2 * 16 * in_dim + 4 * in_dim + 2 * 4096 + 4 * out_dim
    per_layer += 2 * 2 * KVD * ctx_len
    lm = 2 * 16 * D + 4 * D + 2 * 4096 + 4 * V
    return cfg["n_layers"] * per_layer + lm + 2 * D


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "walk_hbm_traffic_mistral7b_effort025.md")


def walk_traffic():
    """HBM bytes per walk launch from the committed counter summary, or None."""
    try:
        for line in open(TRAFFIC_PROFILE):
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) == 2 and cells[0] == "traffic_bytes_per_launch":
                return float(cells[1])
    except OSError:
        pass
    return None


def cpu_baseline(iam, model, cfg, pos, effort, budget_s=12.0):
    """Time the oracle on a bounded sample of the same decode step."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as O

    c1 = dict(cfg)
    c1["n_layers"] = 1
    c1["max_ctx"] = cfg["max_ctx"]

    def read(name, dtype):
        if name in ("embed",):
            return np.zeros(16, dtype)          # unused: the sample feeds hidden states
        return model.read_tensor(name, dtype)

    orc = O.OracleModel(c1, read)
    # layer 0's KV cache as filled on the GPU, so attention spans the real context
    kv = cfg["max_ctx"] * cfg["n_kv_heads"] * cfg["head_dim"]
    p, n = model.tensor("kcache")
    orc.kc[:] = model.read_tensor("kcache", np.uint16)[:kv]
    orc.vc[:] = model.read_tensor("vcache", np.uint16)[:kv]
    h = model.read_tensor("hidden", np.float32)
    t_layer = []
    t0 = time.perf_counter()
    k = 0
    k_max = min(256, cfg["max_ctx"] - pos - 2)   # positions pos .. pos + k stay in the cache
    while time.perf_counter() - t0 < budget_s * 0.85 and k < k_max:
        t = time.perf_counter()
        h = orc.layer_forward(0, pos + k, effort, h)
        t_layer.append(time.perf_counter() - t)
        k += 1
    t = time.perf_counter()
    orc.forward(0, pos + k, effort, hidden_in=h)          # embed skipped, 1 layer + final norm + LM head
    t_model1 = time.perf_counter() - t
    tl = float(np.median(t_layer))
    t_lm = max(t_model1 - tl, 0.0)
    per_token = cfg["n_layers"] * tl + t_lm
    return {"value": round(1.0 / per_token, 4), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"C oracle, 1 thread: {k} decoder layers at positions {pos}..{pos + k - 1} "
                      f"(median {tl * 1e3:.0f} ms/layer) + 1 final-norm/LM-head pass "
                      f"({t_lm * 1e3:.0f} ms), effort {effort}, scaled to {cfg['n_layers']} layers"}


CONFIG1_COPIES = 40   # 40 x 32 MB of buckets: past the 256 MB Infinity Cache


def run_config1(args, iam, ctx):
    """Config 1 of the workload set (`--config1`): one 4096x4096 bucketMul at
    effort 0.25, W ~ N(0, 0.02^2) bucketized on the GPU, x ~ N(0, 1), seed 0.
    Timed as the decode step runs a matrix group (iam_bucketmul_fused: input,
    cutoff, selection and walk in one launch, the reduce in a second) and as
    the reference's calcDispatch + mul (multi: a cutoff launch, the walk, the
    reduce).  CONFIG1_COPIES copies of the bucketized matrix are used in
    turn, so none is in the Infinity Cache when it is read again; kernel
    durations come from per-dispatch events.  Bytes per call:
    2*S*C + 2*R + 4*in + 2*4096 + 4*m (selected rows, one stats value per row,
    x, probes, y)."""
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
    reps = args.config1_reps
    res = {}
    for mode in ("fused", "multi"):
        def call(m):
            if mode == "fused":
                ctx.fused([m], x, in_dim, [y], args.effort)
            else:
                ctx.multi([m], [x], [in_dim], [y], args.effort)
        for m in mats:
            call(m)
        ctx.sync()
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
        for name in ("bucket_cutoff", "bucket_walk", "bucket_reduce"):
            ms, calls = ctx.kernel_stat(name)
            if calls:
                parts[name.split("_")[1] + "_us"] = round(ms / calls * 1e3, 2)
                t_ms += ms / reps
        S = rows / reps
        B = 2 * S * C + 2 * R + 4 * in_dim + 2 * 4096 + 4 * out_dim
        res[mode] = dict(time_us=round(t_ms * 1e3, 2), **parts, selected_rows=round(S),
                         bytes_per_call=round(B), achieved_GBs=round(B / (t_ms * 1e-3) / 1e9, 1))
        log(f"config 1, {mode}: {t_ms * 1e3:.2f} us per call ({parts}), S = {S:.0f}, "
            f"{B / 1e6:.2f} MB -> {B / (t_ms * 1e-3) / 1e9:.0f} GB/s")
    stream_gbs = ctx.read_bandwidth(2 << 30, 10)
    for d in bufs + [x, y]:
        d.free()
    f = res["fused"]
    out = {
        "metric": "config 1: one 4096x4096 bucketMul at effort 0.25 (cutoff, selection, walk, reduce), "
                  "achieved GB/s of the selected rows + stats + x + probes + y",
        "value": f["achieved_GBs"], "unit": "GB/s", "n_gpus": 1, "steps": reps, "higher_is_better": True,
        "dtype": "f64" if args.acc == "fp64" else "f32", "data": "synthetic (seed 0)",
        "config": {"workload": "W 4096x4096 fp16 N(0, 0.02^2) in bucket layout, x 4096 fp32 N(0,1), "
                               f"effort {args.effort}, {CONFIG1_COPIES} rotating copies of W"},
        "frac": round(f["achieved_GBs"] / HBM_PEAK_GBS, 4),
        "frac_of_stream": round(f["achieved_GBs"] / stream_gbs, 4), "stream_read_GBs": round(stream_gbs, 1),
        "fused": res["fused"], "cutoff_launch": res["multi"],
    }
    print(json.dumps(out), flush=True)


SKEW_EFFORTS = [0.05, 1.0]
SKEW_SEQUENCES = 8


def run_skew(args, iam, ctx):
    """Skew stress on the same model (`--skew`): every layer's K and V filled
    with N(0,1) fp16 values for all 4096 positions, then SKEW_SEQUENCES
    sequences decoded back-to-back near the end of the context, each with its
    own seeded 1% of hidden channels (41 of 4096) scaled 20x at the
    embedding, at efforts 0.05 and 1.0 (graph-replayed steps)."""
    cfg = dict(MISTRAL)
    model = iam.Model(ctx, iam.ModelConfig(**cfg))
    model.synthesize(0)
    for name, tid in (("kcache", 9001), ("vcache", 9002)):
        ptr, nbytes = model.tensor(name)
        ctx.gen_f16(0, tid, nbytes // 2, 0.0, 1.0, ptr)
    n = args.skew_steps
    start = cfg["max_ctx"] - SWEEP_WARMUP - n - SWEEP_COUNT - 1
    if n < 1 or start < 1:
        sys.exit(f"--skew-steps {n} must be in [1, {cfg['max_ctx'] - SWEEP_WARMUP - SWEEP_COUNT - 2}]")
    rng = np.random.default_rng(5)
    res = {}
    for e in SKEW_EFFORTS:
        steps = counted = 0
        secs = 0.0
        wbytes = 0
        for sq in range(SKEW_SEQUENCES):
            scale = np.ones(cfg["dim"], np.float32)
            scale[rng.choice(cfg["dim"], cfg["dim"] // 100, replace=False)] = 20.0
            model.set_embed_scale(scale)
            model.set_position(start)
            model.write_tensor("token", np.array([int(rng.integers(0, cfg["vocab"]))], np.int32))
            ctx.set_walk_counting(False)
            model.decode(SWEEP_WARMUP, e)
            ctx.sync()
            t0 = time.perf_counter()
            model.decode(n, e)
            ctx.sync()
            secs += time.perf_counter() - t0
            steps += n
            ctx.set_walk_counting(True)
            ctx.walk_counters(reset=True)
            model.decode(SWEEP_COUNT, e)
            ctx.sync()
            b, _, _ = ctx.walk_counters(reset=True)
            wbytes += b
            counted += SWEEP_COUNT
        bpt = wbytes / counted + per_token_fixed_bytes(cfg, start + SWEEP_WARMUP + n // 2)
        tps = steps / secs
        res[str(e)] = {"tok_s": round(tps, 2), "ms_per_token": round(secs / steps * 1e3, 4),
                       "bytes_per_token": round(bpt), "achieved_GBs": round(bpt * tps / 1e9, 1),
                       "frac": round(bpt * tps / 1e9 / HBM_PEAK_GBS, 4)}
        log(f"skew, effort {e}: {tps:.1f} tok/s over {steps} steps, {bpt / 1e9:.3f} GB/token")
    out = {
        "metric": "skew stress: decode tok/s at efforts 0.05 and 1.0, context 4096, 8 sequences",
        "value": res[str(SKEW_EFFORTS[0])]["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": n,
        "warmup": SWEEP_WARMUP, "higher_is_better": True, "vs_baseline": None,
        "dtype": "f64" if args.acc == "fp64" else "f32",
        "dtype_detail": "fp16 weights, fp32 activations, %s products and accumulation" % args.acc,
        "data": "synthetic (random-init weights, N(0,1) KV cache, random token ids)",
        "config": {"workload": "Mistral-7B-shape decode, 1 percent of hidden channels x20 at the embedding, "
                               f"positions {start}..{start + SWEEP_WARMUP + n + SWEEP_COUNT - 1} of 4096",
                   "sequences": SKEW_SEQUENCES, "efforts": SKEW_EFFORTS},
        "efforts": res,
    }
    print(json.dumps(out), flush=True)
    model.close()


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
    ap.add_argument("--acc", choices=["fp64", "fp32"], default="fp64",
                    help="walk/attention accumulation (fp64: results equal the correctly rounded sums)")
    ap.add_argument("--eager", action="store_true",
                    help="launch every kernel from the host instead of replaying a captured graph")
    ap.add_argument("--skew", action="store_true",
                    help="run the skew stress (efforts 0.05 and 1.0 at context 4096, 8 sequences) instead")
    ap.add_argument("--skew-steps", type=int, default=32, help="timed decode steps per sequence and effort")
    ap.add_argument("--config1", action="store_true",
                    help="time config 1 instead (one 4096x4096 bucketMul, rotating copies of W)")
    ap.add_argument("--config1-reps", type=int, default=400, help="timed calls per mode of --config1")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        sys.exit(2)
    if args.profile_steps < 1:
        sys.exit("--profile-steps must be at least 1 (they give the walk's bytes and launch times)")
    cfg = dict(MISTRAL)
    sweep_efforts = [e for e in SWEEP_EFFORTS if e != args.effort] if args.sweep_steps > 0 else []
    total = (args.prompt + args.warmup + args.steps + args.profile_steps + 1
             + len(sweep_efforts) * (SWEEP_WARMUP + args.sweep_steps + SWEEP_COUNT))
    if total > cfg["max_ctx"]:
        sys.exit(f"prompt + warmup + steps + profile steps ({total}) exceed the KV capacity {cfg['max_ctx']}")

    iam = load_iam()
    ctx = iam.Ctx(0)
    ctx.set_accumulation(args.acc)
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
    ctx.set_walk_counting(True)
    dt = t1 - t0
    tok_s = args.steps / dt

    # per-kernel times: eager decode steps in which every kernel is launched
    # with a pair of HIP events stamped by its own dispatch on the library's
    # stream (hipExtLaunchKernelGGL), so each elapsed time is that kernel's
    # duration
    ctx.kernel_stats_reset()
    ctx.walk_counters(reset=True)
    ctx.profiling(True)
    model.decode(args.profile_steps, args.effort, use_graph=False)
    ctx.sync()
    ctx.profiling(False)
    pbytes, prows, pmats = ctx.walk_counters(reset=True)
    walk_ms, walk_calls = ctx.kernel_stat("bucket_walk")
    log(ctx.kernel_stats())
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

    # the same decode at the other efforts of the configs, continuing the
    # sequence: tok/s and the roofline fraction of the bytes touched per token
    sweep = {}
    pos_now = args.prompt + args.warmup + args.steps + args.profile_steps
    for e in sweep_efforts:
        ctx.set_walk_counting(False)
        model.decode(SWEEP_WARMUP, e, use_graph=use_graph)
        ctx.sync()
        t0 = time.perf_counter()
        model.decode(args.sweep_steps, e, use_graph=use_graph)
        ctx.sync()
        dt_e = time.perf_counter() - t0
        ctx.set_walk_counting(True)
        ctx.walk_counters(reset=True)
        model.decode(SWEEP_COUNT, e, use_graph=use_graph)
        ctx.sync()
        eb, _, _ = ctx.walk_counters(reset=True)
        pos_e = pos_now + SWEEP_WARMUP + args.sweep_steps // 2
        bpt = eb / SWEEP_COUNT + per_token_fixed_bytes(cfg, pos_e)
        tps = args.sweep_steps / dt_e
        sweep[str(e)] = {"tok_s": round(tps, 2), "ms_per_token": round(dt_e / args.sweep_steps * 1e3, 4),
                         "bytes_per_token": round(bpt), "achieved_GBs": round(bpt * tps / 1e9, 1),
                         "frac": round(bpt * tps / 1e9 / HBM_PEAK_GBS, 4)}
        log(f"effort {e}: {tps:.1f} tok/s, {bpt / 1e9:.3f} GB/token -> {bpt * tps / 1e9:.0f} GB/s")
        pos_now += SWEEP_WARMUP + args.sweep_steps + SWEEP_COUNT
    cpu = None
    if not args.no_cpu_baseline:
        t = time.perf_counter()
        cpu = cpu_baseline(iam, model, cfg, pos_now, args.effort)
        log(f"cpu baseline: {cpu['value']} tok/s ({time.perf_counter() - t:.1f} s)")

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
        "dtype": "f64" if args.acc == "fp64" else "f32",
        "dtype_detail": "fp16 weights, fp32 activations, %s products and accumulation" % args.acc,
        "data": "synthetic (random-init weights, random prompt ids)",
        "config": {"workload": "Mistral-7B-shape greedy decode, effort 0.25, 512-token prompt, "
                               "bucket-layout LM head, fp16 GQA KV cache (4096 positions)",
                   "effort": args.effort, "prompt_tokens": args.prompt, "layers": cfg["n_layers"],
                   "accumulation": args.acc, "graph_replay": use_graph,
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
        "effort_sweep": sweep,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    model.close()
    ctx.close()


if __name__ == "__main__":
    main()
