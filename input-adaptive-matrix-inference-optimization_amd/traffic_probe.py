#!/usr/bin/env python3
"""Workload for the HBM traffic counters of the bucket walk.

Runs a few eager decode steps of the Mistral-7B-shape model (the same launch
mix as bench.py: per layer q/k/v, o, w1/w3, w2 walks, plus the LM head) and
one device-to-device copy of a known size for the counter calibration.  Run
it under `rocprofv3 --pmc FETCH_SIZE` and again under `--pmc WRITE_SIZE`, then
summarize with counter_summary.py.  Prints one JSON line with the walk's
algorithmic bytes (2 * selected rows * bucket columns, counted on the device)
per launch and the copy size.
"""
import argparse
import importlib.util
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--prompt", type=int, default=8)
    ap.add_argument("--steps", type=int, default=4)
    ap.add_argument("--effort", type=float, default=0.25)
    ap.add_argument("--copy-mib", type=int, default=256)
    args = ap.parse_args()
    spec = importlib.util.spec_from_file_location("iam", os.path.join(HERE, "iam.py"))
    iam = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(iam)
    cfg = dict(n_layers=args.layers, dim=4096, ffn_dim=14336, n_heads=32, n_kv_heads=8, head_dim=128,
               vocab=32000, max_ctx=1024, rope_theta=10000.0, norm_eps=1e-5)
    ctx = iam.Ctx(0)
    model = iam.Model(ctx, iam.ModelConfig(**cfg))
    model.synthesize(0)
    prompt = np.random.default_rng(0).integers(0, cfg["vocab"], args.prompt).astype(np.int32)
    model.generate(prompt, 1, args.effort, use_graph=False)
    ctx.sync()
    ctx.walk_counters(reset=True)
    model.decode(args.steps, args.effort, use_graph=False)
    ctx.sync()
    wbytes, wrows, wmats = ctx.walk_counters(reset=True)
    launches_per_step = 4 * args.layers + 1
    nbytes = args.copy_mib << 20
    a, b = ctx.alloc(nbytes), ctx.alloc(nbytes)
    ctx.copy(b, a, nbytes)
    ctx.sync()
    print(json.dumps({"walk_bytes_per_launch": wbytes / (args.steps * launches_per_step),
                      "walk_launches_timed": args.steps * launches_per_step,
                      "prefill_walk_launches": args.prompt * launches_per_step,
                      "copy_bytes": nbytes}), flush=True)
    a.free()
    b.free()
    model.close()
    ctx.close()


if __name__ == "__main__":
    main()
