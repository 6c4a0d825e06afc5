#!/usr/bin/env python3
"""Write golden vectors for the bucket-layout producer.

The reference's bucketize_fp16_packed (preprocess_layer_fixed_gpu.py:110-242)
is the only function on the path whose exact output no closed form pins: its
tie order comes from torch.argsort(descending=True) (:170) and its probe and
stats means from numpy float32 summation orders (:154, :213).  This script
imports that one function from the reference checkout, runs it on small seeded
matrices, and stores inputs and outputs as data in bucketize_fixtures.npz.
It runs in the build container only; the fixtures travel, the reference does
not.

    python tests/golden/make_fixtures.py /root/reference
"""
import json
import os
import sys

import numpy as np


def cases():
    rng = np.random.default_rng(0)
    out = {}
    # plain Gaussian, bucket count 2 (8-accumulator branch of the pairwise sum)
    out["g64x32"] = (rng.normal(0, 0.02, size=(64, 32))).astype(np.float16)
    # heavy ties: values from a tiny set, both signs, zeros and negative zeros
    vals = np.array([0.0, -0.0, 0.5, -0.5, 0.25, -0.25, 1.0, -1.0], dtype=np.float16)
    out["ties48x48"] = rng.choice(vals, size=(48, 48)).astype(np.float16)
    # exact-magnitude ties inside otherwise random buckets
    w = rng.normal(0, 0.02, size=(32, 24)).astype(np.float16)
    w[1::4, :] = -w[0::4, :]
    w[2::8, :] = w[0::8, :]
    out["mixties32x24"] = w
    # 200 buckets: the recursive branch of numpy's pairwise sum (n > 128)
    out["g3200x8"] = rng.normal(0, 0.02, size=(3200, 8)).astype(np.float16)
    # LM-head width: 2000 buckets
    out["g32000x2"] = rng.normal(0, 0.02, size=(32000, 2)).astype(np.float16)
    # subnormal and large magnitudes
    w = rng.normal(0, 1e-5, size=(16, 16)).astype(np.float16)
    w[:, :4] = rng.normal(0, 100.0, size=(16, 4)).astype(np.float16)
    out["range16x16"] = w
    out["orderdisc3200x7"] = order_discriminating_columns()
    return out


def order_discriminating_columns():
    """Columns whose fp16 probes or stats differ between float32 sequential,
    float32 pairwise and float64 summation.  With N(0, 0.02^2) weights the
    float32 partial sums are exact, so log-uniform magnitudes are used to make
    the accumulation order visible after fp16 rounding."""
    rng = np.random.default_rng(7)
    out, ncol = 3200, 4096
    nb = out // 16
    mag = np.exp2(rng.uniform(-14, 4, size=(out, ncol)))
    sgn = rng.choice([-1.0, 1.0], size=(out, ncol))
    W = (mag * sgn).astype(np.float16)
    A = np.abs(W.astype(np.float32))
    seq = np.zeros(ncol, np.float32)
    for j in range(out):
        seq = seq + A[j]
    pw = np.add.reduce(np.ascontiguousarray(A.T), axis=1)
    dbl = A.astype(np.float64).sum(0)
    f16 = np.float16
    ps = (seq / np.float32(out)).astype(f16)
    pp = (pw / np.float32(out)).astype(f16)
    pd = (dbl / out).astype(f16)
    pcols = np.nonzero((ps != pp) | (ps != pd))[0]
    rows = np.ascontiguousarray((-np.sort(-A.T.reshape(ncol, nb, 16), axis=2, kind="stable"))
                                .transpose(0, 2, 1))
    s_pw = (np.add.reduce(rows, axis=2) / np.float32(nb)).astype(f16)
    sq = np.zeros((ncol, 16), np.float32)
    for b in range(nb):
        sq = sq + rows[:, :, b]
    s_sq = (sq / np.float32(nb)).astype(f16)
    s_d = (rows.astype(np.float64).sum(2) / nb).astype(f16)
    scols = np.nonzero(((s_pw != s_sq) | (s_pw != s_d)).any(1))[0]
    cols = np.unique(np.concatenate([pcols[:6], scols[:6]]))
    return np.ascontiguousarray(W[:, cols])


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path.insert(0, ref)
    import torch  # noqa: F401  (the reference module needs it)
    from preprocess_layer_fixed_gpu import bucketize_fp16_packed

    arrays = {}
    meta = {"numpy": np.__version__, "torch": torch.__version__, "cases": []}
    for name, W in cases().items():
        bm = bucketize_fp16_packed(W, bsize=16)
        arrays[f"{name}__W"] = W.view(np.uint16)
        arrays[f"{name}__buckets"] = np.ascontiguousarray(bm.buckets).view(np.uint16)
        arrays[f"{name}__stats"] = np.ascontiguousarray(bm.stats).view(np.uint16)
        arrays[f"{name}__probes"] = np.ascontiguousarray(bm.probes).view(np.uint16)
        meta["cases"].append({"name": name, "out_dim": int(W.shape[0]), "in_dim": int(W.shape[1]),
                              "buckets_shape": list(bm.buckets.shape),
                              "stats_shape": list(bm.stats.shape),
                              "probes_shape": list(bm.probes.shape)})
    here = os.path.dirname(os.path.abspath(__file__))
    np.savez_compressed(os.path.join(here, "bucketize_fixtures.npz"), **arrays)
    with open(os.path.join(here, "bucketize_fixtures.json"), "w") as f:
        json.dump(meta, f, indent=1)
    print("wrote", len(meta["cases"]), "cases")


if __name__ == "__main__":
    main()
