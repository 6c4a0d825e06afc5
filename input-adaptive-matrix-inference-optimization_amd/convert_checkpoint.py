#!/usr/bin/env python3
"""A Hugging Face Mistral checkpoint (safetensors shards) -> the reference's
weights directory, with every projection bucketized on the GPU.

The reference's front end does this with torch on the host:
- preprocess_layer_fixed_gpu.py: load_weight_to_fp16 (:91-108, bf16 -> fp32
  -> fp16), bucketize_fp16_packed (:110-242), save_bucketmul_binary
  (:245-282) and preprocess_layer (:285-330) for the seven projections of a
  layer;
- extract_layer_norms.py: the two RMSNorm gains of every layer, fp16 .npy;
- extract_embeddings.py: embed_tokens, the final norm and lm_head, fp16 .npy.

Here the safetensors files are parsed directly (an 8-byte header length, a
JSON header, raw little-endian tensors), bf16 is widened to fp32 exactly and
rounded to fp16 to nearest even (what torch's .to(float32).to(float16) does),
and each projection goes through iam_bucketize on the device, whose bytes
equal the reference bucketizer's.  Written, per layer L and projection
P in q, k, v, o, gate, up, down:
  layer{L}_{P}_proj_bucketmul_fp16_{buckets,stats,probes}.bin + _meta.txt
  layer{L}_input_layernorm.npy, layer{L}_post_attention_layernorm.npy
and embed_tokens.npy, norm_weight.npy, lm_head.npy.  --dense-copies also
writes the reference's layer{L}_{P}_proj_fp16.npy copies, which its C++ path
does not read.

Usage:
  python convert_checkpoint.py --model-dir /path/to/Mistral-7B-v0.3 --out weights/
"""
import argparse
import importlib.util
import json
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

PROJECTIONS = [("q", "self_attn.q_proj"), ("k", "self_attn.k_proj"), ("v", "self_attn.v_proj"),
               ("o", "self_attn.o_proj"), ("gate", "mlp.gate_proj"), ("up", "mlp.up_proj"),
               ("down", "mlp.down_proj")]


def _load_iam():
    spec = importlib.util.spec_from_file_location("iam", os.path.join(HERE, "iam.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


class SafeTensors:
    """Tensors of a checkpoint directory: model.safetensors.index.json and its
    shards, or a single model.safetensors.  Files are memory-mapped; a tensor
    is read when asked for."""

    def __init__(self, model_dir):
        self.files = {}     # shard path -> (memmap, data offset, header)
        self.where = {}     # tensor name -> shard path
        index = os.path.join(model_dir, "model.safetensors.index.json")
        if os.path.exists(index):
            with open(index) as f:
                wmap = json.load(f)["weight_map"]
            for name, shard in wmap.items():
                self.where[name] = os.path.join(model_dir, shard)
        else:
            single = os.path.join(model_dir, "model.safetensors")
            if not os.path.exists(single):
                raise FileNotFoundError(f"{model_dir}: no model.safetensors.index.json or model.safetensors")
            for name in self._header(single)[2]:
                if name != "__metadata__":
                    self.where[name] = single

    def _header(self, path):
        if path not in self.files:
            with open(path, "rb") as f:
                (n,) = struct.unpack("<Q", f.read(8))
                header = json.loads(f.read(n))
            self.files[path] = (np.memmap(path, dtype=np.uint8, mode="r"), 8 + n, header)
        return self.files[path]

    def names(self):
        return sorted(self.where)

    def __contains__(self, name):
        return name in self.where

    def fp16(self, name):
        """The tensor as fp16 (numpy float16, its own shape)."""
        if name not in self.where:
            raise KeyError(f"tensor {name} not in the checkpoint")
        mm, base, header = self._header(self.where[name])
        info = header[name]
        begin, end = info["data_offsets"]
        raw = np.asarray(mm[base + begin:base + end])
        shape = tuple(info["shape"])
        dt = info["dtype"]
        with np.errstate(over="ignore"):   # beyond the fp16 range is +-inf, as in torch
            if dt == "BF16":
                bits = raw.view("<u2").astype(np.uint32) << 16      # bf16 -> fp32 is exact
                out = bits.view(np.float32).astype(np.float16)     # then round to nearest even
            elif dt == "F16":
                out = raw.view("<f2").astype(np.float16)
            elif dt == "F32":
                out = raw.view("<f4").astype(np.float16)
            else:
                raise ValueError(f"tensor {name}: dtype {dt} is not BF16, F16 or F32")
        return out.reshape(shape)


def write_bucket_files(path, buckets, stats, probes, out_dim, in_dim):
    """The four files of one bucketized matrix in the reference's layout:
    raw little-endian fp16 arrays of shapes (1, R, C), (1, R, 4), (1, in) and
    the metadata text whose keys binary_loader.hpp reads."""
    R = in_dim * 16
    C = out_dim // 16
    buckets.astype("<u2").tofile(path + "_buckets.bin")
    stats.astype("<u2").tofile(path + "_stats.bin")
    probes.astype("<u2").tofile(path + "_probes.bin")
    nb, ns, npb = R * C * 2, R * 4 * 2, in_dim * 2
    with open(path + "_meta.txt", "w") as f:
        f.write("# BucketMul Weight Metadata\n# All arrays are FP16 (2 bytes per element)\n\n")
        f.write(f"buckets_shape: 1 {R} {C}\nstats_shape: 1 {R} 4\nprobes_shape: 1 {in_dim}\n")
        f.write(f"in_dim: {in_dim}\nout_dim: {out_dim}\nbsize: 16\ndtype: float16\n")
        f.write(f"\n# File sizes:\n# buckets: {nb} bytes ({nb / 2**20:.2f} MB)\n"
                f"# stats: {ns} bytes ({ns / 2**20:.2f} MB)\n# probes: {npb} bytes ({npb / 2**20:.2f} MB)\n")


def bucketize_on_device(ctx, W):
    """iam_bucketize of a dense fp16 (out_dim, in_dim) matrix: returns the
    buckets (R, C), stats (R, 4) and probes (in_dim,) as uint16."""
    out_dim, in_dim = W.shape
    if out_dim % 16:
        raise ValueError(f"out_dim {out_dim} is not a multiple of 16")
    R, C = in_dim * 16, out_dim // 16
    dw = ctx.upload(np.ascontiguousarray(W).view(np.uint16))
    db = ctx.empty(R * C, np.uint16)
    ds = ctx.empty(R * 4, np.uint16)
    dp = ctx.empty(in_dim, np.uint16)
    try:
        ctx.bucketize(dw, out_dim, in_dim, db, ds, dp)
        return db.read().reshape(R, C), ds.read().reshape(R, 4), dp.read()
    finally:
        for d in (dw, db, ds, dp):
            d.free()


def layer_count(st, model_dir):
    cfg = os.path.join(model_dir, "config.json")
    if os.path.exists(cfg):
        with open(cfg) as f:
            n = json.load(f).get("num_hidden_layers")
        if n:
            return int(n)
    n = 0
    while f"model.layers.{n}.input_layernorm.weight" in st:
        n += 1
    return n


def convert(model_dir, out_dir, layers=None, dense_copies=False, ctx=None, log=print):
    """Convert the checkpoint in model_dir into out_dir; returns the layers
    written.  ctx: an iam.Ctx to bucketize on (default: a new one on device 0)."""
    iam = _load_iam()
    own = ctx is None
    if own:
        ctx = iam.Ctx(0)
    try:
        st = SafeTensors(model_dir)
        os.makedirs(out_dir, exist_ok=True)
        if layers is None:
            layers = list(range(layer_count(st, model_dir)))
        for L in layers:
            for short, hf in PROJECTIONS:
                W = st.fp16(f"model.layers.{L}.{hf}.weight")
                if dense_copies:
                    np.save(os.path.join(out_dir, f"layer{L}_{short}_proj_fp16.npy"), W)
                b, s, p = bucketize_on_device(ctx, W)
                write_bucket_files(os.path.join(out_dir, f"layer{L}_{short}_proj_bucketmul_fp16"), b, s, p,
                                   W.shape[0], W.shape[1])
            for key, hf in (("input_layernorm", "input_layernorm"),
                            ("post_attention_layernorm", "post_attention_layernorm")):
                np.save(os.path.join(out_dir, f"layer{L}_{key}.npy"), st.fp16(f"model.layers.{L}.{hf}.weight"))
            log(f"layer {L}: 7 projections bucketized, norms written")
        embed = st.fp16("model.embed_tokens.weight")
        np.save(os.path.join(out_dir, "embed_tokens.npy"), embed)
        np.save(os.path.join(out_dir, "norm_weight.npy"), st.fp16("model.norm.weight"))
        # a checkpoint with tied embeddings has no lm_head: the embedding is the head
        lm = st.fp16("lm_head.weight") if "lm_head.weight" in st else embed
        np.save(os.path.join(out_dir, "lm_head.npy"), lm)
        log(f"embed_tokens {embed.shape}, norm_weight, lm_head {lm.shape} written")
        return layers
    finally:
        if own:
            ctx.close()


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--model-dir", required=True, help="directory with the safetensors shards (and config.json)")
    ap.add_argument("--out", required=True, help="output weights directory")
    ap.add_argument("--layers", default=None, help="comma-separated layer indices (default: all)")
    ap.add_argument("--dense-copies", action="store_true",
                    help="also write layer{L}_{P}_proj_fp16.npy, as the reference's script does")
    args = ap.parse_args(argv)
    layers = [int(v) for v in args.layers.split(",")] if args.layers else None
    convert(args.model_dir, args.out, layers, args.dense_copies,
            log=lambda *a: print(*a, file=sys.stderr, flush=True))


if __name__ == "__main__":
    main()
