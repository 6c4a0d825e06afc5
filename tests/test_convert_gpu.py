"""The checkpoint converter end to end: a one-layer Mistral-shaped
checkpoint in Hugging Face safetensors form (two shards and an index; bf16
projections and embeddings, an fp32 and an fp16 norm) -> the reference's
weights directory, bucketized on the GPU.

Checks: the bucket files' bytes equal the oracle bucketizer's (pinned by the
reference's own fixtures) on the fp16 the reference's front end would make;
the .npy files hold those fp16 values; greedy decode through the drop-in
binary on the converted directory gives the oracle model's tokens."""
import json
import os
import subprocess

import numpy as np
import pytest

from conftest import f32_to_bf16_bits, write_safetensors

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DROPIN = os.path.join(ROOT, "input-adaptive-matrix-inference-optimization_amd", "bin", "iam_dropin")
CFG = dict(n_layers=1, dim=4096, ffn_dim=4096, n_heads=32, n_kv_heads=8, head_dim=128, vocab=256,
           max_ctx=16, rope_theta=10000.0, norm_eps=1e-5)
HF = {"q": ("self_attn.q_proj", (4096, 4096)), "k": ("self_attn.k_proj", (1024, 4096)),
      "v": ("self_attn.v_proj", (1024, 4096)), "o": ("self_attn.o_proj", (4096, 4096)),
      "gate": ("mlp.gate_proj", (4096, 4096)), "up": ("mlp.up_proj", (4096, 4096)),
      "down": ("mlp.down_proj", (4096, 4096))}
MAT = {"q": "wq", "k": "wk", "v": "wv", "o": "wo", "gate": "w1", "up": "w3", "down": "w2"}


def bf16_to_f16(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float16)


@pytest.fixture(scope="module")
def converted(O, conv, ctx, tmp_path_factory):
    src = str(tmp_path_factory.mktemp("hf"))
    out = str(tmp_path_factory.mktemp("weights"))
    V, D = CFG["vocab"], CFG["dim"]
    shard1, shard2, f16 = {}, {}, {}
    for k, (short, (hf, shp)) in enumerate(HF.items()):
        bits = f32_to_bf16_bits(O.gen_f32(4, 700 + k, shp[0] * shp[1], 0.0, 0.02)).reshape(shp)
        (shard1 if k < 4 else shard2)[f"model.layers.0.{hf}.weight"] = ("BF16", shp, bits)
        f16[short] = bf16_to_f16(bits)
    g_in = (1.0 + 0.01 * O.gen_f32(4, 720, D, 0.0, 1.0)).astype(np.float32)        # fp32 in the file
    g_post = (1.0 + 0.01 * O.gen_f32(4, 721, D, 0.0, 1.0)).astype(np.float16)      # fp16 in the file
    shard1["model.layers.0.input_layernorm.weight"] = ("F32", (D,), g_in)
    shard1["model.layers.0.post_attention_layernorm.weight"] = ("F16", (D,), g_post)
    emb = f32_to_bf16_bits(O.gen_f32(4, 722, V * D, 0.0, 0.02)).reshape(V, D)
    fnorm = f32_to_bf16_bits(1.0 + 0.01 * O.gen_f32(4, 723, D, 0.0, 1.0))
    lm = f32_to_bf16_bits(O.gen_f32(4, 724, V * D, 0.0, 0.02)).reshape(V, D)
    shard1["model.embed_tokens.weight"] = ("BF16", (V, D), emb)
    shard2["model.norm.weight"] = ("BF16", (D,), fnorm)
    shard2["lm_head.weight"] = ("BF16", (V, D), lm)
    write_safetensors(os.path.join(src, "model-00001-of-00002.safetensors"), shard1)
    write_safetensors(os.path.join(src, "model-00002-of-00002.safetensors"), shard2)
    wmap = {n: "model-00001-of-00002.safetensors" for n in shard1}
    wmap.update({n: "model-00002-of-00002.safetensors" for n in shard2})
    with open(os.path.join(src, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wmap}, f)
    with open(os.path.join(src, "config.json"), "w") as f:
        json.dump({"num_hidden_layers": 1, "hidden_size": D}, f)
    layers = conv.convert(src, out, ctx=ctx, log=lambda *a: None)
    assert layers == [0]
    f16["attn_gain"], f16["ffn_gain"] = g_in.astype(np.float16), g_post
    f16["embed"], f16["final_gain"], f16["lm"] = bf16_to_f16(emb), bf16_to_f16(fnorm), bf16_to_f16(lm)
    return out, f16


def read_bucket_files(d, name):
    meta = {}
    for line in open(os.path.join(d, name + "_meta.txt")):
        if line.strip() and not line.startswith("#"):
            k, v = line.split(":", 1)
            meta[k.strip()] = v.split()
    _, R, C = map(int, meta["buckets_shape"])
    b = np.fromfile(os.path.join(d, name + "_buckets.bin"), "<u2").reshape(R, C)
    s = np.fromfile(os.path.join(d, name + "_stats.bin"), "<u2").reshape(R, 4)
    p = np.fromfile(os.path.join(d, name + "_probes.bin"), "<u2")
    return b, s, p, meta


@pytest.mark.parametrize("short", ["q", "k", "down"])
def test_bucket_files_match_oracle(O, converted, short):
    out, f16 = converted
    b, s, p, meta = read_bucket_files(out, f"layer0_{short}_proj_bucketmul_fp16")
    ob, os_, op = O.bucketize(f16[short].view(np.uint16))
    out_dim, in_dim = HF[short][1]
    assert meta["in_dim"] == [str(in_dim)] and meta["out_dim"] == [str(out_dim)]
    assert np.array_equal(b, ob) and np.array_equal(s, os_) and np.array_equal(p, op)


def test_npy_files_hold_the_fp16_values(converted):
    out, f16 = converted
    for fname, key in (("layer0_input_layernorm.npy", "attn_gain"),
                       ("layer0_post_attention_layernorm.npy", "ffn_gain"),
                       ("embed_tokens.npy", "embed"), ("norm_weight.npy", "final_gain"), ("lm_head.npy", "lm")):
        a = np.load(os.path.join(out, fname))
        assert a.dtype == np.float16 and np.array_equal(a.view(np.uint16), f16[key].view(np.uint16)), fname


def test_generate_from_converted_checkpoint(O, converted):
    out, f16 = converted
    t = {}
    for short, m in MAT.items():
        b, s, p, _ = read_bucket_files(out, f"layer0_{short}_proj_bucketmul_fp16")
        t[f"layer0.{m}.buckets"], t[f"layer0.{m}.stats"], t[f"layer0.{m}.probes"] = b, s, p
    t["layer0.attn_gain"], t["layer0.ffn_gain"] = f16["attn_gain"], f16["ffn_gain"]
    t["embed"], t["final_gain"] = f16["embed"], f16["final_gain"]
    lb, ls, lp = O.bucketize(f16["lm"].view(np.uint16))
    t["lm_head.buckets"], t["lm_head.stats"], t["lm_head.probes"] = lb, ls, lp
    prompt = [5, 77, 200, 13]
    n_new = 6
    assert os.path.exists(DROPIN), "bin/iam_dropin not built (run __graft_entry__.build())"
    r = subprocess.run([DROPIN, "generate", "-d", out, "-p", ",".join(map(str, prompt)), "-n", str(n_new),
                        "-e", "0.25", "--max-ctx", str(CFG["max_ctx"]), "--theta", "10000"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    toks = [int(v) for v in r.stdout.split("tokens:")[1].split("\n")[0].split()]
    # the drop-in model's default head: the reference's dense lm_head.npy (matmul16x32)
    orc = O.OracleModel(CFG, lambda name, dtype: np.ascontiguousarray(t[name]).view(dtype).ravel(),
                        lm_dense=f16["lm"].view(np.uint16))
    seq = list(prompt)
    for pos in range(len(prompt) + n_new - 1):
        lo = orc.forward(seq[pos], pos, 0.25)
        if pos >= len(prompt) - 1:
            seq.append(O.argmax(lo))
    assert toks == seq[len(prompt):]
