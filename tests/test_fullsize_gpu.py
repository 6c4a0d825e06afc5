"""The Mistral-7B-shape model the decode benchmark runs (32 layers, dim 4096,
32 query / 8 KV heads of 128, FFN 14336, vocabulary 32000, 4096 positions),
checked against the oracle stage by stage on the GPU's own intermediates
(teacher forcing, model.hpp:152-231, test_generation.cpp:231-276):

- attention stage of layer L: the oracle's norm, q/k/v bucketMul, RoPE,
  attention over the device's KV cache of L, o bucketMul and residual add,
  from the device's layer input; against the device's mid state and the K/V
  row the step appended;
- FFN stage of layer L: the oracle's norm, w1/w3 bucketMul, SiLU gate, w2
  bucketMul and residual add, from the device's mid state; against the
  device's layer output;
- LM head: the oracle's final norm + bucket-layout LM head on the device's
  final hidden state; against the device's logits, and the token the device
  picked against the oracle's first maximum.

Each stage starts from bit-identical inputs, so its cutoffs and selected
rows are the oracle's and the outputs differ only in the order of exact fp64
additions: at most 1 fp32 ulp (1 fp16 ulp for the K/V rows).

Covered: greedy decode from a 512-token prompt to position ~4094 with the
stages of layers 0, 15 and 31 checked near 512, at 2048 and near 4095
(effort 0.25), and the hidden state entering every layer checked at one
position; the FFN block through the fused path at efforts 1.0, 0.5, 0.25
and 0.125; the skew stress (1% of the hidden channels scaled 20x) at
positions 4055-4094 over a KV cache filled with N(0,1) values, for 8 channel
sets at efforts 0.05 and 1.0.

Untethered: after a device prefill, the oracle model takes a copy of the
device's KV cache and token and both sides decode greedily on their own for
8 steps (test_generation.cpp:231-276) at efforts 0.25 and 1.0: the picked
tokens must be identical at every step and the logits within 1 ulp of the
oracle's."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CFG = dict(n_layers=32, dim=4096, ffn_dim=14336, n_heads=32, n_kv_heads=8, head_dim=128, vocab=32000,
           max_ctx=4096, rope_theta=10000.0, norm_eps=1e-5)
KVD = CFG["n_kv_heads"] * CFG["head_dim"]
LAYERS = [0, 15, 31]


def ulps(a, b):
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


def ulps16(a, b):
    ia = np.asarray(a, np.uint16).astype(np.int64)
    ib = np.asarray(b, np.uint16).astype(np.int64)
    ia = np.where(ia & 0x8000, -(ia & 0x7FFF), ia)
    ib = np.where(ib & 0x8000, -(ib & 0x7FFF), ib)
    return np.abs(ia - ib)


@pytest.fixture(scope="module")
def big(iam, ctx):
    m = iam.Model(ctx, iam.ModelConfig(**CFG))
    m.synthesize(0)
    yield m
    m.close()


class Stages:
    """Oracle stages on one layer's device weights (read once per layer)."""

    def __init__(self, O, iam, ctx, model):
        self.O, self.iam, self.ctx, self.m = O, iam, ctx, model
        self.rope = O.rope_table(CFG["rope_theta"], CFG["head_dim"], CFG["max_ctx"])
        self.L = None
        self.w = {}

    def read_range(self, name, off, n, dtype):
        p, size = self.m.tensor(name)
        out = np.empty(n, dtype=dtype)
        assert off + out.nbytes <= size
        self.iam.check(self.iam.lib().iam_read(self.ctx.h, out.ctypes.data_as(C.c_void_p), C.c_void_p(p),
                                               C.c_size_t(off), C.c_size_t(out.nbytes)))
        return out

    def layer(self, L):
        if self.L != L:
            self.w = {}
            for w in ("wq", "wk", "wv", "wo", "w1", "w3", "w2"):
                s = self.m.read_tensor(f"layer{L}.{w}.stats", np.uint16).reshape(-1, 4)
                b = self.m.read_tensor(f"layer{L}.{w}.buckets", np.uint16).reshape(s.shape[0], -1)
                self.w[w] = (b, s, self.m.read_tensor(f"layer{L}.{w}.probes", np.uint16))
            self.w["attn_gain"] = self.m.read_tensor(f"layer{L}.attn_gain", np.uint16)
            self.w["ffn_gain"] = self.m.read_tensor(f"layer{L}.ffn_gain", np.uint16)
            self.L = L
        return self.w

    def bm(self, w, x, effort):
        b, s, p = w
        y, _, _, _ = self.O.bucketmul(x, s, p, b, effort)
        return y

    def attention(self, L, pos, effort, h_in):
        O, w = self.O, self.layer(L)
        hn = O.rmsnorm_gain(h_in, w["attn_gain"], CFG["norm_eps"])
        q, k, v = (self.bm(w[n], hn, effort) for n in ("wq", "wk", "wv"))
        qr = O.rope(q, self.rope[pos], CFG["n_heads"], CFG["head_dim"])
        kr = O.rope(k, self.rope[pos], CFG["n_kv_heads"], CFG["head_dim"])
        off = L * CFG["max_ctx"] * KVD * 2
        kc = self.read_range("kcache", off, (pos + 1) * KVD, np.uint16)
        vc = self.read_range("vcache", off, (pos + 1) * KVD, np.uint16)
        att = O.attention_f16kv(qr, kc, vc, pos + 1, CFG["n_heads"], CFG["n_kv_heads"], CFG["head_dim"])
        o = self.bm(w["wo"], att, effort)
        h_mid = (np.asarray(h_in, np.float32) + o).astype(np.float32)
        return h_mid, O.f32_to_f16(kr), O.f32_to_f16(v), kc[pos * KVD:], vc[pos * KVD:]

    def ffn(self, L, effort, h_mid):
        O, w = self.O, self.layer(L)
        hn = O.rmsnorm_gain(h_mid, w["ffn_gain"], CFG["norm_eps"])
        g = self.bm(w["w1"], hn, effort)
        u = self.bm(w["w3"], hn, effort)
        d = self.bm(w["w2"], O.silu_mul(g, u), effort)
        return (np.asarray(h_mid, np.float32) + d).astype(np.float32)

    def check_layer(self, L, pos, effort):
        m = self.m
        h_in = m.read_tensor(f"layer{L}.h_in", np.float32)
        h_mid = m.read_tensor(f"layer{L}.h_mid", np.float32)
        out = m.read_tensor(f"layer{L + 1}.h_in" if L + 1 < CFG["n_layers"] else "hidden", np.float32)
        want_mid, kr, vr, kdev, vdev = self.attention(L, pos, effort, h_in)
        assert ulps16(kdev, kr).max() <= 1, ("K row", L, pos, effort)
        assert ulps16(vdev, vr).max() <= 1, ("V row", L, pos, effort)
        assert ulps(h_mid, want_mid).max() <= 1, ("attention stage", L, pos, effort)
        want_out = self.ffn(L, effort, h_mid)
        assert ulps(out, want_out).max() <= 1, ("FFN stage", L, pos, effort)

    def check_head(self, effort, picked):
        """The device's logits and picked token against the oracle's final
        norm + LM head on the device's final hidden state."""
        O, m = self.O, self.m
        h = m.read_tensor("hidden", np.float32)
        hn = m.read_tensor("hidden_norm", np.float32)
        assert np.array_equal(hn.view(np.uint32),
                              O.rmsnorm_gain(h, m.read_tensor("final_gain", np.uint16), CFG["norm_eps"]).view(np.uint32))
        s = m.read_tensor("lm_head.stats", np.uint16).reshape(-1, 4)
        b = m.read_tensor("lm_head.buckets", np.uint16).reshape(s.shape[0], -1)
        y, _, _, _ = O.bucketmul(hn, s, m.read_tensor("lm_head.probes", np.uint16), b, effort)
        assert ulps(m.read_tensor("logits", np.float32), y).max() <= 1, ("LM head", effort)
        assert picked == O.argmax(y), ("token", effort)


def checked_step(st, effort, layers):
    """One device step (the device picks the next token) with its stages
    checked; returns the position it ran at."""
    m = st.m
    pos = int(m.read_tensor("pos", np.int32)[0])
    m.step_device(effort)
    st.ctx.sync()
    assert int(m.read_tensor("pos", np.int32)[0]) == pos + 1
    for L in layers:
        st.check_layer(L, pos, effort)
    st.check_head(effort, int(m.read_tensor("token", np.int32)[0]))
    return pos


def test_fullsize_every_layer_input(O, iam, ctx, big):
    """The hidden state entering each of the 32 layers at one position,
    against the oracle layer run on the device's input of the layer before
    (teacher forcing, layer by layer): within 1 ulp."""
    st = Stages(O, iam, ctx, big)
    big.reset_caches()
    prompt = O.gen_tokens(0, 92, 40, CFG["vocab"])
    big.generate(prompt, 1, 0.25, use_graph=True)
    pos = checked_step(st, 0.25, [])
    for L in range(CFG["n_layers"]):
        h_in = big.read_tensor(f"layer{L}.h_in", np.float32)
        h_mid = big.read_tensor(f"layer{L}.h_mid", np.float32)
        out = big.read_tensor(f"layer{L + 1}.h_in" if L + 1 < CFG["n_layers"] else "hidden", np.float32)
        want_mid = st.attention(L, pos, 0.25, h_in)[0]
        assert ulps(h_mid, want_mid).max() <= 1, ("attention stage", L)
        assert ulps(out, st.ffn(L, 0.25, h_mid)).max() <= 1, ("FFN stage", L)
    print(f"  every layer checked at position {pos}", flush=True)


def test_fullsize_synthesized_matrices_match_generator(O, big):
    """Spot check of the device synthesis at full size: layer 31's wk
    (buckets, stats, probes) equals the oracle generator + bucketizer."""
    W = O.gen_f16(0, 1000 + 16 * 31 + 1, 1024 * 4096, 0.0, 0.02).reshape(1024, 4096)
    b, s, p = O.bucketize(W)
    assert np.array_equal(big.read_tensor("layer31.wk.buckets", np.uint16), b.ravel())
    assert np.array_equal(big.read_tensor("layer31.wk.stats", np.uint16), s.ravel())
    assert np.array_equal(big.read_tensor("layer31.wk.probes", np.uint16), p)


def test_fullsize_decode_stages(O, iam, ctx, big):
    """Config 4 (+ config 2's FFN efforts, config 3's 2048-position layer):
    a 512-token random prompt, then greedy decode to position ~4094 at
    effort 0.25, the device's stages checked near 512 (the FFN at efforts
    1.0, 0.5, 0.25 and 0.125), at 2048 and near 4095."""
    st = Stages(O, iam, ctx, big)
    big.reset_caches()
    prompt = O.gen_tokens(0, 90, 512, CFG["vocab"])
    big.generate(prompt, 1, 0.25, use_graph=True)   # prefill; the device holds the picked token at 512
    for effort in (1.0, 0.5, 0.25, 0.125):
        pos = checked_step(st, effort, [0, 31] if effort != 0.25 else LAYERS)
        print(f"  checked position {pos} at effort {effort}", flush=True)
    pos = int(big.read_tensor("pos", np.int32)[0])
    big.decode(2048 - pos, 0.25, use_graph=True)
    pos = checked_step(st, 0.25, [15])
    print(f"  checked position {pos}", flush=True)
    big.decode(4092 - pos - 1, 0.25, use_graph=True)
    for _ in range(3):
        pos = checked_step(st, 0.25, LAYERS)
        print(f"  checked position {pos}", flush=True)
    assert pos == 4094


@pytest.mark.parametrize("effort", [0.05, 1.0])
def test_fullsize_skew_stages(O, iam, ctx, big, effort):
    """Config 5: 8 sequences, each with its own set of 1% hidden channels
    scaled 20x at the embedding, decoded for 2 steps at positions 4055-4094
    over a KV cache of N(0,1) values; the embedding row, the LM head and the
    picked token checked at every step, all stages of layers 0, 15 and 31 on
    the first step of the first and last sequences."""
    st = Stages(O, iam, ctx, big)
    big.reset_caches()
    rng = np.random.default_rng(5)
    n = CFG["n_layers"] * CFG["max_ctx"] * KVD
    big.write_tensor("kcache", rng.standard_normal(n, dtype=np.float32).astype(np.float16).view(np.uint16))
    big.write_tensor("vcache", rng.standard_normal(n, dtype=np.float32).astype(np.float16).view(np.uint16))
    try:
        for seq in range(8):
            scale = np.ones(CFG["dim"], np.float32)
            scale[np.random.default_rng(100 + seq).choice(CFG["dim"], CFG["dim"] // 100, replace=False)] = 20.0
            big.set_embed_scale(scale)
            start = 4055 + 5 * seq
            big.set_position(start)
            tok = int(O.gen_tokens(seq, 80, 1, CFG["vocab"])[0])
            big.write_tensor("token", np.array([tok], np.int32))
            for step in range(2):
                layers = LAYERS if step == 0 and seq in (0, 7) else []
                t_in = int(big.read_tensor("token", np.int32)[0])
                pos = checked_step(st, effort, layers)
                assert pos == start + step
                h0 = big.read_tensor("layer0.h_in", np.float32)
                row = O.f16_to_f32(st.read_range("embed", t_in * CFG["dim"] * 2, CFG["dim"], np.uint16))
                assert np.array_equal(h0.view(np.uint32), (row * scale).astype(np.float32).view(np.uint32))
            print(f"  sequence {seq} checked at positions {start}-{start + 1}", flush=True)
    finally:
        big.set_embed_scale(None)


@pytest.mark.parametrize("effort", [0.25, 1.0])
def test_fullsize_untethered_greedy(O, iam, ctx, big, effort):
    """test_generation.cpp:231-276 at the benchmarked shape with both sides
    running free: a device prefill of a 512-token prompt, then the oracle
    model takes the device's KV cache and picked token, and device and
    oracle each decode 8 greedy steps on their own intermediates.  Tokens
    identical at every step; logits within 1 ulp."""
    big.reset_caches()
    prompt = O.gen_tokens(0, 93, 512, CFG["vocab"])
    big.generate(prompt, 1, effort, use_graph=True)
    ctx.sync()
    pos = int(big.read_tensor("pos", np.int32)[0])
    tok = int(big.read_tensor("token", np.int32)[0])
    assert pos == 512
    orc = O.OracleModel(CFG, big.read_tensor)
    orc.kc[:] = big.read_tensor("kcache", np.uint16)
    orc.vc[:] = big.read_tensor("vcache", np.uint16)
    worst_ulps, worst_rel = 0, 0.0
    for step in range(8):
        lo = orc.forward(tok, pos, effort)
        big.step_device(effort)
        ctx.sync()
        lg = big.read_tensor("logits", np.float32)
        dtok = int(big.read_tensor("token", np.int32)[0])
        otok = O.argmax(lo)
        u = int(ulps(lg, lo).max())
        r = float(np.abs(lg.astype(np.float64) - lo).max() / np.abs(lo).max())
        worst_ulps, worst_rel = max(worst_ulps, u), max(worst_rel, r)
        print(f"  effort {effort} position {pos}: token {dtok} (oracle {otok}), logits within {u} ulps, "
              f"{r:.1e} of the largest", flush=True)
        assert dtok == otok, (effort, pos)
        assert u <= 1, (effort, pos, u, r)
        tok = otok
        pos += 1
    print(f"  effort {effort}: 8 free-running steps, largest logit difference {worst_ulps} ulps", flush=True)
