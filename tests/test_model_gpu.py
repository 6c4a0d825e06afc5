"""The whole decode step (iam_model_*) against the oracle's model on a small
Mistral-shaped configuration: 2 layers, dim 4096 (32 heads x 128, 8 KV
heads), FFN 4096, vocabulary 512, 64 positions.

Bar: synthesized weights byte-identical to the oracle generator + bucketizer;
logits within 1e-3 relative L2 per step; greedy tokens identical, eager and
graph-replayed."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CFG = dict(n_layers=2, dim=4096, ffn_dim=4096, n_heads=32, n_kv_heads=8, head_dim=128, vocab=512,
           max_ctx=64, rope_theta=10000.0, norm_eps=1e-5)
def tid_layer(L, k):
    return 1000 + 16 * L + k


@pytest.fixture(scope="module")
def model(iam, ctx):
    cfg = iam.ModelConfig(**CFG)
    m = iam.Model(ctx, cfg)
    m.synthesize(0)
    yield m
    m.close()


def OracleModel(O, m):
    return O.OracleModel(CFG, m.read_tensor)


def test_synthesized_weights_match_oracle(O, model):
    for L, w, k, shape in [(0, "wk", 1, (1024, 4096)), (1, "w2", 6, (4096, 4096))]:
        W = O.gen_f16(0, tid_layer(L, k), shape[0] * shape[1], 0.0, 0.02).reshape(shape)
        b, s, p = O.bucketize(W)
        assert np.array_equal(model.read_tensor(f"layer{L}.{w}.buckets", np.uint16), b.ravel())
        assert np.array_equal(model.read_tensor(f"layer{L}.{w}.stats", np.uint16), s.ravel())
        assert np.array_equal(model.read_tensor(f"layer{L}.{w}.probes", np.uint16), p)
        assert np.array_equal(model.read_tensor(f"layer{L}.{w}.stats3", np.uint16), s[:, 3])
    assert np.array_equal(model.read_tensor("layer1.ffn_gain", np.uint16), O.gen_f16(0, tid_layer(1, 8), 4096, 1.0, 0.01))
    assert np.array_equal(model.read_tensor("embed", np.uint16), O.gen_f16(0, 10, 512 * 4096, 0.0, 0.02))
    assert np.array_equal(model.read_tensor("final_gain", np.uint16), O.gen_f16(0, 11, 4096, 1.0, 0.01))


@pytest.mark.parametrize("effort", [0.25, 1.0])
def test_forward_logits_and_greedy_match_oracle(O, ctx, model, effort):
    orc = OracleModel(O, model)
    model.reset_caches()
    prompt = O.gen_tokens(0, 99, 6, CFG["vocab"]).tolist()
    dlog = ctx.empty(CFG["vocab"], np.float32)
    toks_gpu, toks_orc = [], []
    seq = list(prompt)
    for pos in range(len(prompt) + 8):
        tok = seq[pos]
        model.forward(tok, pos, effort, dlog)
        lg = dlog.read()
        lo = orc.forward(tok, pos, effort)
        assert np.linalg.norm(lg - lo) / np.linalg.norm(lo) < 1e-3, pos
        ng, no = int(np.argmax(lg)), O.argmax(lo)
        if pos >= len(prompt) - 1:
            toks_gpu.append(ng)
            toks_orc.append(no)
            seq.append(ng)
    assert toks_gpu == toks_orc
    # the KV caches written along the way agree with the oracle's fp16 caches
    kc = model.read_tensor("kcache", np.uint16).view(np.float16).astype(np.float32)
    ko = orc.kc.view(np.float16).astype(np.float32)
    n = len(seq) - 1
    per_layer = CFG["max_ctx"] * 8 * 128
    for L in range(CFG["n_layers"]):
        a = kc[L * per_layer:L * per_layer + n * 1024]
        b = ko[L * per_layer:L * per_layer + n * 1024]
        assert np.linalg.norm(a - b) / np.linalg.norm(b) < 1e-3
    dlog.free()


def test_generate_graph_equals_eager_equals_oracle(O, model):
    orc = OracleModel(O, model)
    prompt = O.gen_tokens(0, 98, 5, CFG["vocab"]).tolist()
    n_new = 10
    model.reset_caches()
    eager = model.generate(prompt, n_new, 0.25, use_graph=False).tolist()
    model.reset_caches()
    graph = model.generate(prompt, n_new, 0.25, use_graph=True).tolist()
    model.reset_caches()
    graph2 = model.generate(prompt, n_new, 0.25, use_graph=True).tolist()   # replays the captured step
    assert eager == graph == graph2
    seq = list(prompt)
    want = []
    for pos in range(len(prompt) + n_new - 1):
        lo = orc.forward(seq[pos], pos, 0.25)
        if pos >= len(prompt) - 1:
            t = O.argmax(lo)
            want.append(t)
            seq.append(t)
    assert eager == want[:n_new]


def test_model_rejects_bad_config(iam, ctx):
    bad = dict(CFG)
    bad["dim"] = 2048
    bad["n_heads"] = 16
    with pytest.raises(iam.IamError):
        iam.Model(ctx, iam.ModelConfig(**bad))
