"""One Mistral-7B-shaped transformer layer (dim 4096, 32 query / 8 KV heads of
128, FFN 14336) composed from the C-ABI kernels in the order
TransformerLayer::forward chains them (transformer_layer.hpp:75-122), at
positions 0, 37, 500 and 2047 of a 2048-token fp16 KV cache prefilled with
random rows.

Every stage is checked with teacher forcing (the oracle receives the GPU's
own input to that stage): cutoff bits, selected-row counts, RMSNorm outputs
and the appended K/V rows are bit-exact, and with the default fp64
accumulation every other output is within 1 ulp of the oracle's (fp64
evaluation rounded once on both sides).  The untethered layer, each side on
its own intermediates, is checked too: with fp32 accumulation the two would
part at the first row whose importance lies within fp32 summation noise of a
cutoff, and fp64 accumulation removes that noise."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CFG = dict(n_layers=1, dim=4096, ffn_dim=14336, n_heads=32, n_kv_heads=8, head_dim=128, vocab=512,
           max_ctx=2048, rope_theta=10000.0, norm_eps=1e-5)
D, F, NH, NKV, HD, T = 4096, 14336, 32, 8, 128, 2048


def ulps(a, b):
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


def rel(a, b):
    b = np.asarray(b, np.float64)
    return np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30)


@pytest.fixture(scope="module")
def layer(iam, ctx):
    m = iam.Model(ctx, iam.ModelConfig(**CFG))
    m.synthesize(3)
    host = {}
    for w in ("wq", "wk", "wv", "wo", "w1", "w3", "w2"):
        s = m.read_tensor(f"layer0.{w}.stats", np.uint16)
        b = m.read_tensor(f"layer0.{w}.buckets", np.uint16)
        host[w] = (b.reshape(s.size // 4, -1), s.reshape(-1, 4), m.read_tensor(f"layer0.{w}.probes", np.uint16))
    host["attn_gain"] = m.read_tensor("layer0.attn_gain", np.uint16)
    host["ffn_gain"] = m.read_tensor("layer0.ffn_gain", np.uint16)
    yield m, host
    m.close()


def mul_stage(O, ctx, m, host, names, dx, dys, in_size, effort, forced):
    """One fused bucketMul launch group; with forced, check each product
    against the oracle on the GPU's own input."""
    mats = [m.matrix(f"layer0.{n}") for n in names]
    ctx.multi(mats, [dx] * len(names), [in_size] * len(names), dys, effort)
    if not forced:
        return
    x = dx.read()
    for k, (n, dy) in enumerate(zip(names, dys)):
        b, s, p = host[n]
        oy, ocut, omask, oS = O.bucketmul(x, s, p, b, effort)
        cut, S = ctx.dispatch_info(k)
        assert np.float32(cut).view(np.uint32) == np.float32(ocut).view(np.uint32), (n, cut, ocut)
        assert S == oS, n
        assert ulps(dy.read(), oy).max() <= 1, n


def run_layer(iam, O, ctx, m, host, h, pos, effort, forced):
    """The layer on the GPU; returns its output.  With forced,
    every stage is checked against the oracle fed the GPU's stage input."""
    eps = CFG["norm_eps"]
    kc_p, _ = m.tensor("kcache")
    vc_p, _ = m.tensor("vcache")
    rope_p, _ = m.tensor("rope")
    ga, _ = m.tensor("layer0.attn_gain")
    gf, _ = m.tensor("layer0.ffn_gain")
    e = lambda n: ctx.empty(n, np.float32)
    dh, dhn, dq, dk, dv, dqr, datt, do = ctx.upload(h), e(D), e(D), e(NKV * HD), e(NKV * HD), e(D), e(D), e(D)
    dg, du, ds, dd = e(F), e(F), e(F), e(D)
    dpos = ctx.upload(np.array([pos], np.int32))
    bufs = [dh, dhn, dq, dk, dv, dqr, datt, do, dg, du, ds, dd, dpos]

    ctx.rmsnorm_gain(dh, ga, D, eps, dhn)
    if forced:
        assert np.array_equal(dhn.read().view(np.uint32), O.rmsnorm_gain(h, host["attn_gain"], eps).view(np.uint32))
    mul_stage(O, ctx, m, host, ["wq", "wk", "wv"], dhn, [dq, dk, dv], D, effort, forced)
    if forced:
        kc_before = m.read_tensor("kcache", np.uint16).reshape(T, NKV, HD)
    ctx.rope_kv_append(dq, dk, dv, rope_p, dpos, NH, NKV, HD, T, dqr, kc_p, vc_p)
    kc = m.read_tensor("kcache", np.uint16).reshape(T, NKV, HD)
    vc = m.read_tensor("vcache", np.uint16).reshape(T, NKV, HD)
    if forced:
        table = O.rope_table(CFG["rope_theta"], HD, T)
        q, k, v = dq.read(), dk.read(), dv.read()
        assert np.array_equal(dqr.read().view(np.uint32), O.rope(q, table[pos], NH, HD).view(np.uint32))
        assert np.array_equal(kc[pos], O.f32_to_f16(O.rope(k, table[pos], NKV, HD)).reshape(NKV, HD))
        assert np.array_equal(vc[pos], O.f32_to_f16(v).reshape(NKV, HD))
        assert np.array_equal(np.delete(kc, pos, 0), np.delete(kc_before, pos, 0))
    ctx.attention(dqr, kc_p, vc_p, dpos, NH, NKV, HD, T, datt)
    if forced:
        want = O.attention_f16kv(dqr.read(), kc, vc, pos + 1, NH, NKV, HD)
        assert ulps(datt.read(), want).max() <= 1
    mul_stage(O, ctx, m, host, ["wo"], datt, [do], D, effort, forced)
    h_before = dh.read() if forced else None
    ctx.add_rmsnorm_gain(dh, do, gf, D, eps, dhn)
    if forced:
        h1 = h_before + do.read()
        assert np.array_equal(dh.read().view(np.uint32), h1.view(np.uint32))
        assert np.array_equal(dhn.read().view(np.uint32), O.rmsnorm_gain(h1, host["ffn_gain"], eps).view(np.uint32))
    mul_stage(O, ctx, m, host, ["w1", "w3"], dhn, [dg, du], D, effort, forced)
    ctx.silu_mul(dg, du, F, ds)
    if forced:
        assert ulps(ds.read(), O.silu_mul(dg.read(), du.read())).max() <= 1
    mul_stage(O, ctx, m, host, ["w2"], ds, [dd], F, effort, forced)
    h_before = dh.read() if forced else None
    ctx.add(dh, dd, D, dh)
    out = dh.read()
    if forced:
        assert np.array_equal(out.view(np.uint32), (h_before + dd.read()).view(np.uint32))
    for b in bufs:
        b.free()
    return out


def prefill(O, m, pos, seed):
    rng = np.random.default_rng(seed)
    kc = np.zeros((T, NKV, HD), np.float16)
    vc = np.zeros((T, NKV, HD), np.float16)
    kc[:pos] = rng.normal(0, 1, (pos, NKV, HD))
    vc[:pos] = rng.normal(0, 1, (pos, NKV, HD))
    m.write_tensor("kcache", kc.view(np.uint16))
    m.write_tensor("vcache", vc.view(np.uint16))
    return kc.view(np.uint16), vc.view(np.uint16)


@pytest.mark.parametrize("pos,effort", [(0, 0.25), (37, 0.25), (2047, 0.25), (2047, 1.0), (500, 0.05)])
def test_layer_teacher_forced(iam, O, ctx, layer, pos, effort):
    m, host = layer
    prefill(O, m, pos, pos)
    h = O.gen_f32(0, 300 + pos, D, 0.0, 1.0)
    run_layer(iam, O, ctx, m, host, h, pos, effort, forced=True)


def test_layer_untethered(iam, O, ctx, layer, capsys):
    """The layer output against orc_layer_forward on the same input and cache
    (oracle.c restates transformer_layer.hpp:75-122), each side running on
    its own intermediates."""
    m, host = layer
    pos = 2047
    kc, vc = prefill(O, m, pos, 11)
    h = O.gen_f32(0, 400, D, 0.0, 1.0)
    out = run_layer(iam, O, ctx, m, host, h, pos, 0.25, forced=False)
    orc = O.OracleModel(CFG, m.read_tensor)
    orc.kc[:] = kc.ravel()
    orc.vc[:] = vc.ravel()
    want = orc.layer_forward(0, pos, 0.25, h)
    r = rel(out, want)
    with capsys.disabled():
        print(f"\n  untethered layer output rel L2 vs oracle at pos {pos}: {r:.3e}, max ulps {ulps(out, want).max()}")
    assert ulps(out, want).max() <= 2
