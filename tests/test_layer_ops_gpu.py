"""Layer kernels, the synthetic generator and the GPU bucketizer against the
oracle (through libiam.so)."""
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def ulps(a, b):
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


def rel(a, b):
    b = np.asarray(b, np.float64)
    return np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30)


def test_generator_bytes_match_oracle(O, ctx):
    for tid, n, mean, sigma in [(1, 100003, 0.0, 0.02), (7, 4096, 1.0, 0.01), (3, 5000, 0.0, 1.0)]:
        d16 = ctx.empty(n, np.uint16)
        ctx.gen_f16(0, tid, n, mean, sigma, d16)
        assert np.array_equal(d16.read(), O.gen_f16(0, tid, n, mean, sigma))
        d32 = ctx.empty(n, np.float32)
        ctx.gen_f32(5, tid, n, mean, sigma, d32)
        assert np.array_equal(d32.read().view(np.uint32), O.gen_f32(5, tid, n, mean, sigma).view(np.uint32))
        d16.free()
        d32.free()


def _gpu_bucketize(ctx, W):
    out_dim, in_dim = W.shape
    dw = ctx.upload(np.ascontiguousarray(W, np.uint16))
    db = ctx.empty(out_dim * in_dim, np.uint16)
    ds = ctx.empty(in_dim * 16 * 4, np.uint16)
    dp = ctx.empty(in_dim, np.uint16)
    ctx.bucketize(dw, out_dim, in_dim, db, ds, dp)
    r = db.read(), ds.read(), dp.read()
    for d in (dw, db, ds, dp):
        d.free()
    return r


def test_gpu_bucketizer_matches_reference_fixtures(ctx):
    d = np.load(os.path.join(HERE, "golden", "bucketize_fixtures.npz"))
    meta = json.load(open(os.path.join(HERE, "golden", "bucketize_fixtures.json")))
    for case in meta["cases"]:
        name = case["name"]
        b, s, p = _gpu_bucketize(ctx, d[f"{name}__W"])
        assert np.array_equal(b, d[f"{name}__buckets"].ravel()), name
        assert np.array_equal(s, d[f"{name}__stats"].ravel()), name
        assert np.array_equal(p, d[f"{name}__probes"].ravel()), name


@pytest.mark.parametrize("shape", [(4096, 4096), (1024, 4096), (32000, 512), (4096, 1536)])
def test_gpu_bucketizer_matches_oracle(O, ctx, shape):
    W = O.gen_f16(3, 77, shape[0] * shape[1], 0.0, 0.02).reshape(shape)
    b, s, p = _gpu_bucketize(ctx, W)
    ob, os_, op = O.bucketize(W)
    assert np.array_equal(b, ob.ravel()) and np.array_equal(s, os_.ravel()) and np.array_equal(p, op)


def test_rmsnorm_and_add(O, ctx):
    x = O.gen_f32(0, 31, 4096, 0.0, 1.0)
    dlt = O.gen_f32(0, 32, 4096, 0.0, 0.5)
    g = O.gen_f16(0, 33, 4096, 1.0, 0.01)
    dx, dd, dg, do = ctx.upload(x), ctx.upload(dlt), ctx.upload(g), ctx.empty(4096, np.float32)
    ctx.rmsnorm_gain(dx, dg, 4096, 1e-5, do)
    got = do.read()
    want = O.rmsnorm_gain(x, g, 1e-5)
    # same fp32 operation order as the oracle (256 block sums, then a tree)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    ctx.add_rmsnorm_gain(dx, dd, dg, 4096, 1e-5, do)
    h = dx.read()
    assert np.array_equal(h.view(np.uint32), (x + dlt).view(np.uint32))
    assert np.array_equal(do.read().view(np.uint32), O.rmsnorm_gain(x + dlt, g, 1e-5).view(np.uint32))
    ctx.add(dx, dd, 4096, do)
    assert np.array_equal(do.read().view(np.uint32), (x + dlt + dlt).view(np.uint32))
    for d_ in (dx, dd, dg, do):
        d_.free()


def test_silu_mul(O, ctx):
    g = O.gen_f32(0, 34, 14336, 0.0, 2.0)
    u = O.gen_f32(0, 35, 14336, 0.0, 1.0)
    dg, du, do = ctx.upload(g), ctx.upload(u), ctx.empty(14336, np.float32)
    ctx.silu_mul(dg, du, 14336, do)
    # both evaluate in fp64 and round once
    assert ulps(do.read(), O.silu_mul(g, u)).max() <= 1
    for d_ in (dg, du, do):
        d_.free()


def test_rope_table_host_matches_oracle(iam, O):
    t = iam.rope_table(10000.0, 128, 300)
    assert np.array_equal(t.view(np.uint32), O.rope_table(10000.0, 128, 300).view(np.uint32))
    t = iam.rope_table(1e6, 128, 64)
    assert np.array_equal(t.view(np.uint32), O.rope_table(1e6, 128, 64).view(np.uint32))


def test_rope_kv_append_and_attention(iam, O, ctx):
    n_heads, n_kv, hd, max_ctx = 32, 8, 128, 640
    table = iam.rope_table(10000.0, hd, max_ctx)
    rng = np.random.default_rng(0)
    kc = rng.normal(0, 1, (max_ctx, n_kv, hd)).astype(np.float16)
    vc = rng.normal(0, 1, (max_ctx, n_kv, hd)).astype(np.float16)
    q = O.gen_f32(0, 40, n_heads * hd, 0.0, 0.3)
    k = O.gen_f32(0, 41, n_kv * hd, 0.0, 1.0)
    v = O.gen_f32(0, 42, n_kv * hd, 0.0, 1.0)
    dt = ctx.upload(table)
    dkc, dvc = ctx.upload(kc.view(np.uint16)), ctx.upload(vc.view(np.uint16))
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    dqr, dout = ctx.empty(n_heads * hd, np.float32), ctx.empty(n_heads * hd, np.float32)
    for pos in (0, 1, 63, 64, 255, 256, 511, 600, 639):
        dpos = ctx.upload(np.array([pos], np.int32))
        ctx.rope_kv_append(dq, dk, dv, dt, dpos, n_heads, n_kv, hd, max_ctx, dqr, dkc, dvc)
        qr = dqr.read()
        assert np.array_equal(qr.view(np.uint32), O.rope(q, table[pos], n_heads, hd).view(np.uint32))
        kcache = dkc.read().reshape(max_ctx, n_kv, hd)
        vcache = dvc.read().reshape(max_ctx, n_kv, hd)
        assert np.array_equal(kcache[pos], O.f32_to_f16(O.rope(k, table[pos], n_kv, hd)).reshape(n_kv, hd))
        assert np.array_equal(vcache[pos], O.f32_to_f16(v).reshape(n_kv, hd))
        ctx.attention(dqr, dkc, dvc, dpos, n_heads, n_kv, hd, max_ctx, dout)
        want = O.attention_f16kv(qr, kcache, vcache, pos + 1, n_heads, n_kv, hd)
        # fp64 evaluation on both sides, rounded once
        assert ulps(dout.read(), want).max() <= 1, pos
        ctx.set_accumulation("fp32")
        ctx.attention(dqr, dkc, dvc, dpos, n_heads, n_kv, hd, max_ctx, dout)
        ctx.set_accumulation("fp64")
        assert rel(dout.read(), want) < 1e-5, pos
        dpos.free()
    # a position past the capacity writes nothing
    before = dkc.read()
    dpos = ctx.upload(np.array([max_ctx], np.int32))
    ctx.rope_kv_append(dq, dk, dv, dt, dpos, n_heads, n_kv, hd, max_ctx, dqr, dkc, dvc)
    assert np.array_equal(dkc.read(), before)
    for d_ in (dt, dkc, dvc, dq, dk, dv, dqr, dout, dpos):
        d_.free()


def test_attention_long_context(iam, O, ctx):
    """Contexts of up to 8192 positions: the 64-position chunks dealt to at
    most 32 runs per head (1 chunk per run up to 2048 positions, then 2, ...,
    4 at 8192) and the last run's sum over the runs, at positions on and off
    chunk and run-length boundaries, with a 4-query-head GQA (heads paired
    per workgroup) and a 1:1 layout (one head per workgroup)."""
    rng = np.random.default_rng(3)
    for n_heads, n_kv, max_ctx, positions in ((32, 8, 8192, (1023, 2047, 2048, 2112, 4095, 4096, 8191)),
                                              (8, 8, 4160, (63, 4159))):
        hd = 128
        kc = rng.normal(0, 1, (max_ctx, n_kv, hd)).astype(np.float16)
        vc = rng.normal(0, 1, (max_ctx, n_kv, hd)).astype(np.float16)
        q = rng.normal(0, 0.3, n_heads * hd).astype(np.float32)
        dkc, dvc = ctx.upload(kc.view(np.uint16)), ctx.upload(vc.view(np.uint16))
        dq, dout = ctx.upload(q), ctx.empty(n_heads * hd, np.float32)
        for pos in positions:
            dpos = ctx.upload(np.array([pos], np.int32))
            ctx.attention(dq, dkc, dvc, dpos, n_heads, n_kv, hd, max_ctx, dout)
            want = O.attention_f16kv(q, kc.view(np.uint16), vc.view(np.uint16), pos + 1, n_heads, n_kv, hd)
            assert ulps(dout.read(), want).max() <= 1, (n_heads, n_kv, pos)
            dpos.free()
        for d_ in (dkc, dvc, dq, dout):
            d_.free()


def test_attention_overflow(O, ctx):
    """No maximum is subtracted (aux.cl:204-225): evaluated in fp64, a score
    above log(DBL_MAX) ~ 709.78 makes that head's outputs NaN and one just
    below (701.4) gives the oracle's result; in fp32 (IAM_ACC_FP32) the limit
    is log(FLT_MAX) ~ 88.72 (87.1 finite, 89.4 NaN).  The other head (all
    scores 0 over equal V rows) is 1.0 either way."""
    hd, n_tok, max_ctx = 128, 3, 64
    k = np.zeros((max_ctx, 1, hd), np.float16)
    k[1, 0, :] = 1.0
    v = np.ones((max_ctx, 1, hd), np.float16)
    dk, dv = ctx.upload(k.view(np.uint16)), ctx.upload(v.view(np.uint16))
    dpos, dout = ctx.upload(np.array([n_tok - 1], np.int32)), ctx.empty(2 * hd, np.float32)
    prev = ctx.get_accumulation()
    try:
        for acc, cases in (("fp64", ((62.0, True), (63.0, False))), ("fp32", ((7.7, True), (7.9, False)))):
            ctx.set_accumulation(acc)
            for qv, finite in cases:   # s = 128 qv / sqrt(128)
                q = np.full(2 * hd, qv, np.float32)
                q[hd:] = 0.0
                dq = ctx.upload(q)
                ctx.attention(dq, dk, dv, dpos, 2, 1, hd, max_ctx, dout)
                got = dout.read()
                assert np.all(np.isfinite(got[:hd])) == finite, (acc, qv)
                assert np.all(np.isnan(got[:hd])) == (not finite), (acc, qv)
                np.testing.assert_allclose(got[hd:], 1.0, rtol=1e-6)
                if acc == "fp64" and finite:
                    want = O.attention_f16kv(q, k.view(np.uint16), v.view(np.uint16), n_tok, 2, 1, hd)
                    assert ulps(got, want).max() <= 1
                dq.free()
    finally:
        ctx.set_accumulation(prev)
        for d_ in (dk, dv, dpos, dout):
            d_.free()


def test_embed_and_argmax(O, ctx):
    vocab, cols = 1000, 4096
    tab = O.gen_f16(0, 50, vocab * cols, 0.0, 0.02)
    dtab, dout = ctx.upload(tab), ctx.empty(cols, np.float32)
    for tok in (0, 7, 999):
        dt = ctx.upload(np.array([tok], np.int32))
        ctx.embed(dtab, cols, vocab, dt, dout)
        assert np.array_equal(dout.read(), O.f16_to_f32(tab[tok * cols:(tok + 1) * cols]))
        dt.free()
    dt = ctx.upload(np.array([vocab], np.int32))       # outside the vocabulary -> zeros
    ctx.embed(dtab, cols, vocab, dt, dout)
    assert not dout.read().any()
    v = np.array([1, 5, 3, 5, 5, -1] + [0] * 40000, np.float32)
    dv, di = ctx.upload(v), ctx.empty(1, np.int32)
    ctx.argmax(dv, len(v), di)
    assert di.read()[0] == 1
    w = O.gen_f32(0, 51, 32000, 0.0, 1.0)
    w[[100, 20000, 31999]] = w.max() + 1.0
    dw = ctx.upload(w)
    ctx.argmax(dw, 32000, di)
    assert di.read()[0] == 100 == O.argmax(w)
    for d_ in (dtab, dout, dt, dv, di, dw):
        d_.free()


def test_read_bandwidth(iam, ctx):
    """The streaming-read measurement: a plausible figure over 1 GiB (past
    the 256 MB Infinity Cache, so at most the 8 TB/s HBM peak), and bad
    arguments are refused."""
    g = ctx.read_bandwidth(1 << 30, 4)
    assert 500.0 < g < 8400.0, g
    with pytest.raises(iam.IamError):
        ctx.read_bandwidth(1000, 4)
    with pytest.raises(iam.IamError):
        ctx.read_bandwidth(1 << 30, 0)
