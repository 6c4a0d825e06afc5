"""The reference's own fp32 forms through libiam.so, against the oracle:

- matmul16x32, the reference's dense fp16 LM head (aux.cl:454-490): the
  same fp32 operations in the same order, so bit-exact;
- the reference's KV cache layout (K and V repeated to every query head,
  fp32, model.hpp:97-98): the RoPE + append bit-exact, and its fp32
  attention (aux.cl:204-225, :370-384, :497-540) within 2e-6 of the largest
  output (the device's expf and the C library's may differ by one ulp;
  everything else is the same operations in the same order), bit-exact for
  one position (p = e / e = 1), NaN past the exp overflow as in the
  reference;
- the decode step with the dense LM head (iam_model_set_lm_dense): greedy
  tokens equal to the oracle model's with the same head, the head's logits
  bit-exact on the device's own normalized hidden state."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def ulps(a, b):
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


@pytest.mark.parametrize("rows,cols", [(32000, 4096), (1003, 4096), (77, 1000), (64, 16384), (5, 4100)])
def test_matmul_f16_dense_bit_exact(O, ctx, rows, cols):
    W = O.gen_f16(9, 700 + cols % 97, rows * cols, 0.0, 0.02).reshape(rows, cols)
    x = O.gen_f32(9, 701, cols, 0.0, 1.0)
    dw, dx, dy = ctx.upload(W), ctx.upload(x), ctx.empty(rows, np.float32)
    ctx.matmul_f16_dense(dw, dx, rows, cols, dy)
    got = dy.read()
    assert np.array_equal(got.view(np.uint32), O.matmul_f16_dense(W, x).view(np.uint32)), (rows, cols)
    for d in (dw, dx, dy):
        d.free()


def _caches(rng, max_ctx, n_heads, hd, n_fill):
    kc = np.zeros((max_ctx, n_heads, hd), np.float32)
    vc = np.zeros((max_ctx, n_heads, hd), np.float32)
    kc[:n_fill] = rng.standard_normal((n_fill, n_heads, hd), dtype=np.float32)
    vc[:n_fill] = rng.standard_normal((n_fill, n_heads, hd), dtype=np.float32)
    return kc, vc


def test_rope_kv_append_f32_and_attention(iam, O, ctx):
    """Append at a run of positions (split edges included) into the fp32
    repeated-head caches, then attention over 0..pos."""
    n_heads, n_kv, hd, max_ctx = 32, 8, 128, 2048
    rng = np.random.default_rng(41)
    table = iam.rope_table(1e6, hd, max_ctx)
    kc, vc = _caches(rng, max_ctx, n_heads, hd, max_ctx)
    dt, dkc, dvc = ctx.upload(table), ctx.upload(kc), ctx.upload(vc)
    dqr, dout = ctx.empty(n_heads * hd, np.float32), ctx.empty(n_heads * hd, np.float32)
    worst = 0
    for pos in (0, 1, 63, 64, 65, 700, 2047):
        q = rng.normal(0, 0.3, n_heads * hd).astype(np.float32)
        k = rng.normal(0, 1, n_kv * hd).astype(np.float32)
        v = rng.normal(0, 1, n_kv * hd).astype(np.float32)
        dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
        dpos = ctx.upload(np.array([pos], np.int32))
        ctx.rope_kv_append_f32(dq, dk, dv, dt, dpos, n_heads, n_kv, hd, max_ctx, dqr, dkc, dvc)
        qr, kr, vr = O.rope_kv_rep32(q, k, v, table[pos], n_heads, n_kv, hd)
        assert np.array_equal(dqr.read().view(np.uint32), qr.view(np.uint32)), pos
        kcache = dkc.read().reshape(max_ctx, n_heads, hd)
        vcache = dvc.read().reshape(max_ctx, n_heads, hd)
        assert np.array_equal(kcache[pos].ravel().view(np.uint32), kr.view(np.uint32)), pos
        assert np.array_equal(vcache[pos].ravel().view(np.uint32), vr.view(np.uint32)), pos
        ctx.attention_f32(dqr, dkc, dvc, dpos, n_heads, hd, max_ctx, dout)
        got = dout.read()
        want = O.attention_f32rep(qr, kcache, vcache, pos + 1, n_heads, hd)
        if pos == 0:
            # one position: p = e / e = 1 exactly, the output is the V row
            assert np.array_equal(got.view(np.uint32), vr.view(np.uint32))
        # an ulp of exp moves p by ~1e-7 relative; an output that cancels
        # (p0 v0 + p1 v1 of opposite signs) can then differ by many of its own
        # ulps, so the bar is on the absolute difference, relative to the
        # outputs' scale
        err = float(np.abs(got.astype(np.float64) - want).max())
        worst = max(worst, err)
        assert err <= 2e-6 * max(1.0, float(np.abs(want).max())), (pos, err)
        for d in (dq, dk, dv, dpos):
            d.free()
    print(f"  fp32 attention: largest difference from the oracle {worst:.2e}")
    for d in (dt, dkc, dvc, dqr, dout):
        d.free()


def test_attention_f32_long_context_and_overflow(O, ctx):
    """4096 positions (64 splits); then one score above log(FLT_MAX) makes
    that head NaN, as the reference's unshifted exp does, and leaves the
    others finite."""
    n_heads, hd, max_ctx = 8, 128, 4096
    rng = np.random.default_rng(42)
    kc, vc = _caches(rng, max_ctx, n_heads, hd, max_ctx)
    q = rng.normal(0, 0.3, n_heads * hd).astype(np.float32)
    dkc, dvc, dq = ctx.upload(kc), ctx.upload(vc), ctx.upload(q)
    dout = ctx.empty(n_heads * hd, np.float32)
    dpos = ctx.upload(np.array([max_ctx - 1], np.int32))
    ctx.attention_f32(dq, dkc, dvc, dpos, n_heads, hd, max_ctx, dout)
    want = O.attention_f32rep(q, kc, vc, max_ctx, n_heads, hd)
    got = dout.read()
    assert np.abs(got - want).max() <= 2e-6 * np.abs(want).max()
    # head 3, position 10: q . k / sqrt(128) = 89 > 88.72
    k2 = kc.copy()
    k2[10, 3, :] = 0.0
    k2[10, 3, 0] = 1.0
    q2 = q.copy()
    q2[3 * hd] = np.float32(89.0 * np.sqrt(np.float32(128.0)))
    dkc.write(k2)
    dq.write(q2)
    ctx.attention_f32(dq, dkc, dvc, dpos, n_heads, hd, max_ctx, dout)
    got = dout.read().reshape(n_heads, hd)
    want = O.attention_f32rep(q2, k2, vc, max_ctx, n_heads, hd).reshape(n_heads, hd)
    assert np.all(np.isnan(got[3])) and np.all(np.isnan(want[3]))
    others = [h for h in range(n_heads) if h != 3]
    assert np.all(np.isfinite(got[others]))
    for d in (dkc, dvc, dq, dout, dpos):
        d.free()


CFG = dict(n_layers=2, dim=4096, ffn_dim=4096, n_heads=32, n_kv_heads=8, head_dim=128, vocab=512,
           max_ctx=64, rope_theta=10000.0, norm_eps=1e-5)


@pytest.mark.parametrize("use_graph", [False, True])
def test_model_dense_lm_head(iam, O, ctx, use_graph):
    """The decode step with the reference's dense LM head: the device's
    logits equal the oracle's dense head on the device's own normalized
    hidden state bit for bit, and greedy tokens (the device picks them)
    equal the oracle model's with the same head."""
    m = iam.Model(ctx, iam.ModelConfig(**CFG))
    try:
        m.synthesize(0)
        lm = O.gen_f16(0, 900, CFG["vocab"] * CFG["dim"], 0.0, 0.02).reshape(CFG["vocab"], CFG["dim"])
        dlm = ctx.upload(lm)
        m.set_lm_dense(dlm)
        prompt = [5, 77, 300]
        n_new = 6
        toks = m.generate(prompt, n_new, 0.25, use_graph=use_graph)
        orc = O.OracleModel(CFG, m.read_tensor, lm_dense=lm)
        seq = list(prompt)
        for pos in range(len(prompt) + n_new - 1):
            lo = orc.forward(seq[pos], pos, 0.25)
            if pos >= len(prompt) - 1:
                seq.append(O.argmax(lo))
        assert list(toks) == seq[len(prompt):]
        # the last step's head on the device's own hidden state
        hn = m.read_tensor("hidden_norm", np.float32)
        want = O.matmul_f16_dense(lm, hn)
        assert np.array_equal(m.read_tensor("logits", np.float32).view(np.uint32), want.view(np.uint32))
        m.set_lm_dense(None)
        dlm.free()
    finally:
        m.close()
