"""iam_bucketmul_fused_noalloc (the matrix group with its scratch in the
library's fixed per-GPU array) against iam_bucketmul_fused on the same
inputs.

Both add exact fp64 products with atomics whose order depends on which
workgroups arrive first, and round each output once, so each output is
within an fp64 rounding of the correctly rounded sum: the two calls agree
within 1 fp32 ulp (usually bit for bit) and each within 1 ulp of the
oracle's fp64 sums; the normalized input is computed in a fixed fp32 order
and is bit-identical.  Checked on two calls in a row, the second with a
smaller group, a third with the LM-head shape, then a repeat of the first;
groups beyond the array's limits are refused with IAM_E_INVALID; and on a
fresh context the entry point allocates nothing (the context's allocated
bytes do not change and no dispatch scratch is created)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def ulps(a, b):
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


def make_matrix(ctx, iam, tid, out_dim, in_dim, keep):
    """A bucketized N(0, 0.02^2) fp16 matrix with compact stats; also the
    host copies the oracle reads (stats in the reference's 4-channel form)."""
    u16 = np.uint16
    W = ctx.empty(out_dim * in_dim, u16)
    ctx.gen_f16(3, tid, out_dim * in_dim, 0.0, 0.02, W)
    R, C = in_dim * 16, out_dim // 16
    b, s, p = ctx.empty(R * C, u16), ctx.empty(R * 4, u16), ctx.empty(max(in_dim, 4096), u16)
    ctx.bucketize(W, out_dim, in_dim, b, s, p)
    s3 = ctx.stats_compact(s, R)
    ctx.sync()
    host = (b.read().reshape(R, C), s.read().reshape(R, 4), p.read())
    W.free()
    s.free()
    keep += [b, s3, p]
    return iam.BucketMatrix(b.ptr, s3.ptr, p.ptr, R, C, 1, 0), host


@pytest.fixture(scope="module")
def mats(iam, ctx):
    keep = []
    m = {"q": make_matrix(ctx, iam, 900, 4096, 4096, keep),
         "k": make_matrix(ctx, iam, 901, 1024, 4096, keep),
         "v": make_matrix(ctx, iam, 902, 1024, 4096, keep),
         "lm": make_matrix(ctx, iam, 903, 32000, 4096, keep)}
    yield m
    for b in keep:
        b.free()


def run_both(ctx, group, effort, norm, seed):
    """The group through fused and through fused_noalloc: (outputs, x) of
    each, and the input the cutoff saw."""
    f32 = np.float32
    D = 4096
    h, x1, x2 = ctx.empty(D, f32), ctx.empty(D, f32), ctx.empty(D, f32)
    gain = ctx.empty(D, np.uint16)
    ctx.gen_f32(seed, 1, D, 0.0, 1.0, h)
    ctx.gen_f16(seed, 2, D, 1.0, 0.01, gain)
    if not norm:
        ctx.copy(x1, h, D * 4)
        ctx.copy(x2, h, D * 4)
    outs = [ctx.empty(m.bucket_cols * 16, f32) for m, _ in group]
    outs2 = [ctx.empty(m.bucket_cols * 16, f32) for m, _ in group]
    kw = dict(h=h, gain=gain) if norm else {}
    ctx.fused([m for m, _ in group], x1, D, outs, effort, **kw)
    ctx.fused_noalloc([m for m, _ in group], x2, D, outs2, effort, **kw)
    ctx.sync()
    res = ([o.read(f32) for o in outs], x1.read(f32), [o.read(f32) for o in outs2], x2.read(f32))
    for b in outs + outs2 + [h, x1, x2, gain]:
        b.free()
    return res


def test_noalloc_equals_fused_on_consecutive_calls(O, ctx, mats):
    prev = ctx.get_accumulation()
    ctx.set_accumulation("fp64")
    try:
        # first call: the q/k/v group with the RMSNorm input; second: one
        # 1024-output matrix at another effort (a smaller share of the
        # array); third: the LM-head shape; then the first again
        cases = [([mats["q"], mats["k"], mats["v"]], 0.25, True, 11),
                 ([mats["k"]], 0.5, False, 12),
                 ([mats["lm"]], 0.125, True, 13),
                 ([mats["q"], mats["k"], mats["v"]], 0.25, True, 11)]
        first = None
        for group, effort, norm, seed in cases:
            ya, xa, yb, xb = run_both(ctx, group, effort, norm, seed)
            assert np.array_equal(xa.view(np.uint32), xb.view(np.uint32))
            for a, b, (_, (hb, hs, hp)) in zip(ya, yb, group):
                assert ulps(a, b).max() <= 1, (len(group), effort)
                assert np.count_nonzero(b) > 0
                want, _, _, _ = O.bucketmul(xb, hs, hp, hb, effort)
                assert ulps(b, want).max() <= 1, (len(group), effort)
            if first is None:
                first = yb
        for a, b in zip(first, yb):
            assert ulps(a, b).max() <= 1
    finally:
        ctx.set_accumulation(prev)


def test_noalloc_refuses_groups_beyond_its_limits(iam, ctx, mats):
    f32 = np.float32
    x, y = ctx.empty(4096, f32), ctx.empty(8193 * 16, f32)
    q = mats["q"][0]
    try:
        big = iam.BucketMatrix(q.buckets, q.stats, q.probes, q.expert_rows, 8193, 1, 0)   # 131088 outputs
        with pytest.raises(iam.IamError) as e:
            ctx.fused_noalloc([big], x, 4096, [y], 0.25)
        assert e.value.code == -1 and "scratch limit" in str(e.value)
        with pytest.raises(iam.IamError) as e:
            ctx.fused_noalloc([mats["k"][0]] * 4, x, 4096, [y] * 4, 0.25)
        assert e.value.code == -1
    finally:
        x.free()
        y.free()


def test_noalloc_allocates_nothing(iam, O):
    """On a context of its own: after the caller's buffers are allocated,
    two no-allocation calls (the second smaller) leave the context's
    allocated bytes unchanged, create no dispatch scratch (the parity
    queries still report no dispatch) and give the oracle's results."""
    c2 = iam.Ctx(0)
    keep = []
    try:
        k, (hb, hs, hp) = make_matrix(c2, iam, 904, 1024, 4096, keep)
        v, (vb, vs, vp) = make_matrix(c2, iam, 905, 1024, 4096, keep)
        xin = O.gen_f32(21, 1, 4096, 0.0, 1.0)
        x = c2.upload(xin)
        y1, y2 = c2.empty(1024, np.float32), c2.empty(1024, np.float32)
        keep += [x, y1, y2]
        c2.sync()
        before = c2.mem_status()[0]
        c2.fused_noalloc([k, v], x, 4096, [y1, y2], 0.25)
        c2.sync()
        assert c2.mem_status()[0] == before
        assert ulps(y1.read(np.float32), O.bucketmul(xin, hs, hp, hb, 0.25)[0]).max() <= 1
        assert ulps(y2.read(np.float32), O.bucketmul(xin, vs, vp, vb, 0.25)[0]).max() <= 1
        c2.fused_noalloc([v], x, 4096, [y1], 0.5)
        c2.sync()
        assert c2.mem_status()[0] == before
        assert ulps(y1.read(np.float32), O.bucketmul(xin, vs, vp, vb, 0.5)[0]).max() <= 1
        with pytest.raises(iam.IamError) as e:
            c2.dispatch_info(0)
        assert e.value.code == iam.IAM_E_STATE
    finally:
        for b in keep:
            b.free()
        c2.close()
