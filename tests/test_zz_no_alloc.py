"""iam_bucketmul_fused_noalloc (the matrix group with its scratch in the
library's fixed per-GPU array) against iam_bucketmul_fused on the same
inputs: bit-identical outputs and normalized input (fp64 accumulation rounds
each output once, so both equal the correctly rounded sums), on two calls in
a row, the second with a smaller group; then a repeat of the first call, and
groups beyond the array's limits refused with IAM_E_INVALID."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def make_matrix(ctx, iam, tid, out_dim, in_dim, keep):
    """A bucketized N(0, 0.02^2) fp16 matrix with compact stats."""
    u16 = np.uint16
    W = ctx.empty(out_dim * in_dim, u16)
    ctx.gen_f16(3, tid, out_dim * in_dim, 0.0, 0.02, W)
    R, C = in_dim * 16, out_dim // 16
    b, s, p = ctx.empty(R * C, u16), ctx.empty(R * 4, u16), ctx.empty(max(in_dim, 4096), u16)
    ctx.bucketize(W, out_dim, in_dim, b, s, p)
    s3 = ctx.stats_compact(s, R)
    ctx.sync()
    W.free()
    s.free()
    keep += [b, s3, p]
    return iam.BucketMatrix(b.ptr, s3.ptr, p.ptr, R, C, 1, 0)


def bits(buf, n):
    return buf.read(np.float32, n).view(np.uint32)


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
    """The group through fused and through fused_noalloc: (outputs, x) of each."""
    f32 = np.float32
    D = 4096
    h, x1, x2 = ctx.empty(D, f32), ctx.empty(D, f32), ctx.empty(D, f32)
    gain = ctx.empty(D, np.uint16)
    ctx.gen_f32(seed, 1, D, 0.0, 1.0, h)
    ctx.gen_f16(seed, 2, D, 1.0, 0.01, gain)
    if not norm:
        ctx.copy(x1, h, D * 4)
        ctx.copy(x2, h, D * 4)
    outs = [ctx.empty(m.bucket_cols * 16, f32) for m in group]
    outs2 = [ctx.empty(m.bucket_cols * 16, f32) for m in group]
    kw = dict(h=h, gain=gain) if norm else {}
    ctx.fused(group, x1, D, outs, effort, **kw)
    ctx.fused_noalloc(group, x2, D, outs2, effort, **kw)
    ctx.sync()
    res = ([bits(o, m.bucket_cols * 16) for o, m in zip(outs, group)], bits(x1, D),
           [bits(o, m.bucket_cols * 16) for o, m in zip(outs2, group)], bits(x2, D))
    for b in outs + outs2 + [h, x1, x2, gain]:
        b.free()
    return res


def test_noalloc_equals_fused_on_consecutive_calls(ctx, mats):
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
            assert np.array_equal(xa, xb)
            for a, b in zip(ya, yb):
                assert np.array_equal(a, b), (len(group), effort)
                assert np.count_nonzero(a) > 0
            if first is None:
                first = yb
        for a, b in zip(first, yb):
            assert np.array_equal(a, b)
    finally:
        ctx.set_accumulation(prev)


def test_noalloc_refuses_groups_beyond_its_limits(iam, ctx, mats):
    f32 = np.float32
    x, y = ctx.empty(4096, f32), ctx.empty(8193 * 16, f32)
    try:
        big = iam.BucketMatrix(mats["q"].buckets, mats["q"].stats, mats["q"].probes, mats["q"].expert_rows,
                               8193, 1, 0)   # 131088 outputs, past the 131072 limit
        with pytest.raises(iam.IamError) as e:
            ctx.fused_noalloc([big], x, 4096, [y], 0.25)
        assert e.value.code == -1 and "scratch limit" in str(e.value)
        with pytest.raises(iam.IamError) as e:
            ctx.fused_noalloc([mats["k"]] * 4, x, 4096, [y] * 4, 0.25)
        assert e.value.code == -1
    finally:
        x.free()
        y.free()
