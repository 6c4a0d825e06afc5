"""bucketMul on the GPU (through libiam.so) against the CPU oracle.

Bar: the cutoff bits and the selected row set are bit-exact.  With the
default fp64 accumulation y equals the oracle's fp64-accumulated sums rounded
to fp32, up to 1 ulp where an fp64 rounding difference (the workgroups'
atomic additions come in any order) straddles an fp32 rounding boundary
(about 1e-7 of the outputs); with fp32 accumulation y is within 1e-5
relative L2.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

RTOL_L2 = 1e-3
_cache = {}


def ulps(a, b):
    """Per-element distance in fp32 units in the last place."""
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


def make_matrix(O, out_dim, in_dim, seed=0, tid=1):
    key = (out_dim, in_dim, seed, tid)
    if key not in _cache:
        W = O.gen_f16(seed, tid, out_dim * in_dim, 0.0, 0.02).reshape(out_dim, in_dim)
        _cache[key] = O.bucketize(W)
    return _cache[key]


def rel_l2(a, b):
    nb = np.linalg.norm(b)
    return np.linalg.norm(a.astype(np.float64) - b) / (nb if nb > 0 else 1.0)


def run_gpu(ctx, b, s, p, x, effort, in_size=None, expert_no=0, expert_rows=None, split=True, fused=None):
    """split: calc_dispatch + mul; else full_mul (both with the cutoff
    launch); fused (the iam module): the walk computes the cutoff itself
    (iam_bucketmul_fused)."""
    R = expert_rows if expert_rows is not None else b.shape[0]
    C = b.shape[1]
    in_size = in_size if in_size is not None else R // 16
    db, ds, dp, dx = ctx.upload(b), ctx.upload(s), ctx.upload(p), ctx.upload(x)
    dy = ctx.empty(16 * C, np.float32)
    if fused is not None:
        mat = fused.BucketMatrix(db.ptr, ds.ptr, dp.ptr, R, C, 4, 3)
        ctx.fused([mat], dx, in_size, [dy], effort, expert_no=expert_no)
    elif split:
        ctx.calc_dispatch(dx, ds, dp, expert_no, in_size, C, R, effort)
        ctx.mul(db, C, dy)
    else:
        ctx.full_mul(dx, ds, dp, db, expert_no, in_size, C, R, effort, dy)
    y = dy.read()
    walked = ctx.walk_count(0)
    cut, S = ctx.dispatch_info(0)
    rows = ctx.dispatch_rows(0)
    for d in (db, ds, dp, dx, dy):
        d.free()
    # the walk selects its rows itself: it must have taken the listed set's size
    assert walked == S, (walked, S)
    return y, cut, S, rows


def check_against_oracle(O, ctx, b, s, p, x, effort, block=1, **kw):
    """block: the oracle selects in blocks of that many inputs (the GPU's
    setting is the context's)."""
    y, cut, S, rows = run_gpu(ctx, b, s, p, x, effort, **kw)
    in_size = kw.get("in_size")
    expert_no = kw.get("expert_no", 0)
    R = kw.get("expert_rows") or b.shape[0]
    if in_size is None:
        in_size = R // 16
    q = O.effort_quantile(effort)
    ocut = O.find_cutoff(x, p, q, exp_no=expert_no)
    mask, oS = O.select_rows_block(x, s, ocut, R, in_size, block, exp_no=expert_no)
    bb = b.reshape(-1, b.shape[-1])
    oy = O.bucket_walk(bb, mask, x, R, exp_no=expert_no)
    assert np.float32(cut).view(np.uint32) == np.float32(ocut).view(np.uint32), (cut, ocut)
    assert S == oS
    assert np.array_equal(rows, np.nonzero(mask)[0].astype(np.uint32))
    assert rel_l2(y, oy) <= RTOL_L2
    if ctx.get_accumulation() == "fp64":
        d = ulps(y, oy)
        assert d.max() <= 1 and np.count_nonzero(d) <= max(2, y.size // 10000), (d.max(), np.count_nonzero(d))
    return y, oy, cut, S


@pytest.mark.parametrize("effort", [1.0, 0.5, 0.25, 0.125, 0.05])
def test_square_4096_parity(O, ctx, effort):
    """One 4096x4096 matrix (wq/wo shape), x ~ N(0,1), seed 0."""
    b, s, p = make_matrix(O, 4096, 4096)
    x = O.gen_f32(0, 2, 4096, 0.0, 1.0)
    y, oy, cut, S = check_against_oracle(O, ctx, b, s, p, x, effort)
    assert rel_l2(y, oy) < 1e-5       # fp32 accumulation in another order


def test_full_and_split_agree(O, ctx):
    b, s, p = make_matrix(O, 4096, 4096)
    x = O.gen_f32(0, 3, 4096, 0.0, 1.0)
    y1, c1, S1, r1 = run_gpu(ctx, b, s, p, x, 0.25, split=True)
    y2, c2, S2, r2 = run_gpu(ctx, b, s, p, x, 0.25, split=False)
    assert c1 == c2 and S1 == S2 and np.array_equal(r1, r2)
    assert rel_l2(y1, y2.astype(np.float64)) < 1e-6


@pytest.mark.parametrize("shape", [(14336, 4096), (1024, 4096), (32000, 4096)],
                         ids=["w1_14336x4096", "wk_1024x4096", "lmhead_32000x4096"])
def test_mistral_shapes_parity(O, ctx, shape):
    b, s, p = make_matrix(O, *shape, tid=5)
    x = O.gen_f32(0, 6, 4096, 0.0, 1.0)
    for effort in (0.25, 1.0):
        check_against_oracle(O, ctx, b, s, p, x, effort)


def test_down_projection_shape(O, ctx):
    """w2: in 14336, out 4096 (R = 229376).  The cutoff sees x[0:4096] only;
    selection covers all 14336 inputs."""
    b, s, p = make_matrix(O, 4096, 14336, tid=7)
    x = O.gen_f32(0, 8, 14336, 0.0, 0.3)
    x[4096:] *= 3.0      # the tail is invisible to the cutoff but still selected against it
    check_against_oracle(O, ctx, b, s, p, x, 0.25)


def test_zero_input_selects_all(O, ctx):
    b, s, p = make_matrix(O, 256, 4096, tid=9)
    x = np.zeros(4096, np.float32)
    y, cut, S, rows = run_gpu(ctx, b, s, p, x, 0.25)
    assert cut == 0.0 and S == 4096 * 16 and not y.any()


def test_skewed_channels(O, ctx):
    b, s, p = make_matrix(O, 4096, 4096)
    x = O.gen_f32(0, 10, 4096, 0.0, 1.0)
    rng = np.random.default_rng(0)
    x[rng.choice(4096, 41, replace=False)] *= 20.0
    for effort in (0.05, 1.0):
        check_against_oracle(O, ctx, b, s, p, x, effort)


def _cutoff_patterns():
    """x vectors that, with every probe 2^-6 (importance = fl(1e5 * |x| / 64),
    the values of the oracle's known-answer cases), drive the bisection
    through those paths while the walk still selects 11k-29k rows: name, x,
    effort, (rounds, converged) of the oracle's trace."""
    x = np.zeros(4096, np.float32)
    x[:1025], x[1025:] = 64e-4, 64e-5                # 1025 at 10, the rest at 1: hit in round 1
    yield "exact_hit_round1", x, 0.25, (1, 1)
    yield "constant", np.full(4096, 0.64, np.float32), 0.5, (1, 1)   # min == max
    yield "ramp_gap", np.arange(4096, dtype=np.float32) * np.float32(2.0 ** -14), 0.25, (11, 1)
    x = np.zeros(4096, np.float32)
    x[:1023], x[1023:1028] = 0.64, 0.32              # 1000 x1023, 500 x5: float midpoints stall
    yield "round_limit_ties", x, 0.25, (20, 0)
    x = np.zeros(4096, np.float32)
    x[:3000] = -0.64                                 # 3000 ties: the bracket never gets below 256 values
    yield "round_limit_wide_bracket", x, 0.25, (20, 0)


@pytest.mark.parametrize("pattern", [p[0] for p in _cutoff_patterns()])
def test_cutoff_edge_paths(O, iam, ctx, pattern):
    """The search's edge paths on the GPU, bit-exact against the oracle: the
    standalone cutoff kernel (calc_dispatch + mul, 4 waves, 16 importances
    per thread), and the walk's own search (iam_bucketmul_fused, 8 waves, 8
    per thread) on a 256-output matrix and on the LM-head shape."""
    name, x, effort, (rounds, conv) = next(p for p in _cutoff_patterns() if p[0] == pattern)
    probes = np.full(4096, 0x2400, np.uint16)
    _, tr = O.find_cutoff(x, probes, O.effort_quantile(effort), trace=True)
    assert (tr.rounds, tr.converged) == (rounds, conv)     # the pattern takes the intended path
    b, s, _ = make_matrix(O, 256, 4096, tid=9)
    check_against_oracle(O, ctx, b, s, probes, x, effort, split=True)
    check_against_oracle(O, ctx, b, s, probes, x, effort, fused=iam)
    b, s, _ = make_matrix(O, 32000, 4096, tid=5)
    check_against_oracle(O, ctx, b, s, probes, x, effort, fused=iam)


def _search_input(kind, rng):
    """(x, probes) of one importance pattern of the search: heavy-tailed,
    skewed, tied, constant, an outlier, tiny, with infinities or NaNs,
    overflowing midpoints, two adjacent floats, zero, bimodal, quantized."""
    n = 4096
    p = rng.normal(0, 0.02, n).astype(np.float16).view(np.uint16)
    const_p = np.full(n, 0x2400, np.uint16)          # 2^-6
    z = rng.normal(0, 1, n).astype(np.float32)
    x = z.copy()
    if kind == "skew":
        x[rng.choice(n, 41, replace=False)] *= 20.0
    elif kind == "ties":
        x, p = np.floor(np.abs(z) * 4).astype(np.float32), const_p
    elif kind == "constant":
        x, p = np.full(n, 0.64, np.float32), const_p
    elif kind == "outlier":
        x[7] = 1e4
    elif kind == "tiny":
        x = (z * np.float32(1e-38)).astype(np.float32)
    elif kind == "inf":
        x[::3] = np.inf
    elif kind == "nan":
        x[::5] = np.nan
    elif kind == "huge":
        x = (rng.random(n) * 1e36).astype(np.float32)
    elif kind == "adjacent":
        x = np.where(np.arange(n) < 2048, np.float32(0.64), np.nextafter(np.float32(0.64), np.float32(1)))
        x, p = x.astype(np.float32), const_p
    elif kind == "zero":
        x = np.zeros(n, np.float32)
    elif kind == "all_nan":
        x = np.full(n, np.nan, np.float32)
    elif kind == "nan_inf":
        x = np.where(np.arange(n) % 2 == 1, np.float32(np.nan), np.float32(np.inf)).astype(np.float32)
    elif kind == "few_nans":
        x[: 1 + int(rng.integers(0, 4))] = np.nan
    elif kind == "bimodal":
        x = (z + np.where(rng.random(n) < 0.5, 10.0, 0.0)).astype(np.float32)
    elif kind == "quantized":      # about three equal keys per value near any rank
        x, p = (np.round(z * 600) / 600).astype(np.float32), const_p
    return x, p


_SEARCH_KINDS = ["normal", "skew", "ties", "constant", "outlier", "tiny", "inf", "nan", "huge",
                 "adjacent", "zero", "all_nan", "nan_inf", "few_nans", "bimodal", "quantized"]


@pytest.mark.parametrize("kind", _SEARCH_KINDS)
def test_cutoff_search_kinds(O, iam, ctx, kind):
    """The cutoff search bit-exact against the oracle on 16 importance
    patterns at efforts that give the quantiles 0..3, 4092..4095 and the
    usual ones: the standalone cutoff kernel (4 waves, radix search) and the
    walk's own search (8 waves) on 256 and 32000 outputs; the selected row
    count matches too.  On the walk's windowed search these patterns take
    every route: the three smallest keys (quantile 0, effort 1), a listed
    small window (e.g. normal at the other extreme quantiles), the fine
    bins read directly (normal at 1023), the fine bins' keys gathered and
    ranked (quantized at 1023), and the radix search after a decline at the
    window (all_nan) or at the list (constant)."""
    rng = np.random.default_rng(100 + _SEARCH_KINDS.index(kind))
    x, p = _search_input(kind, rng)
    quants = [0, 1, 2, 3, 100, 1023, 2047, 3071, 3583, 3890, 4092, 4093, 4094, 4095]
    efforts = sorted({float(np.float32(1.0 - (q + 0.5) / 4095.0)) for q in quants} | {1.0, 0.0})
    mats = []
    for out_dim, tid in ((256, 9), (32000, 5)):
        b, s, _ = make_matrix(O, out_dim, 4096, tid=tid)
        db, ds = ctx.upload(b), ctx.upload(s)
        mats.append((b, s, db, ds))
    dp, dx = ctx.upload(p), ctx.upload(x)
    with np.errstate(all="ignore"):
        for effort in efforts:
            q = O.effort_quantile(effort)
            ocut = O.find_cutoff(x, p, q)
            for mi, (b, s, db, ds) in enumerate(mats):
                R, C = b.shape
                _, oS = O.select_rows(x, s, ocut, R, R // 16)
                runs = ["split", "fused"] if mi == 0 else ["fused"]
                for how in runs:
                    dy = ctx.empty(16 * C, np.float32)
                    if how == "split":
                        ctx.calc_dispatch(dx, ds, dp, 0, R // 16, C, R, effort)
                        ctx.mul(db, C, dy)
                    else:
                        ctx.fused([iam.BucketMatrix(db.ptr, ds.ptr, dp.ptr, R, C, 4, 3)], dx, R // 16, [dy], effort)
                    cut, S = ctx.dispatch_info(0)
                    assert np.float32(cut).view(np.uint32) == np.float32(ocut).view(np.uint32), \
                        (kind, effort, q, how, C, cut, ocut)
                    assert S == oS and ctx.walk_count(0) == S, (kind, effort, how, S, oS)
                    dy.free()
    for _, _, db, ds in mats:
        db.free()
        ds.free()
    dp.free()
    dx.free()


_HINT_KINDS = ["normal", "skew", "ties", "constant", "outlier", "tiny", "inf", "nan", "huge",
               "adjacent", "zero", "few_nans", "bimodal", "quantized"]


@pytest.mark.parametrize("kind", _HINT_KINDS)
def test_search_hints(O, iam, ctx, kind):
    """The walk's search started from a hint finds the oracle's cutoff bit
    for bit, whatever the hint: the exact cutoff and its neighbouring float
    (the window's centre on a key), 10% off (inside the window or at its
    edge), a factor 8 off (the window misses: the full search runs), and
    hints that are no hint (0, negative, NaN, +inf, -inf, tiny, huge); also
    the hint the previous call left, from a scaled input (as the next decode
    step finds it).  The selected row count and the walk's count match
    too."""
    rng = np.random.default_rng(300 + _HINT_KINDS.index(kind))
    x, p = _search_input(kind, rng)
    # ranks t = 4096 - quantile; the walk takes a hint for 64 <= t <= 4032
    quants = [0, 3, 64, 65, 1023, 3071, 3890, 4031, 4032, 4092, 4095]
    efforts = sorted({float(np.float32(1.0 - (q + 0.5) / 4095.0)) for q in quants} | {0.25})
    b, s, _ = make_matrix(O, 256, 4096, tid=9)
    R, C = b.shape
    db, ds, dp = ctx.upload(b), ctx.upload(s), ctx.upload(p)
    dy = ctx.empty(16 * C, np.float32)
    mat = iam.BucketMatrix(db.ptr, ds.ptr, dp.ptr, R, C, 4, 3)
    ctx.set_search_hints(True)
    try:
        with np.errstate(all="ignore"):
            for scale in (1.0, 1.03):
                xs = (x * np.float32(scale)).astype(np.float32)
                dx = ctx.upload(xs)
                for effort in efforts:
                    q = O.effort_quantile(effort)
                    ocut = np.float32(O.find_cutoff(xs, p, q))
                    _, oS = O.select_rows(xs, s, ocut, R, R // 16)
                    hints = [None, ocut, np.nextafter(ocut, np.float32(np.inf)), ocut * np.float32(1.1),
                             ocut * np.float32(0.9), ocut * np.float32(8), ocut / np.float32(8), 0.0, -1.0,
                             np.nan, np.inf, -np.inf, 1e-31, 2e30]
                    for h in hints:
                        if h is not None:      # None: the hint the previous call left
                            ctx.set_search_hint(0, float(h))
                        ctx.fused([mat], dx, R // 16, [dy], effort)
                        cut, S = ctx.dispatch_info(0)
                        assert np.float32(cut).view(np.uint32) == ocut.view(np.uint32), (kind, scale, effort, h, cut, ocut)
                        assert S == oS and ctx.walk_count(0) == S, (kind, scale, effort, h, S, oS)
                dx.free()
    finally:
        ctx.set_search_hints(False)
    for d in (db, ds, dp, dy):
        d.free()


@pytest.mark.parametrize("in_dim", [4096, 8192])
def test_fused_norm_input(O, iam, ctx, in_dim):
    """iam_bucketmul_fused with a norm input: x = RMSNorm(h) * gain is the
    oracle's bit for bit (inside the walk for 4096 inputs, a separate RMSNorm
    launch for 8192); cutoff, rows and y match the oracle on that x; two
    matrices share the input."""
    rng = np.random.default_rng(in_dim)
    h = rng.normal(0, 1.5, in_dim).astype(np.float32)
    gain = O.gen_f16(3, 50, in_dim, 1.0, 0.01)
    mats = [make_matrix(O, 256, in_dim, tid=60), make_matrix(O, 512, in_dim, tid=61)]
    want_x = O.rmsnorm_gain(h, gain, 1e-5)
    dh, dg, dx = ctx.upload(h), ctx.upload(gain), ctx.empty(max(in_dim, 4096), np.float32)
    bufs, descs, ys = [], [], []
    for b, s, p in mats:
        db, ds, dp = ctx.upload(b), ctx.upload(s), ctx.upload(p)
        bufs += [db, ds, dp]
        descs.append(iam.BucketMatrix(db.ptr, ds.ptr, dp.ptr, b.shape[0], b.shape[1], 4, 3))
        ys.append(ctx.empty(16 * b.shape[1], np.float32))
    ctx.fused(descs, dx, in_dim, ys, 0.25, h=dh, gain=dg, eps=1e-5)
    x = dx.read()[:in_dim]
    assert np.array_equal(x.view(np.uint32), want_x.view(np.uint32))
    for k, (b, s, p) in enumerate(mats):
        cut, S = ctx.dispatch_info(k)
        oy, ocut, omask, oS = O.bucketmul(x, s, p, b, 0.25, in_size=in_dim)
        assert np.float32(cut).view(np.uint32) == np.float32(ocut).view(np.uint32)
        assert S == oS and ctx.walk_count(k) == oS
        d = ulps(ys[k].read(), oy)
        assert d.max() <= 1 and np.count_nonzero(d) <= 2
    for d in bufs + ys + [dh, dg, dx]:
        d.free()


@pytest.mark.parametrize("out_dim", [16, 32, 48, 64, 80, 2048 + 16])
def test_narrow_and_ragged_columns(O, ctx, out_dim):
    """bucket_cols 1..129: the 2-byte load path (bucket_cols not a multiple of
    4), the 8-byte one, and partial last tiles."""
    b, s, p = make_matrix(O, out_dim, 4096, tid=11)
    x = O.gen_f32(0, 12, 4096, 0.0, 1.0)
    check_against_oracle(O, ctx, b, s, p, x, 0.25)


def test_in_size_skips_rows(O, ctx):
    b, s, p = make_matrix(O, 256, 4096, tid=13)
    x = O.gen_f32(0, 14, 4096, 0.0, 1.0)
    y, oy, cut, S = check_against_oracle(O, ctx, b, s, p, x, 0.5, in_size=3000)
    rows = ctx.dispatch_rows(0)
    assert rows.max() < 3000 * 16


def test_expert_offset(O, ctx):
    b0, s0, p0 = make_matrix(O, 256, 4096, tid=15)
    b1, s1, p1 = make_matrix(O, 256, 4096, tid=16)
    b = np.concatenate([b0, b1])
    s = np.concatenate([s0, s1])
    p = np.concatenate([p0, p1])
    x = O.gen_f32(0, 17, 4096, 0.0, 1.0)
    y, oy, cut, S = check_against_oracle(O, ctx, b, s, p, x, 0.25, expert_no=1,
                                         expert_rows=4096 * 16)
    y1, cut1, S1, _ = run_gpu(ctx, b1, s1, p1, x, 0.25)
    assert cut == cut1 and S == S1 and rel_l2(y, y1.astype(np.float64)) < 1e-6


def test_stats_channel_three_only(O, ctx):
    b, s, p = make_matrix(O, 256, 4096, tid=18)
    s2 = s.copy()
    s2[:, :3] = np.float16(60000.0).view(np.uint16)
    x = O.gen_f32(0, 19, 4096, 0.0, 1.0)
    y1, c1, S1, r1 = run_gpu(ctx, b, s, p, x, 0.25)
    y2, c2, S2, r2 = run_gpu(ctx, b, s2, p, x, 0.25)
    assert c1 == c2 and S1 == S2 and np.array_equal(r1, r2) and rel_l2(y1, y2.astype(np.float64)) < 1e-6


def test_multi_matches_single(iam, O, ctx):
    """q/k/v-style fused launch (shared x, three matrices, compact stats for one)."""
    shapes = [(4096, 4096, 21), (1024, 4096, 22), (1024, 4096, 23)]
    mats, bufs, outs, ref = [], [], [], []
    x = O.gen_f32(0, 24, 4096, 0.0, 1.0)
    dx = ctx.upload(x)
    for idx, (o, i, tid) in enumerate(shapes):
        b, s, p = make_matrix(O, o, i, tid=tid)
        db, ds, dp = ctx.upload(b), ctx.upload(s), ctx.upload(p)
        m = iam.BucketMatrix(db.ptr, ds.ptr, dp.ptr, b.shape[0], b.shape[1], 4, 3)
        if idx == 2:
            d3 = ctx.stats_compact(ds, b.shape[0])
            bufs.append(d3)
            m = iam.BucketMatrix(db.ptr, d3.ptr, dp.ptr, b.shape[0], b.shape[1], 1, 0)
        mats.append(m)
        bufs += [db, ds, dp]
        outs.append(ctx.empty(o, np.float32))
        ref.append(O.bucketmul(x, s, p, b, 0.25))
    ctx.multi(mats, [dx] * 3, [4096] * 3, outs, 0.25)
    for k in range(3):
        y = outs[k].read()
        oy, ocut, omask, oS = ref[k]
        cut, S = ctx.dispatch_info(k)
        assert np.float32(cut).view(np.uint32) == np.float32(ocut).view(np.uint32)
        assert S == oS and ctx.walk_count(k) == oS
        assert np.array_equal(ctx.dispatch_rows(k), np.nonzero(omask)[0].astype(np.uint32))
        assert rel_l2(y, oy) < 1e-5
    for d in bufs + outs + [dx]:
        d.free()


def test_invalid_arguments_raise(iam, O, ctx):
    b, s, p = make_matrix(O, 64, 4096, tid=25)
    db, ds, dp = ctx.upload(b), ctx.upload(s), ctx.upload(p)
    small_x = ctx.empty(1000, np.float32)          # cutoff needs 4096 inputs
    dy = ctx.empty(64, np.float32)
    with pytest.raises(iam.IamError) as e:
        ctx.calc_dispatch(small_x, ds, dp, 0, 4096, 4, 65536, 0.25)
    assert e.value.code == iam.IAM_E_INVALID
    dx = ctx.upload(O.gen_f32(0, 1, 4096, 0, 1))
    with pytest.raises(iam.IamError):
        ctx.calc_dispatch(dx, ds, dp, 1, 4096, 4, 65536, 0.25)   # expert 1 does not exist
    with pytest.raises(iam.IamError):
        ctx.calc_dispatch(dx, ds, dp, 0, 4096, 4, 65536, float("nan"))
    ctx.calc_dispatch(dx, ds, dp, 0, 4096, 4, 65536, 0.25)
    with pytest.raises(iam.IamError):
        ctx.mul(db, 8, dy)                                        # shape differs from dispatch
    for d in (db, ds, dp, small_x, dy, dx):
        d.free()


@pytest.mark.parametrize("mode", ["fp64", "fp32"])
def test_accumulation_modes_repeat(O, ctx, mode):
    """Repeated runs: fp64 stays within 1 ulp of the oracle on every run;
    fp32 (the reference's fp32 products, added in fp64) within 1e-5 relative
    L2 of the oracle's fp32 walk, and the runs agree to 1e-6 (the sums are
    added in whatever order the workgroups arrive)."""
    b, s, p = make_matrix(O, 14336, 4096, tid=31)
    x = O.gen_f32(0, 32, 4096, 0.0, 1.0)
    ctx.set_accumulation(mode)
    try:
        runs = [run_gpu(ctx, b, s, p, x, 0.25)[0] for _ in range(3)]
    finally:
        ctx.set_accumulation("fp64")
    oy = O.bucketmul(x, s, p, b, 0.25)[0]
    for r in runs:
        if mode == "fp64":
            assert ulps(r, oy).max() <= 1
        else:
            assert rel_l2(r, oy) < 1e-5
        assert rel_l2(r, runs[0].astype(np.float64)) < 1e-6


def test_walk_counting_switch(O, iam, ctx):
    """With counting off the outputs stay within 1 ulp, the counters do not
    move and walk_count still reports the slot's rows (the per-slice counts
    are always written); back on, the counters add up the oracle's
    selected-row count."""
    b, s, p = make_matrix(O, 4096, 4096)
    x = O.gen_f32(0, 77, 4096, 0.0, 1.0)
    y_on, cut, S, rows = run_gpu(ctx, b, s, p, x, 0.25, split=False)
    db, ds, dp, dx = ctx.upload(b), ctx.upload(s), ctx.upload(p), ctx.upload(x)
    dy = ctx.empty(16 * b.shape[1], np.float32)
    ctx.walk_counters(reset=True)
    ctx.set_walk_counting(False)
    try:
        ctx.full_mul(dx, ds, dp, db, 0, 4096, b.shape[1], b.shape[0], 0.25, dy)
        assert ulps(dy.read(), y_on).max() <= 1
        assert ctx.walk_counters(reset=True) == (0, 0, 0)
        assert ctx.walk_count(0) == S
    finally:
        ctx.set_walk_counting(True)
    ctx.full_mul(dx, ds, dp, db, 0, 4096, b.shape[1], b.shape[0], 0.25, dy)
    assert ctx.walk_count(0) == S
    assert ctx.walk_counters(reset=True) == (2 * S * b.shape[1], S, 1)
    for d in (db, ds, dp, dx, dy):
        d.free()


@pytest.mark.parametrize("block", [2, 16])
@pytest.mark.parametrize("shape,effort", [((4096, 4096), 0.25), ((14336, 4096), 0.05), ((4096, 14336), 0.125)],
                         ids=["square", "w1", "w2"])
def test_block_structured_selection(O, iam, ctx, block, shape, effort):
    """Block-structured selection (opt-in, blocks of `block` inputs for
    efforts below 0.5): cutoff bits, the selected rows, their count and y
    against the oracle's block selection and walk, through calc_dispatch +
    mul and through the fused walk; at effort 0.75 (above 0.5) the
    reference's per-row selection."""
    b, s, p = make_matrix(O, *shape, tid=40 + block)
    x = O.gen_f32(0, 41, shape[1], 0.0, 1.0)
    ctx.set_selection_block(block, 0.5)
    try:
        y, oy, cut, S = check_against_oracle(O, ctx, b, s, p, x, effort, block=block)
        fine, _ = O.select_rows(x, s, cut, b.shape[0], shape[1])
        assert S > int(fine.sum())                      # blocks add rows
        yf = run_gpu(ctx, b, s, p, x, effort, fused=iam)[0]
        assert ulps(yf, oy).max() <= 1
        check_against_oracle(O, ctx, b, s, p, x, 0.75, block=1)
    finally:
        ctx.set_selection_block(1)
    assert ctx.get_selection_block()[0] == 1
