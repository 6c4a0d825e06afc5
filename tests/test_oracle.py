"""Pins for the CPU oracle (oracle/oracle.c).  CPU only.

Each test checks the oracle against something that fixes the answer
independently: numpy's IEEE conversions, the reference's own known-answer
cases and golden vectors, hand-traced search runs, closed forms and brute
force.  A planted mistake (wrong channel, > instead of >=, a dropped term,
a transposed index) fails at least one of them.
"""
import json
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")


# ------------------------------------------------------------------ fp16 ---

def test_f32_to_f16_matches_numpy(O):
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[~np.isnan(f)]
    special = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, np.inf, -np.inf,
                        2.0**-24, 2.0**-25, 2.0**-25 * 1.0000001, 3 * 2.0**-26, 2.0**-14,
                        2.0**-14 - 2.0**-25, 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11],
                       dtype=np.float32)
    sub = (rng.uniform(-1, 1, 100000) * 2.0**-13).astype(np.float32)
    allf = np.concatenate([f, special, sub])
    got = O.f32_to_f16(allf)
    with np.errstate(over="ignore"):
        want = allf.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_f64_to_f16_matches_numpy(O):
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**63, size=1 << 20, dtype=np.uint64)
    d = bits.view(np.float64)
    d = d[np.isfinite(d)]
    small = rng.normal(0, 0.02, 1 << 18)                      # the generator's range
    sub = rng.uniform(-1, 1, 1 << 16) * 2.0**-14                # fp16 subnormals
    # exact ties between fp16 neighbours and values one double ulp either side
    h = rng.integers(0, 0x7bff, 4096, dtype=np.uint16).view(np.float16).astype(np.float64)
    h2 = np.nextafter(h.astype(np.float16), np.float16(np.inf)).astype(np.float64)
    mid = (h + h2) / 2
    ties = np.concatenate([mid, np.nextafter(mid, np.inf), np.nextafter(mid, -np.inf), -mid])
    special = np.array([0.0, -0.0, 65504.0, 65519.999, 65520.0, 1e300, -1e300, np.inf, -np.inf,
                        2.0**-24, 2.0**-25, 2.0**-25 * (1 + 2.0**-52), 3 * 2.0**-26, 2.0**-14])
    alld = np.concatenate([d, small, sub, ties, special])
    with np.errstate(over="ignore"):
        want = alld.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.f64_to_f16(alld), want)


def test_f16_to_f32_all_codes(O):
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.f16_to_f32(codes)
    want = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_verify_packing_cases(O):
    """preprocess_layer_fixed_gpu.py:340-361: position exact, value within 1%."""
    import ctypes
    cases = [(1.5, 0), (-0.5, 7), (0.0, 15), (3.14159, 8), (-2.71828, 3)]
    for value, pos in cases:
        packed = O.lib().orc_pack_fp16(value, pos)
        v = ctypes.c_float()
        p = ctypes.c_int()
        O.lib().orc_unpack_fp16(packed, ctypes.byref(v), ctypes.byref(p))
        assert p.value == pos
        assert abs(v.value - value) / (abs(value) + 1e-8) < 0.01
        # the packed code keeps the top 12 bits of the fp16 value
        assert packed & 0xFFF0 == np.float16(value).view(np.uint16) & 0xFFF0


# ------------------------------------------------------ bucket layout ---

def _fixtures():
    d = np.load(os.path.join(GOLD, "bucketize_fixtures.npz"))
    meta = json.load(open(os.path.join(GOLD, "bucketize_fixtures.json")))
    return d, meta


@pytest.mark.parametrize("name", [c["name"] for c in _fixtures()[1]["cases"]])
def test_bucketize_matches_reference_fixtures(O, name):
    d, meta = _fixtures()
    W = d[f"{name}__W"]
    b, s, p = O.bucketize(W)
    assert np.array_equal(b.ravel(), d[f"{name}__buckets"].ravel())
    assert np.array_equal(s.ravel(), d[f"{name}__stats"].ravel())
    assert np.array_equal(p.ravel(), d[f"{name}__probes"].ravel())


def test_order_fixture_discriminates():
    """The order fixture must fail a bucketizer that sums in another order:
    sequential / float64 stats and pairwise / float64 probes all differ."""
    d, _ = _fixtures()
    W = d["orderdisc3200x7__W"].view(np.float16).astype(np.float32)
    out, inn = W.shape
    nb = out // 16
    A = np.abs(W)
    ref_p = d["orderdisc3200x7__probes"].view(np.float16).ravel()
    p_pw = (np.add.reduce(np.ascontiguousarray(A.T), axis=1) / np.float32(out)).astype(np.float16)
    p_64 = (A.astype(np.float64).sum(0) / out).astype(np.float16)
    assert (p_pw != ref_p).any() or (p_64 != ref_p).any()
    ref_s = d["orderdisc3200x7__stats"].view(np.float16).reshape(inn * 16, 4)[:, 3]
    rows = np.ascontiguousarray((-np.sort(-A.T.reshape(inn, nb, 16), axis=2, kind="stable"))
                                .transpose(0, 2, 1)).reshape(inn * 16, nb)
    sq = np.zeros(inn * 16, np.float32)
    for b in range(nb):
        sq = sq + rows[:, b]
    s_seq = (sq / np.float32(nb)).astype(np.float16)
    s_64 = (rows.astype(np.float64).sum(1) / nb).astype(np.float16)
    assert (s_seq != ref_s).any()
    assert (s_64 != ref_s).any()


def test_bucketize_invariants(O):
    rng = np.random.default_rng(3)
    W = rng.normal(0, 0.02, size=(256, 40)).astype(np.float16)
    b, s, p = O.bucketize(W.view(np.uint16))
    out, inn = W.shape
    nb = out // 16
    bb = b.reshape(inn, 16, nb)
    # positions within each (input, bucket) column form a permutation of 0..15
    pos = bb & 15
    assert np.array_equal(np.sort(pos, axis=1), np.broadcast_to(np.arange(16)[None, :, None], pos.shape))
    # the position points back at the original weight; |value| non-increasing in rank
    Wb = W.view(np.uint16).T.reshape(inn, nb, 16)
    orig = np.take_along_axis(Wb, pos.transpose(0, 2, 1).astype(np.int64), axis=2).transpose(0, 2, 1)
    assert np.array_equal(orig & 0xFFF0, bb & 0xFFF0)
    mag = np.abs(orig.view(np.float16).astype(np.float32))
    assert (np.diff(mag, axis=1) <= 0).all()
    # stats channels equal; stats non-increasing in rank
    assert (s == s[:, :1]).all()
    st = s[:, 3].view(np.float16).astype(np.float32).reshape(inn, 16)
    assert (np.diff(st, axis=1) <= 0).all()


def test_pairwise_sum_matches_numpy(O):
    rng = np.random.default_rng(5)
    for n in [0, 1, 7, 8, 9, 15, 16, 127, 128, 129, 200, 255, 256, 1000, 2000, 4097]:
        a = (rng.exponential(1.0, n) * np.exp2(rng.uniform(-20, 10, n))).astype(np.float32)
        got = O.lib().orc_np_pairwise_sum_f32(a, n)
        want = np.add.reduce(a) if n else np.float32(0)
        assert np.float32(got).view(np.uint32) == np.float32(want).view(np.uint32) or (n == 0 and got == 0)


# ---------------------------------------------------------------- cutoff ---

def test_effort_quantile_kat(O):
    # bucket_mul.hpp:164, target = 4096 - quantile
    kat = {1.0: 4096, 0.5: 2049, 0.25: 1025, 0.125: 513, 0.05: 206}
    for e, target in kat.items():
        assert 4096 - O.effort_quantile(e) == target


def test_importance_matches_reference_harness(O):
    """test_cutoff_binary_search.cpp:223-237 restates the importance as
    CUTOFF_SCALE * |input * fp16_to_float(probe)| in float."""
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, 4096).astype(np.float32)
    probes = rng.uniform(0, 0.05, 8192).astype(np.float16)
    for exp_no in (0, 1):
        got = O.importance(x, probes.view(np.uint16), exp_no)
        pv = probes[exp_no * 4096:(exp_no + 1) * 4096].astype(np.float32)
        want = np.float32(100000.0) * np.abs(x * pv)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_cutoff_zero_input(O):
    # all importances 0: bound 0, count 0 < target, range 0 < 1e-5 -> 0 after 1 round
    c, tr = O.find_cutoff_imp(np.zeros(4096, np.float32), O.effort_quantile(0.25), trace=True)
    assert c == 0.0 and tr.rounds == 1 and tr.converged == 1


def test_cutoff_exact_hit_round1(O):
    imp = np.zeros(4096, np.float32)
    imp[:1025] = 10.0
    imp[1025:] = 1.0
    c, tr = O.find_cutoff_imp(imp, O.effort_quantile(0.25), trace=True)
    # min 1, max 10, bound 5.5 counts exactly 1025 = target
    assert c == 5.5 and tr.rounds == 1 and tr.counts[0] == 1025


def test_cutoff_ramp_gap_convergence(O):
    """imp = 0..4095, target 1025: hand-traced; stops in round 11 when the
    bracket counts are 1024 and 1026 (|gap| < 3) and returns the bound tested
    in that round."""
    imp = np.arange(4096, dtype=np.float32)
    c, tr = O.find_cutoff_imp(imp, O.effort_quantile(0.25), trace=True)
    want_bounds = [2047.5, 3071.25, 2559.375, 2815.3125, 2943.28125, 3007.265625, 3039.2578125,
                   3055.25390625, 3063.251953125, 3067.2509765625, 3069.25048828125]
    want_counts = [2048, 1024, 1536, 1280, 1152, 1088, 1056, 1040, 1032, 1028, 1026]
    assert tr.rounds == 11 and tr.converged == 1
    assert list(tr.bounds[:11]) == want_bounds
    assert list(tr.counts[:11]) == want_counts
    assert c == np.float32(3069.25048828125)


def test_cutoff_round_limit_float_ties(O):
    """1023 values at 1000, 5 at 500, the rest 0, target 1025.  The bracket
    closes on 500 from below; from round 18 the float midpoints round (ties to
    even), the bracket never shrinks below 1e-5 and the counts stay 1023/1028,
    so all 20 rounds run and the untested midpoint 500 - 2^-11 is returned.
    Hand-traced: bound_19 = 500 - 62*2^-15, bound_20 = 500 - 31*2^-15."""
    imp = np.zeros(4096, np.float32)
    imp[:1023] = 1000.0
    imp[1023:1028] = 500.0
    c, tr = O.find_cutoff_imp(imp, O.effort_quantile(0.25), trace=True)
    assert tr.rounds == 20 and tr.converged == 0
    assert tr.bounds[0] == 500.0 and tr.counts[0] == 1023
    assert tr.bounds[1] == 250.0 and tr.counts[1] == 1028
    assert tr.bounds[18] == np.float32(500 - 62 * 2.0**-15)
    assert tr.bounds[19] == np.float32(500 - 31 * 2.0**-15)
    assert c == np.float32(500 - 2.0**-11)


def test_cutoff_bracket_invariants(O):
    rng = np.random.default_rng(11)
    for trial in range(40):
        x = rng.normal(0, 1, 4096).astype(np.float32)
        if trial % 4 == 1:
            x[rng.choice(4096, 41, replace=False)] *= 20     # skewed channels
        if trial % 4 == 2:
            x = np.round(x * 4) / 4                           # many ties
        probes = np.abs(rng.normal(0.016, 0.002, 4096)).astype(np.float16)
        for effort in (1.0, 0.5, 0.25, 0.125, 0.05):
            q = O.effort_quantile(effort)
            c, tr = O.find_cutoff(x, probes.view(np.uint16), q, trace=True)
            imp = O.importance(x, probes.view(np.uint16))
            assert tr.init_min <= c <= tr.init_max
            cnt = int((imp > c).sum())
            assert tr.final_max_count <= cnt <= tr.final_min_count
            if effort == 1.0 and tr.converged and tr.final_max - tr.final_min >= 1e-5:
                assert (imp <= c).sum() <= 2


def test_cutoff_constant_importance(O):
    # every |x*p| equal: min == max, one round
    x = np.ones(4096, np.float32)
    probes = np.full(4096, 0.015625, np.float16)
    c, tr = O.find_cutoff(x, probes.view(np.uint16), O.effort_quantile(0.5), trace=True)
    assert c == np.float32(1562.5) and tr.rounds == 1


# ------------------------------------------------------------- selection ---

def test_select_rows_channel3_ge_and_in_size(O):
    rng = np.random.default_rng(2)
    in_dim = 64
    R = in_dim * 16
    x = rng.normal(0, 1, 4096).astype(np.float32)
    stats = np.zeros((R, 4), np.float16)
    stats[:, 3] = np.abs(rng.normal(0.02, 0.01, R)).astype(np.float16)
    stats[:, :3] = np.float16(60000.0)     # garbage in channels 0..2
    imp3 = np.float32(100000.0) * np.abs(np.repeat(x[:in_dim], 16) * stats[:, 3].astype(np.float32))
    cutoff = np.float32(np.sort(imp3)[R // 2])   # an importance value: tie case included
    mask, s = O.select_rows(x, stats.view(np.uint16), cutoff, R, in_dim)
    want = (imp3 >= cutoff)
    assert np.array_equal(mask.astype(bool), want)
    assert s == want.sum()
    assert mask[np.argmin(np.abs(imp3 - cutoff))] == 1           # >= at equality
    mask2, _ = O.select_rows(x, stats.view(np.uint16), cutoff, R, in_dim // 2)
    assert not mask2[R // 2:].any()                              # rows past in_size skipped
    assert np.array_equal(mask2[:R // 2], mask[:R // 2])


def test_select_rows_expert_offset(O):
    rng = np.random.default_rng(4)
    R = 32 * 16
    x = rng.normal(0, 1, 4096).astype(np.float32)
    stats = np.abs(rng.normal(0.02, 0.01, (2 * R, 4))).astype(np.float16)
    m0, _ = O.select_rows(x, stats.view(np.uint16), 1000.0, R, 32, exp_no=0)
    m1, _ = O.select_rows(x, stats.view(np.uint16), 1000.0, R, 32, exp_no=1)
    imp1 = np.float32(100000.0) * np.abs(np.repeat(x[:32], 16) * stats[R:, 3].astype(np.float32))
    assert np.array_equal(m1.astype(bool), imp1 >= 1000.0)
    assert not np.array_equal(m0, m1)


@pytest.mark.parametrize("block", [1, 2, 8, 16])
def test_select_rows_block_is_any_over_the_block(O, block):
    """Block-structured selection against a numpy any-over-the-block of the
    per-row test, with a partial last block (in_size not a multiple of the
    block) and rows past in_size; invariants: it contains the per-row
    selection, is constant over each block for every rank, and block 1 is
    the per-row selection."""
    rng = np.random.default_rng(20 + block)
    in_dim = 100
    R = in_dim * 16
    in_size = 90
    x = rng.standard_cauchy(4096).astype(np.float32)          # heavy-tailed inputs
    stats = np.abs(rng.normal(0.02, 0.01, (R, 4))).astype(np.float16)
    fine, s_fine = O.select_rows(x, stats.view(np.uint16), 300.0, R, in_size)
    mask, s = O.select_rows_block(x, stats.view(np.uint16), 300.0, R, in_size, block)
    f = fine.reshape(in_dim, 16).astype(bool)
    nb = (in_dim + block - 1) // block
    pad = np.zeros((nb * block, 16), bool)
    pad[:in_dim] = f
    want = np.repeat(pad.reshape(nb, block, 16).any(axis=1), block, axis=0)[:in_dim]
    want[in_size:] = False                                    # rows past in_size stay skipped
    assert np.array_equal(mask.reshape(in_dim, 16).astype(bool), want)
    assert s == want.sum()
    assert (mask >= fine).all()
    if block == 1:
        assert np.array_equal(mask, fine) and s == s_fine
    else:
        assert s > s_fine
        m = mask.reshape(in_dim, 16).astype(bool)
        assert not m[in_size:].any()
        for b0 in range(0, in_size - in_size % block, block):   # whole blocks below in_size
            blk = m[b0:b0 + block]
            assert (blk == blk[0]).all()


def test_select_rows_block_one_hot(O):
    """x zero but for input 37: only its block's rows, with the ranks input 37
    passes, are selected, in every input of the block."""
    R = 64 * 16
    x = np.zeros(4096, np.float32)
    x[37] = 3.0
    stats = np.full((R, 4), np.float16(0.01), np.float16)
    stats[37 * 16:38 * 16, 3] = np.linspace(0.05, 0.001, 16).astype(np.float16)
    cutoff = np.float32(100000.0 * 3.0 * np.float32(np.float16(0.02)))
    mask, s = O.select_rows_block(x, stats.view(np.uint16), cutoff, R, 64, 8)
    ranks = np.float32(100000.0) * np.abs(np.float32(3.0) * stats[37 * 16:38 * 16, 3].astype(np.float32)) >= cutoff
    want = np.zeros((64, 16), bool)
    want[32:40] = ranks
    assert np.array_equal(mask.reshape(64, 16).astype(bool), want)
    assert s == 8 * ranks.sum() and 0 < ranks.sum() < 16


# ------------------------------------------------------------------ walk ---

def _packed_dense(b, in_dim):
    """W~[c*16 + pos, i] = value of the packed code, from the bucket layout."""
    R, C_ = b.shape
    Wt = np.zeros((16 * C_, in_dim), np.float64)
    codes = b.reshape(in_dim, 16, C_)
    vals = codes.view(np.float16).astype(np.float64)
    for i in range(in_dim):
        for k in range(16):
            o = np.arange(C_) * 16 + (codes[i, k] & 15)
            Wt[o, i] = vals[i, k]
    return Wt


def test_walk_all_rows_is_dense_gemv(O):
    rng = np.random.default_rng(6)
    out_dim, in_dim = 128, 48
    W = rng.normal(0, 0.02, (out_dim, in_dim)).astype(np.float16)
    b, s, p = O.bucketize(W.view(np.uint16))
    x = rng.normal(0, 1, in_dim).astype(np.float32)
    y = O.bucket_walk(b, np.ones(in_dim * 16, np.uint8), x, in_dim * 16)
    Wt = _packed_dense(b, in_dim)
    np.testing.assert_allclose(y, Wt @ x.astype(np.float64), rtol=1e-6, atol=1e-7)
    # the packed matrix is W with 4 low mantissa bits replaced: close to W x
    yw = W.astype(np.float64) @ x.astype(np.float64)
    assert np.linalg.norm(y - yw) / np.linalg.norm(yw) < 1.5e-2   # 4 of 10 mantissa bits replaced
    y32 = O.bucket_walk(b, np.ones(in_dim * 16, np.uint8), x, in_dim * 16, acc64=False)
    np.testing.assert_allclose(y32, y, rtol=1e-4, atol=1e-6)


def test_walk_one_hot_and_zero(O):
    rng = np.random.default_rng(7)
    out_dim, in_dim = 64, 32
    W = rng.normal(0, 0.02, (out_dim, in_dim)).astype(np.float16)
    b, s, p = O.bucketize(W.view(np.uint16))
    x = np.zeros(in_dim, np.float32)
    x[5] = 2.0
    mask = np.zeros(in_dim * 16, np.uint8)
    mask[5 * 16:5 * 16 + 16] = 1
    y = O.bucket_walk(b, mask, x, in_dim * 16)
    Wt = _packed_dense(b, in_dim)
    np.testing.assert_array_equal(y, (2.0 * Wt[:, 5]).astype(np.float32))
    mask[5 * 16 + 3:5 * 16 + 16] = 0          # only ranks 0..2 of input 5
    y = O.bucket_walk(b, mask, x, in_dim * 16)
    top = np.argsort(-np.abs(W[:, 5].astype(np.float32)).reshape(-1, 16), axis=1, kind="stable")[:, :3]
    want = np.zeros(out_dim, np.float32)
    for bk in range(out_dim // 16):
        for pp in top[bk]:
            want[bk * 16 + pp] = 2.0 * Wt[bk * 16 + pp, 5]
    np.testing.assert_array_equal(y, want)
    y0 = O.bucket_walk(b, np.ones(in_dim * 16, np.uint8), np.zeros(in_dim, np.float32), in_dim * 16)
    assert not y0.any()


def test_bucketmul_zero_x_selects_everything(O):
    rng = np.random.default_rng(8)
    W = rng.normal(0, 0.02, (64, 4096)).astype(np.float16)
    b, s, p = O.bucketize(W.view(np.uint16))
    y, cut, mask, S = O.bucketmul(np.zeros(4096, np.float32), s, p, b, 0.25)
    assert cut == 0.0 and S == 4096 * 16 and not y.any()


# ----------------------------------------------------------- layer ops ---

def test_rmsnorm_gain_closed_form(O):
    rng = np.random.default_rng(9)
    x = rng.normal(0, 1, 4096).astype(np.float32)
    g = (1 + rng.normal(0, 0.01, 4096)).astype(np.float16)
    got = O.rmsnorm_gain(x, g.view(np.uint16), 1e-5)
    xd = x.astype(np.float64)
    want = xd / np.sqrt(np.mean(xd * xd) + 1e-5) * g.astype(np.float64)
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-7)


def test_silu_closed_form(O):
    rng = np.random.default_rng(10)
    g = rng.normal(0, 3, 5000).astype(np.float32)
    u = rng.normal(0, 1, 5000).astype(np.float32)
    want = u.astype(np.float64) * g / (1 + np.exp(-g.astype(np.float64)))
    np.testing.assert_allclose(O.silu_mul(g, u), want, rtol=1e-6, atol=1e-9)


def test_rope_table_and_rotation(O):
    t = O.rope_table(10000.0, 128, 64)
    i = np.arange(64)
    freq = (1.0 / np.power(10000.0, 2.0 * i / 128)).astype(np.float32)
    ang = (np.arange(64, dtype=np.float32)[:, None] * freq[None, :]).astype(np.float32)
    np.testing.assert_allclose(t[..., 0], np.cos(ang.astype(np.float64)), atol=2e-7)
    np.testing.assert_allclose(t[..., 1], np.sin(ang.astype(np.float64)), atol=2e-7)
    rng = np.random.default_rng(12)
    x = rng.normal(0, 1, 4 * 128).astype(np.float32)
    pos = 37
    got = O.rope(x, t[pos], 4, 128)
    xh = x.reshape(4, 128).astype(np.float64)
    c = np.concatenate([t[pos, :, 0], t[pos, :, 0]]).astype(np.float64)
    s = np.concatenate([t[pos, :, 1], t[pos, :, 1]]).astype(np.float64)
    rot = np.concatenate([-xh[:, 64:], xh[:, :64]], axis=1)     # rotate-half
    np.testing.assert_allclose(got.reshape(4, 128), xh * c + rot * s, rtol=1e-6, atol=1e-6)
    # rotation preserves the norm of each (d, d+64) pair
    np.testing.assert_allclose(np.linalg.norm(got.reshape(4, 128), axis=1),
                               np.linalg.norm(xh, axis=1), rtol=1e-5)


def test_attention_closed_form(O):
    rng = np.random.default_rng(13)
    n_heads, n_kv, hd, n_tok = 8, 2, 128, 37
    q = rng.normal(0, 1, n_heads * hd).astype(np.float32)
    k = rng.normal(0, 1, (n_tok, n_kv, hd)).astype(np.float16)
    v = rng.normal(0, 1, (n_tok, n_kv, hd)).astype(np.float16)
    got = O.attention_f16kv(q, k.view(np.uint16), v.view(np.uint16), n_tok, n_heads, n_kv, hd)
    want = np.zeros((n_heads, hd))
    for h in range(n_heads):
        kv = h // (n_heads // n_kv)
        s = k[:, kv].astype(np.float64) @ q[h * hd:(h + 1) * hd].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s) / np.exp(s).sum()
        want[h] = p @ v[:, kv].astype(np.float64)
    np.testing.assert_allclose(got.reshape(n_heads, hd), want, rtol=1e-5, atol=1e-6)


def test_attention_f16kv_has_no_max_subtraction(O):
    """The reference's softmax exponentiates the scores as they are
    (aux.cl:204-225): one score above log(DBL_MAX) ~ 709.78 overflows the
    fp64 evaluation and that head's outputs are NaN (a max-subtracted softmax
    would stay finite); just below, every output is finite."""
    hd, n_tok = 128, 3
    k = np.zeros((n_tok, 1, hd), np.float16)
    k[1, 0, :] = 1.0
    v = np.ones((n_tok, 1, hd), np.float16)
    for qv, finite in ((62.0, True), (63.0, False)):   # s = 128 * qv / sqrt(128): 701.4, 712.7
        q = np.full(2 * hd, qv, np.float32)
        q[hd:] = 0.0                                    # head 1: all scores 0
        got = O.attention_f16kv(q, k.view(np.uint16), v.view(np.uint16), n_tok, 2, 1, hd)
        assert np.all(np.isfinite(got[:hd])) == finite
        assert np.all(np.isnan(got[:hd])) == (not finite)
        np.testing.assert_allclose(got[hd:], 1.0, rtol=1e-7)   # softmax of equal scores over equal rows


def _att32_inputs(rng, n_tok, n_heads, hd, scale=1.0):
    q = rng.normal(0, scale, n_heads * hd).astype(np.float32)
    k = rng.normal(0, 1, (n_tok, n_heads, hd)).astype(np.float32)
    v = rng.normal(0, 1, (n_tok, n_heads, hd)).astype(np.float32)
    return q, k, v


def test_attention_f32rep_textbook(O):
    """Against softmax attention in float64 without a max subtracted, over
    3 splits of positions (the fixed order of the fp32 sums changes only
    roundings)."""
    rng = np.random.default_rng(31)
    n_heads, hd, n_tok = 4, 128, 150
    q, k, v = _att32_inputs(rng, n_tok, n_heads, hd, 0.3)
    got = O.attention_f32rep(q, k, v, n_tok, n_heads, hd).reshape(n_heads, hd)
    for h in range(n_heads):
        s = k[:, h].astype(np.float64) @ q[h * hd:(h + 1) * hd].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s) / np.exp(s).sum()
        np.testing.assert_allclose(got[h], p @ v[:, h].astype(np.float64), rtol=2e-5, atol=2e-6)


def test_attention_f32rep_one_position_and_equal_keys(O):
    """One position: p = e/e = 1 exactly, so the output is that V row bit for
    bit.  Equal keys at every position: equal scores, p = 1/n up to
    rounding, the output is the mean of V."""
    rng = np.random.default_rng(32)
    n_heads, hd = 4, 128
    q, k, v = _att32_inputs(rng, 1, n_heads, hd, 0.3)
    got = O.attention_f32rep(q, k, v, 1, n_heads, hd)
    assert np.array_equal(got.view(np.uint32), v.ravel().view(np.uint32))
    n_tok = 200
    q, k, v = _att32_inputs(rng, n_tok, n_heads, hd, 0.3)
    k[:] = k[0]
    got = O.attention_f32rep(q, k, v, n_tok, n_heads, hd).reshape(n_heads, hd)
    np.testing.assert_allclose(got, v.astype(np.float64).mean(axis=0), rtol=1e-5, atol=1e-6)


def test_attention_f32rep_score_tree_order(O):
    """dotSetScore2 adds the products by the work-group tree (p[i] +=
    p[i + stride] for stride 64 .. 1, aux.cl:519-525).  Products 2^27 at
    d = 0, 1 at d = 64 and -2^27 at d = 1: the tree forms 2^27 + 1 = 2^27
    first (an fp32 rounding) and ends at 0, where a sequential sum ends at 1.
    With a zero V row for the other position the output is p * v, and
    p = e0 / (e0 + e1) with e0 = exp(0) = 1 tells the score apart."""
    hd = 128
    q = np.zeros(hd, np.float32)
    k = np.zeros((2, 1, hd), np.float32)
    q[0], k[0, 0, 0] = 2.0 ** 14, 2.0 ** 13
    q[64], k[0, 0, 64] = 1.0, 1.0
    q[1], k[0, 0, 1] = -(2.0 ** 14), 2.0 ** 13
    v = np.zeros((2, 1, hd), np.float32)
    v[0, 0, :] = 1.0
    got = O.attention_f32rep(q, k, v, 2, 1, hd)
    # position 0 scores 0 (the tree), position 1 scores 0: p0 = 1 / 2 exactly
    assert np.all(got == np.float32(0.5))


def test_attention_f32rep_overflow_is_nan(O):
    """No maximum is subtracted: a score above log(FLT_MAX) ~ 88.72 makes
    exp(s) inf and the head's outputs NaN (inf / inf), as in the
    reference; at 88.0 they are finite."""
    hd = 128
    for s_target, finite in ((88.0, True), (89.0, False)):
        q = np.zeros(hd, np.float32)
        q[0] = np.float32(s_target * np.sqrt(np.float32(hd)))   # q[0] * k[0] / sqrt(128) ~ s_target
        k = np.zeros((2, 1, hd), np.float32)
        k[0, 0, 0] = 1.0
        v = np.ones((2, 1, hd), np.float32)
        got = O.attention_f32rep(q, k, v, 2, 1, hd)
        assert np.all(np.isfinite(got)) == finite
        assert np.all(np.isnan(got)) == (not finite)


def test_rope_kv_rep32(O):
    """The appended row: RoPE of q and k, K and V repeated to every query
    head by index (head h reads KV head h // rep, repeat4x32)."""
    rng = np.random.default_rng(33)
    n_heads, n_kv, hd = 32, 8, 128
    t = O.rope_table(10000.0, hd, 8)
    q = rng.normal(0, 1, n_heads * hd).astype(np.float32)
    k = rng.normal(0, 1, n_kv * hd).astype(np.float32)
    v = rng.normal(0, 1, n_kv * hd).astype(np.float32)
    qo, kr, vr = O.rope_kv_rep32(q, k, v, t[5], n_heads, n_kv, hd)
    assert np.array_equal(qo.view(np.uint32), O.rope(q, t[5], n_heads, hd).view(np.uint32))
    kk = O.rope(k, t[5], n_kv, hd).reshape(n_kv, hd)
    assert np.array_equal(kr.reshape(n_heads, hd), kk[np.arange(n_heads) // 4])
    assert np.array_equal(vr.reshape(n_heads, hd), v.reshape(n_kv, hd)[np.arange(n_heads) // 4])


def test_matmul_f16_dense(O):
    """matmul16x32: against a float64 GEMV; one-hot x gives the column
    exactly; and the order of the sums: work-item l adds its columns
    l, l + 256, ... in order, then the 256-way tree (aux.cl:472-487).  Row
    products 2^27 (column 0), 1 (column 256) and -2^27 (column 128): work-item
    0 forms 2^27 + 1 = 2^27, the tree's first level cancels it: 0 (a
    sequential sum over the columns gives 1)."""
    rng = np.random.default_rng(34)
    rows, cols = 48, 4096
    W = rng.normal(0, 0.02, (rows, cols)).astype(np.float16)
    x = rng.normal(0, 1, cols).astype(np.float32)
    got = O.matmul_f16_dense(W.view(np.uint16), x)
    np.testing.assert_allclose(got, W.astype(np.float64) @ x.astype(np.float64), rtol=1e-4, atol=1e-5)
    e = np.zeros(cols, np.float32)
    e[777] = 1.0
    assert np.array_equal(O.matmul_f16_dense(W.view(np.uint16), e), W[:, 777].astype(np.float32))
    W2 = np.zeros((1, 512), np.float16)
    x2 = np.zeros(512, np.float32)
    W2[0, 0], x2[0] = 2048.0, 2.0 ** 16
    W2[0, 256], x2[256] = 1.0, 1.0
    W2[0, 128], x2[128] = -2048.0, 2.0 ** 16
    assert O.matmul_f16_dense(W2.view(np.uint16), x2)[0] == 0.0


def test_argmax_first_max(O):
    v = np.array([1, 5, 3, 5, 5, -1], np.float32)
    assert O.argmax(v) == 1 == int(np.argmax(v))
    rng = np.random.default_rng(14)
    for _ in range(20):
        w = rng.integers(0, 50, 1000).astype(np.float32)
        assert O.argmax(w) == int(np.argmax(w))


# ------------------------------------------------------------- generator ---

def test_generator_statistics_and_determinism(O):
    a = O.gen_f32(0, 7, 200000, 0.0, 1.0)
    b = O.gen_f32(0, 7, 200000, 0.0, 1.0)
    c = O.gen_f32(1, 7, 200000, 0.0, 1.0)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert abs(a.mean()) < 0.01 and abs(a.var() - 1.0) < 0.01
    assert np.abs(a).max() < 6.0
    h = O.gen_f16(0, 9, 100000, 0.0, 0.02)
    hf = h.view(np.float16).astype(np.float32)
    assert abs(hf.std() - 0.02) < 5e-4
    t = O.gen_tokens(0, 3, 100000, 32000)
    assert t.min() >= 0 and t.max() < 32000 and len(np.unique(t)) > 30000


# ----------------------------------------------------------------- model ---

def test_model_forward_is_the_layer_composition(O):
    """orc_model_forward (transformer_layer.hpp:75-122, model.hpp:152-231)
    equals the primitives chained in the reference order: RMSNorm(attn gain)
    -> q,k,v -> RoPE of q and k at pos -> fp16 K/V rows at pos -> attention
    over pos+1 tokens -> o -> +residual -> RMSNorm(ffn gain) -> w1, w3 ->
    SiLU(w1)*w3 -> w2 -> +residual; final RMSNorm -> LM head."""
    cfg = dict(n_layers=1, dim=4096, ffn_dim=4096, n_heads=32, n_kv_heads=8, head_dim=128, vocab=256,
               max_ctx=4, rope_theta=10000.0, norm_eps=1e-5)
    D, F, V, KVD = 4096, 4096, 256, 1024
    shapes = {"wq": (D, D), "wk": (KVD, D), "wv": (KVD, D), "wo": (D, D), "w1": (F, D), "w3": (F, D), "w2": (D, F)}
    mats = {}
    for k, (name, shp) in enumerate(shapes.items()):
        W = O.gen_f16(5, 500 + k, shp[0] * shp[1], 0.0, 0.02).reshape(shp)
        mats[name] = O.bucketize(W)
    lm = O.bucketize(O.gen_f16(5, 520, V * D, 0.0, 0.02).reshape(V, D))
    t = {"layer0.attn_gain": O.gen_f16(5, 530, D, 1.0, 0.01), "layer0.ffn_gain": O.gen_f16(5, 531, D, 1.0, 0.01),
         "embed": O.gen_f16(5, 532, V * D, 0.0, 0.02), "final_gain": O.gen_f16(5, 533, D, 1.0, 0.01),
         "lm_head.buckets": lm[0], "lm_head.stats": lm[1], "lm_head.probes": lm[2]}
    for name, (b, st, pr) in mats.items():
        t[f"layer0.{name}.buckets"], t[f"layer0.{name}.stats"], t[f"layer0.{name}.probes"] = b, st, pr
    orc = O.OracleModel(cfg, lambda name, dtype: np.ascontiguousarray(t[name]).view(dtype).ravel())
    table = O.rope_table(10000.0, 128, 4)
    kc = np.zeros((4, KVD), np.uint16)
    vc = np.zeros((4, KVD), np.uint16)

    def mm(name, x):
        b, st, pr = mats[name]
        return O.bucketmul(x, st, pr, b, 0.25)[0]

    for pos, tok in enumerate([17, 200, 3]):
        got = orc.forward(tok, pos, 0.25)
        h = O.f16_to_f32(t["embed"].reshape(V, D)[tok])
        hn = O.rmsnorm_gain(h, t["layer0.attn_gain"], 1e-5)
        q, k, v = mm("wq", hn), mm("wk", hn), mm("wv", hn)
        qr, kr = O.rope(q, table[pos], 32, 128), O.rope(k, table[pos], 8, 128)
        kc[pos], vc[pos] = O.f32_to_f16(kr), O.f32_to_f16(v)
        att = O.attention_f16kv(qr, kc, vc, pos + 1, 32, 8, 128)
        h = h + mm("wo", att)
        hn = O.rmsnorm_gain(h, t["layer0.ffn_gain"], 1e-5)
        h = h + mm("w2", O.silu_mul(mm("w1", hn), mm("w3", hn)))
        hn = O.rmsnorm_gain(h, t["final_gain"], 1e-5)
        want = O.bucketmul(hn, lm[1], lm[2], lm[0], 0.25)[0]
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), pos
        assert np.array_equal(orc.kc.reshape(4, KVD)[pos], kc[pos])
