"""The walk lists the rows certain to be selected before the cutoff is known:
those whose importance reaches an upper bound hi > cutoff taken from the
coarse window of the cutoff search (cutoff_upper in csrc/search.h).  Here
the bound is restated in numpy and checked against the oracle's bisection
(bucketMul.cl:68-214) on adversarial importance vectors at quantiles across
the range, edge ranks included: every cutoff lies strictly below hi; also
for the hinted window (the previous decode step's cutoff of the matrix),
where hi comes from the window's upper end.  The
same bound with its slack term removed fails on some of these vectors, so
the cases reach the bound's edge.  On the GPU the bucket-walk parity tests
(selected count and outputs against the oracle) cover the device's use of
it."""
import numpy as np

f32 = np.float32
N = 4096   # importances per search (the probes)


def keys(v):
    """Order-preserving 32-bit keys of numbers >= +0; NaN -> 0."""
    b = v.view(np.uint32).astype(np.uint64)
    k = np.where(b >> 31, ~b & 0xFFFFFFFF, b | 0x80000000)
    return np.where(np.isnan(v), 0, k).astype(np.uint64)


def key_float(k):
    k = int(k)
    b = (k & 0x7FFFFFFF) if (k & 0x80000000) else (~k & 0xFFFFFFFF)
    return float(np.uint32(b).view(np.float32))


def bound_hi(edge, gmn, gmx):
    """cutoff_upper's fp32 formula, every operation rounded to nearest:
    (edge + max(1.0002e-5, (gmax - gmin) 2^-20 + gmax 2^-23)) (1 + 2^-20)"""
    d = f32(f32(gmx) - f32(gmn))
    s = f32(f32(d * f32(2.0**-20)) + f32(f32(gmx) * f32(2.0**-23)))
    dl = max(f32(1.0002e-5), s)
    return f32(f32(f32(edge) + dl) * f32(1.0 + 2.0**-20))


def upper_bound(imp, t, slack=True):
    """cutoff_upper: the coarse bin (bits 30..20 of the key) of rank
    max(1, t - 2) among the numbers, its upper edge plus
    delta = max(1.0001e-5, (gmax - gmin) 2^-20 + gmax 2^-23), formed in fp32
    as the device does (bound_hi); without the slack, the edge alone.  None
    where the device's window search declines (a NaN importance) or gives
    no bound (t < 3, an infinite importance)."""
    if np.isnan(imp).any():
        return None
    k = keys(imp)
    nums = k[k != 0]
    if len(nums) == 0 or nums.min() < 0x80000000:
        return None
    kmx = int(nums.max())
    if t < 3 or kmx >= 0xFF800000:
        return None
    srt = np.sort(nums)[::-1]
    kmin = max(1, t - 2)
    if kmin > len(nums):
        return None
    dhi = int(srt[kmin - 1] >> 20) & 2047
    gmn, gmx = key_float(int(nums.min())), key_float(kmx)
    edge = np.uint32((dhi + 1) << 20).view(np.float32)
    return bound_hi(edge, gmn, gmx) if slack else f32(edge)


def vectors(rng):
    n = N
    yield "normal", np.abs(rng.normal(0, 1, n)).astype(f32) * f32(1600)
    yield "ties", np.round(np.abs(rng.normal(0, 3, n))).astype(f32)
    yield "two values", np.where(rng.random(n) < 0.5, f32(1), f32(2)).astype(f32)
    yield "constant", np.full(n, 5.0, f32)
    yield "tiny", (np.abs(rng.normal(0, 1, n)) * 1e-30).astype(f32)
    yield "huge", (np.abs(rng.normal(0, 1, n)) * 1e30).astype(f32)
    yield "60 decades", (10.0 ** rng.uniform(-30, 30, n)).astype(f32)
    yield "mostly zero", np.where(rng.random(n) < 0.7, f32(0), np.abs(rng.normal(0, 1, n)).astype(f32))
    yield "adjacent floats", (f32(1000) + np.arange(n) * f32(2**-13)).astype(f32)
    yield "eighths", (np.round(np.abs(rng.normal(0, 1, n)) * 8) / 8).astype(f32)
    yield "bimodal", np.concatenate([np.abs(rng.normal(0, 1, n // 2)), 1e4 + np.abs(rng.normal(0, 1, n // 2))]).astype(f32)
    yield "range 1e-5", (f32(1) + rng.random(n).astype(f32) * f32(1e-5)).astype(f32)
    yield "subnormal", (rng.random(n) * 1e-40).astype(f32)
    v = np.abs(rng.normal(0, 1, n)).astype(f32)
    v[rng.random(n) < 0.1] = np.nan
    yield "10% NaN", v
    v = np.abs(rng.normal(0, 1, n)).astype(f32)
    v[rng.random(n) < 0.99] = np.nan
    yield "99% NaN", v


def quantiles(rng):
    fixed = [0, 1, 2, 3, 4, 100, 1000, 2047, 3071, 3583, 3890, 4090, 4092, 4093, 4094, 4095]
    return sorted(set(fixed + [int(q) for q in rng.integers(0, N, 6)]))


def test_bound_hi_exceeds_exact_sum():
    """bound_hi (the device's fp32 formula) is at least the exact edge + delta
    (in exact rational arithmetic), also where every rounding goes down."""
    from fractions import Fraction as Fr
    rng = np.random.default_rng(11)
    cases = 0
    for _ in range(20000):
        gmx = f32(10.0 ** rng.uniform(-30, 30))
        gmn = f32(float(gmx) * rng.choice([0.0, rng.random(), 1.0]))
        edge = f32(float(gmx) * rng.uniform(0.0, 1.5))
        hi = bound_hi(edge, gmn, gmx)
        if not np.isfinite(hi):
            continue
        dl = max(Fr(10001, 10**9), (Fr(float(gmx)) - Fr(float(gmn))) * Fr(1, 2**20) + Fr(float(gmx)) * Fr(1, 2**23))
        assert Fr(float(hi)) >= Fr(float(edge)) + dl, (edge, gmn, gmx, hi)
        cases += 1
    assert cases > 15000


def test_certain_rows_bound_holds(O):
    rng = np.random.default_rng(7)
    checked, tightest = 0, np.inf
    for rep in range(8):
        for name, imp in vectors(rng):
            rng.shuffle(imp)
            for q in quantiles(rng):
                hi = upper_bound(imp, N - q)
                if hi is None:
                    continue
                c = O.find_cutoff_imp(imp, q)
                assert np.isfinite(c), (name, q, c)
                assert c < hi, (name, q, c, hi)
                if c > 0:
                    tightest = min(tightest, (float(hi) - float(c)) / float(c))
                checked += 1
    assert checked > 1500
    print(f"  {checked} cases, smallest relative gap hi - cutoff: {tightest:.2e}")


def test_bound_without_slack_fails_somewhere(O):
    """The upper edge of the coarse bin alone is no bound: a cutoff can lie
    up to the bisection's final bracket width above u_{t-2}."""
    rng = np.random.default_rng(8)
    broken = 0
    for name, imp in vectors(rng):
        rng.shuffle(imp)
        for q in quantiles(rng):
            hi = upper_bound(imp, N - q, slack=False)
            if hi is not None and not (O.find_cutoff_imp(imp, q) < hi):
                broken += 1
    assert broken > 0


def hinted_upper(imp, t, hint):
    """cutoff_upper of a hinted window: None where the device would not use
    the hint, declines (a NaN importance) or the window [7/8 hint, 8/7 hint)
    misses ranks t-2 .. t+2; else the window's upper end plus delta, formed
    as the device does (bound_hi)."""
    if not (1e-30 <= hint <= 1e30) or np.isnan(imp).any():
        return None
    k = keys(imp)
    nums = k[k != 0]
    if len(nums) == 0 or nums.min() < 0x80000000:
        return None
    kmx = int(nums.max())
    if t < 3 or kmx >= 0xFF800000:
        return None
    klo = int(keys(np.array([f32(hint) * f32(0.875)], f32))[0])
    khi = int(keys(np.array([f32(hint) * f32(1.142857142857)], f32))[0])
    above = int(np.count_nonzero(nums >= khi))
    inside = int(np.count_nonzero((nums >= klo) & (nums < khi)))
    kmin, kmax = max(1, t - 2), min(len(nums), t + 2)
    if not (above < kmin and above + inside >= kmax):
        return None
    gmn, gmx = key_float(int(nums.min())), key_float(kmx)
    return bound_hi(f32(key_float(khi)), gmn, gmx)


def test_hinted_window_bound_holds(O):
    """The same bound from a hinted window (the previous step's cutoff of
    the matrix): wherever the window holds ranks t-2 .. t+2, every cutoff
    lies strictly below its upper end plus delta."""
    rng = np.random.default_rng(9)
    checked = 0
    for rep in range(4):
        for name, imp in vectors(rng):
            rng.shuffle(imp)
            for q in quantiles(rng):
                c = O.find_cutoff_imp(imp, q)
                if not np.isfinite(c) or c <= 0:
                    continue
                for f in (1.0, 1.0 + 2.0**-23, 1.05, 0.95, 1.12, 0.89, 1.14, 0.876):
                    hi = hinted_upper(imp, N - q, float(f32(c) * f32(f)))
                    if hi is None:
                        continue
                    assert c < hi, (name, q, f, c, hi)
                    checked += 1
    assert checked > 1000
