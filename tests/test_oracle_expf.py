"""Pins for oracle/or_zexpf, the reference's @exp(f32): the compiler runtime's
expf (src/sampler.zig:219-240, src/model.zig:2505; build.zig:14 links no libc),
restated from musl's / FreeBSD's published expf.  Each check is chosen so that
a plausible restatement mistake fails one of them: a wrong constant or a
dropped term breaks the 1-ulp bound, an f64 evaluation (or contraction into
FMAs) makes it correctly rounded, a wrong threshold moves a special value."""
import numpy as np
import pytest


def f32(u):
    return np.array([u], np.uint32).view(np.float32)[0]


def bits(x):
    return np.asarray(x, np.float32).view(np.uint32).astype(np.int64)


def ulp_gap(got, ref64):
    """f32 ulps between got and the correctly rounded ref64 (same sign, >= 0)."""
    return np.abs(bits(got) - bits(np.asarray(ref64, np.float64).astype(np.float32)))


@pytest.mark.parametrize("lo,hi,step", [(0xC2CFF1B4, 0x80000000, 389), (0x00000000, 0x42B17217, 397)])
def test_within_one_ulp_dense(oracle, lo, hi, step):
    """Every 389th / 397th float over the whole finite, non-zero result range
    (negative arguments down to -103.972, positive up to 88.7228): at most one
    ulp from exp(x), as the published algorithm states."""
    if lo > hi:
        lo, hi = hi, lo
    u = np.arange(lo, hi, step, dtype=np.uint64).astype(np.uint32)
    x = u.view(np.float32)
    got = oracle.zexpf_array(x)
    ref = np.exp(x.astype(np.float64))
    gap = ulp_gap(got, ref)
    assert gap.max() <= 1, (x[gap.argmax()], got[gap.argmax()], ref[gap.argmax()])


def test_not_correctly_rounded(oracle):
    """The port is not the f64-rounded exp: on [-20, 0] (the sampler's terms)
    it differs from the correctly rounded value on a small fraction of
    arguments -- about 0.77% of every 701st float there."""
    u = np.arange(0x80000000, 0xC1A00000, 701, dtype=np.uint64).astype(np.uint32)
    x = u.view(np.float32)
    got = oracle.zexpf_array(x)
    cr = np.exp(x.astype(np.float64)).astype(np.float32)
    frac = np.mean(got != cr)
    assert 0.003 < frac < 0.02, frac


def test_special_values_and_thresholds(oracle):
    e = oracle.zexpf
    assert e(0.0) == 1.0 and e(-0.0) == 1.0
    assert np.isnan(e(float("nan")))
    assert e(float("inf")) == float("inf") and e(float("-inf")) == 0.0
    assert e(f32(0x42B17218)) == float("inf")                      # 88.722839: overflow
    assert np.isfinite(e(f32(0x42B17217))) and e(f32(0x42B17217)) > 3.4e38
    assert e(f32(0xC2CFF1B5)) == 0.0                               # -103.972084: underflow
    t = e(f32(0xC2CFF1B4))                                         # just above: at most the smallest subnormal
    assert 0.0 <= t < 2e-45
    # |x| <= 2^-13 returns 1 + x (one f32 addition)
    for u in [0x39000000, 0x38FFFFFF, 0x38000000, 0xB9000000, 0xB8800000, 0x00000001]:
        x = f32(u)
        assert e(x) == np.float32(np.float32(1.0) + x), hex(u)


def test_reduction_branches_agree_at_their_boundaries(oracle):
    """The three argument-reduction branches (k = 0, k = +-1, k from
    invln2*x) meet at |x| = ln2/2 and 1.5 ln2; the result stays within one ulp
    of exp on both sides of each (a wrong k or hi/lo split at a boundary
    would be off by a factor near 2)."""
    for b in [0x3EB17218, 0x3F851592, 0xBEB17218, 0xBF851592]:
        u = np.arange(b - 64, b + 64, dtype=np.uint64).astype(np.uint32)
        x = u.view(np.float32)
        gap = ulp_gap(oracle.zexpf_array(x), np.exp(x.astype(np.float64)))
        assert gap.max() <= 1, hex(b)


def test_subnormal_results_round_once(oracle):
    """Results below 2^-126 (k <= -126) come from one rounding of y * 2^k,
    so they stay within one subnormal ulp of exp."""
    u = np.arange(0xC2AEAC50, 0xC2CFF1B4, 101, dtype=np.uint64).astype(np.uint32)
    x = u.view(np.float32)
    got = oracle.zexpf_array(x)
    ref = np.exp(x.astype(np.float64))
    assert (got > 0).all()
    assert ulp_gap(got, ref).max() <= 1


def test_sampler_uses_zexpf(oracle):
    """The oracle's sampler evaluates its terms with or_zexpf: a two-entry row
    whose second term is one of the arguments where or_zexpf and the
    correctly rounded exp differ returns that term's or_zexpf value in its
    weights (probs * total)."""
    u = np.arange(0xBF000000, 0xC1A00000, 7, dtype=np.uint64).astype(np.uint32)
    x = u.view(np.float32)
    got = oracle.zexpf_array(x)
    cr = np.exp(x.astype(np.float64)).astype(np.float32)
    d = x[(got != cr) & (x < -0.5)][0]
    p = oracle.params(temp=1.0, top_k=2, top_p=1.0, min_p=0.0, repeat_penalty=1.0)
    logits = np.array([0.0, d], np.float32)
    tok, _, diag = oracle.sample_row(p, logits, [0.5, 0.5], cap=2)
    w1 = oracle.zexpf(d)
    total = np.float32(np.float32(1.0) + np.float32(w1))
    assert diag["probs"][1] == np.float32(np.float32(w1) / total)
