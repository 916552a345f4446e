"""Pins for the oracle beyond the reference's KATs: hand-derived values and
independent formulations (numpy / scipy / brute force), each chosen so that a
plausible restatement mistake -- a wrong tie rule, a tempered top-p, an f64
or reassociated sum, `<` for `<=`, a dropped term -- fails."""
import numpy as np
import pytest


def exp32(x):
    """The reference's @exp(f32) (oracle/or_zexpf, pinned in test_oracle_expf.py)."""
    from oracle import pyoracle

    return np.float32(pyoracle.zexpf(float(np.float32(x))))


# ------------------------------------------------------------------ top-k
@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("k", [1, 7, 40, 0])
def test_topk_order_is_value_desc_id_asc(oracle, seed, k):
    """Insertion top-k (k < V, sampler.zig:203-209) and stable sort (k = V,
    :198-201) both yield the first k of lexsort(id asc, value desc), with
    -0.0 tying +0.0."""
    rng = np.random.default_rng(seed)
    V = 300
    x = rng.integers(-3, 4, V).astype(np.float32)  # heavy ties
    x[x == 0] = np.where(rng.random((x == 0).sum()) < 0.5, -0.0, 0.0)
    p = oracle.params(temp=1.0, top_k=k, top_p=1.0, min_p=0.0)
    kk = V if k == 0 else k
    _, _, diag = oracle.sample_row(p, x, [0.5, 0.5], cap=kk)
    order = np.lexsort((np.arange(V), -x.astype(np.float64)))[:kk]
    assert np.array_equal(diag["ids"], order.astype(np.uint32))


# ------------------------------------------------------------------ top-p
def _sorted_candidates(x, k):
    order = np.lexsort((np.arange(x.size), -x.astype(np.float64)))[:k]
    return x[order], order


@pytest.mark.parametrize("seed", range(8))
def test_top_p_keep_is_sequential_f32_over_untempered_weights(oracle, seed):
    """keep = first i with acc_i >= top_p * total, acc and total sequential f32
    sums of exp(v - max) over the top-k (sampler.zig:215-228), independent of
    temperature.  numpy's float32 add.accumulate is a sequential sum."""
    rng = np.random.default_rng(100 + seed)
    x = (rng.standard_normal(2000) * 2).astype(np.float32)
    k, top_p = 64, np.float32(rng.uniform(0.3, 0.99))
    v, _ = _sorted_candidates(x, k)
    e = np.array([exp32(vi - v[0]) for vi in v], np.float32)
    acc = np.add.accumulate(e, dtype=np.float32)
    keep = int(np.argmax(acc >= np.float32(top_p) * acc[-1])) + 1
    for temp in (0.3, 1.0, 2.5):  # a tempered top-p would move keep
        p = oracle.params(temp=temp, top_k=k, top_p=float(top_p), min_p=0.0)
        _, _, diag = oracle.sample_row(p, x, [0.5, 0.5], cap=k)
        assert diag["keep"] == keep


def test_top_p_uses_f32_sequential_total_not_f64():
    """Terms of exactly half an ulp vanish in a sequential f32 sum (ties to
    even) but not in f64: 1 + 1000 * 2^-24 stays 1.0f."""
    e = np.array([1.0] + [2.0 ** -24] * 1000, np.float32)
    assert np.add.accumulate(e, dtype=np.float32)[-1] == np.float32(1.0)
    assert float(np.sum(e.astype(np.float64))) > 1.00005


def test_top_p_f32_total_decides_keep(oracle):
    """Logits whose untempered weights are 1 and many tiny equal terms: the
    sequential f32 total stays 1.0 so top_p = 0.9999 keeps only token 0; an
    f64 total would keep more."""
    tiny = np.float32(np.log(2.0 ** -24 * 1.0000001))  # exp32(tiny) rounds to about 2^-24
    x = np.full(300, tiny, np.float32)
    x[0] = 0.0
    p = oracle.params(temp=1.0, top_k=300, top_p=0.9999, min_p=0.0)
    _, _, diag = oracle.sample_row(p, x, [0.5, 0.5], cap=300)
    e = exp32(tiny)
    assert e < 2.0 ** -23  # below one ulp of 1.0: lost in f32, kept in f64
    assert diag["keep"] == 1


# ------------------------------------------------------------------ min-p
def test_min_p_cut_is_strictly_below(oracle):
    """min-p keeps candidates with exp(v - max) >= min_p (the cut uses `<`,
    sampler.zig:230) and never keeps fewer than one (:231)."""
    x = np.array([10.0, 9.0, 6.0, 1.0] + [-50.0] * 6, np.float32)
    e1 = float(exp32(np.float32(9.0) - np.float32(10.0)))
    for min_p, keep in [(0.10, 2), (e1, 2), (np.nextafter(np.float32(e1), np.float32(1)), 1), (1.5, 1)]:
        p = oracle.params(temp=1.0, top_k=10, top_p=1.0, min_p=float(min_p))
        _, _, diag = oracle.sample_row(p, x, [0.5, 0.5], cap=10)
        assert diag["keep"] == keep, (min_p, diag["keep"])


# ------------------------------------------------------------------- draw
def test_draw_boundary_uses_le(oracle):
    """r = u * total; r -= w_i; the first r <= 0 wins (sampler.zig:270-274).
    Weights 1, 0.5, 0.5 (exact, total 2): u = 0.5 lands exactly on the first
    boundary and must pick candidate 0, u just above picks candidate 1."""
    ln = np.float32(np.log(0.5))
    x = np.array([0.0, ln, ln] + [-80.0] * 5, np.float32)
    p = oracle.params(temp=1.0, top_k=8, top_p=1.0, min_p=0.0)
    _, _, diag = oracle.sample_row(p, x, [0.5, 0.5], cap=8)
    w = np.array([exp32(v) for v in x[:3]], np.float32)
    assert w[0] == 1.0 and w[1] == np.float32(0.5) and diag["total"] == 2.0
    tot = diag["total"]
    u0 = w[0] / tot  # r = u0 * total == w_0 exactly
    assert oracle.sample_row(p, x, [u0, 0.5])[0] == 0
    assert oracle.sample_row(p, x, [np.nextafter(u0, np.float32(1)), 0.5])[0] == 1


@pytest.mark.parametrize("temp", [0.6, 1.0, 1.7])
def test_draw_frequencies_follow_tempered_weights(oracle, temp):
    """Sweeping u over a fine grid, each kept candidate is drawn with
    frequency w_i / total where w_i = exp((v_i - max) / T) (sampler.zig:236-242)."""
    rng = np.random.default_rng(int(temp * 10))
    x = (rng.standard_normal(500)).astype(np.float32)
    p = oracle.params(temp=temp, top_k=12, top_p=1.0, min_p=0.0)
    v, ids = _sorted_candidates(x, 12)
    w = np.exp((v.astype(np.float64) - v[0]) / temp)
    w /= w.sum()
    N = 20000
    counts = {}
    for u in (np.arange(N, dtype=np.float64) + 0.5) / N:
        t = oracle.sample_row(p, x, [np.float32(u), 0.5])[0]
        counts[t] = counts.get(t, 0) + 1
    for i, tid in enumerate(ids):
        assert abs(counts.get(int(tid), 0) / N - w[i]) < 2e-3


# ------------------------------------------------------------------- XTC
def test_xtc_removes_leading_run_above_threshold(oracle):
    """XTC drops c[0 .. pos_last) where pos_last is the last index of the
    leading run with p >= threshold (sampler.zig:251-266).  Probabilities
    0.4, 0.3, 0.2, 0.1 with threshold 0.25: the run is {0, 1}, pos_last = 1,
    so candidate 0 is removed and 1, 2, 3 remain."""
    x = np.log(np.array([0.4, 0.3, 0.2, 0.1] + [1e-30] * 4)).astype(np.float32)
    p = oracle.params(temp=1.0, top_k=8, top_p=1.0, min_p=0.0, xtc_probability=1.0, xtc_threshold=0.25,
                      xtc_min_keep=1)
    toks = set()
    for u in np.linspace(0, 1, 400, endpoint=False):
        t, _, diag = oracle.sample_row(p, x, [0.0, u], cap=8)
        assert diag["start"] == 1
        toks.add(t)
    assert toks == {1, 2, 3}
    # chance above the probability: no exclusion, two draws consumed
    p2 = oracle.params(temp=1.0, top_k=8, top_p=1.0, min_p=0.0, xtc_probability=0.5, xtc_threshold=0.25)
    _, _, diag = oracle.sample_row(p2, x, [0.75, 0.1], cap=8)
    assert diag["start"] == 0 and diag["ndraws"] == 2


# -------------------------------------------------------------- penalties
def test_repetition_penalty_hand_values(oracle):
    """sampler.zig:91-100: positive logits are divided, non-positive
    multiplied, each distinct id once."""
    x = np.array([3.0, -2.0, 0.0, 6.0, 1.5], np.float32)
    out = oracle.apply_penalty(x, [0, 1, 2, 0, 0, 1], 1.5)
    assert out.tolist() == [2.0, -3.0, 0.0, 6.0, 1.5]


def test_frequency_presence_hand_values(oracle):
    """Extension: l -= count * freq + presence for ids in the window, after
    the repetition step.  id 0 appears 3 times: 3 - (3*0.5 + 0.25) = 1.25;
    id 3 once: 6 - (0.5 + 0.25) = 5.25; with rp 2: id 0 -> 1.5 - 1.75."""
    x = np.array([3.0, 7.0, 1.0, 6.0], np.float32)
    out = oracle.apply_penalty(x, [0, 3, 0, 0], 1.0, 0.5, 0.25)
    assert out.tolist() == [1.25, 7.0, 1.0, 5.25]
    out = oracle.apply_penalty(x, [0, 3, 0, 0], 2.0, 0.5, 0.25)
    assert out.tolist() == [1.5 - 1.75, 7.0, 1.0, 3.0 - 0.75]


def test_dry_matches_brute_force(oracle):
    """DRY edits (sampler.zig:104-187) against an O(L^2) restatement: for each
    earlier position, the longest common suffix with the current context
    (bounded by the breaker limit) names the continuation token."""
    rng = np.random.default_rng(9)
    for trial in range(60):
        L = int(rng.integers(3, 60))
        hist = rng.integers(0, 5, L).tolist()
        brk = [4] if trial % 3 == 0 else []
        allowed = int(rng.integers(1, 4))
        ids, d = oracle.dry_edits(hist, brk, 0.8, 1.75, allowed, 1024)
        R = hist[::-1]
        rep_limit = next((i for i, t in enumerate(R) if t in brk), L)
        expect = {}
        if L > allowed and rep_limit >= allowed:
            for kpos in range(1, L):
                n = 0
                while n < min(L - kpos, rep_limit) and R[n] == R[kpos + n]:
                    n += 1
                if n >= allowed and R[kpos - 1] not in brk:
                    expect[R[kpos - 1]] = max(expect.get(R[kpos - 1], 0), n)
        got = dict(zip(ids.tolist(), d.tolist()))
        assert set(got) == set(expect), (hist, brk, allowed)
        for t, n in expect.items():
            assert abs(got[t] - 0.8 * 1.75 ** (n - allowed)) < 1e-5 * got[t]


# ----------------------------------------------------------------- argmax
def _lane16_model(x):
    """Independent numpy model of the 2x8-lane SIMD argmax."""
    V = x.size
    body = (V // 16) * 16
    cls = x[:body].reshape(-1, 16)
    first = np.argmax(cls, axis=0)  # first maximum per class
    cmax = cls[first, np.arange(16)]
    cidx = first * 16 + np.arange(16)
    seq = [(cmax[c], cidx[c]) for j in range(8) for c in (j, j + 8)] + [(x[i], i) for i in range(body, V)]
    best, second, bi = -np.inf, -np.inf, 0
    for v, i in seq:
        if v > best:
            second, best, bi = best, v, i
        elif v > second:
            second = v
    return int(bi), float(best - second) if second > -np.inf else 10.0


def test_argmax_lane16_hand_cases(oracle):
    x = np.zeros(32, np.float32)
    x[3] = x[8] = 5.0  # equal maxima: class 8 is reduced before class 3
    assert oracle.argmax_with_margin(x) == (8, 0.0)
    y = np.zeros(32, np.float32)
    y[3], y[19] = 5.0, 4.0  # both in class 3: the 4 is hidden from the margin
    assert oracle.argmax_with_margin(y) == (3, 5.0)
    assert oracle.argmax_true(y) == (3, 1.0)
    z = np.full(20, -np.inf, np.float32)
    assert oracle.argmax_with_margin(z) == (0, 10.0)


@pytest.mark.parametrize("V", [16, 17, 33, 100, 1000, 4097])
def test_argmax_lane16_model(oracle, V):
    rng = np.random.default_rng(V)
    for _ in range(20):
        x = rng.integers(-2, 3, V).astype(np.float32)
        assert oracle.argmax_with_margin(x) == _lane16_model(x)


def test_argmax_small_v_path(oracle):
    """V < 16 (sampler.zig:535-551): exact first max; margin x[best] - x[second]."""
    assert oracle.argmax_with_margin(np.array([1, 3, 3, 2], np.float32)) == (1, 0.0)
    assert oracle.argmax_with_margin(np.array([5], np.float32)) == (0, 10.0)
    assert oracle.argmax_with_margin(np.array([2, 7, 1], np.float32)) == (1, 5.0)


# ----------------------------------------------------------------- entropy
@pytest.mark.parametrize("seed", range(4))
def test_entropy_topk_vs_scipy(oracle, seed):
    from scipy.special import softmax
    from scipy.stats import entropy

    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(5000) * 2).astype(np.float32)
    if seed == 1:
        x[7] += 15.0
    if seed == 2:
        x[rng.random(5000) < 0.5] = -np.inf
    H, ids, probs = oracle.entropy_topk(x, 8)
    p = softmax(x.astype(np.float64))
    assert abs(H - entropy(p)) <= 1e-9 * max(1.0, entropy(p))
    order = np.lexsort((np.arange(x.size), -x.astype(np.float64)))[:8]
    assert np.array_equal(ids, order.astype(np.uint32))
    np.testing.assert_allclose(probs, p[order], rtol=1e-12)


# -------------------------------------------------------------------- mask
def test_apply_mask_bit_order(oracle):
    """id t is allowed iff bit (t & 31) of word t >> 5 is set."""
    words = np.array([0b1010, 1 << 31, 0x1], np.uint32)
    x = np.arange(70, dtype=np.float32)
    out = oracle.apply_mask(x, words)
    allowed = np.nonzero(np.isfinite(out))[0].tolist()
    assert allowed == [1, 3, 63, 64]


# ------------------------------------------------------------------ final-logit softcap
@pytest.mark.parametrize("cap", [30.0, 15.0, 50.0, 1.0])
def test_softcap_is_tanh(oracle, cap):
    """model.zig:2492-2510 computes cap*tanh(l/cap) through exp: within a few
    f32 ulps of cap of the f64 closed form (a dropped factor 2, a wrong sign or
    an unclamped exp fails by far more); |result| <= cap; odd within ulps."""
    rng = np.random.default_rng(int(cap))
    ls = np.concatenate([rng.standard_normal(2000) * cap * 2, rng.standard_normal(500) * 1e-3,
                         np.linspace(-12 * cap, 12 * cap, 2001), [0.0, -0.0, 1e-30, -1e-30]]).astype(np.float32)
    got = np.array([oracle.softcap(x, cap) for x in ls], np.float64)
    want = cap * np.tanh(ls.astype(np.float64) / cap)
    assert np.max(np.abs(got - want)) <= cap * 2.0 ** -22
    assert np.all(np.abs(got) <= cap)
    neg = np.array([oracle.softcap(-x, cap) for x in ls], np.float64)
    assert np.max(np.abs(neg + got)) <= cap * 2.0 ** -22


def test_softcap_saturates_and_special_values(oracle):
    """|l| >= 9 cap clamps to the same value as l = +-9 cap; -inf gives the
    low end (a masked, pruned logit stays finite until the mask); NaN takes
    the -9 end, the maxnum rule of @max (a NaN operand yields the other)."""
    cap = 30.0
    hi, lo = oracle.softcap(9 * cap, cap), oracle.softcap(-9 * cap, cap)
    assert hi == -lo and 0.9999 * cap < hi <= cap
    for x in [9.5 * cap, 1e6, 3.4e38, np.inf]:
        assert oracle.softcap(x, cap) == hi
        assert oracle.softcap(-x, cap) == lo
    assert oracle.softcap(float("nan"), cap) == lo
    assert oracle.softcap(0.0, cap) == 0.0


@pytest.mark.parametrize("cap", [30.0, 15.0, 1.0])
def test_softcap_tail_is_tanh(oracle, cap):
    """The scalar tail (model.zig:2511-2513) is cap * tanh(l / cap) with no
    clamp: within two f32 ulps of cap * tanh(fl(l / cap)) in f64 (half an ulp
    each for the rounded tanh, scaled by cap, and for the product), odd,
    tanh(+-inf) = +-1, signed zero kept, NaN propagated."""
    rng = np.random.default_rng(int(cap) + 100)
    ls = np.concatenate([rng.standard_normal(2000) * cap * 2, rng.standard_normal(500) * 1e-3 * cap,
                         np.linspace(-12 * cap, 12 * cap, 2001)]).astype(np.float32)
    got = np.array([oracle.softcap_tail(x, cap) for x in ls], np.float64)
    q = (ls.astype(np.float64) / cap).astype(np.float32).astype(np.float64)  # fl(l / cap)
    want = cap * np.tanh(q)
    ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - want) <= 2.0 * ulp + 1e-45)
    neg = np.array([oracle.softcap_tail(-x, cap) for x in ls], np.float64)
    assert np.array_equal(neg, -got)
    assert oracle.softcap_tail(np.inf, cap) == cap and oracle.softcap_tail(-np.inf, cap) == -cap
    assert np.signbit(oracle.softcap_tail(-0.0, cap)) and oracle.softcap_tail(0.0, cap) == 0.0
    assert np.isnan(oracle.softcap_tail(float("nan"), cap))


def test_softcap_tail_covers_the_last_v_mod_32(oracle):
    """Only ids >= 32*floor(V/32) take the tail.  Near zero the body's
    (e^2z - 1)/(e^2z + 1) loses most of its bits to the cancellation in
    e^2z - 1, the tail does not, so a row of small logits tells the two apart
    by position: sampling it with the cap matches a row capped with the body
    formula below 32*floor(V/32) and the tail formula above it."""
    cap = 30.0
    for V in (33, 45, 64 + 31, 320):
        body = V // 32 * 32
        x = (np.arange(V, dtype=np.float32) + 1.0) * np.float32(1e-3)  # distinct small logits, rising with id
        capped = np.array([oracle.softcap(v, cap) if i < body else oracle.softcap_tail(v, cap)
                           for i, v in enumerate(x)], np.float32)
        tail_vals = np.array([oracle.softcap_tail(v, cap) for v in x[body:]], np.float32)
        body_vals = np.array([oracle.softcap(v, cap) for v in x[body:]], np.float32)
        if V > body:
            assert not np.array_equal(tail_vals, body_vals)  # the formulas differ on these inputs
        pk = dict(temp=0.7, top_k=0, top_p=1.0, min_p=0.0)
        _, _, d1 = oracle.sample_row(oracle.params(final_logit_softcap=cap, **pk), x, [0.5, 0.5], cap=V)
        _, _, d2 = oracle.sample_row(oracle.params(**pk), capped, [0.5, 0.5], cap=V)
        assert np.array_equal(d1["row"], capped)  # the row as the sampler saw it
        assert np.array_equal(d1["ids"], d2["ids"]) and np.array_equal(d1["vals"], d2["vals"])


@pytest.mark.parametrize("seed", range(4))
def test_softcap_precedes_mask_and_penalty(oracle, seed):
    """The cap belongs to the forward (model.zig:2492), so it runs before the
    grammar mask (gen.zig:457-460) and the penalties (sampler.zig:191):
    sampling raw logits with the cap equals sampling the capped row without
    it, and differs from capping after the penalty."""
    rng = np.random.default_rng(seed)
    V, cap = 320, 5.0
    x = (rng.standard_normal(V) * 8).astype(np.float32)
    win = np.argsort(-x)[:6].astype(np.uint32)
    mask = rng.integers(0, 2**32, V // 32, dtype=np.uint64).astype(np.uint32)
    mask[0] |= 1
    pk = dict(temp=0.9, top_k=50, top_p=0.95, min_p=0.02, repeat_penalty=1.4, penalty_last_n=64)
    capped = np.array([oracle.softcap(v, cap) for v in x], np.float32)
    u = [0.37, 0.81]
    t1, m1, d1 = oracle.sample_row(oracle.params(final_logit_softcap=cap, **pk), x, u, mask=mask, window=win, cap=50)
    t2, m2, d2 = oracle.sample_row(oracle.params(**pk), capped, u, mask=mask, window=win, cap=50)
    assert (t1, m1) == (t2, m2) and np.array_equal(d1["ids"], d2["ids"])
    assert np.array_equal(d1["probs"], d2["probs"])
    pen_first = oracle.apply_penalty(x, win, 1.4)
    late = np.array([oracle.softcap(v, cap) for v in pen_first], np.float32)
    assert not np.array_equal(late[win], oracle.apply_penalty(capped, win, 1.4)[win])


# ------------------------------------------------------------------ std.math.pow (DRY penalty)
def test_pow_zig_special_cases(oracle):
    """The special cases of std.math.pow, in its order: y = 0 or x = 1 give 1,
    y = 1 gives x, y = +-0.5 take sqrt, 0 and infinities by sign rules."""
    pw = oracle.pow_zig
    assert pw(7.0, 0.0) == 1.0 and pw(1.0, 123.5) == 1.0 and pw(1.0, float("nan")) == 1.0
    assert pw(1.75, 1.0) == np.float32(1.75)
    assert pw(2.0, 0.5) == np.sqrt(np.float32(2.0)) and pw(2.0, -0.5) == np.float32(1) / np.sqrt(np.float32(2.0))
    assert pw(0.0, 3.0) == 0.0 and pw(0.0, -2.0) == np.inf and np.signbit(pw(-0.0, 3.0))
    assert pw(0.5, np.inf) == 0.0 and pw(2.0, np.inf) == np.inf and pw(-1.0, np.inf) == 1.0
    assert pw(np.inf, -1.0) == 0.0 and pw(np.inf, 2.0) == np.inf
    assert np.isnan(pw(-2.0, 0.5 + 0.25))


@pytest.mark.parametrize("base", [1.75, 1.0001, 3.0, 1.1])
def test_pow_zig_integer_and_fractional_powers(oracle, base):
    """Integer exponents by repeated squaring and the fractional part through
    exp(yf*log x): within the squaring chain's error bound of the f64 closed
    form, about (2*yi + 16) f32 rounding errors relative (the error of
    x1^(2^j) doubles with each squaring), where a dropped multiply, a wrong
    exponent carry or an unshifted yf fails by far more; a single squaring
    is exactly fl(x*x)."""
    for y in list(range(0, 60)) + [0.3, 1.6, 2.75, 10.49, 10.51, 88.0 / np.log(np.float32(base))]:
        yf = np.float32(y)
        got = np.float64(oracle.pow_zig(base, float(yf)))
        want = np.float64(np.float32(base)) ** np.float64(yf)
        if not np.isfinite(want) or want > 3e38:
            continue
        tol = (2 * np.floor(abs(yf) + 0.5) + 16) * 2.0 ** -24 * want
        assert abs(got - want) <= tol, (base, y, got, want)
    b = np.float32(base)
    assert oracle.pow_zig(base, 2.0) == np.float32(b * b)  # one squaring, one rounding
