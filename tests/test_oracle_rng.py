"""Pins of the oracle's restatement of Zig's std.Random.DefaultPrng and
Random.float(f32) (src/sampler.zig:40, :52, :249, :270; server.zig:414
reseeds it), from what the mathematics and the published algorithms fix.

- The xoshiro256 linear engine (the state update of or_xoshiro_next) is a
  256 x 256 matrix M over GF(2).  Blackman and Vigna chose its shift and
  rotate so that M has full period 2^256 - 1.  The test checks M^(2^256) = M
  and M^((2^256 - 1) / p) != I for every prime p of 2^256 - 1 (the eleven
  prime factors of the Fermat numbers F0..F7).  It also checks the published
  jump polynomials: JUMP advances the state by 2^128 steps and LONG_JUMP by
  2^192 steps.  Both are coefficient vectors of x^(2^128) and x^(2^192)
  modulo the engine's characteristic polynomial.  A wrong shift, rotate or
  xor order fails these checks.
- The ++ output scrambler (rotl(s0 + s3, 23) + s0) is not pinned by any
  published vector available here: PARITY UNPINNED, as recorded in the
  oracle header.
- Random.float(f32): for crafted states whose outputs are chosen words, the
  value is the real number 2^-(1 + lz) * (1 + m / 2^23), where m is the low 23
  bits of the first draw and lz the leading-zero count (extended by a second
  draw when the first has 41 or more leading zeros).  Each case is computed
  here with math.ldexp, independently of the oracle's bit assembly.
"""
from __future__ import annotations

import math
import random

import numpy as np
import pytest

M64 = (1 << 64) - 1


@pytest.fixture(scope="module")
def oracle():
    from oracle import pyoracle

    pyoracle.lib()
    return pyoracle


def rotl(x, k):
    return ((x << k) | (x >> (64 - k))) & M64


def rotr(x, k):
    return ((x >> k) | (x << (64 - k))) & M64


def clz64(x):
    return 64 - x.bit_length()


# ---------------------------------------------------------------- GF(2) tools
def state_to_bits(s):
    v = np.zeros(256, np.float32)
    for j in range(256):
        v[j] = (s[j // 64] >> (j % 64)) & 1
    return v


def bits_to_state(v):
    s = [0, 0, 0, 0]
    for j in range(256):
        if int(v[j]) & 1:
            s[j // 64] |= 1 << (j % 64)
    return s


def gf2_mul(a, b):
    return np.mod(a @ b, 2.0).astype(np.float32)


@pytest.fixture(scope="module")
def engine(oracle):
    """M (column j = the state update applied to basis state e_j) and the
    table M^(2^i), i = 0..256."""
    M = np.zeros((256, 256), np.float32)
    for j in range(256):
        s = [0, 0, 0, 0]
        s[j // 64] = 1 << (j % 64)
        t, _ = oracle.xoshiro_step(s)
        M[:, j] = state_to_bits(t)
    pw = [M]
    for _ in range(256):
        pw.append(gf2_mul(pw[-1], pw[-1]))
    return M, pw


def mat_pow(pw, e):
    R = np.eye(256, dtype=np.float32)
    i = 0
    while e:
        if e & 1:
            R = gf2_mul(R, pw[i])
        e >>= 1
        i += 1
    return R


def is_probable_prime(n):
    """Miller-Rabin with the first twelve primes as bases: deterministic for
    n < 3.3e24, which covers every factor below."""
    if n < 2:
        return False
    small = [2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37]
    for p in small:
        if n % p == 0:
            return n == p
    d, r = n - 1, 0
    while d % 2 == 0:
        d //= 2
        r += 1
    for a in small:
        x = pow(a, d, n)
        if x in (1, n - 1):
            continue
        for _ in range(r - 1):
            x = x * x % n
            if x == n - 1:
                break
        else:
            return False
    return True


# Prime factors of 2^256 - 1 = F0 F1 ... F7 (Fermat numbers F_n = 2^(2^n) + 1):
# F0..F4 are prime; F5 = 641 * 6700417 (Euler); F6 = 274177 * 67280421310721
# (Landry); F7 = 59649589127497217 * 5704689200685129054721 (Morrison-Brillhart).
PRIMES_2_256_M1 = [3, 5, 17, 257, 65537, 641, 6700417, 274177, 67280421310721, 59649589127497217,
                   5704689200685129054721]


def test_factorisation_of_2_256_minus_1():
    prod = 1
    for p in PRIMES_2_256_M1:
        assert is_probable_prime(p), p
        prod *= p
    assert prod == (1 << 256) - 1


def test_engine_is_linear(oracle, engine):
    """M built from basis states reproduces the update of random states (the
    update is linear over GF(2), as xoshiro's is)."""
    M, _ = engine
    rng = random.Random(7)
    for _ in range(8):
        s = [rng.getrandbits(64) for _ in range(4)]
        t, _ = oracle.xoshiro_step(s)
        assert bits_to_state(gf2_mul(M, state_to_bits(s)[:, None])[:, 0]) == t


def test_engine_full_period(engine):
    """The linear engine has period exactly 2^256 - 1 (Blackman and Vigna
    2018): M^(2^256 - 1) = I and M^((2^256 - 1) / p) != I for every prime p."""
    M, pw = engine
    assert np.array_equal(pw[256], M)  # M^(2^256) = M, i.e. M^(2^256 - 1) = I (M is invertible)
    assert np.linalg.matrix_rank(M) == 256
    I = np.eye(256, dtype=np.float32)
    full = (1 << 256) - 1
    for p in PRIMES_2_256_M1:
        assert not np.array_equal(mat_pow(pw, full // p), I), p


# xoshiro256 jump constants, published with the reference C implementation
# (prng.di.unimi.it/xoshiro256plusplus.c; Zig's std.Random.Xoshiro256.jump
# uses the same): JUMP is equivalent to 2^128 calls to next(), LONG_JUMP to
# 2^192 calls.
JUMP = [0x180EC6D33CFD0ABA, 0xD5A61266F0C9392C, 0xA9582618E03FC9AA, 0x39ABDC4529B1661C]
LONG_JUMP = [0x76E15D3EFEFDCBBF, 0xC5004E441C522FB3, 0x77710069854EE241, 0x39109BB02ACBE635]


def jump_with_next(oracle, s, poly):
    """The published jump loop: xor together the states at the polynomial's
    set bits, stepping with the oracle's own update."""
    acc = [0, 0, 0, 0]
    cur = list(s)
    for w in poly:
        for b in range(64):
            if (w >> b) & 1:
                acc = [a ^ c for a, c in zip(acc, cur)]
            cur, _ = oracle.xoshiro_step(cur)
    return acc


@pytest.mark.parametrize("poly,log2", [(JUMP, 128), (LONG_JUMP, 192)])
def test_jump_polynomials(oracle, engine, poly, log2):
    _, pw = engine
    rng = random.Random(log2)
    for _ in range(3):
        s = [rng.getrandbits(64) for _ in range(4)]
        want = bits_to_state(gf2_mul(pw[log2], state_to_bits(s)[:, None])[:, 0])
        assert jump_with_next(oracle, s, poly) == want


def test_engine_matches_seeding_by_splitmix(oracle):
    """DefaultPrng.init(seed) fills s[0..3] with four splitmix64 outputs."""
    import ctypes as C

    s = (C.c_uint64 * 4)()
    oracle.lib().or_xoshiro_seed(s, 1234567)
    assert [int(x) for x in s] == oracle.splitmix64_seq(1234567, 4)


# ------------------------------------------------------- Random.float(f32)
def crafted_state(w1, u=None, rng=None):
    """A state whose first output is w1 (s0 = 0 makes the output rotl(s3, 23)).
    With u given, s1 is chosen so that the state after one step has s0' = u,
    s3' = rotl(u, 45); the second output then depends on u alone."""
    s3 = rotr(w1, 23)
    s1 = 0 if u is None else (s3 ^ u)
    return [0, s1, (rng.getrandbits(64) if rng else 0), s3]


def expected_float(m, lz):
    return math.ldexp(1.0 + m / 2.0**23, -(1 + lz))


@pytest.mark.parametrize("lz", [0, 1, 2, 7, 22, 23, 24, 39, 40])
def test_rand_f32_single_draw(oracle, lz):
    rng = random.Random(lz)
    for _ in range(20):
        low = rng.getrandbits(63 - lz) if lz < 63 else 0
        w = (1 << (63 - lz)) | low
        s = crafted_state(w, rng=rng)
        _, out = oracle.xoshiro_step(s)
        assert out == w
        v, after = oracle.rand_f32_from(s)
        assert v == expected_float(w & 0x7FFFFF, lz)
        assert after == oracle.xoshiro_step(s)[0]  # one draw consumed
        assert 0.0 <= v < 1.0


def second_output(u):
    s0, s3 = u, rotl(u, 45)
    return (rotl((s0 + s3) & M64, 23) + s0) & M64


@pytest.mark.parametrize("lz1,lz2", [(41, 0), (41, 3), (50, 1), (63, 5), (64, 0), (64, 9)])
def test_rand_f32_second_draw(oracle, lz1, lz2):
    """41 or more leading zeros: the exponent takes 41 + clz(second draw); the
    mantissa stays the first draw's low 23 bits."""
    rng = random.Random(1000 * lz1 + lz2)
    w1 = 0 if lz1 == 64 else ((1 << (63 - lz1)) | rng.getrandbits(63 - lz1))
    if lz1 == 63:
        w1 = 1
    assert clz64(w1) == lz1
    for _ in range(5):
        while True:
            u = rng.getrandbits(64)
            if clz64(second_output(u)) == lz2:
                break
        s = crafted_state(w1, u=u, rng=rng)
        st1, o1 = oracle.xoshiro_step(s)
        assert o1 == w1
        _, o2 = oracle.xoshiro_step(st1)
        assert o2 == second_output(u)
        v, _ = oracle.rand_f32_from(s)
        assert v == expected_float(w1 & 0x7FFFFF, 41 + lz2)


def test_rand_f32_distribution_of_exponents(oracle):
    """P(value < 2^-j) = 2^-j for the crafted exponent ranges: each
    leading-zero count maps to one binade, each binade's mantissas are its 2^23
    evenly spaced values."""
    for lz in range(0, 41, 5):
        lo, hi = expected_float(0, lz), expected_float(0x7FFFFF, lz)
        assert lo == 2.0 ** -(1 + lz) and hi < 2.0 ** -lz
