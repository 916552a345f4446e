"""GPU parity: whole-vocabulary sampling (top_k = 0 or >= V, the std.mem.sort
branch of src/sampler.zig:198-202) and top-k lists longer than 256
(256 < top_k < V), vs the CPU oracle (stable merge sort, sequential f32 sums).

Bar: token ids, margins, keep counts, uniforms consumed, and the kept
candidates' ids, values and probabilities w_i/total are bit-exact (values of
-0.0 may come back as +0.0 from the whole-order pass, which orders them equal).
Rows take one of two device paths: the prefix pass settles keep from the
top-256 prefix and a bounded total, else the exact whole-order pass sorts the
row; the cases below drive both."""
import numpy as np
import pytest

from paritylib import compare_sample, gpu_sample, oracle_sample
from zinfer_amd.workloads import _bf16_round, pack_mask

pytestmark = pytest.mark.gpu


def _rows(rng, kind, rows, V):
    if kind == "normal":
        return (rng.standard_normal((rows, V)) * 3).astype(np.float32)
    if kind == "t3":
        return (rng.standard_t(3, (rows, V)) * 2).astype(np.float32)
    if kind == "ints":  # many exact ties, including -0.0 and +0.0
        x = rng.integers(-4, 5, (rows, V)).astype(np.float32)
        z = x == 0
        x[z & (rng.random((rows, V)) < 0.5)] = -0.0
        return x
    if kind == "neginf":
        x = (rng.standard_normal((rows, V)) * 2).astype(np.float32)
        x[rng.random((rows, V)) < 0.9] = -np.inf
        return x
    if kind == "flat":
        return np.full((rows, V), 1.5, np.float32)
    if kind == "allneginf":
        return np.full((rows, V), -np.inf, np.float32)
    raise ValueError(kind)


CASES = []
_r = np.random.Generator(np.random.PCG64(11))
for i in range(28):
    V = int(_r.choice([257, 300, 1000, 4099, 32000, 70001, 151936]))
    rows = int(_r.choice([1, 3, 6]))
    kind = str(_r.choice(["normal", "normal", "t3", "ints", "neginf", "flat"]))
    if i % 14 == 13:
        kind = "allneginf"
    ks = [0, 0, V, V + 5, V - 1] + [k for k in (257, 300, 1000) if k < V]
    top_k = int(_r.choice(ks))
    pk = dict(temp=float(_r.choice([0.5, 0.7, 1.0, 1.7])), top_k=top_k,
              top_p=float(_r.choice([1.0, 0.98, 0.9, 0.5, 0.1])), min_p=float(_r.choice([0.0, 0.05, 0.05, 0.3])))
    if _r.random() < 0.5:
        pk.update(repeat_penalty=float(_r.choice([1.1, 1.3, 0.9])), penalty_last_n=int(_r.choice([64, 128, 1000])))
    if _r.random() < 0.3:
        pk.update(freq_penalty=float(_r.choice([0.3, 0.0])), presence_penalty=float(_r.choice([0.5, 0.2])))
        pk.setdefault("penalty_last_n", 64)
    if _r.random() < 0.2:
        pk.update(xtc_probability=float(_r.choice([1.0, 0.5])), xtc_threshold=float(_r.choice([0.1, 0.3])),
                  xtc_min_keep=int(_r.choice([1, 2])))
    CASES.append((i, V, rows, kind, pk, bool(_r.random() < 0.25), bool(_r.random() < 0.25),
                  bool(_r.random() < 0.3)))


def _inputs(rng, V, rows, kind, pk, use_mask, use_edits, bf16):
    x = _rows(rng, kind, rows, V)
    if bf16:
        x = _bf16_round(x)
    u = rng.random((rows, 2), dtype=np.float32)
    hist = hist_len = mask = ei = ed = ec = None
    if "penalty_last_n" in pk:
        H = 300
        hist = rng.integers(0, V, (rows, H), dtype=np.uint32)
        hist[:, ::3] = hist[:, :1]
        hist_len = rng.integers(0, H + 1, rows).astype(np.int32)
    if use_mask:
        bits = rng.random((rows, (V + 31) // 32 * 32)) < 0.4
        bits[:, 0] = True
        mask = pack_mask(bits)
    if use_edits:
        E = 16
        ei = np.stack([rng.choice(V, size=E, replace=False).astype(np.uint32) for _ in range(rows)])
        ed = (rng.random(ei.shape) * 3).astype(np.float32)
        ec = rng.integers(0, E + 1, rows).astype(np.int32)
    return x, u, hist, hist_len, mask, ei, ed, ec


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"w{c[0]}-V{c[1]}-r{c[2]}-{c[3]}-k{c[4]['top_k']}")
def test_whole_vocab_matches_oracle(ctx, oracle, case):
    i, V, rows, kind, pk, use_mask, use_edits, bf16 = case
    rng = np.random.Generator(np.random.PCG64(5000 + i))
    x, u, hist, hl, mask, ei, ed, ec = _inputs(rng, V, rows, kind, pk, use_mask, use_edits, bf16)
    g = gpu_sample(ctx, pk, x, u, hist, hl, mask, ei, ed, ec, bf16=bf16)
    o = oracle_sample(oracle, pk, x, u, hist, hl, mask, ei, ed, ec)
    errs = compare_sample(g, o, pk, V, f"w{i}")
    assert not errs, "\n".join(errs[:20])


@pytest.mark.parametrize("mode", ["minp_cut", "nucleus_0.98", "all_kept", "k300", "k_V_minus_1"])
def test_whole_vocab_paths(ctx, oracle, mode):
    """One setting per device path: min-p settles keep inside the prefix; a
    top-p 0.98 nucleus far longer than 256; top_p = 1, min_p = 0 (every entry
    kept, the draw walks the whole order); and top-k lists of 300 and V - 1."""
    V, rows = 32000, 8
    rng = np.random.Generator(np.random.PCG64(77))
    x = (rng.standard_normal((rows, V)) * 3).astype(np.float32)
    u = rng.random((rows, 2), dtype=np.float32)
    pk = {"minp_cut": dict(temp=0.8, top_k=0, top_p=0.95, min_p=0.3),
          "nucleus_0.98": dict(temp=1.0, top_k=0, top_p=0.98, min_p=0.0),
          "all_kept": dict(temp=1.3, top_k=0, top_p=1.0, min_p=0.0),
          "k300": dict(temp=0.7, top_k=300, top_p=0.9, min_p=0.0),
          "k_V_minus_1": dict(temp=0.7, top_k=V - 1, top_p=0.99, min_p=0.01)}[mode]
    g = gpu_sample(ctx, pk, x, u)
    o = oracle_sample(oracle, pk, x, u)
    errs = compare_sample(g, o, pk, V, mode)
    assert not errs, "\n".join(errs[:20])


def test_whole_vocab_top_p_boundary(ctx, oracle):
    """Rows whose dominant entry holds almost exactly top_p of the mass: the
    prefix pass must leave every row its bounds cannot settle to the exact
    pass (keep 1 vs 2 turns on the last bits of the sequential total)."""
    V, rows = 32000, 64
    rng = np.random.Generator(np.random.PCG64(91))
    x = rng.standard_normal((rows, V)).astype(np.float32)
    lead = np.float32(14.77) + np.linspace(-0.08, 0.08, rows).astype(np.float32)
    x[np.arange(rows), rng.integers(0, V, rows)] = lead
    u = rng.random((rows, 2), dtype=np.float32)
    pk = dict(temp=1.0, top_k=0, top_p=0.98, min_p=0.0)
    g = gpu_sample(ctx, pk, x, u)
    o = oracle_sample(oracle, pk, x, u)
    keeps = {int(d["keep"]) for _, _, d in o}
    assert len(keeps) > 1, "the sweep should straddle the top-p boundary"
    errs = compare_sample(g, o, pk, V, "boundary")
    assert not errs, "\n".join(errs[:20])


def test_config5_full_size_parity(ctx, oracle):
    """Config 5 at its real shape: 512 x 151936 bf16, top_k = 0, top_p 0.98,
    repetition 1.1 over 128-token histories, temperature 1.0."""
    from zinfer_amd.workloads import CONFIGS

    w = CONFIGS[5]()
    pk = dict(w.params)
    g = gpu_sample(ctx, pk, w.logits, w.uniforms, w.hist, w.hist_len, bf16=True)
    o = oracle_sample(oracle, pk, w.logits, w.uniforms, w.hist, w.hist_len)
    errs = compare_sample(g, o, pk, w.vocab, w.name)
    assert not errs, "\n".join(errs[:20])


def test_config5_min_p_zero_full_size(ctx, oracle):
    """Config 5 as its text names it, the worst-case nucleus: min_p = 0, so
    top_p = 0.98 alone cuts the whole-vocabulary order (thousands of entries
    per row) and every row takes the exact whole-order pass.  512 x 151936
    bf16, bit-exact."""
    from zinfer_amd.workloads import CONFIGS

    w = CONFIGS[5]()
    pk = dict(w.params, min_p=0.0)
    g = gpu_sample(ctx, pk, w.logits, w.uniforms, w.hist, w.hist_len, bf16=True)
    o = oracle_sample(oracle, pk, w.logits, w.uniforms, w.hist, w.hist_len)
    errs = compare_sample(g, o, pk, w.vocab, w.name + "_minp0")
    assert not errs, "\n".join(errs[:20])
    assert int(np.median([d["keep"] for _, _, d in o])) > 1000  # the nucleus is long


@pytest.mark.parametrize("min_p,top_p", [(0.05, 0.98), (0.3, 0.9), (0.0, 0.98)])
def test_whole_vocab_large_batch(ctx, oracle, min_p, top_p):
    """>= 256 rows: the prefix pass runs one workgroup per row."""
    V, rows = 32000, 256
    rng = np.random.Generator(np.random.PCG64(int(min_p * 100) + int(top_p * 1000)))
    x = _bf16_round((rng.standard_normal((rows, V)) * 3).astype(np.float32))
    u = rng.random((rows, 2), dtype=np.float32)
    hist = rng.integers(0, V, (rows, 128), dtype=np.uint32)
    hl = np.full(rows, 128, np.int32)
    pk = dict(temp=1.0, top_k=0, top_p=top_p, min_p=min_p, repeat_penalty=1.1, penalty_last_n=128)
    g = gpu_sample(ctx, pk, x, u, hist, hl, bf16=True)
    o = oracle_sample(oracle, pk, x, u, hist, hl)
    errs = compare_sample(g, o, pk, V, f"wl{min_p}")
    assert not errs, "\n".join(errs[:20])


@pytest.mark.parametrize("seed,kind,pk_extra,bf16,use_mask", [
    (1, "normal", dict(top_p=1.0, min_p=0.05), True, False),
    (2, "normal", dict(top_p=0.9, min_p=0.3, temp=0.7), False, False),
    (3, "t3", dict(top_p=0.98, min_p=0.02), True, True),
    (4, "ints", dict(top_p=0.95, min_p=0.05), False, False),     # ties, -0.0 / +0.0
    (5, "neginf", dict(top_p=0.98, min_p=0.05), True, False),    # mostly -inf rows
    (6, "flat", dict(top_p=0.98, min_p=0.05), True, False),      # every entry ties the max: whole-order pass
    (7, "normal", dict(top_p=0.98, min_p=0.9), True, False),     # often a single entry above the floor
])
def test_whole_vocab_large_batch_min_p_prefix(ctx, oracle, seed, kind, pk_extra, bf16, use_mask):
    """>= 256 rows with min_p > 0: the prefix is every entry above a floor that
    trails the row maximum (no top-256 selection); penalties that raise values
    (repetition 0.9, negative presence) and rows the floor cannot settle."""
    V, rows = 20000, 256
    rng = np.random.Generator(np.random.PCG64(900 + seed))
    x = _rows(rng, kind, rows, V)
    if bf16:
        x = _bf16_round(x)
    u = rng.random((rows, 2), dtype=np.float32)
    hist = rng.integers(0, V, (rows, 100), dtype=np.uint32)
    hist[:, -6:] = np.argsort(-x, axis=1)[:, :6].astype(np.uint32)
    hl = rng.integers(0, 101, rows).astype(np.int32)
    pk = dict(temp=1.0, top_k=0, repeat_penalty=float(rng.choice([1.1, 0.9])), presence_penalty=-0.3,
              penalty_last_n=100)
    pk.update(pk_extra)
    mask = None
    if use_mask:
        bits = rng.random((rows, (V + 31) // 32 * 32)) < 0.5
        bits[:, 0] = True
        mask = pack_mask(bits)
    g = gpu_sample(ctx, pk, x, u, hist, hl, mask, bf16=bf16)
    o = oracle_sample(oracle, pk, x, u, hist, hl, mask)
    errs = compare_sample(g, o, pk, V, f"mp-{kind}")
    assert not errs, "\n".join(errs[:20])
