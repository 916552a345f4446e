"""GPU parity: argmaxWithMargin (reference 2x8-lane rules and lowest-index),
entropy / top-k / accept (config 4), in-place mask application."""
import numpy as np
import pytest

from paritylib import dev, f32bits, to_device

pytestmark = pytest.mark.gpu


def _argmax_case(rng, V, kind):
    if kind == "ints":
        return rng.integers(-2, 3, V).astype(np.float32)
    if kind == "neginf":
        x = np.full(V, -np.inf, np.float32)
        if V > 3:
            x[rng.integers(0, V, 3)] = rng.standard_normal(3).astype(np.float32)
        return x
    if kind == "allneginf":
        return np.full(V, -np.inf, np.float32)
    if kind == "zeros":
        x = np.zeros(V, np.float32)
        x[rng.random(V) < 0.5] = -0.0
        return x
    return (rng.standard_normal(V) * 3).astype(np.float32)


@pytest.mark.parametrize("V", [1, 2, 3, 15, 16, 17, 31, 32, 33, 100, 1024, 4097, 32000, 65537, 262144])
@pytest.mark.parametrize("kind", ["normal", "ints", "neginf", "allneginf", "zeros"])
def test_argmax_rows(ctx, oracle, V, kind):
    rng = np.random.Generator(np.random.PCG64(V * 7 + len(kind)))
    rows = 3
    x = np.stack([_argmax_case(rng, V, kind) for _ in range(rows)])
    tok, margin, tok_low, margin_true = ctx.argmax_rows(to_device(x), vocab=V)
    tok, margin = tok.cpu().numpy(), margin.cpu().numpy()
    tok_low, margin_true = tok_low.cpu().numpy(), margin_true.cpu().numpy()
    for r in range(rows):
        et, em = oracle.argmax_with_margin(x[r])
        assert tok[r] == et, (r, tok[r], et)
        assert f32bits(margin[r]) == f32bits(em) or (np.isnan(margin[r]) and np.isnan(em)), (r, margin[r], em)
        lt, lm = oracle.argmax_true(x[r])
        assert tok_low[r] == lt, (r, tok_low[r], lt)
        assert margin_true[r] == lm or (np.isnan(margin_true[r]) and np.isnan(lm)), (r, margin_true[r], lm)


def test_argmax_bf16(ctx, oracle):
    from zinfer_amd.workloads import _bf16_round

    rng = np.random.Generator(np.random.PCG64(5))
    x = _bf16_round(rng.standard_normal((4, 151936)).astype(np.float32) * 3)
    tok, margin, tok_low, _ = ctx.argmax_rows(to_device(x, bf16=True), vocab=151936)
    for r in range(4):
        et, em = oracle.argmax_with_margin(x[r])
        assert int(tok[r]) == et and float(margin[r]) == em
        assert int(tok_low[r]) == oracle.argmax_true(x[r])[0]


@pytest.mark.parametrize("k", [1, 8, 64])
def test_entropy_topk_small(ctx, oracle, k):
    rng = np.random.Generator(np.random.PCG64(k))
    rows, V = 5, 20000
    x = (rng.standard_normal((rows, V)) * 2).astype(np.float32)
    x[1, 77] += 15
    x[2, rng.random(V) < 0.5] = -np.inf
    x[3, :] = np.round(x[3, :])  # ties
    draft = np.array([0, 77, 5, 9, 1], np.uint32)
    ent, ids, probs, am, acc = ctx.entropy_topk_rows(to_device(x), k, dev(draft.astype(np.int32)), vocab=V)
    ent, ids, probs, am, acc = (t.cpu().numpy() for t in (ent, ids, probs, am, acc))
    for r in range(rows):
        H, eids, eprobs = oracle.entropy_topk(x[r], k)
        assert abs(ent[r] - H) <= 1e-5 * abs(H) + 1e-7, (r, ent[r], H)
        assert np.array_equal(ids[r].astype(np.uint32), eids), (r, ids[r], eids)
        np.testing.assert_allclose(probs[r], eprobs, rtol=1e-5, atol=1e-30)
        assert am[r] == eids[0]
        assert acc[r] == int(eids[0] == draft[r])


def test_config4_full_size(ctx, oracle):
    from zinfer_amd.workloads import config4

    w = config4()
    ent, ids, probs, am, acc = ctx.entropy_topk_rows(to_device(w.logits), 8, dev(w.draft.astype(np.int32)),
                                                     vocab=w.vocab)
    ent, ids, probs, am, acc = (t.cpu().numpy() for t in (ent, ids, probs, am, acc))
    for r in range(w.rows):
        H, eids, eprobs = oracle.entropy_topk(w.logits[r], 8)
        assert abs(ent[r] - H) <= 1e-5 * abs(H) + 1e-7, (r, ent[r], H)
        assert np.array_equal(ids[r].astype(np.uint32), eids)
        np.testing.assert_allclose(probs[r], eprobs, rtol=1e-5, atol=1e-30)
        assert am[r] == eids[0] and acc[r] == int(eids[0] == w.draft[r])


@pytest.mark.parametrize("bf16", [False, True])
def test_apply_mask_rows(ctx, oracle, bf16):
    from zinfer_amd.workloads import _bf16_round, pack_mask

    rng = np.random.Generator(np.random.PCG64(11))
    rows, V = 3, 1001
    x = (rng.standard_normal((rows, V)) * 2).astype(np.float32)
    if bf16:
        x = _bf16_round(x)
    W = (V + 31) // 32
    mask = pack_mask(rng.random((rows, W * 32)) < 0.3)
    L = to_device(x, bf16=bf16)
    ctx.apply_mask_rows(L, dev(mask), vocab=V)
    got = L[:, :V].float().cpu().numpy()
    for r in range(rows):
        exp = oracle.apply_mask(x[r], mask[r])
        assert np.array_equal(f32bits(got[r]), f32bits(exp))
    assert np.all(L[:, V:].float().cpu().numpy() == 0)  # padding untouched


WALK_CASES = [  # (rows, V, k, bf16): rows x chunks > 256 takes the walking entropy kernel
    (40, 262144, 8, False),    # 6 segments per row, ragged last segment and step
    (60, 131073, 1, False),    # 4 segments, V not a multiple of the step
    (300, 20000, 64, False),   # one workgroup walks each whole row (2 steps)
    (64, 151936, 8, True),     # bf16 steps of 32 elements per thread
]


@pytest.mark.parametrize("rows,V,k,bf16", WALK_CASES)
def test_entropy_walk_rows(ctx, oracle, rows, V, k, bf16):
    """Segments walked by one workgroup each: a running top-k in LDS whose
    k-th value is each later step's threshold.  Rows with ties, -inf runs, a
    dominant logit and increasing values (every step beats the running
    list) cover the threshold's overflow paths."""
    from zinfer_amd.workloads import _bf16_round

    rng = np.random.Generator(np.random.PCG64(rows * 7 + k))
    x = (rng.standard_normal((rows, V)) * 2).astype(np.float32)
    x[1, V - 3] += 15  # dominant logit in the last step
    x[2, rng.random(V) < 0.7] = -np.inf
    x[3, :] = np.round(x[3, :])  # ties across steps and segments
    x[4, :] = np.linspace(-5.0, 5.0, V, dtype=np.float32)  # increasing: each step overflows the running list
    x[5, :] = -np.inf
    x[5, 12345 % V] = 0.0
    if bf16:
        x = _bf16_round(x)
    draft = rng.integers(0, V, rows).astype(np.uint32)
    draft[1] = V - 3
    ent, ids, probs, am, acc = ctx.entropy_topk_rows(to_device(x, bf16=bf16), k, dev(draft.astype(np.int32)),
                                                     vocab=V)
    ent, ids, probs, am, acc = (t.cpu().numpy() for t in (ent, ids, probs, am, acc))
    for r in range(rows):
        H, eids, eprobs = oracle.entropy_topk(x[r], k)
        n = len(eids)
        assert abs(ent[r] - H) <= 1e-5 * abs(H) + 1e-7, (r, ent[r], H)
        assert np.array_equal(ids[r][:n].astype(np.uint32), eids), (r, ids[r][:n], eids)
        np.testing.assert_allclose(probs[r][:n], eprobs, rtol=1e-5, atol=1e-30)
        assert am[r] == eids[0] and acc[r] == int(eids[0] == draft[r])
