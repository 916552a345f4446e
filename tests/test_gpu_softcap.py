"""GPU parity: the final-logit softcap (src/model.zig:2492-2513) fused into the
batched sampler's read of the logits, vs the CPU oracle that caps the row
first and then samples it (mask, penalty, edits, sampleWithMargin).

Bar: as for the uncapped path -- token ids, margins, keep counts, uniforms
consumed, candidate ids/values and probabilities bit-exact.  The cases cover
every kernel that reads logits: the small-batch chunk pass, the one-row-per-
workgroup pass (>= 256 rows, with and without the min-p prefix), the whole-
vocabulary exact pass, greedy argmax, penalty owners' reloads, bf16 rows and
the host Sampler (which caps its host row in place)."""
import numpy as np
import pytest

from paritylib import compare_sample, gpu_sample, oracle_sample
from zinfer_amd.workloads import _bf16_round, pack_mask

pytestmark = pytest.mark.gpu


def _inputs(rng, rows, V, kind, pen, mask, edits):
    if kind == "wide":  # many logits beyond the cap: the tanh saturates
        x = (rng.standard_normal((rows, V)) * 40).astype(np.float32)
    elif kind == "t3":
        x = (rng.standard_t(3, (rows, V)) * 6).astype(np.float32)
    elif kind == "neginf":
        x = (rng.standard_normal((rows, V)) * 10).astype(np.float32)
        x[rng.random((rows, V)) < 0.5] = -np.inf
    else:
        x = (rng.standard_normal((rows, V)) * 3).astype(np.float32)
    hist = hl = m = ei = ed = ec = None
    if pen:
        hist = rng.integers(0, V, (rows, 200), dtype=np.uint32)
        hist[:, -8:] = np.argsort(-x, axis=1)[:, :8].astype(np.uint32)  # penalize some of the leaders
        hl = rng.integers(0, 201, rows).astype(np.int32)
    if mask:
        bits = rng.random((rows, V)) < 0.5
        bits[:, 0] = True
        m = pack_mask(bits)
    if edits:
        E = 8
        ei = np.stack([rng.choice(V, size=E, replace=False).astype(np.uint32) for _ in range(rows)])
        ed = (rng.random(ei.shape) * 2).astype(np.float32)
        ec = rng.integers(0, E + 1, rows).astype(np.int32)
    return x, hist, hl, m, ei, ed, ec


CASES = [
    # (rows, V, kind, params, pen, mask, edits, bf16)
    (1, 32000, "wide", dict(temp=0.8, top_k=40, top_p=0.95, min_p=0.05), True, False, False, False),
    (4, 151936, "t3", dict(temp=1.0, top_k=64, top_p=0.9, min_p=0.0), True, True, True, False),
    (3, 4096, "neginf", dict(temp=0.7, top_k=200, top_p=0.5, min_p=0.3), False, True, False, False),
    (9, 32000, "wide", dict(temp=1.3, top_k=5, top_p=1.0, min_p=0.0), False, False, True, True),
    (2, 131072, "normal", dict(temp=0.9, top_k=0, top_p=0.9, min_p=0.0), True, False, False, False),
    (3, 32000, "wide", dict(temp=0.7, top_k=1000, top_p=0.98, min_p=0.05), True, True, False, False),
    (2, 70016, "t3", dict(temp=1.0, top_k=0, top_p=0.95, min_p=0.05), False, False, False, True),
    (256, 32000, "t3", dict(temp=0.8, top_k=50, top_p=0.9, min_p=0.05), True, False, True, False),
    (300, 20000, "wide", dict(temp=0.8, top_k=40, top_p=0.9, min_p=0.0), False, True, False, False),
    (260, 65536, "normal", dict(temp=1.0, top_k=256, top_p=0.95, min_p=0.05), True, False, False, True),
    (2, 4096, "wide", dict(temp=0.8, top_k=40, top_p=0.95, min_p=0.05, xtc_probability=1.0,
                           xtc_threshold=0.1, xtc_min_keep=1), True, False, False, False),
]


@pytest.mark.parametrize("cap", [30.0, 4.0])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_softcap_rows_match_oracle(ctx, oracle, case, cap):
    rows, V, kind, pk, pen, mask, edits, bf16 = CASES[case]
    rng = np.random.Generator(np.random.PCG64(900 + case))
    x, hist, hl, m, ei, ed, ec = _inputs(rng, rows, V, kind, pen, mask, edits)
    if bf16:
        x = _bf16_round(x)
    pk = dict(pk, final_logit_softcap=cap)
    if pen:
        pk.update(repeat_penalty=1.3, freq_penalty=0.2, presence_penalty=0.4, penalty_last_n=128)
    u = rng.random((rows, 2), dtype=np.float32)
    g = gpu_sample(ctx, pk, x, u, hist, hl, m, ei, ed, ec, bf16=bf16)
    o = oracle_sample(oracle, pk, x, u, hist, hl, m, ei, ed, ec)
    errs = compare_sample(g, o, pk, V, f"softcap case{case}")
    assert not errs, "\n".join(errs[:20])


LATE_KINDS = ["normal", "t3", "wide", "neginf", "flat_top", "huge"]


@pytest.mark.parametrize("cap", [30.0, 4.0])
@pytest.mark.parametrize("kind", LATE_KINDS)
@pytest.mark.parametrize("mask", [False, True])
@pytest.mark.parametrize("pen", [True, False])
def test_softcap_late_select(ctx, oracle, kind, mask, cap, pen):
    """Chunked top-k rows cap only the chunk's raw candidates
    (chunk_select_late with CAPC): with penalties that never raise a logit on
    grids of >= 64 workgroups, and without penalties on any grid.  Exact when
    at least k capped candidates reach the bound on every other capped value,
    else the chunk is streamed again with the softcap.  Saturated rows
    ("wide", "huge": many values far beyond the cap tie after capping),
    -inf-heavy rows and a negative edit force that fallback."""
    rows, V = 16, 128256  # 4 chunks per row: 64 workgroups
    rng = np.random.Generator(np.random.PCG64(3300 + LATE_KINDS.index(kind) + (20 if mask else 0) + (40 if pen else 0)))
    kx = "normal" if kind in ("flat_top", "huge") else kind
    x, hist, hl, m, ei, ed, ec = _inputs(rng, rows, V, kx, pen, mask, pen)
    if kind == "flat_top":  # integer logits: raw ties, and capped ties among them
        x = np.round(x).astype(np.float32)
    elif kind == "huge":  # far beyond 9 caps: the body's clamp makes every capped value equal
        x = (x * 100 + 500).astype(np.float32)
    pk = dict(temp=0.7, top_k=50, top_p=0.9, min_p=0.05, final_logit_softcap=cap)
    if pen:
        ed[::3, 0] = -5.0  # an edit that raises a logit: that chunk's fallback
        pk.update(repeat_penalty=1.15, freq_penalty=0.3, presence_penalty=0.5, penalty_last_n=256)
    u = rng.random((rows, 2), dtype=np.float32)
    g = gpu_sample(ctx, pk, x, u, hist, hl, m, ei, ed, ec)
    o = oracle_sample(oracle, pk, x, u, hist, hl, m, ei, ed, ec)
    errs = compare_sample(g, o, pk, V, f"softcap late {kind}")
    assert not errs, "\n".join(errs[:20])


@pytest.mark.parametrize("kind", ["normal", "huge"])
@pytest.mark.parametrize("pen", [True, False])
def test_softcap_late_select_bf16(ctx, oracle, kind, pen):
    """The candidates-only softcap on bf16 rows (their own kernel instances)."""
    rows, V = 16, 151936
    rng = np.random.Generator(np.random.PCG64(3400 + (1 if kind == "huge" else 0) + (2 if pen else 0)))
    x, hist, hl, m, ei, ed, ec = _inputs(rng, rows, V, "normal", pen, False, pen)
    if kind == "huge":
        x = (x * 100 + 500).astype(np.float32)
    x = _bf16_round(x)
    pk = dict(temp=0.8, top_k=40, top_p=0.95, min_p=0.05, final_logit_softcap=30.0)
    if pen:
        pk.update(repeat_penalty=1.1, freq_penalty=0.1, presence_penalty=0.2, penalty_last_n=128)
    u = rng.random((rows, 2), dtype=np.float32)
    g = gpu_sample(ctx, pk, x, u, hist, hl, m, ei, ed, ec, bf16=True)
    o = oracle_sample(oracle, pk, x, u, hist, hl, m, ei, ed, ec)
    errs = compare_sample(g, o, pk, V, f"softcap late bf16 {kind}")
    assert not errs, "\n".join(errs[:20])


@pytest.mark.parametrize("V", [32, 4096, 151936])
def test_softcap_greedy_matches_oracle(ctx, oracle, V):
    """temp = 0 takes the argmax pass; capped ties (saturated logits) go to the
    lower id."""
    rng = np.random.Generator(np.random.PCG64(V + 5))
    rows = 4
    x = (rng.standard_normal((rows, V)) * 50).astype(np.float32)  # many saturate at +-cap
    hist = rng.integers(0, V, (rows, 64), dtype=np.uint32)
    hl = np.full(rows, 64, np.int32)
    pk = dict(temp=0.0, repeat_penalty=1.2, penalty_last_n=64, final_logit_softcap=30.0)
    u = np.zeros((rows, 2), np.float32)
    g = gpu_sample(ctx, pk, x, u, hist, hl)
    o = oracle_sample(oracle, pk, x, u, hist, hl)
    errs = compare_sample(g, o, pk, V, "softcap greedy")
    assert not errs, "\n".join(errs[:20])


RAGGED = [
    # (rows, V, params): V not a multiple of 32, so ids >= 32*floor(V/32) take the scalar tail
    (3, 1000, dict(temp=0.8, top_k=40, top_p=0.95, min_p=0.05)),
    (4, 32001, dict(temp=1.0, top_k=64, top_p=0.9, min_p=0.0)),
    (2, 151937, dict(temp=0.9, top_k=0, top_p=0.9, min_p=0.0)),
    (2, 4127, dict(temp=0.7, top_k=1000, top_p=0.98, min_p=0.05)),
    (256, 20007, dict(temp=0.8, top_k=50, top_p=0.9, min_p=0.05)),
    (260, 4999, dict(temp=1.0, top_k=0, top_p=0.95, min_p=0.05)),
    (5, 70023, dict(temp=0.0)),
]


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("case", range(len(RAGGED)))
def test_softcap_ragged_vocab_tail(ctx, oracle, case, bf16):
    """The reference's scalar tail (model.zig:2511-2513, cap * tanh(l / cap))
    on the last V mod 32 ids.  The row's leaders sit in the tail and the
    other tail values are small, where the body's exp form and the tail's
    tanh round differently, so the sampled candidates carry tail values."""
    rows, V, pk = RAGGED[case]
    rng = np.random.Generator(np.random.PCG64(4200 + case))
    body = V // 32 * 32
    x = (rng.standard_normal((rows, V)) * 3).astype(np.float32)
    x[:, body:] = (rng.standard_normal((rows, V - body)) * 1e-3).astype(np.float32)
    x[:, V - 1] = 25.0  # a tail leader (capped near cap)
    x[:, body] = 0.25 * (1 + np.arange(rows, dtype=np.float32))
    if bf16:
        x = _bf16_round(x)
    hist = rng.integers(body, V, (rows, 40), dtype=np.uint32)  # penalties on tail ids (owner reloads)
    hl = rng.integers(0, 41, rows).astype(np.int32)
    pk = dict(pk, final_logit_softcap=4.0, repeat_penalty=1.2, penalty_last_n=64)
    u = rng.random((rows, 2), dtype=np.float32)
    g = gpu_sample(ctx, pk, x, u, hist, hl, bf16=bf16)
    o = oracle_sample(oracle, pk, x, u, hist, hl)
    errs = compare_sample(g, o, pk, V, f"softcap ragged case{case}")
    assert not errs, "\n".join(errs[:20])


@pytest.mark.parametrize("V", [8192, 8197])
def test_host_sampler_caps_row_in_place(ctx, oracle, V):
    """The host Sampler caps the caller's row in place (what the reference's
    forward leaves in the logits, the scalar tail included when V is not a
    multiple of 32), then samples and applies the penalty."""
    from zinfer_amd.api import Sampler, params

    pk = dict(temp=0.9, top_k=30, top_p=0.9, min_p=0.02, repeat_penalty=1.3, penalty_last_n=64,
              final_logit_softcap=20.0, seed=99)
    smp = Sampler(ctx, V, params(**pk))
    stream = oracle.rng_floats(99, 100)
    okw = {k: v for k, v in pk.items() if k != "seed"}
    rng = np.random.Generator(np.random.PCG64(8))
    pos, hist = 0, []
    for step in range(12):
        x = (rng.standard_normal(V) * 15).astype(np.float32)
        win = np.array(hist[-64:], np.uint32)
        exp_tok, exp_m, diag = oracle.sample_row(oracle.params(**okw), x, stream[pos:pos + 2], window=win)
        pos += diag["ndraws"]
        got = x.copy()
        tok, m = smp.sample_with_margin(got)
        assert tok == exp_tok and m == exp_m, (step, tok, exp_tok)
        assert np.array_equal(got.view(np.uint32), diag["row"].view(np.uint32)), "in-place row differs"
        smp.accept(tok)
        hist.append(tok)


def test_softcap_gemma_vocab(ctx, oracle):
    """Gemma's 262144-entry vocabulary with cap 30 (model.zig's final_logit_softcapping)."""
    rng = np.random.Generator(np.random.PCG64(262144))
    rows, V = 8, 262144
    x, hist, hl, m, ei, ed, ec = _inputs(rng, rows, V, "wide", True, False, False)
    pk = dict(temp=0.9, top_k=64, top_p=0.95, min_p=0.05, repeat_penalty=1.1, penalty_last_n=128,
              final_logit_softcap=30.0)
    u = rng.random((rows, 2), dtype=np.float32)
    g = gpu_sample(ctx, pk, x, u, hist, hl)
    o = oracle_sample(oracle, pk, x, u, hist, hl)
    errs = compare_sample(g, o, pk, V, "gemma")
    assert not errs, "\n".join(errs[:20])


@pytest.mark.parametrize("mode", ["all", "reject"])
def test_softcap_in_verify(ctx, oracle, mode):
    """Draft verification with the cap set: every row is capped in the read."""
    import torch

    from test_gpu_verify import _oracle_loop, _setup

    V, k = 4096, 5
    pk = dict(temp=0.8, top_k=40, top_p=0.95, min_p=0.05, repeat_penalty=1.2, penalty_last_n=64,
              final_logit_softcap=6.0, seed=31)
    smp, rng, hist, stream = _setup(ctx, oracle, V, pk, 55)
    X = (rng.standard_normal((k + 1, V)) * 6).astype(np.float32)
    ideal, h, pos = [], list(hist), 0
    for i in range(k):
        _, tok, _, pos, h, _ = _oracle_loop(oracle, pk, X[i:i + 1], [], h, stream, pos)
        ideal.append(tok)
        h.append(tok)
    draft = list(ideal)
    if mode == "reject":
        draft[1] = (draft[1] + 5) % V
    exp = _oracle_loop(oracle, pk, X, draft, hist, stream, 0)
    a, nt, m = smp.verify(torch.from_numpy(X).to("cuda"), draft)
    assert (a, nt, np.float32(m)) == (exp[0], exp[1], np.float32(exp[2]))
    assert np.float32(smp.rand_f32()) == np.float32(stream[exp[3]])
