"""GPU parity: batched draft verification (zi_sampler_verify) against the
reference's sequential loop (src/gen.zig:544-587) restated on the CPU oracle:
row i sampled after take(draft[0..i)) (penalty window, DRY history, JSON
validator), the RNG stream consumed row by row, acceptance stopping at the
first mismatch / end-of-generation token / max_accept, the bonus row when every
draft token is accepted.  Bar: accepted count, next token and margin, and the
sampler state afterwards (next draws, history, JSON state) equal the oracle's."""
import numpy as np
import pytest

from zinfer_amd.workloads import synthetic_vocab, vocab_piece

pytestmark = pytest.mark.gpu


def _oracle_loop(oracle, pk, X, draft, hist0, stream, pos, max_accept=1 << 32, eog=(), breakers=(), js=None,
                 tables=None):
    """The reference verify loop; returns (accepted, next, margin, stream position, history, json state)."""
    okw = {k: v for k, v in pk.items() if k != "seed"}
    p = oracle.params(**okw)
    W = pk.get("penalty_last_n", 64)
    hist = list(hist0)
    js = oracle.json_copy(js) if js is not None else None
    k = len(draft)
    a = 0
    for i in range(k + 1):
        win = np.array(hist[-W:], np.uint32) if W else np.zeros(0, np.uint32)
        mask = None
        if js is not None:
            off, buf, eg, eos = tables
            mask = oracle.json_mask(js, off, buf, eg, eos)
        ei = ed = None
        if pk.get("dry_multiplier", 0.0):
            ei, ed = oracle.dry_edits(np.array(hist, np.uint32), np.array(breakers, np.uint32), pk["dry_multiplier"],
                                      pk.get("dry_base", 1.75), pk.get("dry_allowed_length", 2),
                                      pk.get("dry_range", 1024))
        tok, margin, diag = oracle.sample_row(p, X[i], stream[pos:pos + 2], mask=mask, window=win, edit_ids=ei,
                                              edit_deltas=ed)
        pos += diag["ndraws"]
        if i < k and tok == draft[i] and tok not in eog and a < max_accept:
            a += 1
            hist.append(tok)
            if js is not None:
                oracle.json_consume(js, vocab_piece(tables[0], tables[1], tok))
            continue
        return a, tok, margin, pos, hist, js
    raise AssertionError("unreachable")


def _setup(ctx, oracle, V, pk, seed, n_hist=80, breakers=()):
    from zinfer_amd.api import Sampler, params

    smp = Sampler(ctx, V, params(**pk))
    rng = np.random.Generator(np.random.PCG64(seed))
    hist = [int(t) for t in rng.integers(0, V, n_hist)]
    for t in breakers:
        smp.add_breaker(int(t))
    for t in hist:
        smp.accept(t)
    stream = oracle.rng_floats(pk["seed"], 400)
    return smp, rng, hist, stream


CASES = [
    ("penalties", dict(temp=0.8, top_k=40, top_p=0.95, min_p=0.05, repeat_penalty=1.2, penalty_last_n=64), False),
    ("xtc", dict(temp=1.0, top_k=20, top_p=1.0, min_p=0.0, xtc_probability=0.7, xtc_threshold=0.1,
                 penalty_last_n=64), False),
    ("greedy", dict(temp=0.0, repeat_penalty=1.3, penalty_last_n=64), False),
    ("dry", dict(temp=0.7, top_k=30, top_p=0.9, min_p=0.05, dry_multiplier=0.8, dry_base=1.75,
                 dry_allowed_length=2, penalty_last_n=64), False),
    ("bf16", dict(temp=0.9, top_k=50, top_p=0.9, min_p=0.05, repeat_penalty=1.1, freq_penalty=0.2,
                  presence_penalty=0.3, penalty_last_n=128), True),
]


@pytest.mark.parametrize("name,pk,bf16", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("mode", ["all", "reject", "max_accept", "eog"])
def test_verify_matches_sequential_loop(ctx, oracle, name, pk, bf16, mode):
    import torch

    from zinfer_amd.workloads import _bf16_round

    V, k = 3000, 6
    pk = dict(pk, seed=77)
    breakers = [5, 9] if name == "dry" else []
    smp, rng, hist, stream = _setup(ctx, oracle, V, pk, 11 + len(name), breakers=breakers)
    X = (rng.standard_normal((k + 1, V)) * 2.5).astype(np.float32)
    if name == "dry":  # repeats that DRY penalizes
        hist += hist[-6:]
        for t in hist[-6:]:
            smp.accept(t)
    if bf16:
        X = _bf16_round(X)
    # the target's own tokens: a draft of them is accepted whole
    ideal = []
    h, pos = list(hist), 0
    for i in range(k):
        _, tok, _, pos, h, _ = _oracle_loop(oracle, pk, X[i:i + 1], [], h, stream, pos, breakers=breakers)
        ideal.append(tok)
        h.append(tok)
    draft = list(ideal)
    max_accept, eog = 2**32 - 1, ()
    if mode == "reject":
        draft[3] = (draft[3] + 1) % V
    elif mode == "max_accept":
        max_accept = 2
    elif mode == "eog":
        eog = (draft[2],)
    exp = _oracle_loop(oracle, pk, X, draft, hist, stream, 0, max_accept, eog, breakers)
    L = torch.from_numpy(X).to("cuda").to(torch.bfloat16 if bf16 else torch.float32)
    a, nt, m = smp.verify(L, draft, max_accept=max_accept, eog=eog)
    assert (a, nt) == (exp[0], exp[1]), (mode, a, nt, exp[:2])
    assert np.float32(m) == np.float32(exp[2])
    if mode == "all":
        assert a == k
    # sampler state afterwards: the next draw, and a sample that reads the history
    assert np.float32(smp.rand_f32()) == np.float32(stream[exp[3]])
    x = (rng.standard_normal(V) * 2).astype(np.float32)
    okw = {kk: v for kk, v in pk.items() if kk != "seed"}
    W = pk.get("penalty_last_n", 64)
    ei = ed = None
    if pk.get("dry_multiplier", 0.0):
        ei, ed = oracle.dry_edits(np.array(exp[4], np.uint32), np.array(breakers, np.uint32), pk["dry_multiplier"],
                                  pk["dry_base"], pk["dry_allowed_length"], pk.get("dry_range", 1024))
    t2, m2, _ = oracle.sample_row(oracle.params(**okw), x, stream[exp[3] + 1:exp[3] + 3],
                                  window=np.array(exp[4][-W:], np.uint32), edit_ids=ei, edit_deltas=ed)
    got = smp.sample_with_margin(x.copy())
    assert got == (t2, m2)


@pytest.mark.parametrize("mode", ["all", "reject"])
def test_verify_json_mode(ctx, oracle, mode):
    """JSON mode: every row's mask from the validator after the draft prefix
    (GPU masks), and the validator advanced by the accepted pieces."""
    import torch

    from zinfer_amd.api import JsonValidator, Vocab

    V, k = 4099, 6
    off, buf, eog, eos = synthetic_vocab(V)
    pk = dict(temp=0.8, top_k=40, top_p=0.95, min_p=0.05, repeat_penalty=1.1, penalty_last_n=64, seed=5)
    smp, rng, hist, stream = _setup(ctx, oracle, V, pk, 21)
    vocab = Vocab(ctx, off, buf, eog, eos, cache_states=8)
    prefix = b'{"name": "zin'
    js_o = oracle.json_init(True)
    assert oracle.json_consume(js_o, prefix)
    jv = JsonValidator(True)
    assert jv.consume(prefix)
    X = (rng.standard_normal((k + 1, V)) * 2.5).astype(np.float32)
    tables = (off, buf, eog, eos)
    ideal, h, js, pos = [], list(hist), oracle.json_copy(js_o), 0
    for i in range(k):
        _, tok, _, pos, h, js = _oracle_loop(oracle, pk, X[i:i + 1], [], h, stream, pos, js=js, tables=tables)
        ideal.append(tok)
        h.append(tok)
        oracle.json_consume(js, vocab_piece(off, buf, tok))
    draft = list(ideal)
    if mode == "reject":
        draft[2] = (draft[2] + 7) % V
    from paritylib import to_device

    L = to_device(X)[:, :V]  # row stride padded to a multiple of 8
    a, nt, m = smp.verify(L, draft, eog=tuple(int(t) for t in eog) + (eos,), vocab=vocab, json=jv)
    # the oracle loop's eog check uses the same list
    exp = _oracle_loop(oracle, pk, X, draft, hist, stream, 0, eog=tuple(int(t) for t in eog) + (eos,), js=js_o,
                       tables=tables)
    assert (a, nt, np.float32(m)) == (exp[0], exp[1], np.float32(exp[2]))
    # the validator was advanced by the accepted pieces only
    ref = oracle.json_copy(js_o)
    for t in draft[:a]:
        oracle.json_consume(ref, vocab_piece(off, buf, t))
    from test_grammar import _canon_oracle, _canon_product

    assert _canon_product(jv) == _canon_oracle(ref)
    assert np.float32(smp.rand_f32()) == np.float32(stream[exp[3]])
    vocab.close()
