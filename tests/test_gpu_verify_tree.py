"""GPU parity: tree verification (zi_sampler_verify_tree): several draft
branches verified in one launch, each against the reference's sequential loop
(src/gen.zig:544-587, restated on the CPU oracle) from the same sampler state.
Bar: every branch's accepted count, next token and margin equal the oracle
loop's for that branch alone; the chosen branch is the one with the most
accepted tokens (first on ties); with commit the sampler state afterwards
(next draw, history) is the oracle's for that branch, without it unchanged."""
import numpy as np
import pytest

from test_gpu_verify import _oracle_loop, _setup
from zinfer_amd.workloads import synthetic_vocab, vocab_piece

pytestmark = pytest.mark.gpu

CASES = [
    ("penalties", dict(temp=0.8, top_k=40, top_p=0.95, min_p=0.05, repeat_penalty=1.2, penalty_last_n=64)),
    ("xtc", dict(temp=1.0, top_k=20, top_p=1.0, min_p=0.0, xtc_probability=0.7, xtc_threshold=0.1,
                 penalty_last_n=64)),
    ("greedy", dict(temp=0.0, repeat_penalty=1.3, penalty_last_n=64)),
    ("dry", dict(temp=0.7, top_k=30, top_p=0.9, min_p=0.05, dry_multiplier=0.8, dry_base=1.75,
                 dry_allowed_length=2, penalty_last_n=64)),
]


def _ideal(oracle, pk, X, hist, stream, breakers=(), js=None, tables=None):
    """The tokens the target itself samples row by row (a draft of them is accepted whole)."""
    out, h, pos = [], list(hist), 0
    js = oracle.json_copy(js) if js is not None else None
    for i in range(X.shape[0] - 1):
        _, tok, _, pos, h, js = _oracle_loop(oracle, pk, X[i:i + 1], [], h, stream, pos, breakers=breakers, js=js,
                                             tables=tables)
        out.append(tok)
        h.append(tok)
        if js is not None:
            oracle.json_consume(js, vocab_piece(tables[0], tables[1], tok))
    return out


@pytest.mark.parametrize("name,pk", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("commit", [True, False])
def test_tree_matches_sequential_loop_per_branch(ctx, oracle, name, pk, commit):
    import torch

    V = 3000
    pk = dict(pk, seed=91)
    breakers = [5, 9] if name == "dry" else []
    smp, rng, hist, stream = _setup(ctx, oracle, V, pk, 40 + len(name), breakers=breakers)
    if name == "dry":
        hist += hist[-6:]
        for t in hist[-6:]:
            smp.accept(t)
    lens = [6, 6, 3, 5, 0]
    Xs, drafts = [], []
    for j, k in enumerate(lens):
        X = (rng.standard_normal((k + 1, V)) * 2.5).astype(np.float32)
        d = _ideal(oracle, pk, X, hist, stream, breakers)
        if j == 1:
            d[2] = (d[2] + 1) % V  # rejected at 2
        if j == 3:
            d[0] = (d[0] + 11) % V  # rejected at once
        Xs.append(X)
        drafts.append(d)
    exps = [_oracle_loop(oracle, pk, X, d, hist, stream, 0, breakers=breakers) for X, d in zip(Xs, drafts)]
    L = torch.from_numpy(np.concatenate(Xs)).to("cuda")
    acc, nxt, mg, best = smp.verify_tree(L, drafts, commit=commit)
    for j, e in enumerate(exps):
        assert (acc[j], nxt[j]) == (e[0], e[1]), (j, acc[j], nxt[j], e[:2])
        assert np.float32(mg[j]) == np.float32(e[2]), j
    want_best = int(np.argmax([e[0] for e in exps]))
    assert best == want_best and acc[0] == 6 and acc[1] == 2 and acc[3] == 0
    e = exps[best] if commit else (0, 0, 0, 0, hist)
    assert np.float32(smp.rand_f32()) == np.float32(stream[e[3]])
    # a later sample reads the committed history (or the untouched one)
    x = (rng.standard_normal(V) * 2).astype(np.float32)
    okw = {kk: v for kk, v in pk.items() if kk != "seed"}
    W = pk.get("penalty_last_n", 64)
    ei = ed = None
    if pk.get("dry_multiplier", 0.0):
        ei, ed = oracle.dry_edits(np.array(e[4], np.uint32), np.array(breakers, np.uint32), pk["dry_multiplier"],
                                  pk["dry_base"], pk["dry_allowed_length"], pk.get("dry_range", 1024))
    t2, m2, _ = oracle.sample_row(oracle.params(**okw), x, stream[e[3] + 1:e[3] + 3],
                                  window=np.array(e[4][-W:], np.uint32), edit_ids=ei, edit_deltas=ed)
    assert smp.sample_with_margin(x.copy()) == (t2, m2)


def test_tree_json_mode(ctx, oracle):
    """JSON mode: every branch row's mask from the validator after that
    branch's prefix; the validator advanced by the chosen branch only."""
    import torch

    from paritylib import to_device
    from test_grammar import _canon_oracle, _canon_product
    from zinfer_amd.api import JsonValidator, Vocab

    V = 4099
    off, buf, eog, eos = synthetic_vocab(V)
    tables = (off, buf, eog, eos)
    pk = dict(temp=0.8, top_k=40, top_p=0.95, min_p=0.05, repeat_penalty=1.1, penalty_last_n=64, seed=5)
    smp, rng, hist, stream = _setup(ctx, oracle, V, pk, 23)
    vocab = Vocab(ctx, off, buf, eog, eos, cache_states=8)
    prefix = b'{"key": [1, 2'
    js_o = oracle.json_init(True)
    assert oracle.json_consume(js_o, prefix)
    jv = JsonValidator(True)
    assert jv.consume(prefix)
    lens = [4, 5, 2]
    Xs, drafts = [], []
    for j, k in enumerate(lens):
        X = (rng.standard_normal((k + 1, V)) * 2.5).astype(np.float32)
        d = _ideal(oracle, pk, X, hist, stream, js=js_o, tables=tables)
        if j == 0:
            d[1] = (d[1] + 3) % V
        Xs.append(X)
        drafts.append(d)
    eg = tuple(int(t) for t in eog) + (eos,)
    exps = [_oracle_loop(oracle, pk, X, d, hist, stream, 0, eog=eg, js=js_o, tables=tables) for X, d in zip(Xs, drafts)]
    L = to_device(np.concatenate(Xs))[:, :V]
    acc, nxt, mg, best = smp.verify_tree(L, drafts, eog=eg, vocab=vocab, json=jv)
    for j, e in enumerate(exps):
        assert (acc[j], nxt[j], np.float32(mg[j])) == (e[0], e[1], np.float32(e[2])), j
    assert best == int(np.argmax([e[0] for e in exps]))
    ref = oracle.json_copy(js_o)
    for t in drafts[best][:acc[best]]:
        oracle.json_consume(ref, vocab_piece(off, buf, t))
    assert _canon_product(jv) == _canon_oracle(ref)
    assert np.float32(smp.rand_f32()) == np.float32(stream[exps[best][3]])
    vocab.close()
