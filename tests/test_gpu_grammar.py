"""GPU parity: JSON grammar mask generation (JsonValidator.applyMask,
src/grammar.zig:446-479, one lane per token piece) vs the CPU oracle.

Bar: every mask word bit-exact (bits at and above V clear), for states met
while writing JSON (every State / NumState / EscapeState, literals, depth 64,
finished), on a seeded synthetic vocabulary with byte tokens, long pieces,
empty pieces and end-of-generation ids.  The decode test chains GPU masks
into zi_sample_rows and must reproduce the oracle's token sequence."""
import json
import random

import numpy as np
import pytest

from oracle import pyoracle as po
from zinfer_amd.api import JsonValidator, Vocab
from zinfer_amd.workloads import synthetic_vocab, vocab_piece

pytestmark = pytest.mark.gpu

FIXED_PREFIXES = [  # (object_only, prefix) that reach every sub-state
    (True, ""), (False, ""), (True, "{}"), (True, "{"), (True, '{"ab'), (True, '{"a\\'), (True, '{"a\\u'),
    (True, '{"a\\u1'), (True, '{"a\\u1f'), (True, '{"a"'), (True, '{"a":'), (True, '{"a":"x'), (True, '{"a":"\\'),
    (True, '{"a":-'), (True, '{"a":0'), (True, '{"a":12'), (True, '{"a":1.'), (True, '{"a":1.5'),
    (True, '{"a":1e'), (True, '{"a":1e-'), (True, '{"a":1e5'), (True, '{"a":t'), (True, '{"a":fal'),
    (True, '{"a":nul'), (True, '{"a":true'), (True, '{"a":[1,'), (True, '{"a":['), (True, '{"a":{"b":[{'),
    (True, '{"a":1,'), (False, "[" * 64), (False, "[" * 63), (True, '{"a":' + "[" * 63), (False, "[[1],"),
    (False, "[]"), (True, '{"a":{}}  '), (False, '["x",{"y":[true,'),
]


def _states_from_docs(n, seed):
    r = random.Random(seed)
    out = []
    while len(out) < n:
        obj = {"k%d" % i: r.choice([1, -2.5e-3, "s\"\\\n", True, None, [1, {"a": [False]}], {}]) for i in range(4)}
        doc = json.dumps(obj, indent=r.choice([None, 2]), ensure_ascii=r.random() < 0.5).encode()
        out.append((True, doc[: r.randint(0, len(doc))]))
    return out


def _make(object_only, prefix):
    o = po.json_init(object_only)
    p = JsonValidator(object_only)
    data = prefix.encode() if isinstance(prefix, str) else prefix
    assert po.json_consume(o, data) and p.consume(data), prefix
    return o, p


def _oracle_masks(states, off, buf, eog, eos):
    return np.stack([po.json_mask(o, off, buf, eog, eos) for o, _ in states])


def _gpu_masks(vocab, states):
    import torch

    m = vocab.json_mask_rows([p for _, p in states])
    torch.cuda.synchronize()
    return m.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("V", [300, 1000, 4099, 151936])
def test_json_mask_matches_oracle(ctx, V):
    off, buf, eog, eos = synthetic_vocab(V)
    states = [_make(*s) for s in FIXED_PREFIXES + _states_from_docs(28, V)]
    vocab = Vocab(ctx, off, buf, eog, eos, cache_states=0)
    g = _gpu_masks(vocab, states)
    o = _oracle_masks(states, off, buf, eog, eos)
    assert g.shape == o.shape
    bad = np.nonzero((g != o).any(axis=1))[0]
    assert bad.size == 0, [(FIXED_PREFIXES + _states_from_docs(28, V))[i] for i in bad[:5]]
    # every row allows something, and no bit past V is set
    assert all(o[i].any() for i in range(len(states)))
    if V % 32:
        assert not (g[:, -1] >> np.uint32(V % 32)).any()
    vocab.close()


def test_json_mask_cache_paths(ctx):
    """A 3-state cache: hits, replacement, duplicates in one call, and calls
    that need more distinct states than the cache holds."""
    off, buf, eog, eos = synthetic_vocab(4099)
    pool = [_make(*s) for s in FIXED_PREFIXES]
    ref = _oracle_masks(pool, off, buf, eog, eos)
    vocab = Vocab(ctx, off, buf, eog, eos, cache_states=3)
    r = random.Random(9)
    for call in range(12):
        idx = [r.randrange(len(pool)) for _ in range(r.choice([1, 2, 3, 5, 9]))]
        if call % 4 == 0:
            idx = idx + idx[:2]  # duplicates within one call
        g = _gpu_masks(vocab, [pool[i] for i in idx])
        assert np.array_equal(g, ref[idx]), (call, idx)
    vocab.close()


def test_apply_mask_host_row(ctx):
    """applyMask on a host logit row, in place (the reference signature)."""
    off, buf, eog, eos = synthetic_vocab(4099)
    rng = np.random.Generator(np.random.PCG64(5))
    vocab = Vocab(ctx, off, buf, eog, eos, cache_states=4)
    for ob, prefix in FIXED_PREFIXES[:12]:
        o, p = _make(ob, prefix)
        x = rng.standard_normal(4099).astype(np.float32)
        want = po.apply_mask(x, po.json_mask(o, off, buf, eog, eos))
        got = p.apply_mask(x.copy(), vocab)
        assert np.array_equal(got, want), prefix
    vocab.close()


def test_constrained_decode_matches_oracle(ctx, oracle):
    """JSON-mode decoding, 8 rows x 40 steps: GPU masks -> zi_sample_rows ->
    consume the drawn piece; the oracle runs applyMask -> sample_row ->
    consume.  Token sequences must match exactly."""
    import torch

    V, rows, steps = 4099, 8, 40
    off, buf, eog, eos = synthetic_vocab(V)
    vocab = Vocab(ctx, off, buf, eog, eos, cache_states=16)
    rng = np.random.Generator(np.random.PCG64(12))
    pk = dict(temp=0.8, top_k=40, top_p=0.95, min_p=0.05)
    vg = [JsonValidator(r % 2 == 0) for r in range(rows)]
    vo = [po.json_init(r % 2 == 0) for r in range(rows)]
    done = [False] * rows
    seq_g, seq_o = [[] for _ in range(rows)], [[] for _ in range(rows)]
    from paritylib import dev, to_device
    from zinfer_amd.api import params

    p = params(**pk)
    op = oracle.params(**pk)
    for step in range(steps):
        x = (rng.standard_normal((rows, V)) * 2).astype(np.float32)
        u = rng.random((rows, 2), dtype=np.float32)
        mask = vocab.json_mask_rows(vg)
        res = ctx.sample_rows(p, to_device(x), dev(u), vocab=V, mask=mask)
        torch.cuda.synchronize()
        toks = res.tok.cpu().numpy()
        for r in range(rows):
            if done[r]:
                continue
            om = po.json_mask(vo[r], off, buf, eog, eos)
            t_o, _, _ = oracle.sample_row(op, x[r], u[r], mask=om)
            t_g = int(toks[r])
            seq_g[r].append(t_g)
            seq_o[r].append(t_o)
            assert t_g == t_o, (r, step, seq_o[r])
            if t_o in set(eog.tolist()) | {eos}:
                done[r] = True
                continue
            piece = vocab_piece(off, buf, t_o)
            assert vg[r].consume(piece) and po.json_consume(vo[r], piece), (r, step, piece)
    assert sum(len(s) for s in seq_o) == sum(len(s) for s in seq_g) > rows * 10
    vocab.close()
