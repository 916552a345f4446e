"""The committed golden fixtures (tests/golden/*.npz) against the oracle that
wrote them: a regression guard on the oracle itself (CPU only)."""
import json
import os

import numpy as np

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def sample_case(z, i):
    g = lambda k: z[f"c{i}_{k}"]  # noqa: E731
    pk = json.loads(bytes(g("params")).decode())
    mask = g("mask")
    return pk, g("logits"), g("uniforms"), g("hist"), g("hist_len"), (mask if mask.size else None), \
        g("edit_ids"), g("edit_delta"), g("edit_count")


def test_golden_sample_cases_reproduce(oracle):
    z = load("sample_cases.npz")
    for i in range(int(z["count"][0])):
        pk, x, u, hist, hl, mask, ei, ed, ec = sample_case(z, i)
        p = oracle.params(**pk)
        for r in range(x.shape[0]):
            nw = min(int(hl[r]), pk["penalty_last_n"])
            tok, m, d = oracle.sample_row(p, x[r], u[r], mask=None if mask is None else mask[r],
                                          window=hist[r, int(hl[r]) - nw:int(hl[r])], edit_ids=ei[r, :ec[r]],
                                          edit_deltas=ed[r, :ec[r]], cap=z[f"c{i}_cand_ids"].shape[1])
            assert tok == z[f"c{i}_tok"][r] and np.float32(m) == z[f"c{i}_margin"][r], (i, r)
            assert d["keep"] == z[f"c{i}_keep"][r] and d["ndraws"] == z[f"c{i}_ndraws"][r]


def test_golden_argmax_cases_reproduce(oracle):
    z = load("argmax_cases.npz")
    for i in range(int(z["count"][0])):
        t, m = oracle.argmax_with_margin(z[f"a{i}_x"])
        assert t == z[f"a{i}_tok"][0] and np.float32(m) == z[f"a{i}_margin"][0]


def test_golden_entropy_cases_reproduce(oracle):
    z = load("entropy_cases.npz")
    for i in range(int(z["count"][0])):
        H, ids, probs = oracle.entropy_topk(z[f"e{i}_x"], 8)
        assert H == z[f"e{i}_entropy"][0] and np.array_equal(ids, z[f"e{i}_ids"])
