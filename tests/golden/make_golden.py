"""Writes the committed golden fixtures (small seeded cases with the CPU
oracle's expected outputs) to tests/golden/*.npz.

The reference (Zig) cannot run in this image and publishes no vectors for
top-k / top-p / draw, so the expected outputs come from the oracle, whose own
pins are in tests/test_oracle_*.py.  Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import pyoracle as O  # noqa: E402


def pack_mask(bits):
    rows, n = bits.shape
    w = (np.uint64(1) << np.arange(32, dtype=np.uint64))
    return (bits.reshape(rows, n // 32, 32).astype(np.uint64) * w).sum(-1).astype(np.uint32)


def sample_cases():
    rng = np.random.default_rng(2024)
    out = {}
    specs = []
    for i in range(24):
        V = int(rng.choice([5, 16, 33, 257, 1000, 4096]))
        rows = int(rng.integers(1, 4))
        k = int(rng.choice([1, 3, 40, 64]))
        if V <= 64 and i % 3 == 0:
            k = 0
        pk = dict(temp=float(rng.choice([0.0, 0.7, 1.0, 1.3])), top_k=k, top_p=float(rng.choice([1.0, 0.9, 0.5])),
                  min_p=float(rng.choice([0.0, 0.05])), repeat_penalty=float(rng.choice([1.0, 1.2])),
                  freq_penalty=float(rng.choice([0.0, 0.3])), presence_penalty=float(rng.choice([0.0, 0.5])),
                  penalty_last_n=int(rng.choice([16, 64])))
        if i % 5 == 4:
            pk.update(xtc_probability=1.0, xtc_threshold=0.1)
        specs.append((i, V, rows, pk))
        x = (rng.standard_t(3, (rows, V)) * 2).astype(np.float32) if i % 2 else \
            rng.integers(-3, 4, (rows, V)).astype(np.float32)
        u = rng.random((rows, 2), dtype=np.float32)
        hist = rng.integers(0, V, (rows, 80), dtype=np.uint32)
        hl = rng.integers(0, 81, rows).astype(np.int32)
        use_mask = i % 4 == 1
        mask = pack_mask(np.concatenate([rng.random((rows, V)) < 0.5, np.zeros((rows, (-V) % 32), bool)], 1))
        mask[:, 0] |= 1
        ne = rng.integers(0, 5, rows).astype(np.int32)
        eids = np.stack([rng.choice(V, size=min(4, V), replace=False) for _ in range(rows)]).astype(np.uint32)
        ed = (rng.random(eids.shape) * 2).astype(np.float32)
        ne = np.minimum(ne, eids.shape[1]).astype(np.int32)
        kk = V if (k == 0 or k > V) else k
        toks, margins, ndraws, keeps, ns = [], [], [], [], []
        cids = np.zeros((rows, kk), np.uint32)
        cvals = np.zeros((rows, kk), np.float32)
        probs = np.zeros((rows, kk), np.float32)
        p = O.params(**pk)
        for r in range(rows):
            nw = min(int(hl[r]), pk["penalty_last_n"])
            win = hist[r, int(hl[r]) - nw:int(hl[r])]
            t, m, d = O.sample_row(p, x[r], u[r], mask=mask[r] if use_mask else None, window=win,
                                   edit_ids=eids[r, :ne[r]], edit_deltas=ed[r, :ne[r]], cap=kk)
            toks.append(t)
            margins.append(m)
            ndraws.append(d["ndraws"])
            keeps.append(d["keep"])
            ns.append(d["n"])
            cids[r, :len(d["ids"])] = d["ids"]
            cvals[r, :len(d["vals"])] = d["vals"]
            probs[r, :len(d["probs"])] = d["probs"]
        pre = f"c{i}_"
        out.update({pre + "logits": x, pre + "uniforms": u, pre + "hist": hist, pre + "hist_len": hl,
                    pre + "mask": mask if use_mask else np.zeros((0,), np.uint32), pre + "edit_ids": eids,
                    pre + "edit_delta": ed, pre + "edit_count": ne,
                    pre + "params": np.frombuffer(json.dumps(pk).encode(), np.uint8),
                    pre + "tok": np.array(toks, np.uint32), pre + "margin": np.array(margins, np.float32),
                    pre + "ndraws": np.array(ndraws, np.int32), pre + "keep": np.array(keeps, np.int32),
                    pre + "n": np.array(ns, np.int32), pre + "cand_ids": cids, pre + "cand_vals": cvals,
                    pre + "probs": probs})
    out["count"] = np.array([len(specs)], np.int32)
    return out


def argmax_cases():
    rng = np.random.default_rng(7)
    out = {}
    Vs = [1, 2, 15, 16, 17, 31, 48, 100, 1000, 4097]
    for i, V in enumerate(Vs):
        x = rng.integers(-2, 3, V).astype(np.float32)
        if i % 3 == 2:
            x[rng.random(V) < 0.5] = -np.inf
        t, m = O.argmax_with_margin(x)
        tl, ml = O.argmax_true(x)
        out.update({f"a{i}_x": x, f"a{i}_tok": np.array([t], np.uint32), f"a{i}_margin": np.array([m], np.float32),
                    f"a{i}_tok_low": np.array([tl], np.uint32), f"a{i}_margin_true": np.array([ml], np.float32)})
    out["count"] = np.array([len(Vs)], np.int32)
    return out


def entropy_cases():
    rng = np.random.default_rng(11)
    out = {}
    for i in range(6):
        V = int(rng.choice([100, 3000, 20000]))
        x = (rng.standard_normal(V) * 2).astype(np.float32)
        if i == 1:
            x[5] += 15
        if i == 2:
            x[rng.random(V) < 0.7] = -np.inf
        H, ids, probs = O.entropy_topk(x, 8)
        out.update({f"e{i}_x": x, f"e{i}_entropy": np.array([H]), f"e{i}_ids": ids, f"e{i}_probs": probs})
    out["count"] = np.array([6], np.int32)
    return out


if __name__ == "__main__":
    np.savez_compressed(os.path.join(HERE, "sample_cases.npz"), **sample_cases())
    np.savez_compressed(os.path.join(HERE, "argmax_cases.npz"), **argmax_cases())
    np.savez_compressed(os.path.join(HERE, "entropy_cases.npz"), **entropy_cases())
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))
