"""GPU parity: DRY edits on the device (zi_dry_edits_rows) vs the CPU oracle
(or_dry_edits, src/sampler.zig:104-187) and the host restatement
(zi_dry_edits), then fed to zi_sample_rows.

Bar: counts and ids exact, deltas bit-exact, for histories that exercise the
breaker limit, the 128-token cap, long periodic loops (the quadratic worst
case), histories longer than the reference's 4096-token ring, and the early
exits (DRY off, L <= allowed_length, rep_limit < allowed_length)."""
import ctypes as C

import numpy as np
import pytest

from paritylib import compare_sample, dev, gpu_sample, oracle_sample

pytestmark = pytest.mark.gpu


def _hist(rng, kind, n, V=50):
    if kind == "random":
        return rng.integers(0, V, n, dtype=np.uint32)
    if kind == "small":  # a handful of tokens: many repeats of every length
        return rng.integers(0, 4, n, dtype=np.uint32)
    if kind.startswith("period"):
        p = int(kind[6:])
        base = rng.integers(0, V, p, dtype=np.uint32)
        h = np.tile(base, n // p + 1)[:n]
        noise = rng.random(n) < 0.01
        h[noise] = rng.integers(0, V, int(noise.sum()), dtype=np.uint32)
        return h
    if kind == "many":  # > 128 distinct continuations
        return np.resize(rng.integers(0, 400, max(n // 2, 1), dtype=np.uint32), n)
    raise ValueError(kind)


CASES = []
_r = np.random.Generator(np.random.PCG64(44))
for i in range(28):
    kind = str(_r.choice(["random", "small", "period1", "period3", "period7", "many"]))
    n = int(_r.choice([0, 1, 3, 40, 300, 1500, 4096, 5000]))
    pk = dict(dry_multiplier=float(_r.choice([0.8, 0.8, 1.5, 0.0])), dry_base=float(_r.choice([1.75, 1.0, 1.0001, 3.0, 0.9])),
              dry_allowed_length=int(_r.choice([0, 1, 2, 2, 5])), dry_range=int(_r.choice([1024, 1024, 64, 4096, 0, 9000])))
    nb = int(_r.choice([0, 2, 16]))
    CASES.append((i, kind, n, pk, nb))
CASES.append((100, "period1", 4096, dict(dry_multiplier=0.8, dry_base=1.75, dry_allowed_length=2, dry_range=4096), 0))


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"c{c[0]}-{c[1]}-n{c[2]}")
def test_dry_rows_match_oracle_and_host(ctx, oracle, case):
    import torch
    from zinfer_amd._lib import f32p, lib, u32p
    from zinfer_amd.api import params

    i, kind, n, pk, nb = case
    rng = np.random.Generator(np.random.PCG64(300 + i))
    rows = 5
    H = max(n, 1) + 7
    hist = np.zeros((rows, H), np.uint32)
    hl = np.zeros(rows, np.int32)
    for r in range(rows):
        hl[r] = n if r < 3 else int(rng.integers(0, n + 1))
        hist[r, :hl[r]] = _hist(rng, kind, int(hl[r]))
    brk = rng.choice(50, size=nb, replace=False).astype(np.uint32) if nb else None
    p = params(**pk)
    ids, delta, cnt = ctx.dry_edits_rows(p, dev(hist), dev(hl), dev(brk))
    torch.cuda.synchronize()
    ids, delta, cnt = ids.cpu().numpy().astype(np.uint32), delta.cpu().numpy(), cnt.cpu().numpy()
    for r in range(rows):
        h = hist[r, :hl[r]]
        oi, od = oracle.dry_edits(h, brk if brk is not None else np.zeros(0, np.uint32), pk["dry_multiplier"],
                                  pk["dry_base"], pk["dry_allowed_length"], pk["dry_range"])
        assert cnt[r] == len(oi), (r, cnt[r], len(oi))
        assert np.array_equal(ids[r, :cnt[r]], oi), r
        assert np.array_equal(delta[r, :cnt[r]].view(np.uint32), od.view(np.uint32)), (r, delta[r, :cnt[r]], od)
        # the host restatement (zi_dry_edits) agrees as well
        hi = np.zeros(128, np.uint32)
        hd = np.zeros(128, np.float32)
        hb = brk if brk is not None else np.zeros(1, np.uint32)
        hh = np.ascontiguousarray(h) if h.size else np.zeros(1, np.uint32)
        m = lib().zi_dry_edits(hh.ctypes.data_as(u32p), h.size, hb.ctypes.data_as(u32p), nb, C.byref(p),
                               hi.ctypes.data_as(u32p), hd.ctypes.data_as(f32p))
        assert m == len(oi) and np.array_equal(hi[:m], oi) and np.array_equal(hd[:m].view(np.uint32), od.view(np.uint32))


def test_dry_edits_feed_sampling(ctx, oracle):
    """Device DRY edits go straight into zi_sample_rows' edit inputs."""
    import torch
    from zinfer_amd.api import params

    rng = np.random.Generator(np.random.PCG64(77))
    rows, V, H = 6, 32000, 700
    hist = np.stack([np.tile(rng.integers(0, V, 9, dtype=np.uint32), H // 9 + 1)[:H] for _ in range(rows)])
    hl = np.array([H, H - 5, 300, 10, 2, 0], np.int32)
    x = (rng.standard_normal((rows, V)) * 2).astype(np.float32)
    for r in range(rows):  # make the repeated continuations competitive
        x[r, hist[r, :9]] += 4.0
    u = rng.random((rows, 2), dtype=np.float32)
    pk = dict(temp=0.8, top_k=40, top_p=0.95, min_p=0.05, dry_multiplier=0.8, dry_base=1.75, dry_allowed_length=2,
              dry_range=1024)
    ids, delta, cnt = ctx.dry_edits_rows(params(**pk), dev(hist), dev(hl))
    torch.cuda.synchronize()
    ei, ed, ec = ids.cpu().numpy().astype(np.uint32), delta.cpu().numpy(), cnt.cpu().numpy()
    assert ec[:2].min() > 0
    g = gpu_sample(ctx, pk, x, u, edit_ids=ei, edit_delta=ed, edit_count=ec)
    o = oracle_sample(oracle, pk, x, u, edit_ids=ei, edit_delta=ed, edit_count=ec)
    errs = compare_sample(g, o, pk, V, "dry")
    assert not errs, "\n".join(errs[:20])
    for r in range(rows):  # and the edits are the oracle's
        oi, od = oracle.dry_edits(hist[r, :hl[r]], np.zeros(0, np.uint32), 0.8, 1.75, 2, 1024)
        assert np.array_equal(ei[r, :ec[r]], oi) and np.array_equal(ed[r, :ec[r]], od)
