"""GPU parity: zi_sample_rows_pruned (rows whose logits exist only at listed
groups of 8 ids; src/model.zig:2036-2140) vs the CPU oracle on the row the
reference builds (-inf fill, then the groups written: pyoracle.pruned_row),
and vs zi_sample_rows on that dense row.

Bar: token ids, margins, keep counts, uniforms consumed, candidate ids/values
and probabilities bit-exact.  The unlisted positions of the input buffer hold
garbage (huge values, NaN), which the entry must never read."""
import numpy as np
import pytest

from paritylib import compare_sample, dev, gpu_sample, oracle_sample, to_device
from zinfer_amd.workloads import _bf16_round, pack_mask

pytestmark = pytest.mark.gpu


def _groups(rng, V, rows, n_extra, fixed=64, dup=False, bad=False):
    """The reference's candidate list: groups 0..63 plus n_extra others
    (model.zig:2070-2125), per row, in heap (unsorted) order."""
    ngt = (V + 7) // 8
    out = []
    for _ in range(rows):
        extra = rng.choice(np.arange(fixed, ngt), size=min(n_extra, ngt - fixed), replace=False)
        g = np.concatenate([np.arange(min(fixed, ngt)), extra]).astype(np.uint32)
        rng.shuffle(g)
        if dup:
            g = np.concatenate([g, g[:5]])
        if bad:
            g = np.concatenate([g, np.array([ngt, ngt + 7, 0xFFFFFFF0], np.uint32)])
        out.append(g)
    ld = max(len(g) for g in out) + 3
    G = np.zeros((len(out), ld), np.uint32)
    cnt = np.zeros(len(out), np.int32)
    for r, g in enumerate(out):
        G[r, :len(g)] = g
        cnt[r] = len(g)
    return G, cnt


def _case_inputs(rng, rows, V, kind, G, cnt, bf16):
    if kind == "t3":
        x = (rng.standard_t(3, (rows, V)) * 2).astype(np.float32)
    elif kind == "ints":
        x = rng.integers(-3, 4, (rows, V)).astype(np.float32)
    elif kind == "flat":
        x = np.full((rows, V), 0.5, np.float32)
    else:
        x = (rng.standard_normal((rows, V)) * 3).astype(np.float32)
    if bf16:
        x = _bf16_round(x)
    dense = np.stack([pruned_row_np(x[r], G[r, :cnt[r]], V) for r in range(rows)])
    buf = x.copy()
    unl = np.ones((rows, V), bool)
    for r in range(rows):
        g = G[r, :cnt[r]].astype(np.int64)
        g = g[g < (V + 7) // 8]
        ids = (g[:, None] * 8 + np.arange(8)).reshape(-1)
        unl[r, ids[ids < V]] = False
    garbage = np.where(rng.random((rows, V)) < 0.5, np.float32(3e38), np.float32(np.nan))
    buf[unl] = garbage[unl]  # never read
    return buf, dense


def pruned_row_np(x, g, V):
    from oracle import pyoracle

    return pyoracle.pruned_row(x, g, V)


def _gpu_pruned(ctx, pk, buf, u, G, cnt, hist=None, hl=None, mask=None, ei=None, ed=None, ec=None, bf16=False):
    import torch
    from zinfer_amd.api import params

    rows, V = buf.shape
    L = to_device(buf, bf16)
    res = ctx.sample_rows(params(**pk), L, dev(u), vocab=V, hist=dev(hist), hist_len=dev(hl), mask=dev(mask),
                          edit_ids=dev(ei), edit_delta=dev(ed), edit_count=dev(ec),
                          cands=pk.get("temp", 0.8) > 0, groups=dev(G), group_count=dev(cnt))
    torch.cuda.synchronize()
    out = dict(tok=res.tok.cpu().numpy().astype(np.uint32), margin=res.margin.cpu().numpy(),
               ndraws=res.ndraws.cpu().numpy())
    if res.keep is not None:
        out.update(keep=res.keep.cpu().numpy(), cand_ids=res.cand_ids.cpu().numpy().astype(np.uint32),
                   cand_vals=res.cand_vals.cpu().numpy(), probs=res.probs.cpu().numpy())
    return out


CASES = []
_r = np.random.Generator(np.random.PCG64(515))
for i in range(24):
    V = int(_r.choice([4099, 32000, 128256, 151936, 262144]))
    rows = int(_r.choice([1, 4, 9]))
    kind = str(_r.choice(["normal", "t3", "ints", "flat"]))
    n_extra = int(_r.choice([512, 512, 100, 0]))
    pk = dict(temp=float(_r.choice([0.5, 0.8, 1.0, 1.5])), top_k=int(_r.choice([1, 5, 40, 50, 200, 256])),
              top_p=float(_r.choice([1.0, 0.95, 0.9, 0.5])), min_p=float(_r.choice([0.0, 0.0, 0.05, 0.3])))
    if _r.random() < 0.5:
        pk.update(repeat_penalty=float(_r.choice([1.1, 1.3, 0.9])), penalty_last_n=int(_r.choice([64, 256, 1000])))
    if _r.random() < 0.3:
        pk.update(freq_penalty=0.3, presence_penalty=0.5)
        pk.setdefault("penalty_last_n", 64)
    if _r.random() < 0.25:
        pk.update(xtc_probability=1.0, xtc_threshold=float(_r.choice([0.1, 0.3])), xtc_min_keep=1)
    CASES.append((i, V, rows, kind, n_extra, pk, bool(_r.random() < 0.35), bool(_r.random() < 0.3),
                  bool(_r.random() < 0.3), bool(i % 5 == 3), bool(i % 7 == 2)))
# rows with fewer finite entries than k: the list runs on into -inf ids
CASES.append((100, 32000, 3, "normal", 0, dict(temp=0.8, top_k=256, top_p=1.0, min_p=0.0), True, False, False,
              False, False))
CASES.append((101, 4099, 2, "normal", 0, dict(temp=1.0, top_k=200, top_p=0.9, min_p=0.0), True, True, False,
              False, True))


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"c{c[0]}-V{c[1]}-r{c[2]}-{c[3]}-g{c[4]}")
def test_pruned_rows_match_oracle(ctx, oracle, case):
    i, V, rows, kind, n_extra, pk, use_mask, use_edits, bf16, dup, bad = case
    rng = np.random.Generator(np.random.PCG64(7000 + i))
    G, cnt = _groups(rng, V, rows, n_extra, dup=dup, bad=bad)
    buf, dense = _case_inputs(rng, rows, V, kind, G, cnt, bf16)
    u = rng.random((rows, 2), dtype=np.float32)
    hist = hl = mask = ei = ed = ec = None
    if "penalty_last_n" in pk:
        H = 300
        hist = rng.integers(0, V, (rows, H), dtype=np.uint32)
        top = np.argsort(-np.nan_to_num(dense, neginf=-1e30), axis=1)[:, :12].astype(np.uint32)
        hist[:, -12:] = top  # penalize listed leaders, and unlisted ids elsewhere
        hl = rng.integers(0, H + 1, rows).astype(np.int32)
        hl[0] = H
    if use_mask:
        bits = rng.random((rows, (V + 31) // 32 * 32)) < (0.002 if i >= 100 else 0.4)
        bits[:, 0] = True
        mask = pack_mask(bits)
    if use_edits:
        E = 16
        ei = np.stack([rng.choice(V, size=E, replace=False).astype(np.uint32) for _ in range(rows)])
        ei[:, :4] = np.argsort(-np.nan_to_num(dense, neginf=-1e30), axis=1)[:, :4].astype(np.uint32)
        ed = (rng.random(ei.shape) * 3).astype(np.float32)
        ec = rng.integers(0, E + 1, rows).astype(np.int32)
    g = _gpu_pruned(ctx, pk, buf, u, G, cnt, hist, hl, mask, ei, ed, ec, bf16)
    o = oracle_sample(oracle, pk, dense, u, hist, hl, mask, ei, ed, ec)
    errs = compare_sample(g, o, pk, V, f"pruned case{i}")
    assert not errs, "\n".join(errs[:20])


@pytest.mark.parametrize("V", [16, 17, 4099, 32000, 151936])
@pytest.mark.parametrize("kind", ["normal", "ints"])
def test_pruned_greedy_matches_oracle(ctx, oracle, V, kind):
    """temp = 0: the reference argmax (lane-16 classes, tail, margin rule) over
    the row with the -inf fill; ints give ties inside and across classes."""
    rng = np.random.Generator(np.random.PCG64(V * 3 + len(kind)))
    rows = 5
    G, cnt = _groups(rng, V, rows, 40, fixed=min(64, (V + 7) // 8))
    buf, dense = _case_inputs(rng, rows, V, kind, G, cnt, False)
    hist = rng.integers(0, V, (rows, 64), dtype=np.uint32)
    hl = np.full(rows, 64, np.int32)
    pk = dict(temp=0.0, repeat_penalty=1.2, penalty_last_n=64)
    u = np.zeros((rows, 2), np.float32)
    g = _gpu_pruned(ctx, pk, buf, u, G, cnt, hist, hl)
    o = oracle_sample(oracle, pk, dense, u, hist, hl)
    errs = compare_sample(g, o, pk, V, "pruned greedy")
    assert not errs, "\n".join(errs[:20])


@pytest.mark.parametrize("rows,V,bf16", [(64, 128256, False), (256, 151936, True), (32, 262144, False)])
def test_pruned_matches_dense_entry(ctx, rows, V, bf16):
    """Full-size batches: the pruned entry and zi_sample_rows on the filled
    rows agree on every output."""
    rng = np.random.Generator(np.random.PCG64(rows + V))
    G, cnt = _groups(rng, V, rows, 512)
    buf, dense = _case_inputs(rng, rows, V, "t3", G, cnt, bf16)
    u = rng.random((rows, 2), dtype=np.float32)
    hist = rng.integers(0, V, (rows, 256), dtype=np.uint32)
    hl = np.full(rows, 256, np.int32)
    pk = dict(temp=0.7, top_k=50, top_p=0.9, min_p=0.05, repeat_penalty=1.15, freq_penalty=0.3,
              presence_penalty=0.5, penalty_last_n=256)
    g = _gpu_pruned(ctx, pk, buf, u, G, cnt, hist, hl, bf16=bf16)
    d = gpu_sample(ctx, pk, dense, u, hist, hl, bf16=bf16)
    for key in ("tok", "ndraws", "keep", "cand_ids"):
        assert np.array_equal(g[key], d[key]), key
    for key in ("margin", "cand_vals", "probs"):
        assert np.array_equal(g[key].view(np.uint32), d[key].view(np.uint32)), key


@pytest.mark.parametrize("pk,V,bf16", [
    (dict(temp=0.8, top_k=40, top_p=0.95, min_p=0.05, final_logit_softcap=30.0), 32000, False),
    (dict(temp=0.8, top_k=40, top_p=0.95, min_p=0.0, final_logit_softcap=2.0), 4096, True),
    (dict(temp=0.0, repeat_penalty=1.2, penalty_last_n=64, final_logit_softcap=30.0), 32000, False),
    (dict(temp=0.9, top_k=0, top_p=0.95, min_p=0.05), 32000, False),
    (dict(temp=0.9, top_k=1000, top_p=0.9, min_p=0.0), 4099, False),
    (dict(temp=1.0, top_k=0, top_p=1.0, min_p=0.0), 20000, True),
])
def test_pruned_dense_path_matches_oracle(ctx, oracle, pk, V, bf16):
    """Softcap (applied after the fill, so unlisted ids become -cap*tanh(9))
    and top_k > 256 sample the filled rows through the dense path."""
    rng = np.random.Generator(np.random.PCG64(V + len(pk)))
    rows = 4
    G, cnt = _groups(rng, V, rows, 200)
    buf, dense = _case_inputs(rng, rows, V, "normal", G, cnt, bf16)
    u = rng.random((rows, 2), dtype=np.float32)
    hist = hl = None
    if "penalty_last_n" in pk:
        hist = rng.integers(0, V, (rows, 64), dtype=np.uint32)
        hl = np.full(rows, 64, np.int32)
    g = _gpu_pruned(ctx, pk, buf, u, G, cnt, hist, hl, bf16=bf16)
    o = oracle_sample(oracle, pk, dense, u, hist, hl)
    errs = compare_sample(g, o, pk, V, "pruned dense path")
    assert not errs, "\n".join(errs[:20])


def test_pruned_rejects_unsupported(ctx):
    import torch
    from zinfer_amd._lib import ZI_ERR_INVALID, ZI_ERR_UNSUPPORTED, ZiError
    from zinfer_amd.api import params

    V = 4096
    L = torch.zeros((2, V), dtype=torch.float32, device="cuda")
    u = torch.zeros((2, 2), dtype=torch.float32, device="cuda")
    cnt = torch.full((2,), 8, dtype=torch.int32, device="cuda")
    big = torch.zeros((2, 1025), dtype=torch.int32, device="cuda")
    with pytest.raises(ZiError) as ei:
        ctx.sample_rows(params(), L, u, vocab=V, groups=big, group_count=cnt)
    assert ei.value.code == ZI_ERR_UNSUPPORTED
    G = torch.zeros((2, 8), dtype=torch.int32, device="cuda")
    with pytest.raises(ZiError) as ei:
        ctx.sample_rows(params(), L[:, :15], u, vocab=15, groups=G, group_count=cnt)
    assert ei.value.code in (ZI_ERR_UNSUPPORTED, ZI_ERR_INVALID)
    torch.cuda.synchronize()


def test_pruned_counts_clamped_and_empty_rows(ctx, oracle):
    """group_count above groups_ld is clamped to it; a negative or zero count
    leaves the whole row at -inf (the reference's fill alone)."""
    rng = np.random.Generator(np.random.PCG64(31337))
    rows, V = 4, 32000
    G, cnt = _groups(rng, V, rows, 100)
    ld = G.shape[1]
    cnt = np.array([ld + 50, 0, -3, ld - 20], np.int32)
    used = np.clip(cnt, 0, ld)
    x = (rng.standard_normal((rows, V)) * 2).astype(np.float32)
    dense = np.stack([pruned_row_np(x[r], G[r, :used[r]], V) for r in range(rows)])
    u = rng.random((rows, 2), dtype=np.float32)
    for pk in (dict(temp=0.8, top_k=40, top_p=0.95, min_p=0.05), dict(temp=0.0)):
        g = _gpu_pruned(ctx, pk, x, u, G, cnt)
        o = oracle_sample(oracle, pk, dense, u)
        errs = compare_sample(g, o, pk, V, "pruned counts")
        assert not errs, "\n".join(errs[:20])
