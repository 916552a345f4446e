"""GPU parity: the sort-free whole-order pass (zi_whole.hip) -- bf16 rows with
top_k = 0 that the prefix pass cannot settle, sampled without candidate
outputs (src/sampler.zig:190-276, the std.mem.sort branch :198-202).

Bar: token ids, margins, uniforms consumed and keep counts bit-exact against
the CPU oracle (stable sort, sequential f32 sums).  The rows are built so that
the prefix cannot settle them (min_p = 0 with top_p < 1, large nuclei), and
cover exact ties (integer logits, flat rows: groups of thousands of equal
entries), heavy tails, masks, penalties that lower or raise logits, and a
batch of 512 full-size rows (config 5 as its text names it)."""
import numpy as np
import pytest

from paritylib import dev, oracle_sample, to_device
from zinfer_amd.workloads import _bf16_round, pack_mask

pytestmark = pytest.mark.gpu


def _sample(ctx, pk, x, u, hist=None, hist_len=None, mask=None):
    import torch

    from zinfer_amd.api import SampleResult, params

    rows, V = x.shape
    L = to_device(x, True)
    d = L.device
    out = SampleResult(tok=torch.empty(rows, dtype=torch.int32, device=d),
                       margin=torch.empty(rows, dtype=torch.float32, device=d),
                       ndraws=torch.empty(rows, dtype=torch.int32, device=d),
                       keep=torch.empty(rows, dtype=torch.int32, device=d))
    ctx.sample_rows(params(**pk), L, dev(u), vocab=V, hist=dev(hist), hist_len=dev(hist_len, None),
                    mask=dev(mask), out=out)
    torch.cuda.synchronize()
    return (out.tok.cpu().numpy().astype(np.uint32), out.margin.cpu().numpy(), out.ndraws.cpu().numpy(),
            out.keep.cpu().numpy())


def _compare(g, o, label):
    tok, margin, nd, keep = g
    errs = []
    for r, (t, m, diag) in enumerate(o):
        if int(tok[r]) != t:
            errs.append(f"{label} row {r}: tok {tok[r]} vs {t}")
        if not (np.float32(margin[r]) == np.float32(m)):
            errs.append(f"{label} row {r}: margin {margin[r]!r} vs {m!r}")
        if int(nd[r]) != diag["ndraws"]:
            errs.append(f"{label} row {r}: ndraws {nd[r]} vs {diag['ndraws']}")
        if int(keep[r]) != diag["keep"]:
            errs.append(f"{label} row {r}: keep {keep[r]} vs {diag['keep']}")
    return errs


def _rows(rng, kind, rows, V):
    if kind == "normal":
        return (rng.standard_normal((rows, V)) * 3).astype(np.float32)
    if kind == "t3":
        return (rng.standard_t(3, (rows, V)) * 2).astype(np.float32)
    if kind == "ints":  # a handful of values: groups of V/9 equal entries, -0.0 beside +0.0
        x = rng.integers(-4, 5, (rows, V)).astype(np.float32)
        x[(x == 0) & (rng.random((rows, V)) < 0.5)] = -0.0
        return x
    if kind == "flat":
        return np.full((rows, V), 1.5, np.float32)
    if kind == "small":  # values near 0: many binades of distinct bf16 values
        return (rng.standard_normal((rows, V)) * 0.05).astype(np.float32)
    raise ValueError(kind)


CASES = [
    ("normal", 32000, 6, dict(temp=1.0, top_k=0, top_p=0.98, min_p=0.0)),
    ("normal", 151936, 3, dict(temp=0.7, top_k=0, top_p=0.9, min_p=0.0)),
    ("t3", 70001, 4, dict(temp=1.3, top_k=0, top_p=0.95, min_p=0.0)),
    ("ints", 4099, 6, dict(temp=1.0, top_k=0, top_p=0.98, min_p=0.0)),
    ("ints", 32000, 3, dict(temp=0.5, top_k=0, top_p=0.5, min_p=0.0)),
    ("flat", 1000, 2, dict(temp=1.0, top_k=0, top_p=0.9, min_p=0.0)),
    ("flat", 151936, 1, dict(temp=1.0, top_k=0, top_p=0.98, min_p=0.0)),
    ("small", 32000, 4, dict(temp=1.0, top_k=0, top_p=0.98, min_p=0.0)),
    ("normal", 32000, 4, dict(temp=1.0, top_k=0, top_p=0.98, min_p=0.0, repeat_penalty=1.1, penalty_last_n=128)),
    ("normal", 32000, 4, dict(temp=1.0, top_k=0, top_p=0.98, min_p=0.0, repeat_penalty=0.9, penalty_last_n=64)),
    ("ints", 8192, 3, dict(temp=1.0, top_k=0, top_p=0.9, min_p=0.0, repeat_penalty=1.3, penalty_last_n=64,
                           presence_penalty=0.5, freq_penalty=0.3)),
    ("normal", 32000, 3, dict(temp=1.0, top_k=0, top_p=1.0, min_p=0.0)),  # keep = V: every entry
    ("normal", 4099, 3, dict(temp=1.0, top_k=0, top_p=0.98, min_p=0.001)),
]


@pytest.mark.parametrize("case", list(enumerate(CASES)), ids=lambda c: f"s{c[0]}-{c[1][0]}-V{c[1][1]}")
@pytest.mark.parametrize("masked", [False, True])
def test_sortfree_matches_oracle(ctx, oracle, case, masked):
    i, (kind, V, rows, pk) = case
    rng = np.random.Generator(np.random.PCG64(7100 + i + (50 if masked else 0)))
    x = _bf16_round(_rows(rng, kind, rows, V))
    u = rng.random((rows, 2), dtype=np.float32)
    u[0, 0] = np.float32(0.9999999)  # a draw at the far end of the kept list
    hist = hl = mask = None
    if "penalty_last_n" in pk:
        H = 300
        hist = rng.integers(0, V, (rows, H), dtype=np.uint32)
        hist[:, ::3] = hist[:, :1]
        hl = rng.integers(0, H + 1, rows).astype(np.int32)
    if masked:
        bits = rng.random((rows, (V + 31) // 32 * 32)) < 0.6
        bits[:, 0] = True
        mask = pack_mask(bits)
    g = _sample(ctx, pk, x, u, hist, hl, mask)
    o = oracle_sample(oracle, pk, x, u, hist, hl, mask)
    errs = _compare(g, o, f"s{i}")
    assert not errs, "\n".join(errs[:20])


def test_config5_min_p_zero_sortfree(ctx, oracle):
    """Config 5 as named: 512 x 151936 bf16, top_p = 0.98, min_p = 0, repetition
    1.1 over 128-token histories -- every row through the sort-free pass."""
    from zinfer_amd.workloads import CONFIGS

    w = CONFIGS[5]()
    pk = dict(w.params, min_p=0.0)
    g = _sample(ctx, pk, w.logits, w.uniforms, w.hist, w.hist_len)
    o = oracle_sample(oracle, pk, w.logits, w.uniforms, w.hist, w.hist_len)
    errs = _compare(g, o, "c5")
    assert not errs, "\n".join(errs[:20])
