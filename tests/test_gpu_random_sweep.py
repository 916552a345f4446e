"""GPU parity: a seeded random sweep over the sampling entry point
(zi_sample_rows, src/sampler.zig:190-276, with the mask of grammar.zig:446-479
and the softcap of model.zig:2492-2514 fused into the read).

Each case draws a shape, a dtype, a logit distribution and a parameter set,
so that the dispatch lands on every kernel path (chunked with in-stream or
late penalties, one workgroup per row, the min-p prefix, the whole-order
passes, the candidates-only softcap) in combinations the hand-written cases
do not pin down one by one.  Bar: token ids, margins, uniforms consumed and
keep bit-exact; with candidate outputs also the kept ids, values and
probabilities, exactly as in the other parity files."""
import os

import numpy as np
import pytest

from paritylib import compare_sample, dev, gpu_sample, oracle_sample, to_device
from zinfer_amd.workloads import _bf16_round, pack_mask

pytestmark = pytest.mark.gpu

N_CASES = int(os.environ.get("ZI_SWEEP_CASES", "160"))  # seeds 0 .. N_CASES - 1


def _draw(seed):
    rng = np.random.Generator(np.random.PCG64(9000 + seed))
    bf16 = bool(rng.random() < 0.4)
    top_k = int(rng.choice([1, 5, 40, 50, 58, 59, 64, 65, 100, 256, 257, 1000, 0, 0]))
    whole = top_k == 0 or top_k > 256
    rows = int(rng.choice([1, 3, 16, 64, 256, 300] if not whole else [1, 3, 16, 64, 256]))
    Vs = [1000, 4099, 32000, 65536, 128256, 151936]
    V = int(rng.choice(Vs))
    budget = 2_000_000 if whole else 12_000_000  # oracle time: a full sort per whole-vocabulary row
    while rows * V > budget and V > 1000:
        V = int(Vs[max(0, Vs.index(V) - 1)])
    while rows * V > budget and rows > 1:
        rows //= 2
    pk = dict(temp=float(rng.choice([0.5, 0.8, 1.0, 1.3])), top_k=top_k,
              top_p=float(rng.choice([1.0, 0.98, 0.9, 0.5])), min_p=float(rng.choice([0.0, 0.05, 0.2])))
    pen = rng.choice(["none", "rep_up", "rep_down", "freq", "all"])
    if pen in ("rep_up", "all"):
        pk.update(repeat_penalty=float(rng.choice([1.1, 1.3, 2.0])))
    if pen == "rep_down":
        pk.update(repeat_penalty=0.9)
    if pen in ("freq", "all"):
        pk.update(freq_penalty=float(rng.choice([0.0, 0.3])), presence_penalty=float(rng.choice([0.2, 0.5])))
    if pen != "none":
        pk.update(penalty_last_n=int(rng.choice([32, 64, 256])))
    if rng.random() < 0.3:
        pk.update(final_logit_softcap=float(rng.choice([30.0, 5.0])))
    if rng.random() < 0.15:
        pk.update(xtc_probability=1.0, xtc_threshold=float(rng.choice([0.05, 0.1])), xtc_min_keep=1)
    kind = rng.choice(["normal", "wide", "t3", "ints", "neginf"])
    if kind == "normal":
        x = rng.standard_normal((rows, V)) * 3
    elif kind == "wide":
        x = rng.standard_normal((rows, V)) * 12
    elif kind == "t3":
        x = rng.standard_t(3, (rows, V)) * 2
    elif kind == "ints":
        x = rng.integers(-6, 7, (rows, V)).astype(np.float64)
    else:
        x = rng.standard_normal((rows, V)) * 4
        x[rng.random((rows, V)) < 0.4] = -np.inf
    x = x.astype(np.float32)
    if bf16:
        x = _bf16_round(x)
    hist = hl = None
    if pen != "none":
        H = 256
        hist = rng.integers(0, V, (rows, H), dtype=np.uint32)
        hist[:, -4:] = np.argsort(-x, axis=1, kind="stable")[:, :4].astype(np.uint32)  # some leaders
        hl = rng.integers(0, H + 1, rows).astype(np.int32)
    ei = ed = ec = None
    if rng.random() < 0.3:
        E = 8
        ei = np.stack([rng.choice(V, size=E, replace=False) for _ in range(rows)]).astype(np.uint32)
        ed = (rng.random((rows, E)) * 2).astype(np.float32)
        if rng.random() < 0.3:
            ed[:, 0] = -3.0  # an edit that raises a logit
        ec = rng.integers(0, E + 1, rows).astype(np.int32)
    m = None
    if rng.random() < 0.3:
        bits = rng.random((rows, (V + 31) // 32 * 32)) < float(rng.choice([0.05, 0.5, 0.95]))
        bits[:, 0] = True
        m = pack_mask(bits)
    u = rng.random((rows, 2), dtype=np.float32)
    cands = bool(rng.random() < 0.5)
    return dict(rows=rows, V=V, bf16=bf16, pk=pk, x=x, hist=hist, hl=hl, m=m, ei=ei, ed=ed, ec=ec, u=u,
                cands=cands, label=f"seed {seed}: {rows}x{V} {'bf16' if bf16 else 'f32'} {kind} {pen} {pk}")


def _sample_nocands(ctx, c):
    import torch

    from zinfer_amd.api import SampleResult, params

    rows, V = c["x"].shape
    L = to_device(c["x"], c["bf16"])
    d = L.device
    out = SampleResult(tok=torch.empty(rows, dtype=torch.int32, device=d),
                       margin=torch.empty(rows, dtype=torch.float32, device=d),
                       ndraws=torch.empty(rows, dtype=torch.int32, device=d),
                       keep=torch.empty(rows, dtype=torch.int32, device=d))
    ctx.sample_rows(params(**c["pk"]), L, dev(c["u"]), vocab=V, hist=dev(c["hist"]), hist_len=dev(c["hl"], None),
                    mask=dev(c["m"]), edit_ids=dev(c["ei"]), edit_delta=dev(c["ed"]), edit_count=dev(c["ec"]),
                    out=out)
    torch.cuda.synchronize()
    return (out.tok.cpu().numpy().astype(np.uint32), out.margin.cpu().numpy(), out.ndraws.cpu().numpy(),
            out.keep.cpu().numpy())


@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_sweep_matches_oracle(ctx, oracle, seed):
    c = _draw(seed)
    print(c["label"], flush=True)
    o = oracle_sample(oracle, c["pk"], c["x"], c["u"], c["hist"], c["hl"], c["m"], c["ei"], c["ed"], c["ec"])
    if c["cands"]:
        g = gpu_sample(ctx, c["pk"], c["x"], c["u"], c["hist"], c["hl"], c["m"], c["ei"], c["ed"], c["ec"],
                       bf16=c["bf16"])
        errs = compare_sample(g, o, c["pk"], c["V"], c["label"])
    else:
        tok, margin, nd, keep = _sample_nocands(ctx, c)
        errs = []
        for r, (t, mg, diag) in enumerate(o):
            if int(tok[r]) != t:
                errs.append(f"{c['label']} row {r}: tok {tok[r]} vs {t}")
            if not (np.float32(margin[r]) == np.float32(mg)):
                errs.append(f"{c['label']} row {r}: margin {margin[r]!r} vs {mg!r}")
            if int(nd[r]) != diag["ndraws"]:
                errs.append(f"{c['label']} row {r}: ndraws {nd[r]} vs {diag['ndraws']}")
            if int(keep[r]) != diag["keep"]:
                errs.append(f"{c['label']} row {r}: keep {keep[r]} vs {diag['keep']}")
    assert not errs, "\n".join(errs[:20])
