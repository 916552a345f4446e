"""GPU: zi_reserve allocates the lazily allocated scratch up front, after
which whole-vocabulary sampling and the pruned rows' dense path run under
HIP graph capture: each replay (with eager work and synchronisations between
replays) reproduces the eager result, which matches the oracle."""
import numpy as np
import pytest

from paritylib import compare_sample, dev, oracle_sample, to_device

pytestmark = pytest.mark.gpu


def test_reserve_then_capture_whole_order_and_pruned(oracle):
    import torch

    from zinfer_amd._lib import ZI_RESERVE_PRUNED_DENSE, ZI_RESERVE_WHOLE_ORDER
    from zinfer_amd.api import Context, SampleResult, params

    rows, V = 8, 32000
    ctx = Context(0, max_rows=16, max_vocab=V)
    ctx.reserve(ZI_RESERVE_WHOLE_ORDER | ZI_RESERVE_PRUNED_DENSE)
    rng = np.random.Generator(np.random.PCG64(606))
    x = (rng.standard_normal((rows, V)) * 2).astype(np.float32)
    L = to_device(x)
    u = dev(rng.random((rows, 2), dtype=np.float32))
    pw = dict(temp=0.9, top_k=0, top_p=0.98, min_p=0.0)  # whole order, every row sorted
    ng = (V + 7) // 8
    G = np.stack([np.concatenate([np.arange(64), rng.choice(np.arange(64, ng), 512, replace=False)])
                  for _ in range(rows)]).astype(np.int32)
    gd, cd = dev(G), dev(np.full(rows, G.shape[1], np.int32))
    pp = dict(temp=0.8, top_k=40, top_p=0.95, min_p=0.05, final_logit_softcap=20.0)  # pruned: dense path

    def outs():
        return [SampleResult(tok=torch.empty(rows, dtype=torch.int32, device="cuda"),
                             margin=torch.empty(rows, dtype=torch.float32, device="cuda"),
                             ndraws=torch.empty(rows, dtype=torch.int32, device="cuda")) for _ in range(2)]

    def launch(o):
        ctx.sample_rows(params(**pw), L, u, vocab=V, out=o[0])
        ctx.sample_rows(params(**pp), L, u, vocab=V, out=o[1], groups=gd, group_count=cd)

    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        eager = outs()
        launch(eager)
        torch.cuda.synchronize()
        cap = outs()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            launch(cap)
        torch.cuda.synchronize()
        for rep in range(3):
            for o in cap:
                o.tok.fill_(-1)
            g.replay()
            torch.cuda.synchronize()
            for a, b in zip(eager, cap):
                assert torch.equal(a.tok, b.tok) and torch.equal(a.margin, b.margin), f"replay {rep}"
            launch(outs())  # eager work between replays
            torch.cuda.synchronize()
    o1 = oracle_sample(oracle, pw, x, u.cpu().numpy())
    assert [t for t, _, _ in o1] == [int(t) for t in eager[0].tok.cpu().numpy()]
    xp = np.stack([oracle.pruned_row(x[r], G[r], V) for r in range(rows)])
    o2 = oracle_sample(oracle, pp, xp, u.cpu().numpy())
    assert [t for t, _, _ in o2] == [int(t) for t in eager[1].tok.cpu().numpy()]
    ctx.close()


def test_reserve_rejects_unknown_flags():
    from zinfer_amd._lib import ZiError
    from zinfer_amd.api import Context

    ctx = Context(0, max_rows=4, max_vocab=1024)
    with pytest.raises(ZiError):
        ctx.reserve(8)
    ctx.close()
