"""GPU parity against the committed golden fixtures (tests/golden/*.npz)."""
import numpy as np
import pytest

from paritylib import dev, f32bits, gpu_sample, to_device
from test_golden import load, sample_case

pytestmark = pytest.mark.gpu


def test_golden_sample_cases_on_gpu(ctx):
    z = load("sample_cases.npz")
    errs = []
    for i in range(int(z["count"][0])):
        pk, x, u, hist, hl, mask, ei, ed, ec = sample_case(z, i)
        g = gpu_sample(ctx, pk, x, u, hist, hl, mask, ei, ed, ec)
        for r in range(x.shape[0]):
            if g["tok"][r] != z[f"c{i}_tok"][r] or f32bits(g["margin"][r]) != f32bits(z[f"c{i}_margin"][r]):
                errs.append((i, r, "tok/margin"))
            if pk["temp"] > 0:
                n = int(z[f"c{i}_n"][r])
                if g["keep"][r] != z[f"c{i}_keep"][r] or g["ndraws"][r] != z[f"c{i}_ndraws"][r]:
                    errs.append((i, r, "keep/ndraws"))
                if not np.array_equal(g["cand_ids"][r, :n], z[f"c{i}_cand_ids"][r, :n]):
                    errs.append((i, r, "ids"))
                if not np.array_equal(f32bits(g["probs"][r, :n]), f32bits(z[f"c{i}_probs"][r, :n])):
                    errs.append((i, r, "probs"))
    assert not errs, errs[:10]


def test_golden_argmax_cases_on_gpu(ctx):
    z = load("argmax_cases.npz")
    for i in range(int(z["count"][0])):
        x = z[f"a{i}_x"][None, :]
        t, m, tl, mt = (a.cpu().numpy() for a in ctx.argmax_rows(to_device(x), vocab=x.shape[1]))
        assert t[0] == z[f"a{i}_tok"][0] and f32bits(m[0]) == f32bits(z[f"a{i}_margin"][0]), i
        assert tl[0] == z[f"a{i}_tok_low"][0] and mt[0] == z[f"a{i}_margin_true"][0], i


def test_golden_entropy_cases_on_gpu(ctx):
    z = load("entropy_cases.npz")
    for i in range(int(z["count"][0])):
        x = z[f"e{i}_x"][None, :]
        ent, ids, probs, _, _ = ctx.entropy_topk_rows(to_device(x), 8, vocab=x.shape[1])
        H = z[f"e{i}_entropy"][0]
        assert abs(float(ent.cpu()[0]) - H) <= 1e-5 * abs(H) + 1e-7, i
        assert np.array_equal(ids.cpu().numpy()[0].astype(np.uint32), z[f"e{i}_ids"]), i
        np.testing.assert_allclose(probs.cpu().numpy()[0], z[f"e{i}_probs"], rtol=1e-5)
