"""GPU parity: batched sampleWithMargin (zi_sample_rows) vs the CPU oracle.

Bar: token ids, margins, candidate ids/values, keep counts, uniforms consumed
and probabilities w_i/total are bit-exact (the device tail replays the
reference's sequential f32 arithmetic, src/sampler.zig:190-276)."""
import numpy as np
import pytest

from paritylib import compare_sample, gpu_sample, oracle_sample

pytestmark = pytest.mark.gpu


def _rows(rng, kind, rows, V):
    if kind == "normal":
        return (rng.standard_normal((rows, V)) * 3).astype(np.float32)
    if kind == "t3":
        return (rng.standard_t(3, (rows, V)) * 2).astype(np.float32)
    if kind == "ints":  # many exact ties, including -0.0 and +0.0
        x = rng.integers(-4, 5, (rows, V)).astype(np.float32)
        z = x == 0
        x[z & (rng.random((rows, V)) < 0.5)] = -0.0
        return x
    if kind == "neginf":  # most entries -inf (pruned vocab, model.zig:2127-2128)
        x = (rng.standard_normal((rows, V)) * 2).astype(np.float32)
        x[rng.random((rows, V)) < 0.9] = -np.inf
        return x
    if kind == "flat":
        return np.full((rows, V), 1.5, np.float32)
    if kind == "allneginf":  # every candidate -inf: the reference falls back to c[n-1]
        return np.full((rows, V), -np.inf, np.float32)
    if kind == "rising":  # increasing along the row: every later step beats the running top-k
        ramp = np.linspace(-6.0, 6.0, V, dtype=np.float32)
        return (ramp[None, :] + rng.standard_normal((rows, V)).astype(np.float32) * 0.01).astype(np.float32)
    raise ValueError(kind)


CASES = []
_r = np.random.Generator(np.random.PCG64(7))
for i in range(48):
    V = int(_r.choice([1, 2, 7, 15, 16, 17, 100, 255, 256, 1000, 4099, 16385, 32000, 70001, 131072]))
    rows = int(_r.choice([1, 3, 9]))
    kind = str(_r.choice(["normal", "t3", "ints", "neginf", "flat"]))
    if i % 16 == 15:
        kind = "allneginf"
    top_k = int(_r.choice([1, 2, 5, 40, 64, 200, 256]))
    if V <= 256 and _r.random() < 0.3:
        top_k = 0
    pk = dict(temp=float(_r.choice([0.5, 0.7, 1.0, 1.7])), top_k=top_k,
              top_p=float(_r.choice([1.0, 0.95, 0.5, 0.1])), min_p=float(_r.choice([0.0, 0.05, 0.3])))
    if _r.random() < 0.5:
        pk.update(repeat_penalty=float(_r.choice([1.1, 1.3, 0.9])), penalty_last_n=int(_r.choice([64, 256, 1000])))
    if _r.random() < 0.3:
        pk.update(freq_penalty=float(_r.choice([0.3, 0.0])), presence_penalty=float(_r.choice([0.5, 0.2])))
        pk.setdefault("penalty_last_n", 64)
    if _r.random() < 0.25:
        pk.update(xtc_probability=float(_r.choice([1.0, 0.5])), xtc_threshold=float(_r.choice([0.1, 0.15, 0.3])),
                  xtc_min_keep=int(_r.choice([1, 2])))
    CASES.append((i, V, rows, kind, pk, bool(_r.random() < 0.3), bool(_r.random() < 0.3)))


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"c{c[0]}-V{c[1]}-r{c[2]}-{c[3]}")
def test_sample_rows_matches_oracle(ctx, oracle, case):
    i, V, rows, kind, pk, use_mask, use_edits = case
    rng = np.random.Generator(np.random.PCG64(1000 + i))
    x = _rows(rng, kind, rows, V)
    u = rng.random((rows, 2), dtype=np.float32)
    hist = hist_len = mask = ei = ed = ec = None
    if "penalty_last_n" in pk:
        H = 300
        hist = rng.integers(0, V, (rows, H), dtype=np.uint32)
        hist[:, ::3] = hist[:, :1]  # repeats drive the frequency counts
        hist_len = rng.integers(0, H + 1, rows).astype(np.int32)
    if use_mask:
        W = (V + 31) // 32
        bits = rng.random((rows, W * 32)) < 0.4
        bits[:, 0] = True
        from zinfer_amd.workloads import pack_mask
        mask = pack_mask(bits)
    if use_edits:
        E = 16
        ei = np.stack([rng.choice(V, size=min(E, V), replace=False).astype(np.uint32) for _ in range(rows)])
        ed = (rng.random(ei.shape) * 3).astype(np.float32)
        ec = rng.integers(0, ei.shape[1] + 1, rows).astype(np.int32)
    g = gpu_sample(ctx, pk, x, u, hist, hist_len, mask, ei, ed, ec)
    o = oracle_sample(oracle, pk, x, u, hist, hist_len, mask, ei, ed, ec)
    errs = compare_sample(g, o, pk, V, f"case{i}")
    assert not errs, "\n".join(errs[:20])


@pytest.mark.parametrize("V", [16, 17, 1000, 32000, 131073])
def test_greedy_temp0_matches_reference_argmax(ctx, oracle, V):
    rng = np.random.Generator(np.random.PCG64(V))
    rows = 4
    x = rng.integers(-3, 4, (rows, V)).astype(np.float32)  # heavy ties: lane-16 rule decides
    hist = rng.integers(0, V, (rows, 64), dtype=np.uint32)
    hl = np.full(rows, 64, np.int32)
    pk = dict(temp=0.0, repeat_penalty=1.2, penalty_last_n=64)
    u = np.zeros((rows, 2), np.float32)
    g = gpu_sample(ctx, pk, x, u, hist, hl)
    o = oracle_sample(oracle, pk, x, u, hist, hl)
    errs = compare_sample(g, o, pk, V, "greedy")
    assert not errs, "\n".join(errs[:20])


@pytest.mark.parametrize("cfg", [1, 2, 3])
def test_config_full_size_parity(ctx, oracle, cfg):
    from zinfer_amd.workloads import CONFIGS

    w = CONFIGS[cfg]()
    pk = dict(w.params)
    g = gpu_sample(ctx, pk, w.logits, w.uniforms, w.hist, w.hist_len, w.mask)
    o = oracle_sample(oracle, pk, w.logits, w.uniforms, w.hist, w.hist_len, w.mask)
    errs = compare_sample(g, o, pk, w.vocab, w.name)
    assert not errs, "\n".join(errs[:20])
    if cfg == 1:  # the config also asks for greedy argmax on the same row
        pk0 = dict(pk, temp=0.0)
        g0 = gpu_sample(ctx, pk0, w.logits, w.uniforms, w.hist, w.hist_len)
        o0 = oracle_sample(oracle, pk0, w.logits, w.uniforms, w.hist, w.hist_len)
        errs = compare_sample(g0, o0, pk0, w.vocab, "c1-greedy")
        assert not errs, "\n".join(errs)


@pytest.mark.parametrize("H,win", [(600, 256), (1024, 1000), (3000, 256), (5000, 1000)])
def test_long_history_rows(ctx, oracle, H, win):
    """History rows longer than the kernels prefetch (hist_ld > 1024) go
    through the window compaction first; shorter rows are prefetched whole."""
    rng = np.random.Generator(np.random.PCG64(H + win))
    rows, V = 6, 50000
    x = (rng.standard_t(3, (rows, V)) * 2).astype(np.float32)
    u = rng.random((rows, 2), dtype=np.float32)
    hist = rng.integers(0, V, (rows, H), dtype=np.uint32)
    hist[:, 1::4] = rng.integers(0, 40, (rows, (H + 2) // 4), dtype=np.uint32)[:, : hist[:, 1::4].shape[1]]
    top = np.argsort(-x, axis=1)[:, :8].astype(np.uint32)  # penalize some of the leaders
    hist[:, -8:] = top
    hist_len = np.array([H, H - 1, win // 2, 0, H - win + 3, min(H, 37)], np.int32)
    pk = dict(temp=0.8, top_k=50, top_p=0.9, min_p=0.05, repeat_penalty=1.3, freq_penalty=0.2,
              presence_penalty=0.4, penalty_last_n=win)
    g = gpu_sample(ctx, pk, x, u, hist, hist_len)
    o = oracle_sample(oracle, pk, x, u, hist, hist_len)
    errs = compare_sample(g, o, pk, V, f"hist{H}-win{win}")
    assert not errs, "\n".join(errs[:20])


@pytest.mark.parametrize("rows,V,k,kind,pen,mask", [
    (256, 20000, 50, "t3", True, False),
    (300, 32000, 40, "normal", False, True),
    (260, 131072, 256, "normal", True, False),
    (256, 4099, 7, "ints", True, True),
    (512, 17, 5, "flat", False, False),
    (256, 70000, 50, "rising", True, False),
    (256, 40000, 256, "rising", False, False),
])
def test_large_batch_rows(ctx, oracle, rows, V, k, kind, pen, mask):
    """Batches of >= 256 rows run one workgroup per row (the running top-k
    kept across the row's chunks)."""
    rng = np.random.Generator(np.random.PCG64(rows * 7 + V))
    x = _rows(rng, kind, rows, V)
    u = rng.random((rows, 2), dtype=np.float32)
    pk = dict(temp=0.8, top_k=k, top_p=0.9, min_p=0.05)
    hist = hl = m = ei = ed = ec = None
    if pen:
        pk.update(repeat_penalty=1.2, freq_penalty=0.3, presence_penalty=0.4, penalty_last_n=128)
        hist = rng.integers(0, V, (rows, 200), dtype=np.uint32)
        hist[:, -8:] = np.argsort(-x, axis=1)[:, :8].astype(np.uint32)  # penalize some of the leaders
        hl = rng.integers(0, 201, rows).astype(np.int32)
        E = 8
        ei = np.stack([rng.choice(V, size=min(E, V), replace=False).astype(np.uint32) for _ in range(rows)])
        ed = (rng.random(ei.shape) * 2).astype(np.float32)
        ec = rng.integers(0, ei.shape[1] + 1, rows).astype(np.int32)
    if mask:
        from zinfer_amd.workloads import pack_mask
        bits = rng.random((rows, (V + 31) // 32 * 32)) < 0.5
        bits[:, 0] = True
        m = pack_mask(bits)
    g = gpu_sample(ctx, pk, x, u, hist, hl, m, ei, ed, ec)
    o = oracle_sample(oracle, pk, x, u, hist, hl, m, ei, ed, ec)
    errs = compare_sample(g, o, pk, V, f"rows{rows}")
    assert not errs, "\n".join(errs[:20])


LATE_SCENES = ["leaders", "all_leaders", "neg_edit", "nan_free_mix", "rp_below_one"]


# config 2's k; the largest k with the per-wave candidate threshold (kTauWaveMaxK
# = 58, zi_rowpass.hpp) and the first with the bisection; the largest k with the
# late select (kLatePenMaxK = 64, zi_sample_kernels.hpp) and the first without
LATE_KS = [50, 58, 59, 64, 65]


@pytest.mark.parametrize("top_k", LATE_KS)
@pytest.mark.parametrize("scene", LATE_SCENES)
def test_late_penalty_select(ctx, oracle, scene, top_k):
    """Penalties that never raise a logit are applied to the chunk's raw
    candidates only; when penalized leaders drop below the candidate
    threshold (or an edit delta is negative) the kernel penalizes its
    registers and selects again.  Both branches must match the oracle, on
    both sides of the threshold and late-select cutoffs."""
    rng = np.random.Generator(np.random.PCG64(4200 + LATE_SCENES.index(scene) + 10 * LATE_KS.index(top_k)))
    rows, V = 16, 128256  # 64 workgroups: the late-penalty select is taken from that grid size
    x = (rng.standard_t(3, (rows, V)) * 2).astype(np.float32)
    u = rng.random((rows, 2), dtype=np.float32)
    order = np.argsort(-x, axis=1, kind="stable")
    H = 256
    hist = rng.integers(0, V, (rows, H), dtype=np.uint32)
    pk = dict(temp=0.7, top_k=top_k, top_p=0.9, min_p=0.05, repeat_penalty=1.15, freq_penalty=0.3,
              presence_penalty=0.5, penalty_last_n=256)
    ei = ed = ec = None
    if scene == "leaders":  # a few leaders penalized: candidates stay >= k
        hist[:, -3:] = order[:, :3]
    elif scene == "all_leaders":  # every leader penalized hard: the fallback selects again
        hist[:, :200] = order[:, :200]
        pk.update(repeat_penalty=3.0, presence_penalty=4.0)
    elif scene == "neg_edit":  # an edit that raises a logit: fallback in that chunk
        E = 8
        ei = np.stack([rng.choice(V, size=E, replace=False) for _ in range(rows)]).astype(np.uint32)
        ed = (rng.random((rows, E)) * 2).astype(np.float32)
        ed[::2, 0] = -25.0  # lifts a random id into the top-k
        ec = np.full(rows, E, np.int32)
    elif scene == "nan_free_mix":  # penalized leaders with zero edits and short windows
        hist[:, -40:] = order[:, 10:50]
        E = 4
        ei = np.ascontiguousarray(order[:, :E]).astype(np.uint32)
        ed = np.zeros((rows, E), np.float32)
        ed[:, 1] = 0.75
        ec = np.arange(rows, dtype=np.int32) % (E + 1)
    elif scene == "rp_below_one":  # raises negative logits: the in-stream penalty path
        hist[:, -20:] = order[:, :20]
        pk.update(repeat_penalty=0.9)
    hist_len = np.full(rows, H, np.int32)
    hist_len[1] = 0
    hist_len[2] = 17
    g = gpu_sample(ctx, pk, x, u, hist, hist_len, None, ei, ed, ec)
    o = oracle_sample(oracle, pk, x, u, hist, hist_len, None, ei, ed, ec)
    errs = compare_sample(g, o, pk, V, f"late-{scene}")
    assert not errs, "\n".join(errs[:20])
