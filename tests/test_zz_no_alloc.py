"""GPU: zi_sample_rows_noalloc (the allocation-free variant of
zi_sample_rows, static device scratch) against zi_sample_rows on the same
inputs, through the C ABI.  Bit-exact: tokens, margins, uniforms consumed,
keep, candidate ids / values and probabilities.  Two calls in a row reuse the
static scratch, the second on a smaller batch, so anything a call leaves
behind (tickets, lists) would show."""
import ctypes as C

import numpy as np
import pytest

from paritylib import dev, to_device


def _batch(logits, V, hist=None, hist_len=None, mask=None):
    from zinfer_amd._lib import ZI_BF16, ZI_F32, ZiBatch
    import torch

    b = ZiBatch()
    b.logits = logits.data_ptr()
    b.dtype = ZI_BF16 if logits.dtype == torch.bfloat16 else ZI_F32
    b.rows, b.vocab, b.ld = logits.shape[0], V, logits.shape[1]
    if hist is not None:
        b.hist, b.hist_len, b.hist_ld = hist.data_ptr(), hist_len.data_ptr(), hist.shape[1]
    if mask is not None:
        b.mask, b.mask_ld = mask.data_ptr(), mask.shape[1]
    return b


def _outs(rows, k):
    import torch

    from zinfer_amd._lib import ZiSampleOut

    t = dict(tok=torch.full((rows,), -1, dtype=torch.int32, device="cuda"),
             margin=torch.full((rows,), -7.0, dtype=torch.float32, device="cuda"),
             ndraws=torch.full((rows,), -1, dtype=torch.int32, device="cuda"),
             keep=torch.full((rows,), -1, dtype=torch.int32, device="cuda"),
             cand_ids=torch.full((rows, k), -1, dtype=torch.int32, device="cuda"),
             cand_vals=torch.zeros((rows, k), dtype=torch.float32, device="cuda"),
             probs=torch.zeros((rows, k), dtype=torch.float32, device="cuda"))
    o = ZiSampleOut()
    for f in t:
        setattr(o, f, t[f].data_ptr())
    o.cand_ld = k
    return t, o


def _run(ctx, pk, logits, uniforms, V, hist=None, hist_len=None, mask=None):
    """(zi_sample_rows outputs, zi_sample_rows_noalloc outputs) as numpy."""
    import torch

    from zinfer_amd._lib import check, lib
    from zinfer_amd.api import params

    p = params(**pk)
    rows = logits.shape[0]
    k = max(1, V if (p.top_k == 0 or p.top_k > V) else p.top_k)
    b = _batch(logits, V, hist, hist_len, mask)
    stream = torch.cuda.current_stream()
    ta, oa = _outs(rows, k)
    check(lib().zi_set_stream(ctx.h, C.c_void_p(stream.cuda_stream)))
    check(lib().zi_sample_rows(ctx.h, C.byref(p), C.byref(b), C.c_void_p(uniforms.data_ptr()), C.byref(oa)))
    tb, ob = _outs(rows, k)
    check(lib().zi_sample_rows_noalloc(C.byref(p), C.byref(b), C.c_void_p(uniforms.data_ptr()), C.byref(ob),
                                       C.c_void_p(stream.cuda_stream)))
    torch.cuda.synchronize()
    return ({f: v.cpu().numpy() for f, v in ta.items()}, {f: v.cpu().numpy() for f, v in tb.items()})


def _same(a, b, greedy, what):
    fields = ["tok", "margin", "ndraws"] + ([] if greedy else ["keep", "cand_ids", "cand_vals", "probs"])
    for f in fields:
        x, y = np.ascontiguousarray(a[f]), np.ascontiguousarray(b[f])
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), f"{what}: {f} differs"


CASES = [
    # (rows, V, params, bf16, penalties, mask): each run twice, then on a smaller batch
    (64, 128256, dict(temp=0.7, top_k=50, top_p=0.9, min_p=0.05, repeat_penalty=1.15, freq_penalty=0.3,
                      presence_penalty=0.5, penalty_last_n=256), False, True, False),
    (32, 151936, dict(temp=0.7, top_k=40, top_p=0.95), False, False, True),
    (300, 32000, dict(temp=1.0, top_k=64, top_p=0.9, min_p=0.0, repeat_penalty=1.1, penalty_last_n=64), True,
     True, False),
    (8, 262144, dict(temp=0.0, repeat_penalty=1.2, penalty_last_n=64), False, True, False),
    (512, 151936, dict(temp=0.0), True, False, False),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(len(CASES)))
def test_noalloc_matches_sample_rows(ctx, case):
    import torch

    rows, V, pk, bf16, pen, use_mask = CASES[case]
    rng = np.random.Generator(np.random.PCG64(7700 + case))
    for call, r in enumerate([rows, rows, max(1, rows // 3)]):
        x = (rng.standard_t(3, (r, V)) * 2).astype(np.float32)
        L = to_device(x, bf16)
        u = dev(rng.random((r, 2), dtype=np.float32))
        hist = hl = mask = None
        if pen:
            hist = dev(rng.integers(0, V, (r, 256), dtype=np.uint32))
            hl = dev(rng.integers(0, 257, r).astype(np.int32))
        if use_mask:
            from zinfer_amd.workloads import pack_mask

            bits = rng.random((r, V)) < 0.2
            bits[:, 0] = True
            mask = dev(pack_mask(bits))
        a, b = _run(ctx, pk, L, u, V, hist, hl, mask)
        _same(a, b, pk["temp"] <= 0, f"case {case} call {call} rows {r}")
        del L
        torch.cuda.synchronize()


def test_noalloc_rejects_what_it_cannot_serve():
    """Size limits are refused before any HIP call (the whole-order sort, long
    history rows, more rows than the static scratch holds), so this runs
    without a GPU."""
    from zinfer_amd._lib import ZI_ERR_CAPACITY, ZI_ERR_UNSUPPORTED, ZiBatch, ZiSampleOut, lib
    from zinfer_amd.api import params

    o = ZiSampleOut()
    o.tok, o.margin = 16, 16
    b = ZiBatch()
    b.logits, b.dtype, b.rows, b.vocab, b.ld = 16, 0, 4, 1000, 1000
    assert lib().zi_sample_rows_noalloc(C.byref(params(temp=0.8, top_k=0)), C.byref(b), None, C.byref(o),
                                        None) == ZI_ERR_UNSUPPORTED
    assert lib().zi_sample_rows_noalloc(C.byref(params(temp=0.8, top_k=300)), C.byref(b), None, C.byref(o),
                                        None) == ZI_ERR_UNSUPPORTED
    b.hist, b.hist_len, b.hist_ld = 16, 16, 2048
    assert lib().zi_sample_rows_noalloc(C.byref(params(temp=0.8, top_k=40)), C.byref(b), None, C.byref(o),
                                        None) == ZI_ERR_UNSUPPORTED
    b.hist = None
    b.rows = 513
    assert lib().zi_sample_rows_noalloc(C.byref(params(temp=0.8, top_k=40)), C.byref(b), None, C.byref(o),
                                        None) == ZI_ERR_CAPACITY
