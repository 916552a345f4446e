"""Shared helpers: run the same seeded rows through libzinfer_hip (GPU) and the
CPU oracle, and compare (bit-exact for ids / values, as the parity bar asks)."""
from __future__ import annotations

import numpy as np


def to_device(arr2d: np.ndarray, bf16: bool = False, ld: int | None = None):
    import torch

    rows, V = arr2d.shape
    ld = ld or (V + 7) // 8 * 8
    dt = torch.bfloat16 if bf16 else torch.float32
    t = torch.zeros((rows, ld), dtype=dt, device="cuda")
    t[:, :V] = torch.from_numpy(np.ascontiguousarray(arr2d, dtype=np.float32)).to("cuda").to(dt)
    return t


def dev(a, dtype=None):
    import torch

    if a is None:
        return None
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to("cuda")


def windows(hist, hist_len, W):
    out = []
    for r in range(hist.shape[0]):
        hl = int(hist_len[r])
        nw = min(hl, W)
        out.append(hist[r, hl - nw:hl])
    return out


def f32bits(x):
    return np.asarray(x, dtype=np.float32).view(np.uint32)


def gpu_sample(ctx, pkw, logits, uniforms, hist=None, hist_len=None, mask=None, edit_ids=None, edit_delta=None,
               edit_count=None, bf16=False):
    import torch
    from zinfer_amd.api import params

    rows, V = logits.shape
    L = to_device(logits, bf16)
    p = params(**pkw)
    res = ctx.sample_rows(p, L, dev(uniforms), vocab=V, hist=dev(hist), hist_len=dev(hist_len, None),
                          mask=dev(mask), edit_ids=dev(edit_ids), edit_delta=dev(edit_delta),
                          edit_count=dev(edit_count), cands=pkw.get("temp", 0.8) > 0)
    torch.cuda.synchronize()
    out = dict(tok=res.tok.cpu().numpy().astype(np.uint32), margin=res.margin.cpu().numpy(),
               ndraws=res.ndraws.cpu().numpy())
    if res.keep is not None:
        out.update(keep=res.keep.cpu().numpy(), cand_ids=res.cand_ids.cpu().numpy().astype(np.uint32),
                   cand_vals=res.cand_vals.cpu().numpy(), probs=res.probs.cpu().numpy())
    return out


def oracle_sample(oracle, pkw, logits, uniforms, hist=None, hist_len=None, mask=None, edit_ids=None,
                  edit_delta=None, edit_count=None):
    rows, V = logits.shape
    okw = {k: v for k, v in pkw.items() if k != "seed"}
    p = oracle.params(**okw)
    W = pkw.get("penalty_last_n", 64)
    wins = windows(hist, hist_len, W) if hist is not None else [None] * rows
    k = V if (pkw.get("top_k", 40) in (0,) or pkw.get("top_k", 40) > V) else pkw.get("top_k", 40)
    res = []
    for r in range(rows):
        ei = ed = None
        if edit_ids is not None:
            n = int(edit_count[r])
            ei, ed = edit_ids[r, :n], edit_delta[r, :n]
        tok, margin, diag = oracle.sample_row(p, logits[r], uniforms[r], mask=None if mask is None else mask[r],
                                              window=wins[r], edit_ids=ei, edit_deltas=ed, cap=k)
        res.append((tok, margin, diag))
    return res


def compare_sample(g, o, pkw, V, label=""):
    """Bit-exact comparison; returns a list of mismatch descriptions."""
    errs = []
    greedy = pkw.get("temp", 0.8) <= 0
    top_k = pkw.get("top_k", 40)
    whole = (V if (top_k == 0 or top_k > V) else top_k) > 256  # outputs cover the kept entries only
    for r, (tok, margin, diag) in enumerate(o):
        if int(g["tok"][r]) != tok:
            errs.append(f"{label} row {r}: tok gpu={g['tok'][r]} oracle={tok}")
        if f32bits(g["margin"][r]) != f32bits(margin) and not (g["margin"][r] == margin):
            errs.append(f"{label} row {r}: margin gpu={g['margin'][r]!r} oracle={margin!r}")
        if greedy:
            if int(g["ndraws"][r]) != 0:
                errs.append(f"{label} row {r}: greedy ndraws {g['ndraws'][r]}")
            continue
        if int(g["ndraws"][r]) != diag["ndraws"]:
            errs.append(f"{label} row {r}: ndraws gpu={g['ndraws'][r]} oracle={diag['ndraws']}")
        if int(g["keep"][r]) != diag["keep"]:
            errs.append(f"{label} row {r}: keep gpu={g['keep'][r]} oracle={diag['keep']}")
        n = min(diag["keep"], g["cand_ids"].shape[1]) if whole else diag["n"]
        gi = g["cand_ids"][r, :n]
        oi, ov, op = diag["ids"][:n], diag["vals"][:n], diag["probs"][:n]
        if not np.array_equal(gi, oi):
            bad = int(np.nonzero(gi != oi)[0][0])
            errs.append(f"{label} row {r}: cand id[{bad}] gpu={gi[bad]} oracle={oi[bad]}")
        gv = g["cand_vals"][r, :n]
        if not (np.array_equal(f32bits(gv), f32bits(ov)) or (whole and np.array_equal(gv, ov))):
            errs.append(f"{label} row {r}: cand values differ")  # whole-order rows report -0 as +0
        if not np.array_equal(f32bits(g["probs"][r, :n]), f32bits(op)):
            bad = int(np.nonzero(f32bits(g["probs"][r, :n]) != f32bits(op))[0][0])
            errs.append(f"{label} row {r}: prob[{bad}] gpu={g['probs'][r, bad]!r} oracle={op[bad]!r}")
    return errs
