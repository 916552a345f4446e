"""ctypes view of the CPU oracle (oracle/oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product package.  Each wrapper calls
one C restatement of a reference function; see oracle.h for the reference
file:line each one follows and how it is pinned.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")


class OrParams(C.Structure):
    _fields_ = [
        ("temp", C.c_float),
        ("top_k", C.c_uint32),
        ("top_p", C.c_float),
        ("min_p", C.c_float),
        ("repeat_penalty", C.c_float),
        ("freq_penalty", C.c_float),
        ("presence_penalty", C.c_float),
        ("penalty_last_n", C.c_uint32),
        ("dry_multiplier", C.c_float),
        ("dry_base", C.c_float),
        ("dry_allowed_length", C.c_uint32),
        ("dry_range", C.c_uint32),
        ("xtc_probability", C.c_float),
        ("xtc_threshold", C.c_float),
        ("xtc_min_keep", C.c_uint32),
        ("final_logit_softcap", C.c_float),
    ]


class OrResult(C.Structure):
    _fields_ = [("tok", C.c_uint32), ("margin", C.c_float)]


class OrDiag(C.Structure):
    _fields_ = [
        ("ndraws", C.c_int32),
        ("n", C.c_int32),
        ("keep", C.c_int32),
        ("start", C.c_int32),
        ("total", C.c_float),
        ("cap", C.c_int32),
        ("ids", C.POINTER(C.c_uint32)),
        ("vals", C.POINTER(C.c_float)),
        ("probs", C.POINTER(C.c_float)),
    ]


class OrJson(C.Structure):
    """JsonValidator state, src/grammar.zig:59-68 (see or_json in oracle.h)."""
    _fields_ = [
        ("state", C.c_int32),
        ("escape", C.c_int32),
        ("num", C.c_int32),
        ("depth", C.c_uint32),
        ("stack", C.c_uint8 * 64),
        ("lit_expected", C.c_uint8 * 8),
        ("lit_len", C.c_uint8),
        ("lit_idx", C.c_uint8),
        ("object_only", C.c_uint8),
        ("pad_", C.c_uint8),
    ]


class OrAdaptive(C.Structure):
    _fields_ = [
        ("cur_k", C.c_uint64),
        ("max_k", C.c_uint64),
        ("min_k", C.c_uint64),
        ("consecutive_rejections", C.c_uint64),
        ("cooldown_steps", C.c_uint64),
        ("last_margin", C.c_float),
    ]


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        f32p, u32p = C.POINTER(C.c_float), C.POINTER(C.c_uint32)
        L.or_softcap.restype = C.c_float
        L.or_softcap.argtypes = [C.c_float, C.c_float]
        L.or_zexpf.restype = C.c_float
        L.or_zexpf.argtypes = [C.c_float]
        L.or_zexpf_array.restype = None
        L.or_zexpf_array.argtypes = [C.c_void_p, C.c_void_p, C.c_int64]
        L.or_exp32.restype = C.c_float
        L.or_exp32.argtypes = [C.c_float]
        L.or_tanh32.restype = C.c_float
        L.or_tanh32.argtypes = [C.c_float]
        L.or_softcap_tail.restype = C.c_float
        L.or_softcap_tail.argtypes = [C.c_float, C.c_float]
        L.or_pow_zig.restype = C.c_float
        L.or_pow_zig.argtypes = [C.c_float, C.c_float]
        L.or_params_default.argtypes = [C.POINTER(OrParams)]
        L.or_apply_penalty.argtypes = [f32p, C.c_uint32, u32p, C.c_uint32, C.c_float, C.c_float, C.c_float]
        L.or_apply_edits.argtypes = [f32p, C.c_uint32, u32p, f32p, C.c_uint32]
        L.or_dry_edits.restype = C.c_uint32
        L.or_dry_edits.argtypes = [u32p, C.c_uint32, u32p, C.c_uint32, C.c_float, C.c_float,
                                   C.c_uint32, C.c_uint32, u32p, f32p]
        L.or_apply_mask.argtypes = [f32p, C.c_uint32, u32p]
        L.or_argmax_with_margin.restype = OrResult
        L.or_argmax_with_margin.argtypes = [f32p, C.c_uint32]
        L.or_argmax_true.restype = OrResult
        L.or_argmax_true.argtypes = [f32p, C.c_uint32]
        L.or_sample_penalized.restype = OrResult
        L.or_sample_penalized.argtypes = [C.POINTER(OrParams), f32p, C.c_uint32, f32p, C.POINTER(OrDiag)]
        L.or_sample_row.restype = OrResult
        L.or_sample_row.argtypes = [C.POINTER(OrParams), f32p, C.c_uint32, u32p, u32p, C.c_uint32,
                                    u32p, f32p, C.c_uint32, f32p, C.POINTER(OrDiag)]
        L.or_entropy_topk.argtypes = [f32p, C.c_uint32, C.c_uint32, C.POINTER(C.c_double), u32p,
                                      C.POINTER(C.c_double)]
        L.or_adaptive_init.argtypes = [C.POINTER(OrAdaptive), C.c_uint64]
        L.or_adaptive_record_margin.argtypes = [C.POINTER(OrAdaptive), C.c_float]
        L.or_adaptive_next.restype = C.c_uint64
        L.or_adaptive_next.argtypes = [C.POINTER(OrAdaptive)]
        L.or_adaptive_update.argtypes = [C.POINTER(OrAdaptive), C.c_uint64, C.c_uint64, C.c_int, C.c_float]
        L.or_splitmix64_next.restype = C.c_uint64
        L.or_splitmix64_next.argtypes = [C.POINTER(C.c_uint64)]
        L.or_xoshiro_seed.argtypes = [C.POINTER(C.c_uint64), C.c_uint64]
        L.or_xoshiro_next.restype = C.c_uint64
        L.or_xoshiro_next.argtypes = [C.POINTER(C.c_uint64)]
        L.or_rand_f32.restype = C.c_float
        L.or_rand_f32.argtypes = [C.POINTER(C.c_uint64)]
        L.or_bench_sample_rows.restype = C.c_double
        L.or_bench_sample_rows.argtypes = [C.POINTER(OrParams), f32p, C.c_uint32, C.c_uint32, C.c_uint64,
                                           u32p, C.POINTER(C.c_int32), C.c_uint32, u32p, C.c_uint32,
                                           f32p, C.c_uint32, u32p, f32p]
        jp = C.POINTER(OrJson)
        u8p = C.POINTER(C.c_uint8)
        L.or_json_init.argtypes = [jp, C.c_int]
        L.or_json_is_finished.argtypes = [jp]
        L.or_json_step_byte.argtypes = [jp, C.c_uint8]
        L.or_json_try_consume.argtypes = [jp, u8p, C.c_size_t, jp]
        L.or_json_consume.argtypes = [jp, u8p, C.c_size_t]
        L.or_json_mask.argtypes = [jp, u32p, u8p, C.c_uint32, u32p, C.c_uint32, C.c_int64, u32p]
        L.or_bench_json_mask.restype = C.c_double
        L.or_bench_json_mask.argtypes = [jp, C.c_uint32, u32p, u8p, C.c_uint32, u32p, C.c_uint32, C.c_int64,
                                         u32p, C.c_uint32]
        _lib = L
    return _lib


def _p(a, ct):
    return a.ctypes.data_as(C.POINTER(ct)) if a is not None else None


def params(**kw) -> OrParams:
    p = OrParams()
    lib().or_params_default(C.byref(p))
    for k, v in kw.items():
        if not hasattr(p, k):
            raise KeyError(k)
        setattr(p, k, v)
    return p


def softcap(x: float, cap: float) -> float:
    return lib().or_softcap(float(x), float(cap))


def softcap_tail(x: float, cap: float) -> float:
    return lib().or_softcap_tail(float(x), float(cap))


def tanh32(x: float) -> float:
    return lib().or_tanh32(float(x))


def exp32(x: float) -> float:
    """(float)exp((double)x): the correctly rounded stand-in kept for pow."""
    return lib().or_exp32(float(x))


def zexpf(x: float) -> float:
    """The reference's @exp(f32) (compiler-rt expf, oracle.c or_zexpf)."""
    return lib().or_zexpf(float(x))


def zexpf_array(x) -> np.ndarray:
    """or_zexpf over a float32 array."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().or_zexpf_array(x.ctypes.data, y.ctypes.data, x.size)
    return y


def pow_zig(x: float, y: float) -> float:
    return lib().or_pow_zig(float(x), float(y))


def apply_penalty(logits: np.ndarray, window, rp: float, freq: float = 0.0, pres: float = 0.0) -> np.ndarray:
    out = np.ascontiguousarray(logits, dtype=np.float32).copy()
    w = np.ascontiguousarray(window, dtype=np.uint32)
    lib().or_apply_penalty(_p(out, C.c_float), out.size, _p(w, C.c_uint32), w.size, rp, freq, pres)
    return out


def dry_edits(history, breakers, mult, base, allowed, rng):
    h = np.ascontiguousarray(history, dtype=np.uint32)
    b = np.ascontiguousarray(breakers, dtype=np.uint32)
    ids = np.zeros(128, np.uint32)
    deltas = np.zeros(128, np.float32)
    n = lib().or_dry_edits(_p(h, C.c_uint32), h.size, _p(b, C.c_uint32), b.size, mult, base,
                           allowed, rng, _p(ids, C.c_uint32), _p(deltas, C.c_float))
    return ids[:n].copy(), deltas[:n].copy()


def apply_mask(logits: np.ndarray, words) -> np.ndarray:
    out = np.ascontiguousarray(logits, dtype=np.float32).copy()
    w = np.ascontiguousarray(words, dtype=np.uint32)
    lib().or_apply_mask(_p(out, C.c_float), out.size, _p(w, C.c_uint32))
    return out


def argmax_with_margin(x) -> tuple[int, float]:
    a = np.ascontiguousarray(x, dtype=np.float32)
    r = lib().or_argmax_with_margin(_p(a, C.c_float), a.size)
    return int(r.tok), float(r.margin)


def argmax_true(x) -> tuple[int, float]:
    a = np.ascontiguousarray(x, dtype=np.float32)
    r = lib().or_argmax_true(_p(a, C.c_float), a.size)
    return int(r.tok), float(r.margin)


def sample_row(p: OrParams, logits, u, mask=None, window=None, edit_ids=None, edit_deltas=None,
               cap: int = 0):
    """Mask -> penalty -> edits -> sample, as gen.zig drives the Zig sampler.

    Returns (tok, margin, diag_dict); logits are copied, not modified."""
    row = np.ascontiguousarray(logits, dtype=np.float32).copy()
    uu = np.ascontiguousarray(np.asarray(u, dtype=np.float32).reshape(-1)[:2])
    if uu.size < 2:
        uu = np.concatenate([uu, np.zeros(2 - uu.size, np.float32)])
    mk = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint32)
    w = np.zeros(0, np.uint32) if window is None else np.ascontiguousarray(window, dtype=np.uint32)
    ei = None if edit_ids is None else np.ascontiguousarray(edit_ids, dtype=np.uint32)
    ed = None if edit_deltas is None else np.ascontiguousarray(edit_deltas, dtype=np.float32)
    d = OrDiag()
    ids = np.zeros(max(cap, 1), np.uint32)
    vals = np.zeros(max(cap, 1), np.float32)
    probs = np.zeros(max(cap, 1), np.float32)
    d.cap = cap
    d.ids, d.vals, d.probs = _p(ids, C.c_uint32), _p(vals, C.c_float), _p(probs, C.c_float)
    r = lib().or_sample_row(C.byref(p), _p(row, C.c_float), row.size, _p(mk, C.c_uint32),
                            _p(w, C.c_uint32), w.size, _p(ei, C.c_uint32), _p(ed, C.c_float),
                            0 if ei is None else ei.size, _p(uu, C.c_float), C.byref(d))
    n = min(cap, d.n)
    diag = dict(ndraws=d.ndraws, n=d.n, keep=d.keep, start=d.start, total=d.total,
                ids=ids[:n].copy(), vals=vals[:n].copy(), probs=probs[:n].copy(), row=row)
    return int(r.tok), float(r.margin), diag


def entropy_topk(x, k: int):
    a = np.ascontiguousarray(x, dtype=np.float32)
    H = C.c_double()
    ids = np.zeros(k, np.uint32)
    probs = np.zeros(k, np.float64)
    lib().or_entropy_topk(_p(a, C.c_float), a.size, k, C.byref(H), _p(ids, C.c_uint32),
                          _p(probs, C.c_double))
    return float(H.value), ids, probs


class Adaptive:
    def __init__(self, max_k: int):
        self.s = OrAdaptive()
        lib().or_adaptive_init(C.byref(self.s), max_k)

    def next_draft(self) -> int:
        return int(lib().or_adaptive_next(C.byref(self.s)))

    def record_margin(self, m: float) -> None:
        lib().or_adaptive_record_margin(C.byref(self.s), m)

    def update(self, accepted: int, drafted: int, margin=None) -> None:
        lib().or_adaptive_update(C.byref(self.s), accepted, drafted, 0 if margin is None else 1,
                                 0.0 if margin is None else float(margin))


def splitmix64_seq(seed: int, n: int):
    st = C.c_uint64(seed)
    return [int(lib().or_splitmix64_next(C.byref(st))) for _ in range(n)]


def rng_floats(seed: int, n: int):
    s = (C.c_uint64 * 4)()
    lib().or_xoshiro_seed(s, seed)
    return np.array([lib().or_rand_f32(s) for _ in range(n)], dtype=np.float32)


def xoshiro_step(state):
    """One or_xoshiro_next call on the 4-word state: (new state, output)."""
    s = (C.c_uint64 * 4)(*[int(x) & 0xFFFFFFFFFFFFFFFF for x in state])
    out = int(lib().or_xoshiro_next(s))
    return [int(x) for x in s], out


def rand_f32_from(state):
    """or_rand_f32 on the 4-word state: (value, state after the draws)."""
    s = (C.c_uint64 * 4)(*[int(x) & 0xFFFFFFFFFFFFFFFF for x in state])
    v = float(lib().or_rand_f32(s))
    return v, [int(x) for x in s]


def bench_sample_rows(p: OrParams, logits2d, hist, hist_len, mask, uniforms, reps: int):
    L = np.ascontiguousarray(logits2d, dtype=np.float32)
    rows, V = L.shape
    h = None if hist is None else np.ascontiguousarray(hist, dtype=np.uint32)
    hl = None if hist_len is None else np.ascontiguousarray(hist_len, dtype=np.int32)
    mk = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint32)
    u = np.ascontiguousarray(uniforms, dtype=np.float32)
    tok = np.zeros(rows, np.uint32)
    mar = np.zeros(rows, np.float32)
    t = lib().or_bench_sample_rows(C.byref(p), _p(L, C.c_float), rows, V, V,
                                   _p(h, C.c_uint32), _p(hl, C.c_int32), 0 if h is None else h.shape[1],
                                   _p(mk, C.c_uint32), 0 if mk is None else mk.shape[1],
                                   _p(u, C.c_float), reps, _p(tok, C.c_uint32), _p(mar, C.c_float))
    return t, tok, mar


# ---------------------------------------------------------------- grammar


def json_init(object_only: bool = True) -> OrJson:
    """JsonValidator.initObjectOnly / initAny (src/grammar.zig:70-76)."""
    j = OrJson()
    lib().or_json_init(C.byref(j), int(bool(object_only)))
    return j


def json_copy(j: OrJson) -> OrJson:
    c = OrJson()
    C.memmove(C.byref(c), C.byref(j), C.sizeof(OrJson))
    return c


def json_is_finished(j: OrJson) -> bool:
    return bool(lib().or_json_is_finished(C.byref(j)))


def _bytes(piece) -> tuple:
    b = piece.encode() if isinstance(piece, str) else bytes(piece)
    buf = (C.c_uint8 * max(len(b), 1)).from_buffer_copy(b or b"\0")
    return buf, len(b)


def json_consume(j: OrJson, piece) -> bool:
    """consume (src/grammar.zig:437-443): in place."""
    buf, n = _bytes(piece)
    return bool(lib().or_json_consume(C.byref(j), buf, n))


def json_try_consume(j: OrJson, piece):
    """tryConsume (src/grammar.zig:428-434): the new state, or None."""
    buf, n = _bytes(piece)
    out = OrJson()
    ok = lib().or_json_try_consume(C.byref(j), buf, n, C.byref(out))
    return out if ok else None


def json_mask(j: OrJson, piece_off, piece_buf, eog=(), eos=None) -> np.ndarray:
    """applyMask (src/grammar.zig:446-479) as the packed allowed-token mask."""
    off = np.ascontiguousarray(piece_off, dtype=np.uint32)
    buf = np.ascontiguousarray(piece_buf, dtype=np.uint8)
    if buf.size == 0:
        buf = np.zeros(1, np.uint8)
    V = off.size - 1
    e = np.ascontiguousarray(np.asarray(eog, dtype=np.uint32).reshape(-1))
    if e.size == 0:
        e = np.zeros(1, np.uint32)
        ne = 0
    else:
        ne = e.size
    out = np.zeros((V + 31) // 32, np.uint32)
    lib().or_json_mask(C.byref(j), _p(off, C.c_uint32), _p(buf, C.c_uint8), V, _p(e, C.c_uint32), ne,
                       -1 if eos is None else int(eos), _p(out, C.c_uint32))
    return out


def bench_json_mask(states, piece_off, piece_buf, eog, eos, reps: int):
    """Seconds for `reps` passes of json_mask over every state."""
    arr = (OrJson * len(states))(*states)
    off = np.ascontiguousarray(piece_off, dtype=np.uint32)
    buf = np.ascontiguousarray(piece_buf, dtype=np.uint8)
    e = np.ascontiguousarray(np.asarray(eog, dtype=np.uint32).reshape(-1))
    V = off.size - 1
    out = np.zeros((len(states), (V + 31) // 32), np.uint32)
    t = lib().or_bench_json_mask(arr, len(states), _p(off, C.c_uint32), _p(buf, C.c_uint8), V,
                                 _p(e, C.c_uint32), e.size, -1 if eos is None else int(eos),
                                 _p(out, C.c_uint32), reps)
    return t, out


def pruned_row(logits, groups, V: int) -> np.ndarray:
    """The row the reference's pruned lm_head leaves: the whole row is set to
    -inf (src/model.zig:2127-2128), then prunedFineWorker (:1144-1160) writes
    logits[8g .. 8g + 8) for each candidate group g.  Groups past the
    vocabulary are skipped; a repeated group writes the same values again."""
    row = np.full(V, -np.inf, np.float32)
    g = np.asarray(groups, np.int64)
    g = g[(g >= 0) & (g < (V + 7) // 8)]
    if g.size:
        ids = (g[:, None] * 8 + np.arange(8)[None, :]).reshape(-1)
        ids = ids[ids < V]
        row[ids] = np.asarray(logits, np.float32)[ids]
    return row
