"""Torch-facing wrappers over the C ABI (device memory and streams only).

Tensors are passed to libzinfer_hip as raw device pointers; every call is
enqueued on torch's current stream so it orders with the surrounding torch
work.  Nothing here computes a result on the host.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from ._lib import ZiBatch, ZiParams, ZiSampleOut, check, lib

__all__ = ["Context", "Sampler", "params", "SampleResult", "JsonValidator", "Vocab"]

params = _lib.params


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else C.c_void_p(t.data_ptr())


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return _lib.ZI_F32
    if t.dtype == torch.bfloat16:
        return _lib.ZI_BF16
    raise TypeError(f"logits dtype {t.dtype} (need float32 or bfloat16)")


@dataclass
class SampleResult:
    tok: torch.Tensor
    margin: torch.Tensor
    ndraws: torch.Tensor
    keep: Optional[torch.Tensor] = None
    cand_ids: Optional[torch.Tensor] = None
    cand_vals: Optional[torch.Tensor] = None
    probs: Optional[torch.Tensor] = None


class Context:
    """zi_ctx: device scratch + stream for batches of <= max_rows x max_vocab."""

    def __init__(self, device: int = 0, max_rows: int = 512, max_vocab: int = 262144):
        self.device = device
        h = C.c_void_p()
        check(lib().zi_create(C.byref(h), device, max_rows, max_vocab))
        self.h = h

    def close(self):
        if self.h:
            lib().zi_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reserve(self, what: int):
        """zi_reserve: allocate the lazily allocated scratch now (ZI_RESERVE_* bits)."""
        check(lib().zi_reserve(self.h, what))

    def _bind_stream(self):
        s = torch.cuda.current_stream(self.device)
        check(lib().zi_set_stream(self.h, C.c_void_p(s.cuda_stream)))

    @staticmethod
    def batch(logits: torch.Tensor, vocab: Optional[int] = None, hist=None, hist_len=None, mask=None,
              edit_ids=None, edit_delta=None, edit_count=None) -> ZiBatch:
        assert logits.dim() == 2 and logits.stride(1) == 1
        b = ZiBatch()
        b.logits = logits.data_ptr()
        b.dtype = _dtype_code(logits)
        b.rows = logits.shape[0]
        b.vocab = logits.shape[1] if vocab is None else vocab
        b.ld = logits.stride(0)
        if hist is not None:
            b.hist, b.hist_len, b.hist_ld = hist.data_ptr(), hist_len.data_ptr(), hist.stride(0)
        if mask is not None:
            b.mask, b.mask_ld = mask.data_ptr(), mask.stride(0)
        if edit_ids is not None:
            b.edit_ids, b.edit_delta, b.edit_count = edit_ids.data_ptr(), edit_delta.data_ptr(), edit_count.data_ptr()
            b.edit_ld = edit_ids.stride(0)
        return b

    def sample_rows(self, p: ZiParams, logits: torch.Tensor, uniforms: torch.Tensor, *, vocab=None, hist=None,
                    hist_len=None, mask=None, edit_ids=None, edit_delta=None, edit_count=None,
                    cands: bool = False, out: Optional[SampleResult] = None, groups=None,
                    group_count=None) -> SampleResult:
        """zi_sample_rows; with `groups` ([rows, ld] int32/uint32 group ids) and
        `group_count` ([rows] int32), zi_sample_rows_pruned."""
        rows = logits.shape[0]
        dev = logits.device
        if out is None:
            out = SampleResult(tok=torch.empty(rows, dtype=torch.int32, device=dev),
                               margin=torch.empty(rows, dtype=torch.float32, device=dev),
                               ndraws=torch.empty(rows, dtype=torch.int32, device=dev))
            if cands:
                V = logits.shape[1] if vocab is None else vocab
                k = V if (p.top_k == 0 or p.top_k > V) else p.top_k
                out.keep = torch.empty(rows, dtype=torch.int32, device=dev)
                out.cand_ids = torch.full((rows, k), -1, dtype=torch.int32, device=dev)
                out.cand_vals = torch.zeros((rows, k), dtype=torch.float32, device=dev)
                out.probs = torch.zeros((rows, k), dtype=torch.float32, device=dev)
        o = ZiSampleOut()
        o.tok, o.margin, o.ndraws = out.tok.data_ptr(), out.margin.data_ptr(), out.ndraws.data_ptr()
        if out.keep is not None:
            o.keep = out.keep.data_ptr()
        if out.cand_ids is not None:
            o.cand_ids, o.cand_vals, o.probs = out.cand_ids.data_ptr(), out.cand_vals.data_ptr(), out.probs.data_ptr()
            o.cand_ld = out.cand_ids.stride(0)
        b = self.batch(logits, vocab, hist, hist_len, mask, edit_ids, edit_delta, edit_count)
        self._bind_stream()
        if groups is not None:
            check(lib().zi_sample_rows_pruned(self.h, C.byref(p), C.byref(b), _ptr(groups), _ptr(group_count),
                                              groups.stride(0), _ptr(uniforms), C.byref(o)))
        else:
            check(lib().zi_sample_rows(self.h, C.byref(p), C.byref(b), _ptr(uniforms), C.byref(o)))
        return out

    def dry_edits_rows(self, p: ZiParams, hist: torch.Tensor, hist_len: torch.Tensor,
                       breakers: Optional[torch.Tensor] = None, edit_ld: int = 128):
        """zi_dry_edits_rows: per-row DRY edits (ids [rows, edit_ld] int32,
        deltas [rows, edit_ld] f32, counts [rows] int32) on the device."""
        rows, dev = hist.shape[0], hist.device
        ids = torch.zeros((rows, edit_ld), dtype=torch.int32, device=dev)
        delta = torch.zeros((rows, edit_ld), dtype=torch.float32, device=dev)
        cnt = torch.empty(rows, dtype=torch.int32, device=dev)
        nb = 0 if breakers is None else int(breakers.numel())
        self._bind_stream()
        check(lib().zi_dry_edits_rows(self.h, C.byref(p), _ptr(hist), _ptr(hist_len), hist.stride(0), rows,
                                      _ptr(breakers), nb, _ptr(ids), _ptr(delta), _ptr(cnt), edit_ld))
        return ids, delta, cnt

    def argmax_rows(self, logits: torch.Tensor, vocab=None):
        rows, dev = logits.shape[0], logits.device
        tok = torch.empty(rows, dtype=torch.int32, device=dev)
        margin = torch.empty(rows, dtype=torch.float32, device=dev)
        tok_low = torch.empty(rows, dtype=torch.int32, device=dev)
        margin_true = torch.empty(rows, dtype=torch.float32, device=dev)
        b = self.batch(logits, vocab)
        self._bind_stream()
        check(lib().zi_argmax_rows(self.h, C.byref(b), _ptr(tok), _ptr(margin), _ptr(tok_low), _ptr(margin_true)))
        return tok, margin, tok_low, margin_true

    def entropy_topk_rows(self, logits: torch.Tensor, k: int, draft: Optional[torch.Tensor] = None, vocab=None):
        rows, dev = logits.shape[0], logits.device
        ent = torch.empty(rows, dtype=torch.float32, device=dev)
        ids = torch.empty((rows, k), dtype=torch.int32, device=dev)
        probs = torch.empty((rows, k), dtype=torch.float32, device=dev)
        am = torch.empty(rows, dtype=torch.int32, device=dev)
        acc = torch.empty(rows, dtype=torch.uint8, device=dev) if draft is not None else None
        b = self.batch(logits, vocab)
        self._bind_stream()
        check(lib().zi_entropy_topk_rows(self.h, C.byref(b), k, _ptr(draft), _ptr(ent), _ptr(ids), _ptr(probs), k,
                                         _ptr(am), _ptr(acc)))
        return ent, ids, probs, am, acc

    def apply_mask_rows(self, logits: torch.Tensor, mask: torch.Tensor, vocab=None):
        b = self.batch(logits, vocab, mask=mask)
        self._bind_stream()
        check(lib().zi_apply_mask_rows(self.h, C.byref(b)))
        return logits


class Sampler:
    """The host mirror of the Zig Sampler (zi_sampler_*), one host row per call."""

    def __init__(self, ctx: Context, vocab: int, p: ZiParams):
        self.ctx = ctx
        self.vocab = vocab
        h = C.c_void_p()
        check(lib().zi_sampler_init(C.byref(h), ctx.h, vocab, C.byref(p)))
        self.h = h

    def __del__(self):
        try:
            if self.h:
                lib().zi_sampler_deinit(self.h)
                self.h = None
        except Exception:
            pass

    def reset(self):
        lib().zi_sampler_reset(self.h)

    def add_breaker(self, tok: int):
        lib().zi_sampler_add_breaker(self.h, tok)

    def is_breaker(self, tok: int) -> bool:
        return bool(lib().zi_sampler_is_breaker(self.h, tok))

    def accept(self, tok: int):
        lib().zi_sampler_accept(self.h, tok)

    def seed(self, s: int):
        lib().zi_sampler_seed(self.h, s)

    def rand_f32(self) -> float:
        return float(lib().zi_sampler_rand_f32(self.h))

    def apply_dry(self, logits):
        import numpy as np
        a = np.ascontiguousarray(logits, dtype=np.float32)
        lib().zi_sampler_apply_dry(self.h, a.ctypes.data_as(_lib.f32p), a.size)
        return a

    def sample_with_margin(self, logits):
        """logits: a float32 numpy array; modified in place like the reference."""
        import numpy as np
        assert isinstance(logits, np.ndarray) and logits.dtype == np.float32 and logits.flags.c_contiguous
        tok = C.c_uint32()
        m = C.c_float()
        check(lib().zi_sampler_sample_with_margin(self.h, logits.ctypes.data_as(_lib.f32p), logits.size,
                                                  C.byref(tok), C.byref(m)))
        return int(tok.value), float(m.value)

    def sample(self, logits) -> int:
        return self.sample_with_margin(logits)[0]

    def verify(self, logits: torch.Tensor, draft, *, max_accept: int = 2**32 - 1, eog=(), vocab=None,
               json: Optional["JsonValidator"] = None):
        """Draft verification in one batched launch (zi_sampler_verify, src/gen.zig:544-587).
        logits: device [>= len(draft) + 1][V].  Returns (accepted, next_tok, margin)."""
        import numpy as np
        d = np.ascontiguousarray(np.asarray(draft, dtype=np.uint32).reshape(-1))
        e = np.ascontiguousarray(np.asarray(eog, dtype=np.uint32).reshape(-1))
        b = Context.batch(logits, self.vocab)
        a, nt, m = C.c_uint32(), C.c_uint32(), C.c_float()
        self.ctx._bind_stream()
        check(lib().zi_sampler_verify(self.h, C.byref(b), d.ctypes.data_as(_lib.u32p) if d.size else None, d.size,
                                      max_accept, e.ctypes.data_as(_lib.u32p) if e.size else None, e.size,
                                      vocab.h if vocab is not None else None,
                                      C.byref(json.st) if json is not None else None,
                                      C.byref(a), C.byref(nt), C.byref(m)))
        return int(a.value), int(nt.value), float(m.value)

    def verify_tree(self, logits: torch.Tensor, drafts, *, max_accept: int = 2**32 - 1, eog=(), vocab=None,
                    json: Optional["JsonValidator"] = None, commit: bool = True):
        """Tree verification (zi_sampler_verify_tree): `drafts` is a list of
        branches; logits holds each branch's len + 1 rows back to back.
        Returns (accepted[], next[], margin[], best)."""
        import numpy as np
        nb = len(drafts)
        ld = max(1, max(len(d) for d in drafts))
        D = np.zeros((nb, ld), np.uint32)
        ks = np.zeros(nb, np.uint32)
        for j, d in enumerate(drafts):
            D[j, :len(d)] = np.asarray(d, dtype=np.uint32)
            ks[j] = len(d)
        e = np.ascontiguousarray(np.asarray(eog, dtype=np.uint32).reshape(-1))
        b = Context.batch(logits, self.vocab)
        acc = np.zeros(nb, np.uint32)
        nxt = np.zeros(nb, np.uint32)
        mg = np.zeros(nb, np.float32)
        best = C.c_uint32()
        self.ctx._bind_stream()
        check(lib().zi_sampler_verify_tree(self.h, C.byref(b), D.ctypes.data_as(_lib.u32p), ld,
                                           ks.ctypes.data_as(_lib.u32p), nb, max_accept,
                                           e.ctypes.data_as(_lib.u32p) if e.size else None, e.size,
                                           vocab.h if vocab is not None else None,
                                           C.byref(json.st) if json is not None else None, 1 if commit else 0,
                                           acc.ctypes.data_as(_lib.u32p), nxt.ctypes.data_as(_lib.u32p),
                                           mg.ctypes.data_as(_lib.f32p), C.byref(best)))
        return [int(a) for a in acc], [int(t) for t in nxt], [float(m) for m in mg], int(best.value)

    def get_params(self) -> ZiParams:
        p = ZiParams()
        lib().zi_sampler_get_params(self.h, C.byref(p))
        return p

    def set_params(self, p: ZiParams):
        lib().zi_sampler_set_params(self.h, C.byref(p))


def _piece(piece):
    b = piece.encode() if isinstance(piece, str) else bytes(piece)
    return (C.c_uint8 * max(len(b), 1)).from_buffer_copy(b or b"\0"), len(b)


class JsonValidator:
    """The reference's JsonValidator (src/grammar.zig:59-480) over the C ABI:
    the host state machine (zi_json_*) and the GPU mask (Vocab.json_mask_rows)."""

    def __init__(self, object_only: bool = True):
        self.st = _lib.ZiJsonState()
        lib().zi_json_init(C.byref(self.st), int(bool(object_only)))

    @classmethod
    def init_object_only(cls) -> "JsonValidator":  # :70-72
        return cls(True)

    @classmethod
    def init_any(cls) -> "JsonValidator":  # :74-76
        return cls(False)

    def copy(self) -> "JsonValidator":
        c = JsonValidator.__new__(JsonValidator)
        c.st = _lib.ZiJsonState()
        C.memmove(C.byref(c.st), C.byref(self.st), C.sizeof(_lib.ZiJsonState))
        return c

    def is_finished(self) -> bool:  # :78-80
        return bool(lib().zi_json_is_finished(C.byref(self.st)))

    def step_byte(self, b: int) -> bool:  # :195-381
        return bool(lib().zi_json_step_byte(C.byref(self.st), int(b)))

    def consume(self, piece) -> bool:  # :437-443
        buf, n = _piece(piece)
        return bool(lib().zi_json_consume(C.byref(self.st), buf, n))

    def try_consume(self, piece) -> Optional["JsonValidator"]:  # :428-434
        buf, n = _piece(piece)
        out = JsonValidator.__new__(JsonValidator)
        out.st = _lib.ZiJsonState()
        return out if lib().zi_json_try_consume(C.byref(self.st), buf, n, C.byref(out.st)) else None

    def apply_mask(self, logits, vocab: "Vocab"):  # :446-479, host logits in place
        import numpy as np
        assert isinstance(logits, np.ndarray) and logits.dtype == np.float32 and logits.flags.c_contiguous
        check(lib().zi_json_apply_mask(vocab.ctx.h, vocab.h, C.byref(self.st), logits.ctypes.data_as(_lib.f32p),
                                       logits.size))
        return logits


class Vocab:
    """Token pieces on the device (zi_vocab): Tokenizer.piece_off / piece_buf,
    the end-of-generation ids and the eos id (src/tokenizer.zig:35-47)."""

    def __init__(self, ctx: Context, piece_off, piece_buf, eog=(), eos=None, cache_states: int = 64):
        import numpy as np
        self.ctx = ctx
        self.h = None
        off = np.ascontiguousarray(piece_off, dtype=np.uint32)
        buf = np.ascontiguousarray(piece_buf, dtype=np.uint8)
        if buf.size == 0:
            buf = np.zeros(1, np.uint8)
        e = np.ascontiguousarray(np.asarray(eog, dtype=np.uint32).reshape(-1))
        self.V = off.size - 1
        self.words = (self.V + 31) // 32
        h = C.c_void_p()
        check(lib().zi_vocab_create(C.byref(h), ctx.h, off.ctypes.data_as(_lib.u32p), buf.ctypes.data_as(_lib.u8p),
                                    self.V, e.ctypes.data_as(_lib.u32p) if e.size else None, e.size,
                                    -1 if eos is None else int(eos), cache_states))
        self.h = h

    def close(self):
        if self.h:
            lib().zi_vocab_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def json_mask_rows(self, validators, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Packed allowed-token masks [rows][ceil(V/32)] (int32 view of u32), one row per validator."""
        rows = len(validators)
        arr = (_lib.ZiJsonState * rows)(*[v.st for v in validators])
        if out is None:
            out = torch.empty((rows, self.words), dtype=torch.int32, device=f"cuda:{self.ctx.device}")
        assert out.dtype == torch.int32 and out.is_cuda and out.shape[0] >= rows and out.stride(1) == 1
        self.ctx._bind_stream()
        check(lib().zi_json_mask_rows(self.ctx.h, self.h, arr, rows, _ptr(out), out.stride(0)))
        return out
