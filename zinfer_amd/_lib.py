"""ctypes binding of libzinfer_hip (include/zinfer_hip.h).

This is the same binding a maintainer would write for any FFI host: plain C
structs and pointers.  Loading fails loudly when the library has not been
built; there is no fallback implementation.
"""
from __future__ import annotations

import ctypes as C
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libzinfer_hip.so")

ZI_OK = 0
ZI_ERR_INVALID = -1
ZI_ERR_HIP = -2
ZI_ERR_OOM = -3
ZI_ERR_UNSUPPORTED = -4
ZI_ERR_CAPACITY = -5
ZI_F32 = 0
ZI_BF16 = 1
ZI_RESERVE_WHOLE_ORDER = 1
ZI_RESERVE_PRUNED_DENSE = 2

u32p = C.POINTER(C.c_uint32)
f32p = C.POINTER(C.c_float)
i32p = C.POINTER(C.c_int32)


class ZiParams(C.Structure):
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
        ("seed", C.c_uint64),
        ("final_logit_softcap", C.c_float),
    ]


class ZiBatch(C.Structure):
    _fields_ = [
        ("logits", C.c_void_p),
        ("dtype", C.c_int32),
        ("rows", C.c_int32),
        ("vocab", C.c_int32),
        ("ld", C.c_int32),
        ("hist", C.c_void_p),
        ("hist_len", C.c_void_p),
        ("hist_ld", C.c_int32),
        ("mask", C.c_void_p),
        ("mask_ld", C.c_int32),
        ("edit_ids", C.c_void_p),
        ("edit_delta", C.c_void_p),
        ("edit_count", C.c_void_p),
        ("edit_ld", C.c_int32),
    ]


class ZiSampleOut(C.Structure):
    _fields_ = [
        ("tok", C.c_void_p),
        ("margin", C.c_void_p),
        ("ndraws", C.c_void_p),
        ("keep", C.c_void_p),
        ("cand_ids", C.c_void_p),
        ("cand_vals", C.c_void_p),
        ("probs", C.c_void_p),
        ("cand_ld", C.c_int32),
    ]


class ZiAdaptiveDraft(C.Structure):
    _fields_ = [
        ("cur_k", C.c_uint64),
        ("max_k", C.c_uint64),
        ("min_k", C.c_uint64),
        ("consecutive_rejections", C.c_uint64),
        ("cooldown_steps", C.c_uint64),
        ("last_margin", C.c_float),
    ]


class ZiJsonState(C.Structure):
    """JsonValidator state (src/grammar.zig:59-68); see zi_json_state."""
    _fields_ = [
        ("stack", C.c_uint64),
        ("state", C.c_uint8),
        ("escape", C.c_uint8),
        ("num", C.c_uint8),
        ("depth", C.c_uint8),
        ("lit_len", C.c_uint8),
        ("lit_idx", C.c_uint8),
        ("object_only", C.c_uint8),
        ("reserved", C.c_uint8),
        ("lit_expected", C.c_uint8 * 8),
    ]


u8p = C.POINTER(C.c_uint8)
jsp = C.POINTER(ZiJsonState)

# name -> (restype, argtypes); mirrors include/zinfer_hip.h one to one
SIGNATURES = {
    "zi_params_default": (None, [C.POINTER(ZiParams)]),
    "zi_create": (C.c_int32, [C.POINTER(C.c_void_p), C.c_int32, C.c_int32, C.c_int32]),
    "zi_destroy": (None, [C.c_void_p]),
    "zi_set_stream": (C.c_int32, [C.c_void_p, C.c_void_p]),
    "zi_sync": (C.c_int32, [C.c_void_p]),
    "zi_reserve": (C.c_int32, [C.c_void_p, C.c_uint32]),
    "zi_last_error": (C.c_char_p, []),
    "zi_sample_rows_noalloc": (C.c_int32, [C.POINTER(ZiParams), C.POINTER(ZiBatch), C.c_void_p,
                                           C.POINTER(ZiSampleOut), C.c_void_p]),
    "zi_abi_version": (C.c_int32, []),
    "zi_sample_rows": (C.c_int32, [C.c_void_p, C.POINTER(ZiParams), C.POINTER(ZiBatch), C.c_void_p,
                                    C.POINTER(ZiSampleOut)]),
    "zi_sample_rows_pruned": (C.c_int32, [C.c_void_p, C.POINTER(ZiParams), C.POINTER(ZiBatch), C.c_void_p,
                                           C.c_void_p, C.c_int32, C.c_void_p, C.POINTER(ZiSampleOut)]),
    "zi_dry_edits_rows": (C.c_int32, [C.c_void_p, C.POINTER(ZiParams), C.c_void_p, C.c_void_p, C.c_int32,
                                       C.c_int32, C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p,
                                       C.c_int32]),
    "zi_argmax_rows": (C.c_int32, [C.c_void_p, C.POINTER(ZiBatch), C.c_void_p, C.c_void_p, C.c_void_p,
                                    C.c_void_p]),
    "zi_entropy_topk_rows": (C.c_int32, [C.c_void_p, C.POINTER(ZiBatch), C.c_int32, C.c_void_p, C.c_void_p,
                                          C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p]),
    "zi_apply_mask_rows": (C.c_int32, [C.c_void_p, C.POINTER(ZiBatch)]),
    "zi_json_init": (None, [jsp, C.c_int32]),
    "zi_json_is_finished": (C.c_int32, [jsp]),
    "zi_json_step_byte": (C.c_int32, [jsp, C.c_uint8]),
    "zi_json_consume": (C.c_int32, [jsp, u8p, C.c_size_t]),
    "zi_json_try_consume": (C.c_int32, [jsp, u8p, C.c_size_t, jsp]),
    "zi_vocab_create": (C.c_int32, [C.POINTER(C.c_void_p), C.c_void_p, u32p, u8p, C.c_uint32, u32p, C.c_uint32,
                                     C.c_int64, C.c_int32]),
    "zi_vocab_destroy": (None, [C.c_void_p]),
    "zi_json_mask_rows": (C.c_int32, [C.c_void_p, C.c_void_p, jsp, C.c_int32, C.c_void_p, C.c_int32]),
    "zi_json_apply_mask": (C.c_int32, [C.c_void_p, C.c_void_p, jsp, f32p, C.c_uint32]),
    "zi_sampler_init": (C.c_int32, [C.POINTER(C.c_void_p), C.c_void_p, C.c_uint32, C.POINTER(ZiParams)]),
    "zi_sampler_deinit": (None, [C.c_void_p]),
    "zi_sampler_reset": (None, [C.c_void_p]),
    "zi_sampler_add_breaker": (None, [C.c_void_p, C.c_uint32]),
    "zi_sampler_is_breaker": (C.c_int32, [C.c_void_p, C.c_uint32]),
    "zi_sampler_accept": (None, [C.c_void_p, C.c_uint32]),
    "zi_sampler_apply_dry": (None, [C.c_void_p, f32p, C.c_uint32]),
    "zi_sampler_sample_with_margin": (C.c_int32, [C.c_void_p, f32p, C.c_uint32, u32p, f32p]),
    "zi_sampler_sample": (C.c_int32, [C.c_void_p, f32p, C.c_uint32, u32p]),
    "zi_sampler_verify": (C.c_int32, [C.c_void_p, C.POINTER(ZiBatch), u32p, C.c_uint32, C.c_uint32, u32p, C.c_uint32,
                                       C.c_void_p, jsp, u32p, u32p, f32p]),
    "zi_sampler_verify_tree": (C.c_int32, [C.c_void_p, C.POINTER(ZiBatch), u32p, C.c_uint32, u32p, C.c_uint32,
                                            C.c_uint32, u32p, C.c_uint32, C.c_void_p, C.c_void_p, C.c_int32, u32p,
                                            u32p, f32p, u32p]),
    "zi_sampler_get_params": (None, [C.c_void_p, C.POINTER(ZiParams)]),
    "zi_sampler_set_params": (None, [C.c_void_p, C.POINTER(ZiParams)]),
    "zi_sampler_seed": (None, [C.c_void_p, C.c_uint64]),
    "zi_sampler_rand_f32": (C.c_float, [C.c_void_p]),
    "zi_argmax_with_margin": (C.c_int32, [C.c_void_p, f32p, C.c_uint32, u32p, f32p]),
    "zi_dry_edits": (C.c_uint32, [u32p, C.c_uint32, u32p, C.c_uint32, C.POINTER(ZiParams), u32p, f32p]),
    "zi_adaptive_draft_init": (None, [C.POINTER(ZiAdaptiveDraft), C.c_uint64]),
    "zi_adaptive_draft_record_margin": (None, [C.POINTER(ZiAdaptiveDraft), C.c_float]),
    "zi_adaptive_draft_next": (C.c_uint64, [C.POINTER(ZiAdaptiveDraft)]),
    "zi_entropy_margin": (C.c_float, [C.c_float]),
    "zi_adaptive_draft_record_entropy": (None, [C.POINTER(ZiAdaptiveDraft), C.c_float]),
    "zi_adaptive_draft_update": (None, [C.POINTER(ZiAdaptiveDraft), C.c_uint64, C.c_uint64, C.c_int32,
                                        C.c_float]),
}

_lib = None


class ZiError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"zinfer_hip error {code}: {msg}")
        self.code = code


def lib():
    """Loads libzinfer_hip.so (built by zinfer_amd/build.py).  Raises if absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run `python -m zinfer_amd.build` (or __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != ZI_OK:
        raise ZiError(rc, lib().zi_last_error().decode())


def params(**kw) -> ZiParams:
    p = ZiParams()
    lib().zi_params_default(C.byref(p))
    for k, v in kw.items():
        if not hasattr(p, k):
            raise KeyError(k)
        setattr(p, k, v)
    return p
