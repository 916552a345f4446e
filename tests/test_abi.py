"""The C ABI without a GPU: the library loads, exports every symbol the header
declares, the ctypes structs match the C layout, and the host-only entry
points (defaults, DRY edits, AdaptiveDraft, error paths) behave."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "zinfer_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(zi_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from zinfer_amd._lib import SIGNATURES, lib

    L = lib()
    syms = declared_symbols()
    assert len(syms) >= 25
    for s in syms:
        assert hasattr(L, s), s
    assert set(syms) == set(SIGNATURES), set(syms) ^ set(SIGNATURES)


def test_struct_layout_matches_header(tmp_path):
    """Compile a probe against the header with the host C compiler and compare
    sizes and offsets with the ctypes mirrors."""
    from zinfer_amd import _lib

    structs = {"zi_params": _lib.ZiParams, "zi_batch": _lib.ZiBatch, "zi_sample_out": _lib.ZiSampleOut,
               "zi_adaptive_draft": _lib.ZiAdaptiveDraft, "zi_json_state": _lib.ZiJsonState}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "zinfer_hip.h"', "int main(void) {"]
    for name, cls in structs.items():
        lines.append(f'printf("{name} size %zu\\n", sizeof({name}));')
        for f, _ in cls._fields_:
            lines.append(f'printf("{name}.{f} %zu\\n", offsetof({name}, {f}));')
    lines.append("return 0; }")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    got = dict(l.rsplit(" ", 1) for l in out if l)
    for name, cls in structs.items():
        assert int(got[f"{name} size"]) == C.sizeof(cls), name
        for f, _ in cls._fields_:
            assert int(got[f"{name}.{f}"]) == getattr(cls, f).offset, (name, f)


def test_params_default_are_reference_defaults():
    """src/sampler.zig:4-26 (plus neutral extensions, window 64 = :30)."""
    from zinfer_amd._lib import params

    p = params()
    assert (p.temp, p.top_k, p.top_p, p.min_p, p.repeat_penalty) == (np.float32(0.8), 40, np.float32(0.95),
                                                                        np.float32(0.05), 1.0)
    assert (p.freq_penalty, p.presence_penalty, p.penalty_last_n) == (0.0, 0.0, 64)
    assert (p.dry_multiplier, p.dry_base, p.dry_allowed_length, p.dry_range) == (0.0, 1.75, 2, 1024)
    assert (p.xtc_probability, p.xtc_threshold, p.xtc_min_keep, p.seed) == (0.0, np.float32(0.1), 1, 0)


def test_abi_version():
    from zinfer_amd._lib import lib

    assert lib().zi_abi_version() == 1


def test_dry_edits_match_oracle(oracle):
    """The library's host DRY step (sampler.zig:104-187) equals the oracle's on
    random histories with breakers."""
    from zinfer_amd._lib import f32p, lib, params, u32p

    rng = np.random.default_rng(4)
    for trial in range(100):
        L = int(rng.integers(0, 200))
        hist = rng.integers(0, 6, L).astype(np.uint32)
        brk = np.array([5] if trial % 2 else [], np.uint32)
        mult, base, allowed, rnge = 0.8, float(rng.choice([1.75, 2.0, 1.0])), int(rng.integers(1, 4)), 1024
        p = params(dry_multiplier=mult, dry_base=base, dry_allowed_length=allowed, dry_range=rnge)
        ids = np.zeros(128, np.uint32)
        d = np.zeros(128, np.float32)
        n = lib().zi_dry_edits(hist.ctypes.data_as(u32p), L, brk.ctypes.data_as(u32p), brk.size, C.byref(p),
                               ids.ctypes.data_as(u32p), d.ctypes.data_as(f32p))
        eids, ed = oracle.dry_edits(hist, brk, mult, base, allowed, rnge)
        assert np.array_equal(ids[:n], eids) and np.array_equal(d[:n].view(np.uint32), ed.view(np.uint32))


def test_adaptive_draft_kat():
    """gen.zig:845-874 through zi_adaptive_draft_*."""
    from zinfer_amd._lib import ZiAdaptiveDraft, lib

    a = ZiAdaptiveDraft()
    L = lib()
    L.zi_adaptive_draft_init(C.byref(a), 5)
    seq = [L.zi_adaptive_draft_next(C.byref(a))]
    for acc, dr in [(3, 3), (4, 4), (3, 5), (1, 5), (0, 4)]:
        L.zi_adaptive_draft_update(C.byref(a), acc, dr, 1, 2.5)
        seq.append(L.zi_adaptive_draft_next(C.byref(a)))
    L.zi_adaptive_draft_update(C.byref(a), 0, 3, 1, 2.5)
    seq += [L.zi_adaptive_draft_next(C.byref(a)) for _ in range(3)]
    assert seq == [3, 4, 5, 5, 4, 3, 0, 0, 2]
    # the margin thresholds of nextDraft (gen.zig:396-403)
    L.zi_adaptive_draft_init(C.byref(a), 8)
    L.zi_adaptive_draft_record_margin(C.byref(a), 3.5)
    assert L.zi_adaptive_draft_next(C.byref(a)) == 4
    L.zi_adaptive_draft_record_margin(C.byref(a), 0.5)
    assert L.zi_adaptive_draft_next(C.byref(a)) == 1


def test_entropy_margin_inverts_two_token_entropy():
    """zi_entropy_margin(H) is the m at which softmax([m, 0]) has entropy H:
    checked against scipy's entropy of that distribution (a round trip), its
    boundaries and its monotonicity."""
    from scipy.stats import entropy

    from zinfer_amd._lib import lib

    L = lib()
    for m in [0.0, 0.05, 0.5, 0.9, 1.8, 3.0, 7.5, 20.0, 30.0]:  # in f64, p[0] rounds to 1 beyond ~35
        p = np.exp(np.array([m, 0.0]) - m)
        H = float(entropy(p / p.sum()))
        got = L.zi_entropy_margin(H)
        assert abs(got - m) <= 1e-4 * max(1.0, m), (m, H, got)
    assert L.zi_entropy_margin(float(np.log(2.0))) == 0.0
    assert L.zi_entropy_margin(5.0) == 0.0  # a flatter row than any two-token one
    assert L.zi_entropy_margin(float("nan")) == 0.0
    assert L.zi_entropy_margin(0.0) == 100.0
    hs = np.linspace(1e-6, 0.69, 200).astype(np.float32)
    ms = np.array([L.zi_entropy_margin(float(h)) for h in hs])
    assert np.all(np.diff(ms) < 0)


def test_adaptive_draft_entropy_input():
    """record_entropy drives nextDraft exactly as the equivalent margin does."""
    from zinfer_amd._lib import ZiAdaptiveDraft, lib

    L = lib()
    for H, want in [(0.05, 4), (0.3, 3), (0.5, 3), (0.65, 1), (2.0, 1)]:  # cur_k = 3 after init
        a = ZiAdaptiveDraft()
        L.zi_adaptive_draft_init(C.byref(a), 8)
        L.zi_adaptive_draft_record_entropy(C.byref(a), H)
        b = ZiAdaptiveDraft()
        L.zi_adaptive_draft_init(C.byref(b), 8)
        L.zi_adaptive_draft_record_margin(C.byref(b), L.zi_entropy_margin(H))
        assert L.zi_adaptive_draft_next(C.byref(a)) == L.zi_adaptive_draft_next(C.byref(b)) == want, H


def test_invalid_arguments_fail_loudly():
    """Entry points reject bad arguments with a status and a message, never
    silently; without a GPU, zi_create reports the missing device."""
    from zinfer_amd._lib import ZI_OK, lib

    L = lib()
    h = C.c_void_p()
    assert L.zi_create(None, 0, 1, 1) != ZI_OK
    assert L.zi_create(C.byref(h), 0, 0, 100) != ZI_OK
    assert b"max_rows" in L.zi_last_error()
    assert L.zi_create(C.byref(h), 0, 1, 10 ** 7) != ZI_OK
    assert L.zi_sample_rows(None, None, None, None, None) != ZI_OK
    assert L.zi_sync(None) != ZI_OK


def test_no_cpu_fallback_in_product():
    """The product package never imports, links or loads the oracle."""
    pkg = os.path.join(ROOT, "zinfer_amd")
    bad = re.compile(r"(import\s+oracle|from\s+oracle|pyoracle|liboracle|#include\s+[\"<][^\">]*oracle)")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".hpp", ".h")):
                text = open(os.path.join(dirpath, f), errors="ignore").read()
                assert not bad.search(text), f
