"""Seeded synthetic inputs for the five BASELINE.json configurations.

Generated with numpy's PCG64 Generator (seed = 101 * cfg unless given), so the
CPU oracle and the GPU see identical bytes.  Parameters not named by a config
take the reference Params defaults (src/sampler.zig:3-27): min_p = 0.05 in
every config, top_k = 40 in config 3.  The penalty window is the whole
per-row history (256 in config 2, 128 in config 5); the reference's fixed
window of 64 is exercised separately by the parity tests.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from functools import lru_cache
from typing import Optional

import numpy as np


@dataclass
class Workload:
    name: str
    logits: np.ndarray                 # [rows, V] float32 (config 5: float32 holding bf16 values)
    params: dict
    uniforms: np.ndarray               # [rows, 2] float32
    hist: Optional[np.ndarray] = None  # [rows, H] uint32
    hist_len: Optional[np.ndarray] = None
    mask: Optional[np.ndarray] = None  # [rows, ceil(V/32)] uint32
    draft: Optional[np.ndarray] = None
    bf16: bool = False
    extra: dict = field(default_factory=dict)

    @property
    def rows(self):
        return self.logits.shape[0]

    @property
    def vocab(self):
        return self.logits.shape[1]

    def nbytes(self) -> int:
        """Algorithmic bytes of one pass: logits + history + mask + uniforms read, outputs written."""
        elt = 2 if self.bf16 else 4
        b = self.rows * self.vocab * elt
        if self.hist is not None:
            b += self.hist.nbytes + self.hist_len.nbytes
        if self.mask is not None:
            b += self.mask.nbytes
        b += self.rows * 4  # one uniform per row
        b += self.rows * 8  # token id + margin
        return b


def _bf16_round(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even to bfloat16, returned as float32 values."""
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    u = (u + 0x7FFF + lsb) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def _zipf_ids(rng, V: int, n: tuple, s: float) -> np.ndarray:
    ranks = np.arange(1, V + 1, dtype=np.float64)
    cdf = np.cumsum(ranks ** (-s))
    cdf /= cdf[-1]
    perm = rng.permutation(V).astype(np.uint32)
    r = np.searchsorted(cdf, rng.random(n), side="right")
    return perm[np.minimum(r, V - 1)]


def config1(seed: int = 101, V: int = 32000) -> Workload:
    rng = np.random.Generator(np.random.PCG64(seed))
    x = (rng.standard_normal((1, V)) * 3.0).astype(np.float32)
    spikes = rng.choice(V, size=5, replace=False)
    x[0, spikes] += np.float32(12.0)
    hist = rng.integers(0, V, size=(1, 64), dtype=np.uint32)
    u = rng.random((1, 2), dtype=np.float32)
    return Workload("c1_single_row_v32000", x, dict(temp=0.8, top_k=40, top_p=0.95, min_p=0.05,
                    repeat_penalty=1.1, penalty_last_n=64), u, hist, np.full(1, 64, np.int32))


def config2(seed: int = 202, rows: int = 64, V: int = 128256) -> Workload:
    rng = np.random.Generator(np.random.PCG64(seed))
    x = (rng.standard_t(3.0, size=(rows, V)) * 2.0).astype(np.float32)
    hist = _zipf_ids(rng, V, (rows, 256), 1.1)
    u = rng.random((rows, 2), dtype=np.float32)
    return Workload("c2_64x128256_f32_topk_topp", x, dict(temp=0.7, top_k=50, top_p=0.9, min_p=0.05,
                    repeat_penalty=1.15, freq_penalty=0.3, presence_penalty=0.5, penalty_last_n=256),
                    u, hist, np.full(rows, 256, np.int32))


def config3(seed: int = 303, rows: int = 32, V: int = 151936) -> Workload:
    rng = np.random.Generator(np.random.PCG64(seed))
    x = (rng.standard_normal((rows, V)) * 2.5).astype(np.float32)
    W = (V + 31) // 32
    dens = np.exp(rng.uniform(np.log(0.005), np.log(0.30), size=rows))
    bits = rng.random((rows, W * 32)) < dens[:, None]
    bits[:, V:] = False
    for r in range(rows):
        if not bits[r, :V].any():
            bits[r, rng.integers(0, V)] = True
    mask = pack_mask(bits)
    u = rng.random((rows, 2), dtype=np.float32)
    return Workload("c3_32x151936_f32_mask", x, dict(temp=0.7, top_k=40, top_p=0.95, min_p=0.05), u,
                    mask=mask, extra=dict(density=dens))


def config4(seed: int = 404, rows: int = 64, V: int = 262144) -> Workload:
    rng = np.random.Generator(np.random.PCG64(seed))
    x = (rng.standard_normal((rows, V)) * 2.0).astype(np.float32)
    dom = rng.random(rows) < 0.1
    for r in np.nonzero(dom)[0]:
        x[r, rng.integers(0, V)] += np.float32(15.0)
    am = np.argmax(x, axis=1).astype(np.uint32)
    rand_ids = rng.integers(0, V, size=rows, dtype=np.uint32)
    draft = np.where(rng.random(rows) < 0.5, am, rand_ids).astype(np.uint32)
    u = rng.random((rows, 2), dtype=np.float32)
    return Workload("c4_64x262144_f32_entropy_top8", x, dict(k=8), u, draft=draft,
                    extra=dict(dominant=dom))


def config5(seed: int = 505, rows: int = 512, V: int = 151936) -> Workload:
    rng = np.random.Generator(np.random.PCG64(seed))
    x = _bf16_round(rng.standard_normal((rows, V), dtype=np.float32) * np.float32(3.0))
    hist = rng.integers(0, V, size=(rows, 128), dtype=np.uint32)
    u = rng.random((rows, 2), dtype=np.float32)
    return Workload("c5_512x151936_bf16_topp098", x, dict(temp=1.0, top_k=0, top_p=0.98, min_p=0.05,
                    repeat_penalty=1.1, penalty_last_n=128), u, hist, np.full(rows, 128, np.int32), bf16=True)


CONFIGS = {1: config1, 2: config2, 3: config3, 4: config4, 5: config5}


def pack_mask(bits: np.ndarray) -> np.ndarray:
    """[rows, 32*W] bool -> [rows, W] uint32 with id t at bit (t & 31) of word t >> 5."""
    rows, n = bits.shape
    W = n // 32
    weights = (np.uint64(1) << np.arange(32, dtype=np.uint64))
    return (bits.reshape(rows, W, 32).astype(np.uint64) * weights).sum(-1).astype(np.uint32)


def mask_bit(mask: np.ndarray, ids: np.ndarray) -> np.ndarray:
    """Bit t of a packed row mask: (mask[t >> 5] >> (t & 31)) & 1."""
    return (mask[ids >> 5] >> (ids & 31).astype(np.uint32)) & 1


# ------------------------------------------------------------ token pieces

_JSON_FRAGMENTS = [
    "{", "}", "[", "]", ":", ",", '"', '{"', '"}', '":', '": ', '": "', '",', '", "', '"},', '"}]', "},", "}]",
    "],", "]}", "[{", '[{"', '["', '"]', ' {', ' [', ' "', '\n', '\n ', '\n  ', '\n    ', '\t', '\r\n', ' ', '  ',
    '    ', 'true', 'false', 'null', ' true', ' false', ' null', 'tr', 'ue', 'fal', 'se', 'nu', 'll', 't', 'f',
    'n', 'nul', 'fa', 'tru', '0', '1', '2', '9', '10', '12', '123', '2024', '-', '-1', '-0', '0.', '.', '.5', '.25',
    'e', 'E', 'e+', 'e-', 'E+', '1e', '1e10', '3.14', '1.0', '00', '0x', '+1', '\\', '\\n', '\\"', '\\\\', '\\/',
    '\\t', '\\u', '\\u00', '\\u12', '\\u12af', '\\ud83d', '\\q', '\\x', ': {', ': [', ', "', '": {', '": [',
    '": true', '": null', '": 1', '":"', '","', '"],"', '},{"', 'NaN', 'Infinity', '1,', '1}', '1]', '0,', '0}',
]
_WORD_CHARS = "abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ0123456789_-./'"


@lru_cache(maxsize=4)
def synthetic_vocab(V: int = 151936, seed: int = 77):
    """A seeded tokenizer vocabulary for the JSON mask: ids 0-255 are the single
    bytes (control bytes and bytes >= 0x80 included), then JSON fragments, escapes,
    numbers, literals, whitespace runs, word pieces with and without a leading
    space, pieces longer than 12 bytes, a few empty pieces, and three
    end-of-generation ids whose pieces are special-token text.

    Returns (piece_off [V+1] u32, piece_buf u8, eog ids u32, eos id)."""
    assert V >= 300
    rng = np.random.Generator(np.random.PCG64(seed))
    pieces: list = [bytes([b]) for b in range(256)]
    pieces += [f.encode() for f in _JSON_FRAGMENTS]
    specials = [b"<|endoftext|>", b"<|im_end|>", b"</s>"]
    while len(pieces) < V:
        u = rng.random()
        if u < 0.50:  # word piece, often with a leading space
            n = int(rng.integers(1, 11))
            w = "".join(rng.choice(list(_WORD_CHARS[:52]), n))
            pieces.append(((" " if rng.random() < 0.6 else "") + w).encode())
        elif u < 0.62:  # digits / number fragments
            n = int(rng.integers(1, 6))
            w = "".join(rng.choice(list("0123456789"), n))
            w = w + str(rng.choice(["", "", ".", ",", "}", "]", "e", "E+", " "]))
            pieces.append(w.encode())
        elif u < 0.74:  # JSON punctuation mixed with text
            k = int(rng.integers(1, 4))
            parts = [str(rng.choice(_JSON_FRAGMENTS)) for _ in range(k)]
            pieces.append("".join(parts).encode())
        elif u < 0.80:  # whitespace runs
            n = int(rng.integers(1, 20))
            pieces.append("".join(rng.choice([" ", " ", "\n", "\t", "\r"], n)).encode())
        elif u < 0.86:  # long pieces (past the 12 inline bytes)
            n = int(rng.integers(13, 90))
            alphabet = list(_WORD_CHARS + ' "{}[]:,\\')
            pieces.append("".join(rng.choice(alphabet, n)).encode())
        elif u < 0.92:  # arbitrary bytes, including control bytes and UTF-8 tails
            n = int(rng.integers(1, 8))
            pieces.append(bytes(rng.integers(0, 256, n).astype(np.uint8).tolist()))
        elif u < 0.9995:  # string content with escapes
            n = int(rng.integers(1, 6))
            parts = [str(rng.choice(["a", "b", " ", "\\n", "\\\"", "\\u00e9", "\\u12", "x", "\\\\", "é"]))
                     for _ in range(n)]
            pieces.append("".join(parts).encode())
        else:
            pieces.append(b"")
    pieces = pieces[:V]
    # end-of-generation ids: special-token text at fixed positions past the bytes
    eog = np.array([V - 1, V // 2 + 1, 290], np.uint32)
    for i, t in zip(eog.tolist(), specials):
        pieces[i] = t
    eos = int(eog[0])
    lens = np.array([len(p) for p in pieces], np.int64)
    off = np.zeros(V + 1, np.uint32)
    off[1:] = np.cumsum(lens).astype(np.uint32)
    buf = np.frombuffer(b"".join(pieces), dtype=np.uint8).copy()
    for a in (off, buf, eog):
        a.flags.writeable = False  # shared by the cache
    return off, buf, eog, eos


def vocab_piece(off: np.ndarray, buf: np.ndarray, i: int) -> bytes:
    return bytes(buf[int(off[i]):int(off[i + 1])])


def json_prefixes(n: int, seed: int = 606):
    """Seeded JSON documents (json.dumps of random objects: strings with
    escapes, numbers, literals, nested arrays and objects) cut at random
    points: n pairs (object_only, prefix bytes), the validator states of a
    JSON-mode decoding batch."""
    import json
    import random

    r = random.Random(seed)
    vals = [0, -17, 3.25, -1.5e-7, 12345678901, "", "plain text", 'q"uote', "back\\slash", "tab\there", "é€",
            True, False, None]

    def value(depth):
        k = r.random()
        if depth > 0 and k < 0.2:
            return {"k%d" % i: value(depth - 1) for i in range(r.randint(0, 3))}
        if depth > 0 and k < 0.35:
            return [value(depth - 1) for _ in range(r.randint(0, 3))]
        return r.choice(vals)

    out = []
    while len(out) < n:
        obj = {"field_%d" % i: value(r.randint(0, 4)) for i in range(r.randint(1, 5))}
        doc = json.dumps(obj, indent=r.choice([None, 2]), ensure_ascii=r.random() < 0.5).encode()
        out.append((True, doc[: r.randint(0, len(doc) - 1)]))
    return out
