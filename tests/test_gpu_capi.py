"""GPU: a C program (tests/capi/consumer.c, built by build() with gcc against
include/zinfer_hip.h and linked to libzinfer_hip.so) drives the host-row
Sampler API as the Zig shim would (init with a seed, accept the prompt, then
sample + accept per step, and argmaxWithMargin), and its tokens and margins
match the oracle's sequential loop bit for bit."""
import os
import struct
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "capi", "zi_consumer")

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", range(3))
def test_c_consumer_matches_oracle(oracle, tmp_path, case):
    assert os.path.exists(EXE), "tests/capi/zi_consumer missing: run __graft_entry__.build()"
    rng = np.random.Generator(np.random.PCG64(5150 + case))
    rows, V = [(6, 4096), (5, 32000), (4, 151937)][case]
    seed = int(rng.integers(0, 2**32))
    prompt = rng.integers(0, V, 40, dtype=np.uint32)
    temp, top_k, top_p, min_p, rep = [(0.8, 40, 0.95, 0.05, 1.1), (1.0, 0, 0.9, 0.0, 1.3),
                                      (0.7, 64, 0.9, 0.05, 1.0)][case]
    X = (rng.standard_t(3, (rows, V)) * 2).astype(np.float32)
    X[:, prompt[-4:]] += 6.0  # leaders that the penalty then moves
    inp = tmp_path / "in.bin"
    with open(inp, "wb") as f:
        f.write(struct.pack("<4I", rows, V, seed, prompt.size))
        f.write(prompt.astype("<u4").tobytes())
        f.write(struct.pack("<fIfff", temp, top_k, top_p, min_p, rep))
        f.write(X.astype("<f4").tobytes())
    r = subprocess.run([EXE, str(inp)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    got = [ln.split() for ln in r.stdout.strip().splitlines()]
    assert len(got) == rows
    p = oracle.params(temp=temp, top_k=top_k, top_p=top_p, min_p=min_p, repeat_penalty=rep, penalty_last_n=64)
    stream = oracle.rng_floats(seed, 4 * rows + 8)
    hist, pos = [int(t) for t in prompt], 0
    for i in range(rows):
        at, am = oracle.argmax_with_margin(X[i])
        tok, margin, d = oracle.sample_row(p, X[i], stream[pos:pos + 2], window=np.array(hist[-64:], np.uint32))
        pos += d["ndraws"]
        hist.append(tok)
        assert int(got[i][0]) == tok, (i, got[i], tok)
        assert int(got[i][1], 16) == int(np.float32(margin).view(np.uint32))
        assert int(got[i][2]) == at
        assert int(got[i][3], 16) == int(np.float32(am).view(np.uint32))
