"""Benchmark: rows/sec and HBM roofline of the batched sampling path.

One step = one zi_sample_rows launch over one batch of BASELINE config 2
(64 rows x 128256 f32 logits, top_k 50, top_p 0.9, T 0.7, repetition 1.15,
frequency 0.3, presence 0.5 over 256-token histories), inputs resident in HBM.
Steps rotate over enough distinct input batches (>= 512 MiB) that the 256 MiB
Infinity Cache cannot serve them.  The launches are recorded once into a HIP
graph (as a serving loop would) and replayed, so host submission does not
limit the measured rate.

Prints ONE JSON line (rank 0).  Only one GPU is used by this build: --gpus N
with N > 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
METRIC = "rows/sec + HBM GB/s (% of peak), 64×128256 f32 top-k/top-p sampling"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2048, help="timed launches (exactly)")
    ap.add_argument("--warmup", type=int, default=128, help="untimed launches before them (exactly)")
    ap.add_argument("--config", type=int, default=2, help="BASELINE config to run (2 = headline)")
    ap.add_argument("--path", choices=["sample", "json_mask", "verify", "dry", "readfloor"], default="sample",
                    help="sample: zi_sample_rows on --config (the headline); json_mask: zi_json_mask_rows; "
                         "verify: zi_sampler_verify; dry: zi_dry_edits_rows; readfloor: a plain read of "
                         "config 2's bytes (the achievable-bandwidth reference)")
    ap.add_argument("--branches", type=int, default=1,
                    help="verify path: > 1 verifies that many 8-token branches in one call (zi_sampler_verify_tree)")
    ap.add_argument("--softcap", type=float, default=0.0,
                    help="final-logit softcap fused into the read (sample path; 0 = off, the config's default)")
    ap.add_argument("--min-p", type=float, default=None,
                    help="override the config's min_p (config 5 with 0 is the whole-order nucleus case)")
    ap.add_argument("--top-k", type=int, default=None, help="override the config's top_k")
    ap.add_argument("--spike", type=float, default=0.0,
                    help="add this to one seeded entry per row (a dominant token: peaked rows)")
    ap.add_argument("--pruned", type=int, default=0,
                    help="pruned rows (sample path): 64 fixed + this many random groups of 8 ids per row are the "
                         "only logits (zi_sample_rows_pruned; the reference keeps 512); 0 = dense rows")
    ap.add_argument("--rotate-mib", type=int, default=512, help="distinct input bytes cycled through")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="bounded CPU-baseline sample (0 = skip)")
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly instead of replaying a HIP graph")
    ap.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "traffic.md"),
                    help="rocprofv3 counter summary giving HBM bytes per launch")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain device copy of known size (counter calibration)")
    return ap.parse_args()


def copy_calibration(nbytes: int = 256 * 2**20, reps: int = 8):
    """A plain copy of known size: FETCH_SIZE / WRITE_SIZE per dispatch read
    against `nbytes` give the scale factor applied to the sampling kernel."""
    import torch

    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").uniform_()
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes, "reps": reps}), flush=True)


def _entropy_chunks(V: int, rows: int) -> int:
    """Chunks per row of the chunked entropy plan (zi::plan_rows, f32)."""
    ept = 64
    chunks = lambda e: -(-V // (512 * e))
    while ept > 16 and rows * chunks(ept) < 256 and chunks(ept // 2) <= 8:
        ept //= 2
    return chunks(ept)


def read_traffic(path: str, kernel: str, workload: str):
    """HBM bytes per launch from a committed rocprofv3 --pmc summary line:
    `traffic <workload> <kernel> <bytes>`."""
    if not os.path.exists(path):
        return None
    for line in open(path):
        m = re.match(r"\s*traffic\s+(\S+)\s+(\S+)\s+([0-9.eE+]+)", line)
        if m and m.group(1) == workload and m.group(2) == kernel:
            return float(m.group(3))
    return None


def timed_launches(launch, nsets: int, steps: int, warmup: int, stream, use_graph: bool = True):
    """Runs exactly `warmup` untimed then `steps` timed launches, launch i
    working on input set i % nsets, on `stream` (the caller has made it
    current).  With graphs: one graph of all nsets launches, replayed
    steps // nsets times, plus a graph of the first steps % nsets launches
    (likewise for the warmup).  Returns (gpu ms over the timed launches from
    HIP events on `stream`, host wall seconds)."""
    import torch

    graphs = {}

    def graph_of(n):
        if n not in graphs:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for i in range(n):
                    launch(i)
            torch.cuda.synchronize()
            graphs[n] = g
        return graphs[n]

    def run(n):
        if not use_graph:
            for i in range(n):
                launch(i % nsets)
            return
        full, rem = divmod(n, nsets)
        for _ in range(full):
            graph_of(nsets).replay()
        if rem:
            graph_of(rem).replay()

    for i in range(nsets):  # eager first pass: any lazy set-up happens outside the graphs
        launch(i)
    torch.cuda.synchronize()
    if use_graph:  # capture before timing
        graph_of(nsets)
        if steps % nsets:
            graph_of(steps % nsets)
        if warmup % nsets:
            graph_of(warmup % nsets)
    run(warmup)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    run(steps)
    ev1.record(stream)
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1), time.perf_counter() - t0


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_threads() -> int:
    """Worker threads for the all-cores CPU leg: the box's CPU share (its
    OMP_NUM_THREADS), else the visible cores."""
    n = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return max(1, n or (os.cpu_count() or 1))


def bench_readfloor(args):
    """A plain streaming read of config 2's bytes (zi_probe.hip, 1024-thread
    workgroups, 128 KiB each, non-temporal 16-byte loads) in the same harness
    as the sampling path: rotating input sets, graph replay, HIP events.  It
    is the achievable-bandwidth reference for the sampling kernels (and its
    per-launch time includes the same launch overhead)."""
    import ctypes as C

    import torch

    lib = C.CDLL(os.path.join(ROOT, "zinfer_amd", "libzi_probe.so"))
    lib.zi_probe_read.restype = C.c_int32
    lib.zi_probe_read.argtypes = [C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p]
    dev = torch.device("cuda:0")
    nbytes = 64 * 128256 * 4
    nsets = max(1, (args.rotate_mib * 2**20 + nbytes - 1) // nbytes)
    sets = [torch.empty(nbytes // 4, dtype=torch.float32, device=dev).uniform_() for _ in range(nsets)]
    out = torch.empty(((nbytes + 131071) // 131072) * 16, dtype=torch.float32, device=dev)
    stream = torch.cuda.Stream(dev)

    def launch(i):
        rc = lib.zi_probe_read(sets[i].data_ptr(), nbytes, out.data_ptr(), stream.cuda_stream)
        assert rc == 0, rc

    with torch.cuda.stream(stream):
        gpu_ms, wall = timed_launches(launch, nsets, args.steps, args.warmup, stream, not args.no_graph)
    ms = gpu_ms / args.steps
    achieved = nbytes / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "plain streaming read of 64x128256 f32 (achievable-bandwidth reference)",
        "value": round(achieved, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (torch uniform_)",
        "config": {"workload": "readfloor_64x128256_f32", "bytes": nbytes, "rotating_input_sets": nsets,
                   "launch": "eager" if args.no_graph else "hip_graph_replay"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
                     "algorithmic_bytes_per_launch": nbytes, "kernel": "read_kernel"},
        "cpu_baseline": None, "wall_s": round(wall, 3)}), flush=True)


def bench_json_mask(args):
    """JSON grammar masks (zi_json_mask_rows, no state cache): 32 validator
    states (seeded JSON prefixes) over a 151936-token synthetic vocabulary,
    config 3's batch and vocabulary size.  One step = one call for the batch.
    Every mask is checked against the oracle; the CPU baseline times the
    oracle's applyMask restatement on the same states."""
    import numpy as np
    import torch

    from zinfer_amd.api import Context, JsonValidator, Vocab
    from zinfer_amd.workloads import json_prefixes, synthetic_vocab

    V, rows = 151936, 32
    off, buf, eog, eos = synthetic_vocab(V)
    pre = json_prefixes(rows)
    vals = []
    for ob, text in pre:
        v = JsonValidator(ob)
        assert v.consume(text)
        vals.append(v)
    ctx = Context(0, max_rows=64, max_vocab=V)
    vocab = Vocab(ctx, off, buf, eog, eos, cache_states=0)
    W = (V + 31) // 32
    dev = torch.device("cuda:0")
    out = torch.empty((rows, W), dtype=torch.int32, device=dev)
    inner = 16
    stream = torch.cuda.Stream(dev)
    with torch.cuda.stream(stream):
        vocab.json_mask_rows(vals, out=out)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(inner):
                vocab.json_mask_rows(vals, out=out)
        torch.cuda.synchronize()
        reps = max(1, args.steps // inner)
        for _ in range(max(1, args.warmup // inner)):
            graph.replay()
        torch.cuda.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        ev0.record(stream)
        for _ in range(reps):
            graph.replay()
        ev1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    steps = reps * inner
    ms = ev0.elapsed_time(ev1) / steps
    got = out.cpu().numpy().view(np.uint32)

    from oracle import pyoracle

    ostates = []
    for ob, text in pre:
        j = pyoracle.json_init(ob)
        pyoracle.json_consume(j, text)
        ostates.append(j)
    t1, want = pyoracle.bench_json_mask(ostates, off, buf, eog, eos, 1)
    parity = bool(np.array_equal(got, want))
    cpu = None
    if args.cpu_seconds > 0:
        creps = max(1, int(args.cpu_seconds / max(t1, 1e-6)))
        tc, _ = pyoracle.bench_json_mask(ostates, off, buf, eog, eos, creps)
        cpu = {"value": round(rows * creps / tc, 1), "unit": "rows/s", "cores": 1, "kind": "port",
               "sample": f"the same {rows} states x {creps} passes ({tc:.1f} s), oracle/grammar_oracle.c "
                         f"(C restatement of src/grammar.zig:446-479), -O3, 1 thread"}
    # bytes per call: per row the base mask read and the mask written (4 W each), the stack-token
    # list pass reads each list token's class record, tail chunks and id once per row
    # list tokens: pieces holding { } [ ] or , that are not end-of-generation ids (zi_vocab_create)
    hit = np.isin(np.asarray(buf), np.frombuffer(b"{}[],", np.uint8))
    cs = np.concatenate([[0], np.cumsum(hit)])
    lens = np.diff(np.asarray(off)).astype(np.int64)
    listed = (cs[np.asarray(off)[1:]] - cs[np.asarray(off)[:-1]]) > 0
    listed[np.asarray(eog, dtype=np.int64)] = False
    listed[eos] = False
    S = int(listed.sum())
    tail_bytes = int((16 * ((np.maximum(lens[listed] - 12, 0) + 15) // 16)).sum())
    nbytes = rows * (8 * W + S * 20 + tail_bytes)
    achieved = nbytes / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "JSON grammar mask rows/sec (zi_json_mask_rows, 151936-token vocabulary)",
        "value": round(rows / (ms * 1e-3), 1), "unit": "rows/s", "n_gpus": 1, "steps": steps,
        "warmup": max(1, args.warmup // inner) * inner, "ms_per_step": round(ms, 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "u8",
        "data": "synthetic, seeded (zinfer_amd/workloads.py synthetic_vocab, json_prefixes)",
        "config": {"workload": "json_mask_32x151936", "rows": rows, "vocab": V, "stack_tokens": S,
                   "cache_states": 0, "launch": "hip_graph_replay", "parity_vs_oracle": parity},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
                     "algorithmic_bytes_per_launch": nbytes, "kernel": "json_list_kernel"},
        "cpu_baseline": cpu,
        "wall_s": round(wall, 3),
    }), flush=True)
    vocab.close()
    ctx.close()
    if not parity:
        raise SystemExit("json_mask: GPU masks differ from the oracle")


def bench_verify(args):
    """Draft verification (zi_sampler_verify, src/gen.zig:544-587): 8 drafted
    tokens + the bonus row over a 151936-token f32 vocabulary, device logits.
    One step = one verify call (synchronous: the accepted count comes back to
    the host).  For contrast the same rows are also sampled one call per row
    through the host-row Sampler (the reference API shape: host logits in).
    The CPU baseline is the oracle's sequential verify loop."""
    import numpy as np
    import torch

    from zinfer_amd.api import Context, Sampler, params

    V, k = 151936, 8
    nbr = max(1, args.branches)
    rng = np.random.Generator(np.random.PCG64(808))
    Xb, drafts = [], []
    for j in range(nbr):  # branch j: the target agrees with its draft up to token 8 - 2j
        Xj = (rng.standard_normal((k + 1, V)) * 2.5).astype(np.float32)
        dj = [int(t) for t in rng.integers(0, V, k)]
        for i, t in enumerate(dj[:max(0, k - 2 * j)]):
            Xj[i, t] += 25.0  # well above the row maximum
        Xb.append(Xj)
        drafts.append(dj)
    X, draft = Xb[0], drafts[0]
    pk = dict(temp=0.8, top_k=40, top_p=0.95, min_p=0.05, repeat_penalty=1.1, penalty_last_n=64, seed=9)
    hist = [int(t) for t in rng.integers(0, V, 64)]
    ctx = Context(0, max_rows=max(16, nbr * (k + 1)), max_vocab=V)
    dev = torch.device("cuda:0")
    L = torch.from_numpy(np.concatenate(Xb) if nbr > 1 else X).to(dev)
    smp = Sampler(ctx, V, params(**pk))
    for t in hist:
        smp.accept(t)

    def call():
        if nbr > 1:
            return max(smp.verify_tree(L, drafts, commit=False)[0])
        return smp.verify(L, draft)[0]

    for _ in range(max(1, args.warmup // 16)):
        call()
    torch.cuda.synchronize()
    steps = max(16, args.steps)
    accepted = []
    t0 = time.perf_counter()
    for _ in range(steps):
        accepted.append(call())
    wall = time.perf_counter() - t0
    ms = wall * 1e3 / steps
    # one call per row through the host-row sampler, for contrast
    seq = Sampler(ctx, V, params(**pk))
    for t in hist:
        seq.accept(t)
    reps = max(4, steps // 8)
    t1 = time.perf_counter()
    for _ in range(reps):
        for Xj in Xb:
            for i in range(k + 1):
                seq.sample_with_margin(Xj[i].copy())
    ms_seq = (time.perf_counter() - t1) * 1e3 / reps

    from oracle import pyoracle

    op = pyoracle.params(**{kk: v for kk, v in pk.items() if kk != "seed"})
    stream = pyoracle.rng_floats(9, 64)
    cpu = None
    if args.cpu_seconds > 0:
        n_cpu, tc0 = 0, time.perf_counter()
        while time.perf_counter() - tc0 < min(args.cpu_seconds, 10.0):
            for Xj, dj in zip(Xb, drafts):  # one sequential loop per branch
                h, pos = list(hist), 0
                for i in range(k + 1):
                    tok, _, d = pyoracle.sample_row(op, Xj[i], stream[pos:pos + 2],
                                                    window=np.array(h[-64:], np.uint32))
                    pos += d["ndraws"]
                    if i < k and tok == dj[i]:
                        h.append(tok)
                        continue
                    break
            n_cpu += 1
        tc = time.perf_counter() - tc0
        cpu = {"value": round(n_cpu / tc, 2), "unit": "verify calls/s", "cores": 1, "kind": "port",
               "sample": f"{n_cpu} x {nbr} sequential verify loops of {k} drafted tokens + bonus row ({tc:.1f} s), "
                         f"oracle/oracle.c sample_row (C restatement of src/sampler.zig:190-276), 1 thread"}
    nbytes = nbr * (k + 1) * V * 4
    achieved = nbytes / (ms * 1e-3) / 1e9
    entry = "zi_sampler_verify_tree, %d branches of" % nbr if nbr > 1 else "zi_sampler_verify,"
    print(json.dumps({
        "metric": f"draft verification calls/sec ({entry} 8 drafted tokens + bonus row, V=151936 f32)",
        "value": round(1e3 / ms, 1), "unit": "verify calls/s", "n_gpus": 1, "steps": steps,
        "warmup": max(1, args.warmup // 16), "ms_per_step": round(ms, 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic, seeded (bench.py bench_verify): N(0, 2.5^2) rows, draft tokens +25",
        "config": {"workload": f"verify_{nbr}x8_151936_f32" if nbr > 1 else "verify_k8_151936_f32", "drafted": k,
                   "branches": nbr, "vocab": V, **pk,
                   "accepted_mean": float(np.mean(accepted)), "one_call_per_row_ms": round(ms_seq, 4),
                   "timing": "host wall clock per synchronous call"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
                     "algorithmic_bytes_per_launch": nbytes, "kernel": "sample_kernel"},
        "cpu_baseline": cpu,
        "wall_s": round(wall, 3),
    }), flush=True)
    ctx.close()


def bench_dry(args):
    """DRY edits on the device (zi_dry_edits_rows, src/sampler.zig:104-187) for 64
    rows of 1024-token histories (the default dry_range), graph-replayed with
    HIP events on the launch stream.  The histories mix Zipf ids with repeated
    phrases, so every row has repeats to penalize.  Also timed: the worst case,
    period-1 loops over the full 4096-token ring (dry_range 4096)."""
    import numpy as np
    import torch

    from zinfer_amd.api import Context, params

    rows, H = 64, 1024
    rng = np.random.Generator(np.random.PCG64(616))
    hist = np.minimum(rng.zipf(1.2, (rows, H)), 50000).astype(np.uint32)
    for r in range(rows):  # paste a few earlier phrases again
        for _ in range(8):
            ln = int(rng.integers(3, 24))
            a0 = int(rng.integers(0, H - 2 * ln))
            b0 = int(rng.integers(a0 + ln, H - ln))
            hist[r, b0:b0 + ln] = hist[r, a0:a0 + ln]
    hl = np.full(rows, H, np.int32)
    brk = np.array([13, 10, 2, 7], np.uint32)
    pk = dict(dry_multiplier=0.8, dry_base=1.75, dry_allowed_length=2, dry_range=1024)
    p = params(**pk)
    dev = torch.device("cuda:0")
    ctx = Context(0, max_rows=rows, max_vocab=1024)
    hd, ld, bd = torch.from_numpy(hist).to(dev), torch.from_numpy(hl).to(dev), torch.from_numpy(brk).to(dev)

    def timed(hd, ld, p, steps):
        stream = torch.cuda.Stream(dev)
        with torch.cuda.stream(stream):
            out = ctx.dry_edits_rows(p, hd, ld, bd)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for _ in range(16):
                    ctx.dry_edits_rows(p, hd, ld, bd)
            torch.cuda.synchronize()
            reps = max(1, steps // 16)
            for _ in range(max(1, args.warmup // 16)):
                graph.replay()
            torch.cuda.synchronize()
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            ev0.record(stream)
            for _ in range(reps):
                graph.replay()
            ev1.record(stream)
            torch.cuda.synchronize()
        return ev0.elapsed_time(ev1) / (reps * 16), reps * 16, out

    t0 = time.perf_counter()
    ms, steps, (ids, dl, cnt) = timed(hd, ld, p, args.steps)
    wall = time.perf_counter() - t0
    worst = np.tile(np.uint32(5), (rows, 4096))
    ms_worst, _, _ = timed(torch.from_numpy(worst).to(dev), torch.full((rows,), 4096, dtype=torch.int32, device=dev),
                           params(**dict(pk, dry_range=4096)), 64)
    from oracle import pyoracle

    cnt_h = cnt.cpu().numpy()
    ids_h = ids.cpu().numpy().astype(np.uint32)
    parity = all(np.array_equal(ids_h[r, :cnt_h[r]], pyoracle.dry_edits(hist[r], brk, 0.8, 1.75, 2, 1024)[0])
                 for r in range(rows))
    cpu = None
    if args.cpu_seconds > 0:
        n_cpu, tc0 = 0, time.perf_counter()
        while time.perf_counter() - tc0 < min(args.cpu_seconds, 10.0):
            pyoracle.dry_edits(hist[n_cpu % rows], brk, 0.8, 1.75, 2, 1024)
            n_cpu += 1
        tc = time.perf_counter() - tc0
        cpu = {"value": round(n_cpu / tc, 1), "unit": "rows/s", "cores": 1, "kind": "port",
               "sample": f"{n_cpu} rows of the same histories ({tc:.1f} s), oracle/oracle.c or_dry_edits "
                         f"(C restatement of src/sampler.zig:104-187, Z-algorithm), 1 thread"}
    nbytes = rows * (H * 4 + 4) + int(cnt_h.sum()) * 8 + rows * 4
    achieved = nbytes / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "DRY edit rows/sec (zi_dry_edits_rows, 64 rows x 1024-token histories)",
        "value": round(rows / (ms * 1e-3), 1), "unit": "rows/s", "n_gpus": 1, "steps": steps,
        "warmup": max(1, args.warmup // 16) * 16, "ms_per_step": round(ms, 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "u32",
        "data": "synthetic, seeded (bench.py bench_dry): Zipf(1.2) ids with pasted phrases",
        "config": {"workload": "dry_64x1024", "rows": rows, "history": H, **pk, "breakers": len(brk),
                   "edits_mean": float(cnt_h.mean()), "worst_case_ms": round(ms_worst, 4),
                   "worst_case": "period-1 loop, 4096-token ring, dry_range 4096", "parity_vs_oracle": parity},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
                     "algorithmic_bytes_per_launch": nbytes, "kernel": "dry_kernel"},
        "cpu_baseline": cpu,
        "wall_s": round(wall, 3),
    }), flush=True)
    ctx.close()
    if not parity:
        raise SystemExit("dry: device edits differ from the oracle")


def bench_entropy(args, w):
    """Config 4: entropy (nats, T = 1, full vocabulary), top-8 ids and full-vocabulary
    probabilities, argmax and accept = (argmax == draft) per row
    (zi_entropy_topk_rows), 64 x 262144 f32, inputs rotating over >= --rotate-mib."""
    import numpy as np
    import torch

    from zinfer_amd.api import Context

    dev = torch.device("cuda:0")
    rows, V, k = w.rows, w.vocab, int(w.params["k"])
    base = torch.from_numpy(w.logits).to(dev)
    per_set = base.numel() * 4
    nsets = max(1, (args.rotate_mib * 2**20 + per_set - 1) // per_set)
    sets = [torch.roll(base, shifts=i * 97, dims=1).contiguous() if i else base for i in range(nsets)]
    draft = torch.from_numpy(w.draft.astype(np.int32)).to(dev)
    ctx = Context(0, max_rows=rows, max_vocab=V)
    stream = torch.cuda.Stream(dev)
    steps = args.steps
    with torch.cuda.stream(stream):
        gpu_ms, wall = timed_launches(lambda i: ctx.entropy_topk_rows(sets[i], k, draft), nsets, steps, args.warmup,
                                      stream, not args.no_graph)
    ms = gpu_ms / steps
    ent, ids, probs, am, acc = ctx.entropy_topk_rows(sets[0], k, draft)
    torch.cuda.synchronize()
    cpu = None
    if args.cpu_seconds > 0:
        from oracle import pyoracle

        n_cpu, tc0 = 0, time.perf_counter()
        agree = True
        while time.perf_counter() - tc0 < args.cpu_seconds:
            r = n_cpu % rows
            H, oids, _ = pyoracle.entropy_topk(w.logits[r], k)
            if n_cpu < rows:
                agree &= bool(np.array_equal(oids.astype(np.int64), ids[r].cpu().numpy().astype(np.int64)))
            n_cpu += 1
        tc = time.perf_counter() - tc0
        cpu = {"value": round(n_cpu / tc, 1), "unit": "rows/s", "cores": 1, "kind": "port",
               "sample": f"{n_cpu} rows ({tc:.1f} s), oracle/oracle.c or_entropy_topk, 1 thread",
               "top8_ids_match_gpu": agree}
    # per row: the logits and the draft id read; entropy, k ids, k probabilities, argmax, accept written
    nbytes = rows * (V * 4 + 4 + 4 + 8 * k + 4 + 1)
    achieved = nbytes / (ms * 1e-3) / 1e9
    # batches whose chunked grid exceeds one workgroup per CU walk their segments
    kname = "entropy_walk_kernel" if w.rows * _entropy_chunks(w.vocab, w.rows) > 256 else "entropy_kernel"
    print(json.dumps({
        "metric": "rows/sec + HBM GB/s (% of peak), 64x262144 f32 entropy + top-8 + accept",
        "value": round(rows / (ms * 1e-3), 1), "unit": "rows/s", "n_gpus": 1, "steps": steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic, seeded (zinfer_amd/workloads.py): " + w.name,
        "config": {"workload": w.name, "rows": rows, "vocab": V, "k": k, "rotating_input_sets": nsets,
                   "launch": "hip_graph_replay"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": read_traffic(args.traffic, kname, w.name),
                     "algorithmic_bytes_per_launch": nbytes, "kernel": kname},
        "cpu_baseline": cpu,
        "wall_s": round(wall, 3),
    }), flush=True)
    ctx.close()


def main():
    args = parse()
    if args.copy_calibration:
        copy_calibration()
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build runs on one GPU only (the sampling path is row-parallel; "
              "rows would shard across GPUs with no collective, which is not implemented). Use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    if args.path == "json_mask":
        bench_json_mask(args)
        return
    if args.path == "verify":
        bench_verify(args)
        return
    if args.path == "dry":
        bench_dry(args)
        return
    if args.path == "readfloor":
        bench_readfloor(args)
        return

    import numpy as np
    import torch

    from zinfer_amd.api import Context, SampleResult, params
    from zinfer_amd.workloads import CONFIGS

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    w = CONFIGS[args.config]()
    rows, V = w.rows, w.vocab
    if args.softcap > 0:
        w.params = dict(w.params, final_logit_softcap=args.softcap)
    if args.min_p is not None:
        w.params = dict(w.params, min_p=args.min_p)
        w.name += f"_minp{args.min_p:g}"
    if args.top_k is not None:
        w.params = dict(w.params, top_k=args.top_k)
        w.name += f"_k{args.top_k}"
    if args.spike:
        srng = np.random.Generator(np.random.PCG64(77))
        cols = srng.integers(0, V, size=rows)
        w.logits = w.logits.copy()
        w.logits[np.arange(rows), cols] += np.float32(args.spike)
        if w.bf16:
            from zinfer_amd.workloads import _bf16_round
            w.logits = _bf16_round(w.logits)
        w.name += f"_spike{args.spike:g}"
    if args.config == 4:
        bench_entropy(args, w)
        return
    ld = (V + 7) // 8 * 8
    dt = torch.bfloat16 if w.bf16 else torch.float32
    elt = 2 if w.bf16 else 4
    per_set = rows * ld * elt
    nsets = min(1024, max(1, (args.rotate_mib * 2**20 + per_set - 1) // per_set))
    base = torch.zeros((rows, ld), dtype=dt, device=dev)
    base[:, :V] = torch.from_numpy(w.logits).to(dev).to(dt)
    sets = []
    for i in range(nsets):  # distinct bytes per set: cyclic roll keeps the value distribution
        sets.append(torch.roll(base, shifts=i * 97, dims=1).contiguous() if i else base)
    hist = torch.from_numpy(w.hist).to(dev) if w.hist is not None else None
    hist_len = torch.from_numpy(w.hist_len).to(dev) if w.hist is not None else None
    mask = torch.from_numpy(w.mask).to(dev) if w.mask is not None else None
    uni = torch.from_numpy(w.uniforms).to(dev)
    p = params(**w.params)
    gdev = cdev = None
    if args.pruned > 0:  # the reference's candidate groups (src/model.zig:2070-2125): 0..63 + the rest
        from oracle import pyoracle

        grng = np.random.Generator(np.random.PCG64(909))
        ngt = (V + 7) // 8
        G = np.stack([np.concatenate([np.arange(64), grng.choice(np.arange(64, ngt), args.pruned, replace=False)])
                      for _ in range(rows)]).astype(np.int32)
        gdev = torch.from_numpy(G).to(dev)
        cdev = torch.full((rows,), G.shape[1], dtype=torch.int32, device=dev)
        # the CPU leg samples the rows as the reference sees them: -inf outside the groups
        w.logits = np.stack([pyoracle.pruned_row(w.logits[r], G[r], V) for r in range(rows)])
        w.name += f"_pruned{G.shape[1]}"
    ctx = Context(0, max_rows=max(rows, 64), max_vocab=V)
    outs = [SampleResult(tok=torch.empty(rows, dtype=torch.int32, device=dev),
                         margin=torch.empty(rows, dtype=torch.float32, device=dev),
                         ndraws=torch.empty(rows, dtype=torch.int32, device=dev)) for _ in range(nsets)]

    def launch(i):
        ctx.sample_rows(p, sets[i], uni, vocab=V, hist=hist, hist_len=hist_len, mask=mask, out=outs[i],
                        groups=gdev, group_count=cdev)

    stream = torch.cuda.Stream(dev)  # default priority
    steps, wsteps = args.steps, args.warmup
    with torch.cuda.stream(stream):
        gpu_ms, wall = timed_launches(launch, nsets, steps, wsteps, stream, not args.no_graph)

    ms_per_step = gpu_ms / steps
    rows_per_s = rows / (ms_per_step * 1e-3)
    nbytes = w.nbytes()
    if gdev is not None:  # per row: the listed groups' logits, their ids, the count, history, mask bits,
        ng = gdev.shape[1]  # one uniform, token + margin
        per_row = ng * (8 * elt + 4) + 4 + ((w.hist.shape[1] * 4 + 4) if w.hist is not None else 0) \
            + (ng if w.mask is not None else 0) + 4 + 8
        nbytes = rows * per_row
    achieved = nbytes / (ms_per_step * 1e-3) / 1e9
    top_k = w.params.get("top_k", 40)
    k_eff = V if (top_k == 0 or top_k > V) else top_k
    # the launch's dominant kernel: batches of >= 256 rows (kRowLoopRows in zi_sample.hip) run one
    # workgroup per row; a whole-vocabulary nucleus with min_p > 0 runs the min-p prefix kernel there
    if gdev is not None:
        kernel = "pruned_kernel"
    elif rows >= 256:
        kernel = "prefix_kernel" if (k_eff > 256 and w.params.get("min_p", 0.05) > 0) else "row_kernel"
        if (k_eff > 256 and w.params.get("min_p", 0.05) == 0 and w.bf16 and args.softcap <= 0
                and not w.params.get("xtc_probability", 0)):
            # no prefix settles these rows: row_kernel's top-256 pass, then the sort-free whole-order
            # pass, which takes most of the call (achieved is over the whole call)
            kernel = "whole_kernel"
    else:
        kernel = "nucleus_kernel" if k_eff > 256 else "sample_kernel"
    traffic = read_traffic(args.traffic, kernel, w.name)

    # sanity: every replayed batch reproduces the eager result of its set
    ref = SampleResult(tok=torch.empty(rows, dtype=torch.int32, device=dev),
                       margin=torch.empty(rows, dtype=torch.float32, device=dev),
                       ndraws=torch.empty(rows, dtype=torch.int32, device=dev))
    ctx.sample_rows(p, sets[0], uni, vocab=V, hist=hist, hist_len=hist_len, mask=mask, out=ref, groups=gdev,
                    group_count=cdev)
    torch.cuda.synchronize()
    assert torch.equal(ref.tok, outs[0].tok) and torch.equal(ref.margin, outs[0].margin), "replay differs from eager"

    cpu = None
    if args.cpu_seconds > 0:
        from oracle import pyoracle

        op = pyoracle.params(**{k: v for k, v in w.params.items()})
        n_rows_cpu = min(rows, 64)
        L = np.ascontiguousarray(w.logits[:n_rows_cpu])
        t1, tok1, _ = pyoracle.bench_sample_rows(op, L, w.hist[:n_rows_cpu] if w.hist is not None else None,
                                                w.hist_len[:n_rows_cpu] if w.hist is not None else None,
                                                w.mask[:n_rows_cpu] if w.mask is not None else None,
                                                w.uniforms[:n_rows_cpu], 1)
        creps = max(1, int(args.cpu_seconds / max(t1, 1e-6)))
        tc, tokc, _ = pyoracle.bench_sample_rows(op, L, w.hist[:n_rows_cpu] if w.hist is not None else None,
                                                w.hist_len[:n_rows_cpu] if w.hist is not None else None,
                                                w.mask[:n_rows_cpu] if w.mask is not None else None,
                                                w.uniforms[:n_rows_cpu], creps)
        gtok = ref.tok.cpu().numpy().astype(np.uint32)[:n_rows_cpu]
        cpu = {"value": round(n_rows_cpu * creps / tc, 1), "unit": "rows/s", "cores": 1, "kind": "port",
               "sample": f"{n_rows_cpu} rows of the same batch x {creps} passes ({tc:.1f} s), oracle/oracle.c "
                         f"(C restatement of src/sampler.zig:91-276), -O3, 1 thread",
               "tokens_match_gpu": bool(np.array_equal(gtok, tokc)),
               # the north star's count of chosen-token disagreements (top-p boundary or other) on the
               # rows both sides sampled; the kernels are bit-exact, so any nonzero count is a bug
               "id_mismatches": int(np.count_nonzero(gtok != tokc)), "rows_compared": int(n_rows_cpu)}
        # the same sample with rows spread over the host's cores (the reference sampler is
        # single-threaded; this is the planned second leg): one thread per core, each passing
        # over its own slice of the rows; ctypes releases the GIL during the oracle call
        from concurrent.futures import ThreadPoolExecutor

        nth = min(host_threads(), n_rows_cpu)
        bounds = np.linspace(0, n_rows_cpu, nth + 1).astype(int)
        creps_all = max(1, creps * nth // 2)  # about half the 1-core leg's time at full scaling

        def part(i):
            a, b = bounds[i], bounds[i + 1]
            return pyoracle.bench_sample_rows(op, np.ascontiguousarray(L[a:b]),
                                              w.hist[a:b] if w.hist is not None else None,
                                              w.hist_len[a:b] if w.hist is not None else None,
                                              w.mask[a:b] if w.mask is not None else None, w.uniforms[a:b],
                                              creps_all)

        with ThreadPoolExecutor(nth) as ex:
            tw0 = time.perf_counter()
            res = list(ex.map(part, range(nth)))
            tw = time.perf_counter() - tw0
        tok_all = np.concatenate([r[1] for r in res]).astype(np.uint32)
        cpu["all_cores"] = {"value": round(n_rows_cpu * creps_all / tw, 1), "unit": "rows/s", "cores": nth,
                            "cpu_model": cpu_model(),
                            "sample": f"{n_rows_cpu} rows x {creps_all} passes over {nth} threads ({tw:.1f} s)",
                            "tokens_match_gpu": bool(np.array_equal(gtok, tok_all))}

    out = {
        "metric": METRIC,
        "value": round(rows_per_s, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": wsteps,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if w.bf16 else "f32",
        "data": "synthetic, seeded (zinfer_amd/workloads.py): " + w.name,
        "config": {"workload": w.name, "rows": rows, "vocab": V, **{k: v for k, v in w.params.items()},
                   "rotating_input_sets": nsets, "input_bytes_cycled": nsets * per_set,
                   "launch": "eager" if args.no_graph else "hip_graph_replay"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "algorithmic_bytes_per_launch": nbytes, "kernel": kernel},
        "cpu_baseline": cpu,
        "wall_s": round(wall, 3),
    }
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
