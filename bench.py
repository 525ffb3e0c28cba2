#!/usr/bin/env python3
"""Decoded tokens/s of the integer SpiralCore/FBS decode path on one MI355X.

Workload (BASELINE.json's metric: batch 1,024 at width 256): the width-256 artifact of config 3
(64 quaternions, 6 layers, mlp 384, vocab 32,768, window 16, 256 Zipf-sized drawers probing 8,
max 512 members, int32 Q16.16 residual, int64 Q32 state, i16 Q12 writer table), 1,024
independent sequences, Zipf(1.1) prompts of 1,024 tokens, 1,024 greedy decode steps.

Protocol (the reference's fbs-toks, crates/uor-r4-integer/src/bin/fbs-toks.rs:1510-1533): the
prompt is prefilled once (untimed setup; its last choice starts the reply), then each timed
step decodes `gen` greedy tokens for the whole batch from that prefilled state, each step
feeding back the previous choice. value = batch x gen / step time. Inputs and state are
resident in HBM before the timed region; the step is one launch of the decode kernel, timed by
HIP events on its stream.

The same line carries the roofline of that kernel (algorithmic bytes per token x tokens per
launch / launch time, against MI355X's 8 TB/s) and the CPU baseline: the oracle (a C
restatement of the reference's step, one sequence per thread) timed on this host over a
bounded sample of the same decode, whose replies must equal the GPU's.

Beside the metric, `drawer_index` measures the 256-cell CSR drawer index (uor_fbs_index_*):
builds at C5's vocabulary and at --index-large tokens (checked against torch's stable sort),
single-token updates, batched probes (checked against the full scan), and the reference's
single-query protocol with its published RTX 5090 medians beside ours.
"""

from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import re
import sys
import time
from dataclasses import replace

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "uor-r4_amd"), os.path.join(ROOT, "oracle")]

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
# Measured HBM bytes per launch of each config's timed kernel (rocprofv3 FETCH_SIZE and WRITE_SIZE
# passes, scaled by a copy kernel's reading), for the workload each summary names.
TRAFFIC_SUMMARIES = {
    "c2": "fbs_decode_pair_c2_b1024_traffic.md", "c3": "fbs_decode_pair_c3_b1024_traffic.md",
    "c4": "fbs_rows_pair_c4_r1048576_traffic.md", "c5": "fbs_decode_pair8_c5_b16384_traffic.md",
    "hamming": "fbs_decode_pair_ham_c3_b1024_traffic.md"}
D11_TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "d11_score_rows_m1_traffic.md")
# BASELINE.json's configs at their full shapes: (sequences, prompt, decode steps); c4 is
# teacher-forced scoring of (rows, row length).
# Query bytes a candidate-statistics replay may move (the whole batch at C2/C3).
REPLAY_BYTES = 6 << 30
CONFIG_SHAPES = {"c1": (1, 256, 256), "c2": (1024, 512, 512), "c3": (1024, 1024, 1024),
                 "c4": (1 << 20, 128, 0), "c5": (16384, 4096, 4096)}
# The Hamming reads in the served step (--config hamming): C3's artifact with a typed stream read
# after layer 3 and a typed readout read, 8 heads (4 copy, 4 type) keeping 16 positions each;
# (sequences, prompt, decode steps) as C3.
HAMMING_READS = dict(heads=8, depths=(3, 6), kept=16)
HAMMING_SHAPE = (1024, 1024, 1024)
# The discrete M1 panel scorer (uor_d11_score_rows): the reference's ft/dev panel size, the M1
# container's shape (vocabulary 4,096, 4 blocks, context 192, 8 kept cells, relation read
# keeping 8 with 1 sweep, 19-table trunk), rows of 186-192 tokens (the published run's mean
# context is 34,625,934 / 183,206 = 189 tokens per row).
D11_ROWS = 14287
D11_PUBLISHED = {
    "value": 183206, "unit": "response tokens/s", "context_tokens_per_s": 34625934,
    "hardware": "1x RTX 5090 (compute_120)", "rows": 14287,
    "timing": "wall time of DeviceScorer::score (device.rs:120-210): host-to-device copies of "
              "the rows, scratch allocation, launches and device-to-host copies of the records",
    "source": "docs/loop/tasks/m1-close-saved-model/antigravity-110/REPORT.md:32, STATE.md:43"}


def log(msg: str):
    """A progress line on stderr (stdout carries only the JSON line)."""
    print(f"bench.py: {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it, with the family, model and stepping numbers,
    clock and cache the first processor reports (a VM's model name can be as short as
    "AMD EPYC")."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            if not line.strip():
                break  # the first processor's block
            k, _, v = line.partition(":")
            info[k.strip()] = v.strip()
    except OSError:
        return "unknown"
    name = info.get("model name", "unknown")
    extra = [f"{k} {info[k]}" for k in ("cpu family", "model", "stepping") if k in info]
    if "cpu MHz" in info:
        extra.append(f"{float(info['cpu MHz']):.0f} MHz")
    if "cache size" in info:
        extra.append(f"cache {info['cache size']}")
    return f"{name} ({', '.join(extra)})" if extra else name


def cpu_threads(a) -> tuple[int, dict]:
    """Threads for the CPU baseline and what they are: every core this process may run on
    (its affinity), capped at the CPU share the GPU box grants one GPU, which it states in
    OMP_NUM_THREADS (16 there); --cpu-threads overrides."""
    affinity = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    share = int(omp) if omp and omp.isdigit() and int(omp) > 0 else affinity
    threads = a.cpu_threads or max(1, min(affinity, share))
    return threads, {"affinity_cores": affinity, "cpu_count": os.cpu_count(),
                     "omp_num_threads": omp, "cpu_model": cpu_model()}


def cpu_protocol(run, units: int, runs: int, warmup: int = 1, same=None) -> dict:
    """The reference's CPU timing protocol (src/bin/fbs-toks.rs:1513-1610): `warmup` untimed
    runs, then `runs` timed ones that must all give the same result; integer nanoseconds, the
    median (integer mean of the middle two for an even count), the nearest-rank p95, and
    integer units per second at each. Returns the summary and the first timed result."""
    for _ in range(warmup):
        run()
    raw, first = [], None
    for _ in range(runs):
        t0 = time.perf_counter_ns()
        r = run()
        raw.append(time.perf_counter_ns() - t0)
        if first is None:
            first = r
        elif same is not None and not same(first, r):
            raise RuntimeError("timed CPU runs gave different results")
    srt = sorted(raw)
    n = len(srt)
    med = srt[n // 2] if n % 2 else (srt[n // 2 - 1] + srt[n // 2]) // 2
    p95 = srt[max(1, -(-n * 95 // 100)) - 1]
    per_s = lambda ns: units * 1_000_000_000 // max(ns, 1)  # noqa: E731
    return {"warmup_runs": warmup, "timed_runs": runs, "units_per_run": units, "raw_ns": raw,
            "median_ns": med, "p95_ns": p95, "median_per_s": per_s(med),
            "p95_per_s": per_s(p95)}, first


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=3)
    p.add_argument("--warmup", type=int, default=1)
    p.add_argument("--config", default="c3",
                   choices=sorted(CONFIG_SHAPES) + ["m1", "copy", "hamming"],
                   help="BASELINE's configs: c3 (default) is the metric's; c4 scores rows")
    p.add_argument("--batch", type=int, default=None, help="sequences (c4: rows); config's default")
    p.add_argument("--prompt", type=int, default=None, help="prompt tokens (c4: row length)")
    p.add_argument("--gen", type=int, default=None, help="decode steps per timed step")
    p.add_argument("--seed", type=int, default=2026120203)
    p.add_argument("--cpu-seconds", type=float, default=24.0, help="target CPU-baseline sample time")
    p.add_argument("--cpu-threads", type=int, default=0,
                   help="0: the host cores this process may run on, capped at the CPU share the "
                        "box grants one GPU (OMP_NUM_THREADS where set)")
    p.add_argument("--cpu-runs", type=int, default=20,
                   help="timed CPU-baseline runs after one warm-up (fbs-toks' protocol)")
    p.add_argument("--no-writer-memory-pass", action="store_true",
                   help="skip the extra timed pass with the writer's memory of its last query off")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-parts", action="store_true",
                   help="skip the part clocks' launch (the step's phases in cycles, after the "
                        "timed launches)")
    p.add_argument("--serve-steps", type=int, default=64,
                   help="serving-loop launches after the decode (0: none); reported beside the metric")
    p.add_argument("--no-index", action="store_true",
                   help="skip the CSR drawer index measurements (build, update, probe)")
    p.add_argument("--index-large", type=int, default=1 << 24,
                   help="tokens of the large index build (width 32)")
    p.add_argument("--copy-probe-mib", type=int, default=0,
                   help="only run one elementwise copy kernel over this many MiB (the reference "
                        "reading for the FETCH_SIZE / WRITE_SIZE counters) and exit")
    p.add_argument("--d11-trunk-entries", type=int, default=600_000,
                   help="m1: (key, token) entries in each of the six trunk tables it reads")
    a = p.parse_args()
    batch, prompt, gen = CONFIG_SHAPES.get(a.config, (D11_ROWS, 192, 0) if a.config == "m1"
                                           else HAMMING_SHAPE if a.config == "hamming"
                                           else (4096, 1024, 0))
    a.batch = batch if a.batch is None else a.batch
    a.prompt = prompt if a.prompt is None else a.prompt
    a.gen = gen if a.gen is None else a.gen
    return a


def copy_probe(mib: int):
    """One elementwise kernel that reads and writes mib MiB each (y = ~x over int32)."""
    import torch

    n = mib * (1 << 20) // 4
    x = torch.arange(n, dtype=torch.int32, device="cuda:0")
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    torch.bitwise_not(x, out=y)
    torch.cuda.synchronize()
    assert int(y[-1]) == ~(n - 1)
    print(json.dumps({"copy_probe": {"read_bytes": n * 4, "write_bytes": n * 4,
                                     "kernel": "bitwise_not int32"}}))


def workload_key(a) -> str:
    return f"{a.config} batch {a.batch} prompt {a.prompt} gen {a.gen} seed {a.seed}"


def measured_traffic(a, kernel):
    """HBM bytes per timed launch from the config's committed counter summary, if it covers this
    exact workload and kernel; None otherwise."""
    try:
        text = open(os.path.join(ROOT, "profiles", TRAFFIC_SUMMARIES[a.config])).read()
    except (KeyError, OSError):
        return None
    w = re.search(r"^workload: (.+)$", text, re.M)
    k = re.search(r"^kernel: (.+)$", text, re.M)
    t = re.search(r"^traffic_bytes_per_launch: (\d+)$", text, re.M)
    if not w or not k or not t or w.group(1).strip() != workload_key(a) or k.group(1).strip() != kernel:
        return None
    return int(t.group(1))


def algorithmic_bytes_per_token(spec, mean_candidates: float) -> float:
    """Bytes one decoded token moves by the path's definition: its input row, the window read
    and the new history row per layer, the scored candidate rows, the token id. Shared model
    tables and on-chip state are excluded."""
    c = 1 if spec.table == "i8" else 2
    d, L, W = spec.width, spec.layers, spec.window
    return c * d + L * (W * d * 4 + d * 4) + c * d * mean_candidates + 4


# Bytes one token moves in an index build by the path's definition: its two 8-value endpoint
# blocks read, its cell written and read back by the scatter, its member entry written.
INDEX_BUILD_BYTES_PER_TOKEN = 64 + 4 + 4 + 4
# Measured HBM bytes of one 16,777,216-token build (rocprofv3 FETCH_SIZE and WRITE_SIZE passes).
INDEX_TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "fbs_index_build_16m_traffic.md")
# The reference's published single-card kernel medians (RTX 5090, 120 launches per operation
# over V in {64, 256, 1024, 4096} x K in {1, 8, 16}, one query each;
# projects/uor-cuda-inverted-file/RESULTS.md).
INDEX_REFERENCE_MS = {"probe": 0.160144, "full_scan": 0.109856}


def index_section(torch, dev, stream, sp, large: int) -> dict:
    """The CSR drawer index on the device: builds (at C5's vocabulary and at `large` tokens),
    single-token updates, batched probes, and the reference's single-query protocol. Results
    are checked on the device against torch's stable sort and against the full scan."""
    from uor_fbs import hip
    from uor_fbs import index as ix

    L = hip.lib()
    roots = torch.from_numpy(ix.CODEBOOK).to(dev)
    out: dict = {"build": [], "probe": []}

    def ptr(t):
        return C.c_void_p(t.data_ptr())

    def check(code):
        if code:
            raise hip.FbsError(code, L.uor_fbs_last_error().decode())

    def timed(fn, reps, warm=2):
        for _ in range(warm):
            fn()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(reps)]
        for s_, e_ in ev:
            s_.record(stream)
            fn()
            e_.record(stream)
        torch.cuda.synchronize()
        return [s_.elapsed_time(e_) for s_, e_ in ev]

    def random_table(count, seed):
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        t = torch.randint(-(1 << 31), (1 << 31) - 1, (count, 32), dtype=torch.int32, device=dev,
                          generator=g)
        cells = torch.randint(0, 256, (count,), device=dev, generator=g)
        t[:, :8] = roots[cells // 16]
        t[:, 24:] = roots[cells % 16]
        return t, cells

    class Buffers:
        def __init__(self, count):
            z = lambda n: torch.zeros(n, dtype=torch.int32, device=dev)  # noqa: E731
            self.count = count
            self.off, self.mem, self.cells, self.absent = z(257), z(count), z(count), z(1)
            self.ws = z(int(L.uor_fbs_index_workspace_bytes(count)) // 4)
            self.status = z(1)

        def build(self, table):
            check(L.uor_fbs_index_build_async(ptr(table), self.count, 32, ptr(roots), 0,
                                              ptr(self.off), ptr(self.mem), ptr(self.cells),
                                              ptr(self.absent), ptr(self.ws), ptr(self.status), sp))

        def update(self, table, moved):
            check(L.uor_fbs_index_update_async(ptr(table), self.count, 32, ptr(roots), moved,
                                               ptr(self.off), ptr(self.mem), ptr(self.cells),
                                               ptr(self.absent), ptr(self.ws), ptr(self.status),
                                               sp))

    def same_as_sort(b, cells):
        order = torch.sort(cells, stable=True).indices.to(torch.int32)
        offsets = torch.zeros(257, dtype=torch.int64, device=dev)
        offsets[1:] = torch.cumsum(torch.bincount(cells, minlength=256), 0)
        return (int(b.status.item()) == 0 and bool(torch.equal(b.mem, order))
                and bool(torch.equal(b.cells.long(), cells))
                and bool(torch.equal(b.off.long(), offsets)) and int(b.absent.item()) == 0)

    keep = {}
    for count in (65536, large):
        table, cells = random_table(count, count)
        b = Buffers(count)
        ms = timed(lambda: b.build(table), reps=10)
        ok = same_as_sort(b, cells)
        achieved = INDEX_BUILD_BYTES_PER_TOKEN * count / (np.mean(ms) / 1e3) / 1e9
        traffic = None
        if count == 1 << 24 and os.path.exists(INDEX_TRAFFIC_SUMMARY):
            m = re.search(r"^traffic_bytes_per_launch: (\d+)$", open(INDEX_TRAFFIC_SUMMARY).read(),
                          re.M)
            traffic = int(m.group(1)) if m else None
        out["build"].append({
            "tokens": count, "width": 32, "ms": round(float(np.mean(ms)), 4),
            "tokens_per_s": round(count / (np.mean(ms) / 1e3), 1), "equal_stable_sort": ok,
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                         "traffic": traffic, "bytes_per_token": INDEX_BUILD_BYTES_PER_TOKEN}})
        if count == 65536:
            keep["c5"] = (table, cells, b)
        del table, cells
    # Updates at C5's vocabulary: 64 tokens move to other cells, one call each (the row edit is
    # the caller's and stays outside the timing); the result must equal a fresh build.
    table, cells, b = keep["c5"]
    rng = np.random.default_rng(5)
    upd_ms = []
    for _ in range(64):
        moved, c = int(rng.integers(0, 65536)), int(rng.integers(0, 256))
        table[moved, :8], table[moved, 24:] = roots[c // 16], roots[c % 16]
        cells[moved] = c
        upd_ms += timed(lambda: b.update(table, moved), reps=1, warm=0)
        assert int(b.status.item()) == 0, "index update failed"
    out["update"] = {"tokens": 65536, "moves": 64, "ms_per_update": round(float(np.mean(upd_ms)), 4),
                     "launches_per_update": 4, "equal_fresh_build": same_as_sort(b, cells)}
    # Batched probes: 65,536 query rows (root endpoints, random middles) against tables of the
    # reference's size and of C5's vocabulary.
    rows = 65536
    queries, _ = random_table(rows, 77)
    z = lambda n: torch.zeros(n, dtype=torch.int32, device=dev)  # noqa: E731
    pred, adm, top, st = z(rows), z(rows * 16), z(rows * 8), z(rows)
    for count in (4096, 65536):
        if count == 65536:
            tb, bb = table, b
        else:
            tb, _ = random_table(count, 4096)
            bb = Buffers(count)
            bb.build(tb)
        for k in (8, 16):
            def probe():
                check(L.uor_fbs_index_probe_async(ptr(tb), count, 32, ptr(roots), ptr(queries),
                                                  rows, k, ptr(bb.off), ptr(bb.mem), ptr(pred),
                                                  ptr(adm), ptr(top), ptr(st), sp))
            ms = timed(probe, reps=10)
            ok = int(st.abs().sum().item()) == 0
            # Cross-check: the full scan (every token of the table) on the first 512 rows.
            n = 512
            fp, fa, ft, fs = z(n), z(n * 16), z(n * 8), z(n)
            check(L.uor_fbs_index_full_scan_async(ptr(tb), count, 32, ptr(roots), ptr(queries), n,
                                                  k, ptr(bb.off), ptr(fp), ptr(fa), ptr(ft),
                                                  ptr(fs), sp))
            torch.cuda.synchronize()
            ok = ok and bool(torch.equal(ft, top[:n * 8])) and bool(torch.equal(fa, adm[:n * 16]))
            out["probe"].append({"tokens": count, "k": k, "rows": rows,
                                 "ms_per_launch": round(float(np.mean(ms)), 4),
                                 "rows_per_s": round(rows / (np.mean(ms) / 1e3), 1),
                                 "equal_full_scan_first_512": ok})
    # For the CPU leg: the C5 table, its index and the last probe's (k 16) first 64 rows.
    keep["probe_check"] = (queries[:64].cpu().numpy(), table.cpu().numpy(),
                           [b.off.cpu().numpy(), b.mem.cpu().numpy(), b.cells.cpu().numpy()],
                           top[:64 * 8].cpu().numpy().reshape(64, 8))
    # The reference's protocol: one query (its query_at(7)) per launch on its seeded tables.
    single = {"probe": [], "full_scan": []}
    q1 = torch.from_numpy(ix.seeded_query(7)).to(dev)
    o1 = [z(1), z(16), z(8), z(1)]
    for count in (64, 256, 1024, 4096):
        tb = torch.from_numpy(ix.seeded_table(count)).to(dev)
        bb = Buffers(count)
        bb.build(tb)
        for k in (1, 8, 16):
            single["probe"] += timed(lambda: check(L.uor_fbs_index_probe_async(
                ptr(tb), count, 32, ptr(roots), ptr(q1), 1, k, ptr(bb.off), ptr(bb.mem),
                *[ptr(x) for x in o1], sp)), reps=10, warm=3)
            single["full_scan"] += timed(lambda: check(L.uor_fbs_index_full_scan_async(
                ptr(tb), count, 32, ptr(roots), ptr(q1), 1, k, ptr(bb.off),
                *[ptr(x) for x in o1], sp)), reps=10, warm=3)
    out["single_query_ms"] = {
        op: {"median": round(float(np.median(v)), 5), "launches": len(v),
             "reference_rtx5090_median": INDEX_REFERENCE_MS[op]} for op, v in single.items()}
    out["single_query_protocol"] = ("one query (query_at(7)) per launch on the reference tests' "
                                    "seeded tables, V in {64, 256, 1024, 4096} x K in {1, 8, 16}, "
                                    "3 warm-up + 10 timed launches each, HIP events")
    out["_keep"] = keep
    return out


def score_main(a, torch, oracle, art, model, rows, dev, stream, sp) -> dict:
    """C4: teacher-forced scoring of `batch` rows of `prompt` tokens; a step is one score launch
    over every row (each position's choice compared with the next token, the matches summed)."""
    from uor_fbs import hip
    L = hip.lib()
    spec = art.spec
    R, n = a.batch, a.prompt
    d_rows = torch.from_numpy(np.ascontiguousarray(rows, np.uint32).view(np.int32)).to(dev)
    matches = torch.zeros(1, dtype=torch.int64, device=dev)
    status = torch.zeros(R, dtype=torch.int32, device=dev)

    def step():
        matches.zero_()
        code = L.uor_fbs_score_async(model.handle, C.c_void_p(d_rows.data_ptr()), R, n, None,
                                     C.c_void_p(matches.data_ptr()),
                                     C.c_void_p(status.data_ptr()), sp)
        if code:
            raise hip.FbsError(code, L.uor_fbs_last_error().decode())

    log(f"c4: scoring {R} rows x {n}")
    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(a.steps)]
    t0 = time.perf_counter()
    for s_, e_ in ev:
        s_.record(stream)
        step()
        e_.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    assert int(status.abs().sum()) == 0, "scoring failed"
    launch_ms = [s_.elapsed_time(e_) for s_, e_ in ev]
    ms_per_step = wall * 1e3 / a.steps
    positions = R * n
    sample = min(R, 64)
    _, kept, _ = model.sequences(rows[:sample])
    cand = art.drawer_sizes()[kept.astype(np.int64)].sum(-1)
    mean_cand = float(cand.mean())
    bpt = algorithmic_bytes_per_token(spec, mean_cand) + 4  # plus each position's input id
    achieved = bpt * positions / (float(np.mean(launch_ms)) / 1e3) / 1e9
    S = 1
    while S < spec.width // 32:
        S *= 2
    family = "fbs_rows_pair" if model.block_waves(R) == 2 else "fbs_rows"
    if spec.table == "i8":  # the int8 table's own kernels (fbs_rows_pair8, fbs_rows_8)
        family += "8" if family.endswith("pair") else "_8"
    out = {
        "metric": f"teacher-forced scored positions/sec, {R} rows x {n}, width {spec.width} (1 GPU)",
        "value": round(positions / (ms_per_step / 1e3), 1), "unit": "positions/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int64",
        "data": "synthetic (seeded integer artifact and Zipf rows)",
        "config": {"workload": f"c4 artifact: {R} Zipf(1.1) rows of {n} tokens scored per timed "
                               f"step", "key": workload_key(a), "width": spec.width,
                   "layers": spec.layers, "vocab": spec.vocab, "window": spec.window,
                   "drawers": art.drawers, "probes": art.probes, "rows": R, "row_length": n,
                   "parallelism": "none (1 GPU)"},
        "matches": int(matches.item()),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(a, f"{family}<{(spec.width // 4 + 63) // 64}, {S}>"),
                     "bytes_per_position": round(bpt, 1), "mean_candidate_rows": round(mean_cand, 1),
                     "kernel": f"{family}<{(spec.width // 4 + 63) // 64}, {S}>",
                     "launch_ms": [round(x, 3) for x in launch_ms]},
    }
    if not a.no_cpu:
        log("c4: CPU baseline")
        threads, host = cpu_threads(a)
        t0 = time.perf_counter()
        oracle.score(art, rows[:threads], threads=threads)
        per_row = (time.perf_counter() - t0) / threads
        per_run = a.cpu_seconds / (a.cpu_runs + 1)
        n_cpu = int(min(R, max(threads, per_run / per_row)))
        n_cpu -= n_cpu % threads if n_cpu > threads else 0

        def cpu_run():
            st_, m_, arg_ = oracle.score(art, rows[:n_cpu], threads=threads)
            assert st_ == 0
            return m_, arg_

        proto, (cpu_matches, cpu_argmin) = cpu_protocol(
            cpu_run, n_cpu * n, a.cpu_runs,
            same=lambda x, y: x[0] == y[0] and np.array_equal(x[1], y[1]))
        gpu_matches, gpu_argmin = model.score(rows[:n_cpu])
        same = cpu_matches == gpu_matches and np.array_equal(cpu_argmin, gpu_argmin)
        out["cpu_baseline"] = {
            "value": proto["median_per_s"], "unit": "positions/s",
            "cores": min(threads, n_cpu), **host, "kind": "port",
            "sample": f"the first {n_cpu} of the {R} rows per run, oracle C restatement, one row "
                      f"per thread; value = integer median over {a.cpu_runs} timed runs after "
                      f"one warm-up", "p95_positions_per_s": proto["p95_per_s"],
            "protocol": proto, "choices_equal_gpu": bool(same)}
        if not same:
            print("bench.py: CPU scoring differs from the GPU's", file=sys.stderr)
    return out


def d11_main(a, torch, oracle) -> dict:
    """The discrete M1 panel: a step is one uor_d11_score_rows launch over every row (each row's
    read, admitted cells, top 8, hinges and losses)."""
    from uor_fbs import d11
    L = d11.lib()
    art = d11.synthetic(seed=a.seed, trunk_entries=a.d11_trunk_entries)
    R = a.batch
    pre, lens, tg = d11.panel_rows(art, R, a.seed + 1, min_len=186)
    ctx = art.shape.context
    model = d11.IntegerDiscreteModel(art)
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    sp = C.c_void_p(stream.cuda_stream)
    d_pre = torch.from_numpy(pre.view(np.int32)).to(dev)
    d_len = torch.from_numpy(lens).to(dev)
    d_tg = torch.from_numpy(tg.view(np.int32)).to(dev)
    d_out = torch.zeros(R * d11.ROW_DTYPE.itemsize, dtype=torch.uint8, device=dev)
    log(f"m1: {R} rows, {int(lens.sum())} context tokens, trunk tables of "
        f"{a.d11_trunk_entries} entries")

    def step():
        code = L.uor_d11_score_rows_async(model.handle, C.c_void_p(d_pre.data_ptr()),
                                          C.c_void_p(d_len.data_ptr()),
                                          C.c_void_p(d_tg.data_ptr()), R, ctx,
                                          C.c_void_p(d_out.data_ptr()), sp)
        if code:
            raise d11.DiscreteError(L.uor_d11_last_error().decode())

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(a.steps)]
    t0 = time.perf_counter()
    for s_, e_ in ev:
        s_.record(stream)
        step()
        e_.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    launch_ms = [s_.elapsed_time(e_) for s_, e_ in ev]
    recs = d_out.cpu().numpy().view(d11.ROW_DTYPE)
    assert (recs["status"] == 0).all(), "rows failed"
    ms_per_step = wall * 1e3 / a.steps
    # The reference's timing includes the host copies: the same over host buffers.
    host_ms = []
    for _ in range(3):
        t0 = time.perf_counter()
        host = model.score_rows(pre, lens, tg)
        host_ms.append((time.perf_counter() - t0) * 1e3)
    assert np.array_equal(host.view(np.uint32), recs.view(np.uint32)), "host path differs"
    host_best = min(host_ms)
    bytes_per_row = 4 * float(lens.mean()) + 8 + d11.ROW_DTYPE.itemsize
    traffic = None  # the committed counter summary, for the workload it was measured on
    if (R, a.d11_trunk_entries, a.seed) == (D11_ROWS, 600_000, 2026120203) and \
            os.path.exists(D11_TRAFFIC_SUMMARY):
        m = re.search(r"traffic_bytes_per_launch:\s*(\d+)", open(D11_TRAFFIC_SUMMARY).read())
        traffic = int(m.group(1)) if m else None
    achieved = bytes_per_row * R / (float(np.mean(launch_ms)) / 1e3) / 1e9
    ctx_tokens = int(lens.sum())
    out = {
        "metric": f"scored response tokens/sec, discrete M1 panel of {R} rows (1 GPU)",
        "value": round(R / (ms_per_step / 1e3), 1), "unit": "response tokens/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int32",
        "data": "synthetic (seeded discrete container of the M1 shape, uniform rows)",
        "config": {"workload": f"m1: {R} (prefix, target) rows of 186-192 tokens scored per timed "
                               "step", "vocabulary": art.shape.vocabulary,
                   "blocks": art.shape.blocks, "context": ctx, "kept_cells": art.shape.kept_cells,
                   "read": f"{art.shape.read_mode} kept {art.shape.read_kept} sweeps "
                           f"{art.shape.read_sweeps}", "trunk_entries_per_table": a.d11_trunk_entries,
                   "parallelism": "none (1 GPU)"},
        "context_tokens_per_s": round(ctx_tokens / (ms_per_step / 1e3), 1),
        "host_inclusive": {"ms": round(host_best, 3), "response_tokens_per_s": round(R / (host_best / 1e3), 1),
                           "what": "uor_d11_score_rows over host buffers: allocation, copies to "
                                   "and from the device, the launch"},
        "reference_published": D11_PUBLISHED,
        "vs_published_host_inclusive": round(R / (host_best / 1e3) / D11_PUBLISHED["value"], 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": traffic,
                     "bytes_per_row": round(bytes_per_row, 1), "kernel": "d11_score_rows",
                     "launch_ms": [round(x, 3) for x in launch_ms]},
    }
    if not a.no_cpu:
        threads, host = cpu_threads(a)
        cpu_model_ = oracle.D11Oracle(art)  # loaded once, as the reference's from_bytes
        n_cal = threads * 8
        t0 = time.perf_counter()
        cpu_model_.score_rows(pre[:n_cal], lens[:n_cal], tg[:n_cal], threads=threads)
        per_row = (time.perf_counter() - t0) / n_cal
        n_cpu = int(min(R, max(threads, a.cpu_seconds / (a.cpu_runs + 1) / per_row)))
        proto, cpu = cpu_protocol(
            lambda: cpu_model_.score_rows(pre[:n_cpu], lens[:n_cpu], tg[:n_cpu], threads=threads),
            n_cpu, a.cpu_runs, same=lambda x, y: np.array_equal(x.view(np.uint32), y.view(np.uint32)))
        cpu_model_.close()
        same = np.array_equal(cpu.view(np.uint32), recs[:n_cpu].view(np.uint32))
        out["cpu_baseline"] = {
            "value": proto["median_per_s"], "unit": "response tokens/s",
            "cores": min(threads, n_cpu), **host, "kind": "port",
            "sample": f"the first {n_cpu} of the {R} rows per run, oracle C restatement, one row "
                      f"per thread; value = integer median over {a.cpu_runs} timed runs after "
                      f"one warm-up", "p95_response_tokens_per_s": proto["p95_per_s"],
            "protocol": proto, "records_equal_gpu": bool(same)}
        if not same:
            print("bench.py: CPU records differ from the GPU's", file=sys.stderr)
    model.close()
    return out


def copy_main(a, torch, oracle) -> dict:
    """The copy heads' Hamming read: a step is one uor_copy_mean_rows launch reading the last row
    of every stream (C3's width and vocabulary, 4 copy heads keeping 16 positions each)."""
    from uor_fbs import copy as cp
    L = cp.lib()
    heads = cp.synthetic(seed=a.seed)
    R, n = a.batch, a.prompt
    rng = np.random.default_rng(a.seed + 1)
    tok = rng.integers(0, heads.codes.shape[0], (R, n)).astype(np.uint32)
    lens = np.full(R, n, np.int32)
    gpu = cp.CopyHeads(heads)
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    sp = C.c_void_p(stream.cuda_stream)
    d_tok = torch.from_numpy(tok.view(np.int32)).to(dev)
    d_len = torch.from_numpy(lens).to(dev)
    d_out = torch.zeros((R, heads.table.shape[1]), dtype=torch.int64, device=dev)
    d_found = torch.zeros(R, dtype=torch.uint8, device=dev)
    log(f"copy: {R} streams of {n} tokens")

    def step():
        code = L.uor_copy_mean_rows_async(gpu.handle, C.c_void_p(d_tok.data_ptr()),
                                          C.c_void_p(d_len.data_ptr()), None, R, n,
                                          C.c_void_p(d_out.data_ptr()),
                                          C.c_void_p(d_found.data_ptr()), None, sp)
        if code:
            raise cp.CopyError(L.uor_copy_last_error().decode())

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(a.steps)]
    t0 = time.perf_counter()
    for s_, e_ in ev:
        s_.record(stream)
        step()
        e_.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    launch_ms = [s_.elapsed_time(e_) for s_, e_ in ev]
    ms_per_step = wall * 1e3 / a.steps
    copy, kept, width = heads.codes.shape[1], heads.kept, heads.table.shape[1]
    bytes_per_read = 4 * n + copy * kept * width * 2 + width * 8 + 1
    achieved = bytes_per_read * R / (float(np.mean(launch_ms)) / 1e3) / 1e9
    out = {
        "metric": f"copy-head reads/sec, {R} streams of {n} tokens, width {width} (1 GPU)",
        "value": round(R / (ms_per_step / 1e3), 1), "unit": "reads/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int64",
        "data": "synthetic (random 64-bit head codes, uniform streams)",
        "config": {"workload": f"copy: the read at the last row of {R} streams of {n} tokens",
                   "vocab": int(heads.codes.shape[0]), "width": width, "copy_heads": copy,
                   "kept": kept, "rule": heads.rule, "parallelism": "none (1 GPU)"},
        "context_tokens_per_s": round(R * n / (ms_per_step / 1e3), 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "bytes_per_read": bytes_per_read, "kernel": "copy_mean_rows",
                     "launch_ms": [round(x, 3) for x in launch_ms]},
    }
    got_out = d_out.cpu().numpy()
    got_found = d_found.cpu().numpy().astype(bool)
    if not a.no_cpu:
        _, host = cpu_threads(a)
        t0 = time.perf_counter()
        oracle.copy_mean_rows(heads, tok[:8], lens[:8])
        per = (time.perf_counter() - t0) / 8
        n_cpu = int(min(R, max(8, a.cpu_seconds / (a.cpu_runs + 1) / per)))
        proto, (w_out, w_found, _) = cpu_protocol(
            lambda: oracle.copy_mean_rows(heads, tok[:n_cpu], lens[:n_cpu]), n_cpu, a.cpu_runs,
            same=lambda x, y: np.array_equal(x[0], y[0]) and np.array_equal(x[1], y[1]))
        same = np.array_equal(w_out, got_out[:n_cpu]) and np.array_equal(w_found, got_found[:n_cpu])
        out["cpu_baseline"] = {"value": proto["median_per_s"], "unit": "reads/s",
                               "cores": 1, **host, "kind": "port",
                               "sample": f"the first {n_cpu} of the {R} streams per run, oracle "
                                         f"C restatement on one thread (it has no threaded form); "
                                         f"value = integer median over {a.cpu_runs} timed runs "
                                         f"after one warm-up", "protocol": proto,
                               "reads_equal_gpu": bool(same)}
    gpu.close()
    return out


def hamming_bytes_per_token(spec, ham, mean_candidates: float, t_mean: float) -> dict:
    """HBM bytes one decoded token moves with the Hamming reads, by definition: the base path's
    (algorithmic_bytes_per_token) plus, per read, the kept positions' table rows (copy heads,
    2 B a channel) and payloads (type heads, 8 B a channel: read, and this row's written), and
    the session's token ids (4 B a position). The key codes of the earlier positions are
    gathered from a per-read table of vocab x heads words that stays in the L2 caches (2 MiB at
    C3): counted apart, as `code_bytes`."""
    d, copy, types, kept = spec.width, ham.heads // 2, ham.heads - ham.heads // 2, ham.kept
    reads = len(ham.depths)
    per_read = copy * kept * d * 2 + types * kept * d * 8 + d * 8 + 4 * t_mean
    return {"base": algorithmic_bytes_per_token(spec, mean_candidates),
            "reads": reads * per_read, "code_bytes": reads * ham.heads * 8 * t_mean}


def hamming_main(a, torch, oracle) -> dict:
    """The Hamming reads inside the served step: C3's artifact with HAMMING_READS; a step is
    `gen` greedy steps of every sequence resumed from its prefilled session (state, window ring,
    token stream and payload caches; uor_fbs_decode_stream_async with the payloads updated in
    place)."""
    from uor_fbs import hip, synth
    spec = replace(synth.CONFIGS["c3"], context=a.prompt + a.gen + 1,
                   hamming=synth.HammingSpec(**HAMMING_READS))
    art = synth.make_artifact(spec, a.seed)
    prompts = synth.zipf_prompts(spec.vocab, a.batch, a.prompt, a.seed + 1)
    model = hip.Model(art, device=0)
    L = hip.lib()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    sp = C.c_void_p(stream.cuda_stream)
    B, G = a.batch, a.gen
    ptr = lambda t: None if t is None else C.c_void_p(t.data_ptr())  # noqa: E731

    def check(code):
        if code:
            raise hip.FbsError(code, L.uor_fbs_last_error().decode())

    d_prompts = torch.from_numpy(prompts.view(np.int32)).to(dev)
    state = torch.zeros((B, model.state_words), dtype=torch.int64, device=dev)
    hist = torch.zeros((B, model.history_words), dtype=torch.int32, device=dev)
    pos = torch.zeros(B, dtype=torch.int32, device=dev)
    tok = torch.zeros((B, model.stream_words), dtype=torch.int32, device=dev)
    pay = torch.zeros((B, model.payload_words), dtype=torch.int64, device=dev)
    first = torch.zeros((B, 1), dtype=torch.int32, device=dev)
    status = torch.zeros(B, dtype=torch.int32, device=dev)
    log(f"hamming: {B} sequences, payload caches {pay.numel() * 8 / 2**30:.1f} GiB")
    t0 = time.perf_counter()
    check(L.uor_fbs_decode_stream_async(model.handle, ptr(d_prompts), B, a.prompt, 0, ptr(first),
                                        None, None, None, None, None, ptr(state), ptr(hist),
                                        ptr(pos), ptr(tok), ptr(pay), ptr(status), sp))
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    assert int(status.abs().sum()) == 0, "prefill failed"
    log(f"hamming: prefill {prefill_s:.1f} s")
    reply = torch.zeros((B, G), dtype=torch.int32, device=dev)

    def step():
        check(L.uor_fbs_decode_stream_async(model.handle, ptr(first), B, 1, G - 1, ptr(reply),
                                            ptr(state), ptr(hist), ptr(pos), ptr(tok), ptr(pay),
                                            None, None, None, None, ptr(pay), ptr(status), sp))

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(a.steps)]
    t0 = time.perf_counter()
    for s_, e_ in ev:
        s_.record(stream)
        step()
        e_.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    assert int(status.abs().sum()) == 0, "decode failed"
    launch_ms = [s_.elapsed_time(e_) for s_, e_ in ev]
    ms_per_step = wall * 1e3 / a.steps
    tokens = B * G
    # Candidate rows per token from a teacher-forced replay of evenly spaced sequences.
    host_reply = reply.cpu().numpy().view(np.uint32)
    host_first = first.cpu().numpy().view(np.uint32)
    ids = np.linspace(0, B - 1, min(B, 64)).astype(np.int64)
    replay = np.concatenate([prompts[ids], host_first[ids], host_reply[ids, :-1]], axis=1)
    _, kept, _ = model.sequences(replay, want_query=False)
    mean_cand = float(art.drawer_sizes()[kept[:, a.prompt:, :].astype(np.int64)].sum(-1).mean())
    bpt = hamming_bytes_per_token(spec, spec.hamming, mean_cand, a.prompt + G / 2)
    total = bpt["base"] + bpt["reads"]
    achieved = total * tokens / (float(np.mean(launch_ms)) / 1e3) / 1e9
    Q = (spec.width // 4 + 63) // 64
    Sw = 1
    while Sw < spec.width // 32:
        Sw *= 2
    ham_kernel = ("fbs_decode_pair_ham" if model.block_waves(B) == 2 else "fbs_decode_ham") + f"<{Q}, {Sw}>"
    out = {
        "metric": f"decoded tokens/sec at batch {B}, width {spec.width}, with Hamming reads (1 GPU)",
        "value": round(tokens / (ms_per_step / 1e3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int64",
        "data": "synthetic (seeded integer artifact and Hamming reads, Zipf prompts)",
        "config": {"workload": f"hamming: c3 artifact with reads {HAMMING_READS} at batch {B}: "
                               f"prefilled {a.prompt}-token prompts, {G} greedy decode steps per "
                               "timed step", "key": workload_key(a), "batch": B,
                   "prompt": a.prompt, "gen": G, "width": spec.width, "layers": spec.layers,
                   "vocab": spec.vocab, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(a, ham_kernel),
                     "bytes_per_token": {k: round(v, 1) for k, v in bpt.items()},
                     "mean_candidate_rows": round(mean_cand, 1),
                     "kernel": ham_kernel,
                     "launch_ms": [round(x, 3) for x in launch_ms]},
        "prefill_tokens_per_s": round(B * a.prompt / prefill_s, 1),
    }
    if not a.no_cpu:
        _, host = cpu_threads(a)
        n_cpu = 2
        t0 = time.perf_counter()
        want = oracle.decode(art, prompts[:n_cpu], 8, threads=1)
        per_tok = (time.perf_counter() - t0) / (n_cpu * (a.prompt + 8))
        proto, w = cpu_protocol(lambda: oracle.decode(art, prompts[:n_cpu], 8, threads=n_cpu),
                                n_cpu * (a.prompt + 8), min(a.cpu_runs, 3),
                                same=lambda x, y: np.array_equal(x["reply"], y["reply"]))
        same = np.array_equal(w["reply"][:, 1:], host_reply[:n_cpu, :8]) and \
            np.array_equal(w["reply"][:, :1], host_first[:n_cpu])
        out["cpu_baseline"] = {"value": proto["median_per_s"], "unit": "tokens/s",
                               "cores": n_cpu, **host, "kind": "port",
                               "sample": f"{n_cpu} sequences: the prompt and 8 decode steps, oracle "
                                         f"C restatement on {n_cpu} threads; value = integer median "
                                         f"over {min(a.cpu_runs, 3)} timed runs after one warm-up "
                                         f"({per_tok * 1e3:.2f} ms a token on one thread)",
                               "protocol": proto, "tokens_equal_gpu": bool(same)}
    return out


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py: this path runs on one GPU; --gpus {a.gpus} is not supported "
              "(sequences are independent: shard the batch across GPUs, see DESIGN.md)",
              file=sys.stderr)
        sys.exit(2)
    if a.copy_probe_mib:
        copy_probe(a.copy_probe_mib)
        return
    import torch

    import oracle
    from uor_fbs import hip, synth

    if a.config == "m1":
        print(json.dumps(d11_main(a, torch, oracle)))
        return
    if a.config == "copy":
        print(json.dumps(copy_main(a, torch, oracle)))
        return
    if a.config == "hamming":
        print(json.dumps(hamming_main(a, torch, oracle)))
        return
    spec = replace(synth.CONFIGS[a.config], context=a.prompt + a.gen + 1)
    art = synth.make_artifact(spec, a.seed)
    if spec.zipf_drawers:
        prompts = synth.zipf_prompts(spec.vocab, a.batch, a.prompt, a.seed + 1)
    else:
        prompts = synth.uniform_prompts(spec.vocab, a.batch, a.prompt, a.seed + 1)
    model = hip.Model(art, device=0)
    log(f"{a.config}: artifact and inputs ready")
    L = hip.lib()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    sp = C.c_void_p(stream.cuda_stream)
    if a.config == "c4":
        print(json.dumps(score_main(a, torch, oracle, art, model, prompts, dev, stream, sp)))
        return
    B, G = a.batch, a.gen
    sw, hw = model.state_words, model.history_words

    def ptr(t):
        return C.c_void_p(t.data_ptr()) if t is not None else None

    def u32(arr):
        return torch.from_numpy(np.ascontiguousarray(arr, np.uint32).view(np.int32)).to(dev)

    d_prompts = u32(prompts)
    state = torch.zeros((B, sw), dtype=torch.int64, device=dev)
    hist = torch.zeros((B, hw), dtype=torch.int32, device=dev)
    pos = torch.zeros(B, dtype=torch.int32, device=dev)
    first = torch.zeros((B, 1), dtype=torch.int32, device=dev)
    status = torch.zeros(B, dtype=torch.int32, device=dev)

    def check(code):
        if code:
            raise hip.FbsError(code, L.uor_fbs_last_error().decode())

    # Prefill (setup): the whole prompt, its last choice is the reply's first token.
    t0 = time.perf_counter()
    check(L.uor_fbs_decode_async(model.handle, ptr(d_prompts), B, a.prompt, 0, ptr(first), None,
                                 None, None, ptr(state), ptr(hist), ptr(pos), ptr(status), sp))
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    assert int(status.abs().sum()) == 0, "prefill failed"
    log(f"{a.config}: prefill {prefill_s:.1f} s")

    reply = torch.zeros((B, G), dtype=torch.int32, device=dev)

    def step():
        # `gen` greedy steps: the first feeds the prefill's choice, each later one the last.
        check(L.uor_fbs_decode_async(model.handle, ptr(first), B, 1, G - 1, ptr(reply), ptr(state),
                                     ptr(hist), ptr(pos), None, None, None, ptr(status), sp))

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(a.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(a.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(a.steps):
        starts[i].record(stream)
        step()
        ends[i].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    assert int(status.abs().sum()) == 0, "decode failed"
    log(f"{a.config}: {a.steps} timed steps, {wall:.1f} s")
    launch_ms = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    ms_per_step = wall * 1e3 / a.steps
    tokens = B * G
    value = tokens / (ms_per_step / 1e3)

    # Candidate rows per decoded token, exactly, from a teacher-forced replay of the decoded
    # sequences (every one, unless their queries would exceed REPLAY_BYTES: then evenly spaced
    # ones): the prompt, the prefill's choice, then the reply; the replay reproduces the
    # decode's states, queries and kept drawers at positions prompt .. .
    host_reply = reply.cpu().numpy().view(np.uint32)
    host_first = first.cpu().numpy().view(np.uint32)
    per_seq = (a.prompt + G) * spec.width * 4
    n_rep = int(min(B, max(1, REPLAY_BYTES // per_seq)))
    rep_ids = np.linspace(0, B - 1, n_rep).astype(np.int64) if n_rep < B else np.arange(B)
    sizes = art.drawer_sizes()
    cand_sum = scanned_sum = reused_n = 0
    chunk = max(1, min(256, (1 << 29) // per_seq))
    for c0 in range(0, n_rep, chunk):
        ids = rep_ids[c0:c0 + chunk]
        replay = np.concatenate([prompts[ids], host_first[ids], host_reply[ids, :-1]], axis=1)
        _, kept, query = model.sequences(replay)
        cand = sizes[kept[:, a.prompt:, :].astype(np.int64)].sum(-1)
        # The writer takes its previous result when a query repeats its last run's exactly (a
        # sequence settled on a fixed point): those tokens scan no candidate rows. Each launch
        # starts with nothing remembered, so the first generated token always scans.
        q = query[:, a.prompt:]
        reused = np.zeros(q.shape[:2], dtype=bool)
        reused[:, 1:] = (q[:, 1:] == q[:, :-1]).all(-1)
        cand_sum += int(cand.sum())
        scanned_sum += int(np.where(reused, 0, cand).sum())
        reused_n += int(reused.sum())
        del kept, query, q
    n_tok = n_rep * G
    mean_cand = cand_sum / n_tok
    scanned_cand = scanned_sum / n_tok
    bpt = algorithmic_bytes_per_token(spec, mean_cand)
    mean_launch_s = float(np.mean(launch_ms)) / 1e3
    achieved = bpt * tokens / mean_launch_s / 1e9
    bpt_scanned = algorithmic_bytes_per_token(spec, scanned_cand)
    achieved_scanned = bpt_scanned * tokens / mean_launch_s / 1e9

    # The same launches with the writer's memory of its last query off: every decoded token
    # then scans its candidates, so every token moves the algorithmic bytes.
    no_memory = None
    if not a.no_writer_memory_pass:
        os.environ["UOR_FBS_WRITER_MEMORY"] = "0"
        try:
            model_nm = hip.Model(art, device=0)
        finally:
            del os.environ["UOR_FBS_WRITER_MEMORY"]
        reply_nm = torch.zeros_like(reply)

        def step_nm():
            check(L.uor_fbs_decode_async(model_nm.handle, ptr(first), B, 1, G - 1, ptr(reply_nm),
                                         ptr(state), ptr(hist), ptr(pos), None, None, None,
                                         ptr(status), sp))

        step_nm()
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(a.steps)]
        t0 = time.perf_counter()
        for s_, e_ in ev:
            s_.record(stream)
            step_nm()
            e_.record(stream)
        torch.cuda.synchronize()
        wall_nm = time.perf_counter() - t0
        assert int(status.abs().sum()) == 0, "decode without the writer memory failed"
        ms_nm = [s_.elapsed_time(e_) for s_, e_ in ev]
        mean_nm = float(np.mean(ms_nm)) / 1e3
        no_memory = {
            "value": round(tokens / (wall_nm / a.steps), 1),
            "ms_per_step": round(wall_nm * 1e3 / a.steps, 3),
            "frac": round(bpt * tokens / mean_nm / 1e9 / HBM_PEAK_GBS, 4),
            "launch_ms": [round(x, 3) for x in ms_nm],
            "replies_equal": bool(torch.equal(reply_nm, reply)),
            "what": "UOR_FBS_WRITER_MEMORY=0 at model creation: no step takes the writer's "
                    "previous result",
        }
        del model_nm
    S = 1
    while S < spec.width // 32:
        S *= 2
    family = "fbs_decode_pair" if model.block_waves(B) == 2 else "fbs_decode"
    if spec.table == "i8":  # the int8 table's own kernels (fbs_decode_pair8, fbs_decode_8)
        family += "8" if family.endswith("pair") else "_8"
    kernel = f"{family}<{(spec.width // 4 + 63) // 64}, {S}>"
    traffic = measured_traffic(a, kernel)

    out = {
        "metric": f"decoded tokens/sec at batch {B}, width {spec.width} (1 GPU)",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int64",
        "data": "synthetic (seeded integer artifact and Zipf prompts)",
        "config": {
            "workload": f"{a.config} artifact at batch {B}: prefilled {a.prompt}-token prompts, "
                        f"{G} greedy decode steps per timed step", "key": workload_key(a),
            "width": spec.width, "layers": spec.layers, "mlp": spec.mlp, "vocab": spec.vocab,
            "window": spec.window, "drawers": art.drawers, "probes": art.probes,
            "table": spec.table, "batch": B, "prompt": a.prompt, "gen": G,
            "parallelism": "none (1 GPU)",
        },
        # achieved/frac charge each decoded token the bytes it moves: a token that takes the
        # writer's remembered result scans no candidate rows. The figure that charges every
        # token its kept drawers' rows is beside it (_full_scan), and the launch with the
        # memory off in without_writer_memory.
        "roofline": {
            "bound": "hbm", "achieved": round(achieved_scanned, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved_scanned / HBM_PEAK_GBS, 4), "traffic": traffic,
            "algorithmic_bytes_per_launch": round(bpt_scanned * tokens),
            "bytes_per_token": round(bpt_scanned, 1),
            "scanned_candidate_rows": round(scanned_cand, 1),
            "writer_reuse_fraction": round(reused_n / n_tok, 4),
            "bytes_per_token_full_scan": round(bpt, 1), "mean_candidate_rows": round(mean_cand, 1),
            "achieved_full_scan": round(achieved, 1),
            "frac_full_scan": round(achieved / HBM_PEAK_GBS, 4),
            "replay_sequences": n_rep,
            "without_writer_memory": no_memory,
            "kernel": kernel, "launch_ms": [round(x, 3) for x in launch_ms],
        },
        "prefill_tokens_per_s": round(B * a.prompt / prefill_s, 1),
    }
    if B == 1:  # a latency: one sequence (the config's CPU-runnable case)
        out["ms_per_token"] = round(ms_per_step / G, 5)

    if not a.no_parts and model.block_waves(B) == 2:
        # The part clocks (measure_fbs_step_parts): the same launch from the same state on the
        # instrumented kernel, outside the timed region; its replies must equal the decode's.
        names = hip.part_names()
        n_part = len(names)
        parts = torch.zeros((B, 2 * n_part + 2), dtype=torch.int64, device=dev)
        reply_p = torch.zeros_like(reply)
        ev_p = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        ev_p[0].record(stream)
        check(L.uor_fbs_decode_parts_async(model.handle, ptr(first), B, 1, G - 1, ptr(reply_p),
                                           ptr(state), ptr(hist), ptr(pos), None, None, None,
                                           ptr(status), ptr(parts), sp))
        ev_p[1].record(stream)
        torch.cuda.synchronize()
        assert int(status.abs().sum()) == 0, "the part clocks' decode failed"
        raw = parts.cpu().numpy().view(np.uint64)
        steps_run = float(raw[:, 2 * n_part].sum())
        cyc = raw[:, :2 * n_part].reshape(B, 2, n_part).sum(0).astype(np.float64) / steps_run
        total0 = float(cyc[0].sum())
        mhz = float(raw[:, :n_part].sum()) / float(raw[:, 2 * n_part + 1].sum()) * 100.0
        out["parts"] = {
            "what": "cycles per decoded token in each phase of the paired step, wave 0 (the "
                    "recurrence chain) and wave 1 (the window ring), summed over layers; syncN "
                    "is the wait at barrier N; from one launch of the instrumented kernel "
                    "(uor_fbs_decode_parts_async) at this workload",
            "wave0": {n: round(float(c), 1) for n, c in zip(names, cyc[0])},
            "wave1": {n: round(float(c), 1) for n, c in zip(names, cyc[1])},
            "cycles_per_token": round(total0, 1),
            "shader_mhz": round(mhz, 1),
            "launch_ms": round(ev_p[0].elapsed_time(ev_p[1]), 3),
            "replies_equal_decode": bool(torch.equal(reply_p, reply)),
        }

    if a.serve_steps:
        # The serving loop: every sequence is a session in a device slot (a fixed permutation of
        # the slots), and each launch steps all of them by one token from their slot state,
        # updated in place with each slot's serving cache (uor_fbs_serve_slots_async, serve_step
        # for the whole batch; the cache starts empty). From the same prefilled state, its tokens
        # must equal the decode's replies. The same launches without the cache are timed beside.
        K = min(a.serve_steps, G)
        perm = np.random.default_rng(a.seed).permutation(B).astype(np.uint32)
        d_slots = u32(perm)
        s_state, s_hist, s_pos = (torch.empty_like(t) for t in (state, hist, pos))
        s_state[d_slots.long()] = state  # sequence i lives in slot perm[i]
        # A slot's history is its window ring: ring row (p - 1 - r) mod W holds history row r.
        L_, W_, d_ = spec.layers, spec.window, spec.width
        p0 = int(pos[0].item())
        assert bool((pos == p0).all())
        src = torch.from_numpy((p0 - 1 - np.arange(W_)) % W_)
        ring_rows = torch.empty(W_, dtype=torch.int64)
        ring_rows[src] = torch.arange(W_)
        s_hist[d_slots.long()] = hist.view(B, L_, W_, d_)[:, :, ring_rows.to(dev)].reshape(B, -1)
        s_pos[d_slots.long()] = pos
        saved = [t.clone() for t in (s_state, s_hist, s_pos)]
        cache = torch.zeros((B, int(L.uor_fbs_slot_cache_bytes(model.handle))), dtype=torch.uint8,
                            device=dev)

        def serve_loop(cached: bool, handle=model.handle):
            for t, v in zip((s_state, s_hist, s_pos), saved):
                t.copy_(v)
            served = torch.zeros((K + 1, B), dtype=torch.int32, device=dev)
            served[0] = first[:, 0]
            # Each launch's arguments formed before the loop, so that the host enqueues the
            # launches back to back (a caller's serving loop in compiled code issues them with a
            # few microseconds between calls); one event pair brackets the K launches.
            args = [(handle, ptr(d_slots), B, B, ptr(served[k]), 1, 0, ptr(served[k + 1]),
                     ptr(s_state), ptr(s_hist), ptr(s_pos), ptr(cache) if cached else None, None,
                     None, None, None, ptr(status), sp) for k in range(K)]
            fn = L.uor_fbs_serve_slots_async
            ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            ev[0].record(stream)
            for k in range(K):
                check(fn(*args[k]))
            ev[1].record(stream)
            torch.cuda.synchronize()
            wall_ = time.perf_counter() - t0
            assert int(status.abs().sum()) == 0, "serving loop failed"
            same_ = np.array_equal(served[1:].cpu().numpy().view(np.uint32).T, host_reply[:, :K])
            return wall_, [ev[0].elapsed_time(ev[1]) / K], same_

        # The library takes the drawer-major scan for one-token launches where the drawers'
        # sizes are skewed (the largest more than twice the mean).
        sizes_ = art.drawer_sizes()
        drawer_major = (model.block_waves(B) == 2
                        and int(sizes_.max()) * len(sizes_) > 2 * int(sizes_.sum()))
        bare_wall, bare_ms, bare_same = serve_loop(False)
        serve_wall, serve_ms, same_serve = serve_loop(True)
        # The same launches on the path the library did not choose (UOR_FBS_SERVE_SCAN at model
        # creation: the writer inside the step, or the drawer-major scan), for comparison.
        other = None
        if model.block_waves(B) == 2:
            os.environ["UOR_FBS_SERVE_SCAN"] = "fused" if drawer_major else "drawer"
            try:
                model_o = hip.Model(art, device=0)
            finally:
                del os.environ["UOR_FBS_SERVE_SCAN"]
            o_wall, o_ms, o_same = serve_loop(True, model_o.handle)
            other = {"tokens_per_s": round(B * K / o_wall, 1),
                     "ms_per_launch": round(float(np.mean(o_ms)), 4),
                     "tokens_equal_decode": bool(o_same),
                     "what": ("the writer inside the step (one kernel a launch)" if drawer_major
                              else "the drawer-major scan (three kernels a launch)")}
            del model_o
        out["serving"] = {
            "tokens_per_s": round(B * K / serve_wall, 1),
            "ms_per_launch": round(float(np.mean(serve_ms)), 4),
            "launches": K, "sessions": B,
            "kernel": (kernel.replace("fbs_decode", "fbs_prefill") +
                       (" + fbs_serve_scan + fbs_serve_finish" if drawer_major else "")),
            "workload": f"{B} sessions in permuted device slots, one token each per launch, "
                        f"{K} launches from the prefilled state",
            "tokens_equal_decode": bool(same_serve),
            "cache": "each slot's window sums for its next step and the writer's memory, kept "
                     "between launches (empty at the first)",
            "without_cache": {"tokens_per_s": round(B * K / bare_wall, 1),
                              "ms_per_launch": round(float(np.mean(bare_ms)), 4),
                              "tokens_equal_decode": bool(bare_same)},
            "other_path": other,
        }
        if not same_serve:
            print("bench.py: the serving loop's tokens differ from the decode's", file=sys.stderr)

    index = None if a.no_index or a.config != "c3" else index_section(torch, dev, stream, sp,
                                                                          a.index_large)

    if not a.no_cpu:
        log(f"{a.config}: CPU baseline")
        threads, host = cpu_threads(a)
        st_np = state.cpu().numpy()
        hist_np = hist.cpu().numpy()
        pos_np = pos.cpu().numpy().view(np.uint32)
        first_np = first.cpu().numpy().view(np.uint32)
        # Calibrate: a small run, then a sample sized so that a warm-up and --cpu-runs timed
        # runs take about --cpu-seconds: sequences (one per thread at a time) for as many
        # leading decode steps as that allows, fewer sequences where two steps of all are long.
        n_cal, g_cal = min(B, threads), min(G, 4)
        t0 = time.perf_counter()
        oracle.decode(art, first_np[:n_cal], g_cal - 1, threads=threads, in_state=st_np[:n_cal],
                      in_history=hist_np[:n_cal], in_position=pos_np[:n_cal], want_state=False)
        per_tok = (time.perf_counter() - t0) / (n_cal * g_cal)
        per_run = a.cpu_seconds / (a.cpu_runs + 1)
        n_cpu = B if B < threads else (B // threads) * threads
        g_cpu = int(min(G, max(2, per_run / per_tok / n_cpu)))
        if n_cpu > threads and n_cpu * g_cpu * per_tok > 1.5 * per_run:
            n_cpu = max(threads, int(per_run / per_tok / g_cpu) // threads * threads)

        def cpu_run():
            r = oracle.decode(art, first_np[:n_cpu], g_cpu - 1, threads=threads,
                              in_state=st_np[:n_cpu], in_history=hist_np[:n_cpu],
                              in_position=pos_np[:n_cpu], want_state=False)
            assert r["status"] == 0
            return r["reply"]

        proto, cpu_reply = cpu_protocol(cpu_run, n_cpu * g_cpu, a.cpu_runs,
                                        same=np.array_equal)
        same = np.array_equal(cpu_reply, host_reply[:n_cpu, :g_cpu])
        out["cpu_baseline"] = {
            "value": proto["median_per_s"], "unit": "tokens/s",
            "cores": min(threads, n_cpu), **host, "kind": "port",
            "sample": f"{n_cpu} of the {B} prefilled sequences x the first {g_cpu} decode steps "
                      f"per run, oracle C restatement, one sequence per thread; value = integer "
                      f"median over {a.cpu_runs} timed runs after one warm-up",
            "p95_tokens_per_s": proto["p95_per_s"], "protocol": proto,
            "replies_equal_gpu": bool(same),
        }
        if not same:
            print("bench.py: CPU replies differ from the GPU's", file=sys.stderr)
        if index is not None:
            index["cpu_baseline"] = index_cpu_baseline(oracle, index)
    if index is not None:
        index.pop("_keep", None)
        out["drawer_index"] = index
    print(json.dumps(out))


def index_cpu_baseline(oracle, index) -> dict:
    """The oracle's index build on this host at C5's vocabulary (one thread), timed, and its
    index and probes compared with the device's."""
    from uor_fbs import index as ix
    keep = index["_keep"]
    queries, table, (off, mem, cells), top = keep["probe_check"]
    reps, t0 = 0, time.perf_counter()
    while True:
        st, host = oracle.index_build(table, ix.CODEBOOK)
        reps += 1
        if time.perf_counter() - t0 > 2.0:
            break
    cpu_s = (time.perf_counter() - t0) / reps
    same = (st == 0 and np.array_equal(host.offsets, off.view(np.uint32))
            and np.array_equal(host.members, mem.view(np.uint32))
            and np.array_equal(host.cells, cells.view(np.uint32)))
    probes_same = True
    for r in range(len(queries)):
        pst, _, ptop, _ = oracle.index_probe(table, ix.CODEBOOK, queries[r], 16, host)
        probes_same &= pst == 0 and np.array_equal(ptop, top[r].view(np.uint32))
    return {"build_tokens_per_s": round(len(table) / cpu_s, 1), "cores": 1, "kind": "port",
            "sample": f"oracle build of the {len(table)}-token index x {reps}",
            "index_equal_gpu": bool(same), "probes_equal_gpu_first_64": bool(probes_same)}


if __name__ == "__main__":
    main()
