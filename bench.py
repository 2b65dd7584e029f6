"""Benchmark of the MI355X attention path (one GPU).

Headline workload (the configuration the >= 70 % HBM target is quoted on):
continuous-batching decode, 64 sequences, 32 q / 4 kv heads, head_dim 64,
per-sequence context lengths drawn uniform in [512, 32768] (numpy PCG64,
seed 0), paged f32 KV in 16-token blocks with shuffled block tables in one
shared pool.  A step is one nyion_paged_decode_attention call over the whole
batch (one decode launch).  Inputs are resident in HBM before timing; the
2.2 GB the call reads is far larger than the 256 MB Infinity Cache.

metric/unit: achieved algorithmic HBM bandwidth of the decode call in GB/s
(K + V + q + out + block-table bytes, each counted once), with the call's
microseconds beside it.  The other workloads are measured in the same run
and reported under "configs", keyed by their --only selector: c1
(contiguous 128-position node), c2 (22-layer TinyLlama decode step, ctx
4096; c2t the same through the tracked form), c3h (the headline batch on
binary16 KV), c3q (the headline batch on Q4-20B KV), c4 (4-bit KV, 131072
context, window 4096, cold), c5 (causal
prefill of 8192 tokens with its paged KV write, TFLOP/s against the bf16
MFMA peak), abi (gpu_attention_device without scratch against the node with
its scores buffer), zone (decode over zone-geometry pages against 16-token
block tables), gemv / gemv6 (Q4_K and Q6_K weight GEMV) and pool (paged KV pool
with host spill).

Timing: `ms_per_step` is the wall clock over exactly K calls bracketed by
device synchronisation, after the W warm-up calls; before those, each GPU
workload's set-up runs its call back to back for ~60 ms, untimed, so the
clock has left idle (`settle_calls` reports how many for the headline);
per-call statistics (median, p10, p90) come from
an event pair recorded around each of >= 20 further calls on the launching
stream; `roofline.achieved` divides the algorithmic bytes (or FLOPs) of one
launch by the mean launch duration over back-to-back calls timed with HIP
events on the launching stream, which is what the rocprofv3 kernel-trace
average under profiles/ measures.
cpu_baseline: the C restatement of ops::attention (oracle/, the reference's
AVX-512 dot/axpy order, OpenMP over heads) on the host cores, on a bounded
sample of the headline batch (the first sequences, scaled by attended
tokens), at all host cores and at 6 threads (the reference executor's rayon
pool); every CPU figure is the median over the runs that fit its time budget.
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import threading
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
for sub in ("nyion.rs_amd", "oracle", "tests"):
    sys.path.insert(0, os.path.join(ROOT, sub))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = ("decode-attn µs/layer + achieved HBM GB/s (% peak); prefill TFLOP/s (% MFMA)")
ALL = ("c1", "c2", "c2t", "c3", "c3h", "c3q", "c4", "a5", "c5", "abi", "zone", "gemv", "gemv6",
       "pool")


# The GPU run's own input bytes (copied from HBM after the timed calls) and
# its outputs, per workload: the CPU baselines time the oracle on exactly
# these bytes and report how far the GPU's outputs are from the oracle's.
SAMPLES = {}


def _err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    e = float(np.max(np.abs(got - ref)))
    return {"max_abs_err_vs_gpu": e, "rel_err_vs_gpu": e / max(float(np.max(np.abs(ref))), 1e-30)}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", default="", help="comma list of " + ",".join(ALL) + " (default all but gemv6)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--no-graph", action="store_true",
                    help="GEMV section: issue the launches directly instead of replaying graphs")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run a 512 MiB device copy (PMC traffic calibration)")
    ap.add_argument("--sustain", type=float, default=0.0,
                    help="c5: also run the prefill back to back for this many seconds on the "
                         "workload's inputs and on all-zero inputs, sampling power and clock")
    return ap.parse_args()


# ----------------------------------------------------------------------------
# helpers
# ----------------------------------------------------------------------------

def settle(fn, torch, ms=60.0):
    """Workload set-up, untimed: run the call back to back for about `ms` of
    wall clock so that the GPU's clock has left its idle state before the
    warm-up and timed calls (from idle, the first ~100 calls of the 64-sequence
    batch run about 6 % slower while the clock ramps). Returns the number of
    calls made, which the JSON line reports."""
    n, t0 = 0, time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(8):
            fn(n)
            n += 1
        torch.cuda.synchronize()
    return n


def timed(fn, steps, warmup, torch):
    """W untimed, then K timed; synchronize on both sides; ms per call."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        fn(i)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def event_mean(fn, reps, torch):
    """Mean device time per call (ms): HIP events on the launching stream
    around `reps` back-to-back calls (per-call event pairs would add the
    event records' own cost to every call)."""
    st = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    fn(0)
    torch.cuda.synchronize()
    a.record(st)
    for i in range(reps):
        fn(i)
    b.record(st)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def event_pcts(fn, reps, torch):
    """Per-call device time (ms): an event pair on the launching stream
    around each of `reps` calls; returns p10, median, p90."""
    st = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(reps)]
    fn(0)
    torch.cuda.synchronize()
    for i, (e0, e1) in enumerate(evs):
        e0.record(st)
        fn(i)
        e1.record(st)
    torch.cuda.synchronize()
    p10, p50, p90 = np.percentile([e0.elapsed_time(e1) for e0, e1 in evs], [10, 50, 90])
    return float(p10), float(p50), float(p90)


def _us3(p):
    return [round(x * 1e3, 3) for x in p]


def _profile_value(fname, key, workload):
    """A machine-readable line `key workload value` of a summary under profiles/."""
    try:
        for line in open(os.path.join(ROOT, "profiles", fname)):
            f = line.split()
            if len(f) == 3 and f[0] == key and f[1] == workload:
                return float(f[2])
    except OSError:
        pass
    return None


def pmc_traffic(workload):
    """HBM bytes per launch of the decode kernel for `workload`, from the
    calibrated FETCH_SIZE + WRITE_SIZE passes summarised under profiles/."""
    return _profile_value("decode_hbm_traffic_pmc.txt", "traffic_bytes_per_launch", workload)


def hbm_roofline(nbytes, us, traffic):
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic}


def paged_tables(rng, n_seqs, nblk, total):
    perm = rng.permutation(total).astype(np.int32)
    return perm[: n_seqs * nblk].reshape(n_seqs, nblk)


def _cores():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def _cpu_time(fn, budget_s=2.0, max_calls=2000):
    """Median seconds per call of fn after one warm call, over the calls that
    fit in about budget_s (at least three)."""
    fn()
    times, t0 = [], time.perf_counter()
    while True:
        t1 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t1)
        el = time.perf_counter() - t0
        if (el > budget_s and len(times) >= 3) or len(times) >= max_calls:
            return float(np.median(times)), len(times)


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ----------------------------------------------------------------------------
# continuous batch (headline; selector c3, c3h on binary16 KV)
# ----------------------------------------------------------------------------

C3_HQ, C3_HKV, C3_D, C3_BT = 32, 4, 64, 16


def bench_c3(nh, torch, steps, warmup, seed=0, f16=False, q4=False):
    """64-sequence continuous batch; f16=True stores the same K/V draw as
    binary16 rows (half the bytes), q4=True as Q4-20B rows (40 bytes per
    64-element row, quantised on the device)."""
    import workloads as W

    Hq, Hkv, D, bt = C3_HQ, C3_HKV, C3_D, C3_BT
    lens = W.c3_lengths(seed=seed)
    nblk = (lens + bt - 1) // bt
    total = int(nblk.sum())
    rng = np.random.default_rng(seed)
    perm = rng.permutation(total).astype(np.int32)
    tables = np.zeros((64, int(nblk.max())), np.int32)
    off = 0
    for b in range(64):
        tables[b, : nblk[b]] = perm[off: off + nblk[b]]
        off += nblk[b]
    g = torch.Generator(device="cuda").manual_seed(seed)
    kp = torch.randn((total, Hkv, bt, D), generator=g, device="cuda")
    vp = torch.randn((total, Hkv, bt, D), generator=g, device="cuda")
    if f16:
        kp, vp = kp.half(), vp.half()
    if q4:
        rb = 40
        kq = torch.empty((total, Hkv, bt, rb), dtype=torch.uint8, device="cuda")
        vq = torch.empty_like(kq)
        rows = total * Hkv * bt
        nh.q4_quantize(kp, rows, D, kq)
        nh.q4_quantize(vp, rows, D, vq)
        kp, vp = kq, vq
    q = torch.randn((64, Hq, D), generator=g, device="cuda")
    tab = torch.from_numpy(tables).cuda()
    ctx = torch.from_numpy(lens).cuda()
    out = torch.empty_like(q)
    maxc = int(lens.max())
    ws = nh.alloc_workspace(nh.decode_workspace_size(64, Hq, Hkv, D, maxc))
    kvt = nh.KV_F16 if f16 else nh.KV_Q4_20B if q4 else nh.KV_F32
    call1 = nh.prepare_paged_decode(q, kp, vp, tab, ctx, out, Hq, Hkv, D, bt, maxc, kv_dtype=kvt,
                                    workspace=ws)

    def call(i):
        call1()

    if not f16 and not q4:
        # sequences 0 and 1 as [Hkv][L][D] rows, their q and this call's output
        call1()
        torch.cuda.synchronize()
        smp = {"lens": [int(x) for x in lens[:2]], "q": q[:2].cpu().numpy(),
               "out": out[:2].cpu().numpy(), "k": [], "v": []}
        for b in range(2):
            t = torch.arange(int(lens[b]), device="cuda")
            blk = tab[b].long()[t // bt]
            smp["k"].append(kp[blk, :, t % bt].permute(1, 0, 2).contiguous().cpu().numpy())
            smp["v"].append(vp[blk, :, t % bt].permute(1, 0, 2).contiguous().cpu().numpy())
        SAMPLES["c3"] = smp
    toks = int(lens.sum())
    row_bytes = 40 if q4 else D * (2 if f16 else 4)
    nbytes = 2 * toks * Hkv * row_bytes + int(nblk.sum()) * 4 + 2 * 64 * Hq * D * 4
    n_settle = settle(call, torch)
    ms = timed(call, steps, warmup, torch)
    reps = max(steps, 20)
    us = event_mean(call, reps, torch) * 1e3
    pct = event_pcts(call, reps, torch)
    return {"ms_per_call_wall": ms, "us_per_layer": us, "us_p10_p50_p90": _us3(pct),
            "reps": reps, "bytes": nbytes, "tokens": toks, "settle_calls": n_settle,
            "gbs_wall": nbytes / (ms * 1e-3) / 1e9, "gbs": nbytes / (us * 1e-6) / 1e9,
            "gbs_median": nbytes / (pct[1] * 1e-3) / 1e9,
            "roofline": hbm_roofline(nbytes, us, pmc_traffic("c3h" if f16 else "c3q" if q4 else "c3")),
            "partition_tokens": nh.partition_tokens(64, Hkv, D, maxc)}


def cpu_baseline_c3(seed=0, n_sample=2, budget_s=5.0, sample=None):
    """Oracle on the first n_sample sequences of the 64-sequence batch,
    scaled by attended tokens to the batch; at all host cores and at 6
    threads.  With `sample` (the GPU run's own rows of those sequences) the
    oracle runs on those bytes and its outputs are compared with the GPU's."""
    import oracle
    import workloads as W

    lens = W.c3_lengths(seed=seed)
    if sample is not None:
        q = sample["q"]
        lays = [oracle.contiguous_layout(sample["k"][b], sample["v"][b], int(lens[b]), 64)
                for b in range(n_sample)]
        origin = "the GPU run's own q and K/V rows of those sequences, copied from HBM"
    else:
        pb = W.paged_batch([int(x) for x in lens[:n_sample]], seed=seed)
        q = pb.q
        lays = [pb.layout(b) for b in range(n_sample)]
        origin = "a seeded draw of the same shapes"
    toks_sample, toks_all = int(lens[:n_sample].sum()), int(lens.sum())
    nbytes = 2 * toks_all * 4 * 64 * 4 + int(((lens + 15) // 16).sum()) * 4 + 2 * 64 * 32 * 64 * 4
    res = {}
    for label, thr in (("all", _cores()), ("6", 6)):
        def run():
            return [oracle.attention(q[b], lays[b], int(lens[b]), int(lens[b]) - 1, 32, 4, 64,
                                     threads=thr) for b in range(n_sample)]
        dt, n = _cpu_time(run, budget_s=budget_s)
        res[label] = (thr, n, dt, dt * toks_all / toks_sample)
    thr, n, dt, est = res["all"]
    thr6, n6, dt6, est6 = res["6"]
    out = {"value": round(nbytes / est / 1e9, 3), "unit": "GB/s", "cores": thr, "kind": "port",
           "sample": (f"{n} runs over sequences 0-{n_sample - 1} of the batch ({toks_sample} tokens, "
                      f"{dt * 1e3:.1f} ms per run at {thr} threads; inputs: {origin}), scaled by "
                      f"attended tokens to the batch's {toks_all}: {est * 1e3:.1f} ms per call; at "
                      f"6 threads {est6 * 1e3:.1f} ms ({nbytes / est6 / 1e9:.2f} GB/s)"),
           "us_per_layer": est * 1e6, "us_per_layer_6_threads": est6 * 1e6,
           "cpu_model": _cpu_model()}
    if sample is not None:
        ref = np.stack([o.reshape(32, 64) for o in
                        [oracle.attention(q[b], lays[b], int(lens[b]), int(lens[b]) - 1, 32, 4, 64,
                                          threads=thr) for b in range(n_sample)]])
        out.update(_err(sample["out"], ref))
    return out


# ----------------------------------------------------------------------------
# 22-layer decode step, ctx 4096 (selector c2)
# ----------------------------------------------------------------------------

def bench_c2(nh, torch, steps, warmup, seed=0):
    L, ctx, Hq, Hkv, D, bt = 22, 4096, 32, 4, 64, 16
    R = 3  # rotated copies of the whole 22-layer cache (555 MB > the 256 MB MALL)
    nblk = ctx // bt
    rng = np.random.default_rng(seed)
    g = torch.Generator(device="cuda").manual_seed(seed)
    layers = []
    for r in range(R):
        sets = []
        for layer in range(L):
            kp = torch.randn((nblk, Hkv, bt, D), generator=g, device="cuda")
            vp = torch.randn((nblk, Hkv, bt, D), generator=g, device="cuda")
            tab = torch.from_numpy(paged_tables(rng, 1, nblk, nblk)).cuda()
            q = torch.randn((1, Hq, D), generator=g, device="cuda")
            sets.append((q, kp, vp, tab))
        layers.append(sets)
    ctx_t = torch.full((1,), ctx, dtype=torch.int32, device="cuda")
    outs = [torch.empty((1, Hq, D), device="cuda") for _ in range(L)]
    ws_bytes = nh.decode_workspace_size(1, Hq, Hkv, D, ctx)
    ws = nh.alloc_workspace(ws_bytes)

    # argument marshalling done once per (copy, layer): a step then costs only
    # the C-ABI calls, as it would from the compiled executor
    calls = [[nh.prepare_paged_decode(q, kp, vp, tab, ctx_t, outs[layer], Hq, Hkv, D, bt, ctx,
                                      workspace=ws)
              for layer, (q, kp, vp, tab) in enumerate(layers[r])] for r in range(R)]

    def step(i):
        for c in calls[i % R]:
            c()

    bytes_layer = 2 * ctx * Hkv * D * 4 + nblk * 4 + 2 * Hq * D * 4
    settle(step, torch)
    ms = timed(step, steps, warmup, torch)
    pct_step = event_pcts(step, max(steps, 20), torch)
    # layer 0 of the first copy: its rows in position order, q and output
    calls[0][0]()
    torch.cuda.synchronize()
    q0, kp0, vp0, tab0 = layers[0][0]
    t = torch.arange(ctx, device="cuda")
    blk = tab0[0].long()[t // bt]
    SAMPLES["c2"] = {"q": q0[0].cpu().numpy(), "out": outs[0][0].cpu().numpy(),
                     "k": kp0[blk, :, t % bt].permute(1, 0, 2).contiguous().cpu().numpy(),
                     "v": vp0[blk, :, t % bt].permute(1, 0, 2).contiguous().cpu().numpy()}
    reps = max(steps, 20) * L
    one = lambda i: calls[i % R][i % L]()  # noqa: E731
    us_call = event_mean(one, reps, torch) * 1e3
    pct = event_pcts(one, max(steps, 20) * 3, torch)
    return {
        "ms_per_step": ms,
        "step_ms_p10_p50_p90": [round(x, 4) for x in pct_step],
        "us_per_layer": ms * 1e3 / L,
        "gbs": L * bytes_layer / (ms * 1e-3) / 1e9,
        "bytes_per_layer": bytes_layer,
        "call_us_event_mean": us_call,
        "call_us_p10_p50_p90": _us3(pct),
        "roofline": hbm_roofline(bytes_layer, us_call, pmc_traffic("c2")),
        "partition_tokens": nh.partition_tokens(1, Hkv, D, ctx),
        "workspace_bytes": ws_bytes,
    }


def bench_c2_tracked(nh, torch, steps, seed=0):
    """The 22-layer C2 step through the tracked form (ops::attention_tracked,
    the executor's Full decode call, executor.rs:742-755): per layer the
    decode launch also stores the scores, and a second launch adds
    importance[t] = sum_h p_h[t] in f64.  Replayed from a HIP graph (no host
    overhead), 3 rotated caches as for C2.  Also timed pipelined: layer l's
    launch also runs layer l-1's importance sum on workgroups past its
    decode's (two scores buffers in turn), and one importance launch after
    the last layer -- L + 1 launches instead of 2L, the same results."""
    L, ctx, Hq, Hkv, D, bt = 22, 4096, 32, 4, 64, 16
    R = 3
    nblk = ctx // bt
    rng = np.random.default_rng(seed)
    g = torch.Generator(device="cuda").manual_seed(seed)
    sets = []
    for r in range(R):
        for layer in range(L):
            kp = torch.randn((nblk, Hkv, bt, D), generator=g, device="cuda")
            vp = torch.randn((nblk, Hkv, bt, D), generator=g, device="cuda")
            tab = torch.from_numpy(paged_tables(rng, 1, nblk, nblk)).cuda()
            q = torch.randn((1, Hq, D), generator=g, device="cuda")
            sets.append((q, kp, vp, tab))
    ctx_t = torch.full((1,), ctx, dtype=torch.int32, device="cuda")
    out = torch.empty((1, Hq, D), device="cuda")
    imp = torch.zeros((L, 1, ctx + 2), dtype=torch.float64, device="cuda")
    scores = torch.empty((1, Hq, ctx + 2), dtype=torch.float32, device="cuda")
    ws = nh.alloc_workspace(nh.decode_workspace_size(1, Hq, Hkv, D, ctx))

    def step_of(r, tracked):
        def step():
            for layer in range(L):
                q, kp, vp, tab = sets[r * L + layer]
                if tracked:
                    nh.paged_decode_tracked(q, kp, vp, tab, ctx_t, out, imp[layer], Hq, Hkv, D,
                                            bt, max_ctx=ctx, workspace=ws, scores=scores)
                else:
                    nh.paged_decode(q, kp, vp, tab, ctx_t, out, Hq, Hkv, D, bt, max_ctx=ctx,
                                    workspace=ws)
        return step

    scores2 = [torch.empty((1, Hq, ctx + 2), dtype=torch.float32, device="cuda") for _ in range(2)]

    def step_pipelined(r):
        def step():
            for layer in range(L):
                q, kp, vp, tab = sets[r * L + layer]
                first = layer == 0
                nh.paged_decode_tracked_pipelined(
                    q, kp, vp, tab, ctx_t, out, scores2[layer % 2],
                    None if first else scores2[(layer - 1) % 2], None if first else imp[layer - 1],
                    Hq, Hkv, D, bt, max_ctx=ctx, workspace=ws)
            nh.paged_decode_importance(ctx_t, scores2[(L - 1) % 2], imp[L - 1], Hq, max_ctx=ctx)
        return step

    reps = max(steps // R, 5)
    settle(lambda i: step_of(i % R, True)(), torch)
    us = [_graph_us(torch, step_of(r, True), reps) for r in range(R)]
    us_plain = [_graph_us(torch, step_of(r, False), reps) for r in range(R)]
    us_pipe = [_graph_us(torch, step_pipelined(r), reps) for r in range(R)]
    step_us, plain_us, pipe_us = float(np.mean(us)), float(np.mean(us_plain)), float(np.mean(us_pipe))
    bytes_layer = 2 * ctx * Hkv * D * 4 + nblk * 4 + 2 * Hq * D * 4
    return {"timing": "graph replay" if USE_GRAPHS else "direct launches",
            "ms_per_step": step_us * 1e-3, "us_per_layer": step_us / L,
            "untracked_us_per_layer_same_timing": plain_us / L,
            "tracked_over_untracked": step_us / plain_us,
            "pipelined_us_per_layer": pipe_us / L,
            "pipelined_over_untracked": pipe_us / plain_us,
            "gbs": L * bytes_layer / (step_us * 1e-6) / 1e9, "bytes_per_layer": bytes_layer,
            "score_and_importance_bytes_per_layer": Hq * (ctx + 2) * 4 * 2 + (ctx + 2) * 8 * 2}


def cpu_baseline_c2(seed=0, sample=None):
    """Oracle (C restatement of ops::attention) on one C2 layer at a time;
    with `sample`, on the GPU run's own layer-0 bytes, its outputs compared
    with the GPU's."""
    import oracle
    import workloads as W

    if sample is not None:
        q = sample["q"]
        lay = oracle.contiguous_layout(sample["k"], sample["v"], 4096, 64)
        origin = "the GPU run's own layer-0 q and K/V rows, copied from HBM"
    else:
        pb = W.paged_batch([4096], seed=seed)
        q, lay = pb.q[0], pb.layout(0)
        origin = "a seeded draw of the same shapes"
    bytes_layer = 2 * 4096 * 4 * 64 * 4 + 256 * 4 + 2 * 32 * 64 * 4
    res = {}
    for label, thr in (("6", 6), ("all", _cores())):
        dt, n = _cpu_time(lambda: oracle.attention(q, lay, 4096, 4095, 32, 4, 64, threads=thr),
                          budget_s=3.0)
        res[label] = (thr, n, dt * 1e6)
    thr6, n6, us6 = res["6"]
    thra, na, usa = res["all"]
    out = {"value": bytes_layer / (usa * 1e-6) / 1e9, "unit": "GB/s", "cores": thra, "kind": "port",
           "sample": (f"{na} single-layer decode calls (ctx 4096, 32/4 heads, D=64, f32; inputs: "
                      f"{origin}) at {thra} threads: {usa:.0f} us/layer; at 6 threads {us6:.0f} "
                      f"us/layer"),
           "us_per_layer": usa, "us_per_layer_6_threads": us6}
    if sample is not None:
        ref = oracle.attention(q, lay, 4096, 4095, 32, 4, 64, threads=thra).reshape(32, 64)
        out.update(_err(sample["out"], ref))
    return out


def cpu_baseline_c1():
    """Oracle on the contiguous 128-position node (all host cores)."""
    import oracle
    import workloads as W

    q, k, v = W.c1_contiguous(seed=0)
    lay = oracle.contiguous_layout(k, v, 128, 64)
    thr = _cores()
    dt, n = _cpu_time(lambda: oracle.attention(q.reshape(-1), lay, 128, 127, 32, 4, 64, threads=thr))
    nbytes = 278528
    return {"value": dt * 1e6, "unit": "us/layer", "cores": thr, "kind": "port",
            "gbs": nbytes / dt / 1e9,
            "sample": f"{n} calls of the whole node (32/4 heads, D=64, 128 positions)"}


# ----------------------------------------------------------------------------
# 4-bit KV, ctx 131072, window 4096 (selector c4)
# ----------------------------------------------------------------------------

C4_R = 64  # rotated block tables: 63 other windows (>= 660 MB) are read between two uses of one


def c4_tables(rng, R, B, nblk, w, bt, stride):
    """Block tables of R rotation sets for B sequences of nblk logical blocks:
    the blocks a call attends (the window's w/bt last blocks and, with global
    stride s, the blocks of positions s*g, g < 128) get distinct physical
    blocks per (set, sequence), shuffled within that region; all other
    entries point at the region's first block (never read).  Returns
    ([R][B][nblk] int32, physical blocks)."""
    att = list(range(nblk - w // bt, nblk))
    if stride:
        att = sorted(set(att) | {(stride * g) // bt for g in range(128)})
    na = len(att)
    tabs = np.zeros((R, B, nblk), np.int32)
    for r in range(R):
        for b in range(B):
            base = (r * B + b) * na
            tabs[r, b, :] = base
            tabs[r, b, att] = base + rng.permutation(na)
    return tabs, R * B * na


def bench_c4(nh, torch, steps, warmup, seed=0):
    B, ctx, w, Hq, Hkv, D, bt = 8, 131072, 4096, 32, 4, 64, 16
    nblk = ctx // bt
    rb = 40
    rng = np.random.default_rng(seed)
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn((B, Hq, D), generator=g, device="cuda")
    ctxt = torch.full((B,), ctx, dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    res = {}
    for stride in (0, 64):
        tabs, total = c4_tables(rng, C4_R, B, nblk, w, bt, stride)
        kp = torch.empty((total, Hkv, bt, rb), dtype=torch.uint8, device="cuda")
        vp = torch.empty_like(kp)
        rows = total * Hkv * bt
        chunk = 1 << 22
        for pool in (kp, vp):
            flat = pool.view(-1, rb)
            for s in range(0, rows, chunk):
                n = min(chunk, rows - s)
                x = torch.randn((n, D), generator=g, device="cuda")
                nh.q4_quantize(x, n, D, flat[s: s + n])
        tab = torch.from_numpy(tabs).cuda()
        torch.cuda.synchronize()
        ws = nh.alloc_workspace(nh.decode_workspace_size(B, Hq, Hkv, D, ctx, w, stride))
        calls = [nh.prepare_paged_decode(q, kp, vp, tab[r], ctxt, out, Hq, Hkv, D, bt, ctx,
                                         kv_dtype=nh.KV_Q4_20B, window=w, global_stride=stride,
                                         workspace=ws) for r in range(C4_R)]

        def call(i):
            calls[i % C4_R]()

        n_pos = w + (128 if stride else 0)
        nbytes = 2 * B * n_pos * Hkv * rb + 2 * B * Hq * D * 4 + B * (n_pos // bt + 8) * 4
        settle(call, torch)
        ms = timed(call, max(steps, C4_R), warmup, torch)
        reps = max(steps, 2 * C4_R)
        us = event_mean(call, reps, torch) * 1e3
        pct = event_pcts(call, reps, torch)
        if stride == 0:
            # rotation 0: every sequence's window rows [Hkv][4096][40 B], q and output
            calls[0]()
            torch.cuda.synchronize()
            t = torch.arange(ctx - w, ctx, device="cuda")
            smp = {"q": q.cpu().numpy(), "out": out.cpu().numpy(), "k": [], "v": []}
            for b in range(B):
                blk = tab[0, b].long()[t // bt]
                smp["k"].append(kp[blk, :, t % bt].permute(1, 0, 2).contiguous().cpu().numpy())
                smp["v"].append(vp[blk, :, t % bt].permute(1, 0, 2).contiguous().cpu().numpy())
            SAMPLES["c4"] = smp
        res[f"stride{stride}"] = {
            "us_per_layer": us, "us_per_layer_wall": ms * 1e3, "us_p10_p50_p90": _us3(pct),
            "reps": reps, "bytes_packed": nbytes, "gbs_packed": nbytes / (us * 1e-6) / 1e9,
            "cold": f"{C4_R} rotated block tables over {total} physical blocks "
                    f"({2 * total * Hkv * bt * rb / 1e6:.0f} MB of K+V pools)",
            "roofline": hbm_roofline(nbytes, us, pmc_traffic("c4" if stride == 0 else "c4s64"))}
        del kp, vp, tab, calls, ws
        torch.cuda.empty_cache()
    return res


A5_R = 32  # rotated page-base tables for the attention_sparse_q4 line


def a5_zone_tables(rng, R, B, ctx, w, stride, n_kv_heads, row):
    """Zone page bases of R rotation sets for B sequences (one layer): the
    pages the call attends (the window's and the strided globals') get
    distinct, shuffled places in one pool per (set, sequence); every other
    page is absent (never read).  Returns ([R][B][n_pages] int64, pool bytes,
    attended positions)."""
    ve = ctx - 1
    ws = ve - w + 1 if ve > w else 0
    pos = list(range(ws, ve + 1))
    if stride:
        pos = [stride * g for g in range(min(ws // stride, 128))] + pos

    def page(t):  # cache.rs:593-598 page_id / 235-237 block_size_for
        if t < 4096:
            return t >> 5, 32
        if t < 131072:
            return 128 + ((t - 4096) >> 7), 128
        return 1120 + ((t - 131072) >> 10), 1024

    pages = sorted({page(t) for t in pos})
    n_pages = page(ctx - 1)[0] + 1
    bases = np.full((R, B, n_pages), -1, np.int64)
    off = 0
    for r in range(R):
        for b in range(B):
            for i in rng.permutation(len(pages)):
                p, bs = pages[i]
                bases[r, b, p] = off
                off += n_kv_heads * bs * row
    return bases, off, len(pos)


def bench_a5(nh, torch, steps, warmup, seed=0):
    """ops::attention_sparse_q4 (ops.rs:597-723) on the 4-bit window workload's
    shape: 8 sequences, ctx 131072, window 4096, 32/4 heads, D=64, zone pages
    of Q4-20B rows (one layer), global stride 0 and 64, cold (A5_R rotated
    page tables)."""
    B, ctx, w, Hq, Hkv, D = 8, 131072, 4096, 32, 4, 64
    rb = 40
    rng = np.random.default_rng(seed)
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn((B, Hq, D), generator=g, device="cuda")
    ctxt = torch.full((B,), ctx, dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    res = {}
    for stride in (0, 64):
        bases, nbytes_pool, n_pos = a5_zone_tables(rng, A5_R, B, ctx, w, stride, Hkv, rb)
        kp = torch.empty(nbytes_pool, dtype=torch.uint8, device="cuda")
        vp = torch.empty_like(kp)
        rows = nbytes_pool // rb
        chunk = 1 << 22
        for pool in (kp, vp):
            flat = pool.view(-1, rb)
            for s0 in range(0, rows, chunk):
                n = min(chunk, rows - s0)
                x = torch.randn((n, D), generator=g, device="cuda")
                nh.q4_quantize(x, n, D, flat[s0: s0 + n])
        tab = torch.from_numpy(bases).cuda()
        torch.cuda.synchronize()
        calls = [nh.prepare_attention_sparse_q4(q, kp, vp, tab[r], 1, 0, ctxt, out, Hq, Hkv, D, w,
                                                stride, ctx) for r in range(A5_R)]

        def call(i):
            calls[i % A5_R]()

        nbytes = 2 * B * n_pos * Hkv * rb + 2 * B * Hq * D * 4
        settle(call, torch)
        ms = timed(call, max(steps, A5_R), warmup, torch)
        reps = max(steps, 2 * A5_R)
        us = event_mean(call, reps, torch) * 1e3
        pct = event_pcts(call, reps, torch)
        res[f"stride{stride}"] = {
            "us_per_layer": us, "us_per_layer_wall": ms * 1e3, "us_p10_p50_p90": _us3(pct),
            "reps": reps, "positions": n_pos, "bytes_packed": nbytes,
            "gbs_packed": nbytes / (us * 1e-6) / 1e9,
            "cold": f"{A5_R} rotated page tables over {2 * nbytes_pool / 1e6:.0f} MB of K+V pools",
            "roofline": hbm_roofline(nbytes, us, pmc_traffic("a5" if stride == 0 else "a5s64"))}
        del kp, vp, tab, calls
        torch.cuda.empty_cache()
    return res


def cpu_baseline_a5(seed=0):
    """The oracle's attention_sparse_q4 (ops.rs:597-723) on all 8 sequences of
    the 4-bit window workload (window 4096, global stride 0), rows quantised."""
    import oracle

    B, ctx, w, hkv, hd = 8, 131072, 4096, 4, 64
    rng = np.random.default_rng(seed)
    rb = oracle.q4_row_bytes(hd)
    pos = oracle.sparse_positions(ctx, ctx - 1, w, 0)
    lo = int(pos[0])
    # rows [lo, ctx) of each sequence, contiguous per kv head; earlier rows are never read
    ks = [oracle.q4_quantize_rows(rng.standard_normal((hkv * (ctx - lo), hd), dtype=np.float32))
          for _ in range(B)]
    vs = [oracle.q4_quantize_rows(rng.standard_normal((hkv * (ctx - lo), hd), dtype=np.float32))
          for _ in range(B)]
    q = rng.standard_normal((B, 32, hd), dtype=np.float32)
    lays = []
    for b in range(B):
        k = ks[b].reshape(hkv, ctx - lo, rb)
        v = vs[b].reshape(hkv, ctx - lo, rb)
        # a layout whose row of position t is row t - lo of the arrays
        lay = oracle.contiguous_layout(np.ascontiguousarray(k), np.ascontiguousarray(v), ctx - lo,
                                       hd, oracle.KV_Q4)
        lay.k_base -= lo * rb
        lay.v_base -= lo * rb
        lays.append(lay)
    thr = _cores()

    def run():
        for b in range(B):
            oracle.attention_sparse_q4(q[b], lays[b], ctx, ctx - 1, 32, hkv, hd, w, 0, threads=thr)

    dt, n = _cpu_time(run)
    nbytes = 2 * B * len(pos) * hkv * rb
    return {"value": dt * 1e6, "unit": "us/layer", "cores": thr, "kind": "port",
            "gbs_packed": nbytes / dt / 1e9,
            "sample": f"{n} runs of all 8 sequences, window 4096, global stride 0"}


def cpu_baseline_c4(seed=0, sample=None):
    """Oracle on the 4-bit window workload: 8 sequences, ctx 131072, window
    4096 (the attended rows, Q4-20B).  With `sample` (the GPU run's own
    window rows, in position order) the oracle runs on those bytes, its
    outputs compared with the GPU's."""
    import oracle
    import workloads as W

    B, ctx, w, bt, hkv, hd = 8, 131072, 4096, 16, 4, 64
    rb = oracle.q4_row_bytes(hd)
    if sample is not None:
        # the window's rows only: positions ctx-w .. ctx-1 are rows 0 .. w-1
        q = sample["q"]
        lays = [oracle.contiguous_layout(sample["k"][b], sample["v"][b], w, hd, oracle.KV_Q4)
                for b in range(B)]
        pos = np.arange(w, dtype=np.int32)
        origin = "the GPU run's own q and window rows, copied from HBM"
    else:
        rng = np.random.default_rng(seed)
        nblk = ctx // bt
        tables = rng.permutation(B * nblk).astype(np.int32).reshape(B, nblk)
        kp = np.zeros((B * nblk, hkv, bt, rb), np.uint8)
        vp = np.zeros_like(kp)
        pos = oracle.sparse_positions(ctx, ctx - 1, w, 0)
        for b in range(B):
            blk = tables[b, pos // bt]
            kp[blk, :, pos % bt] = oracle.q4_quantize_rows(
                rng.standard_normal((len(pos), hkv, hd), dtype=np.float32))
            vp[blk, :, pos % bt] = oracle.q4_quantize_rows(
                rng.standard_normal((len(pos), hkv, hd), dtype=np.float32))
        q = rng.standard_normal((B, 32, hd), dtype=np.float32)
        pb = W.PagedBatch(q, kp, vp, tables, np.full(B, ctx, np.int32), 32, hkv, hd, bt,
                          oracle.KV_Q4, seed)
        lays = [pb.layout(b) for b in range(B)]
        origin = "a seeded draw of the same shapes"
    thr = _cores()

    def run():
        return [oracle.attention_positions(q[b], lays[b], pos, 32, hkv, hd, threads=thr)
                for b in range(B)]

    dt, n = _cpu_time(run)
    nbytes = 2 * B * len(pos) * hkv * rb
    out = {"value": dt * 1e6, "unit": "us/layer", "cores": thr, "kind": "port",
           "gbs_packed": nbytes / dt / 1e9,
           "sample": f"{n} runs of all 8 sequences, window 4096, global stride 0 (inputs: {origin})"}
    if sample is not None:
        out.update(_err(sample["out"], np.stack([o.reshape(32, hd) for o in run()])))
    return out


# ----------------------------------------------------------------------------
# causal prefill, 8192 tokens (selector c5)
# ----------------------------------------------------------------------------

def bench_c5(nh, torch, steps, warmup, seed=0):
    n, Hq, Hkv, D, bt = 8192, 32, 8, 128, 16
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn((n, Hq, D), generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn((n, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((n, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
    out = torch.empty((n, Hq, D), device="cuda")
    nblk = n // bt
    tab = torch.from_numpy(np.random.default_rng(seed).permutation(nblk).astype(np.int32)).cuda()
    kp = torch.empty((nblk, Hkv, bt, D), device="cuda")
    vp = torch.empty_like(kp)
    flops = 4 * Hq * D * n * (n + 1) / 2

    def attn(i):  # the prefill alone (the kernel also checks V's binary16 range)
        nh.prefill_bf16(q, k, v, out, Hq, Hkv, D)

    def attn_kv(i):  # the configuration's work: prefill plus the paged KV write of the chunk
        nh.prefill_bf16(q, k, v, out, Hq, Hkv, D, k_pool=kp, v_pool=vp, block_table=tab,
                        block_tokens=bt)

    # the same chunk written into Q4-20B pools (the quantising write is its own
    # launch after the attention kernel)
    rbq = 4 * D // 32 * 5
    kq = torch.empty((nblk, Hkv, bt, rbq), dtype=torch.uint8, device="cuda")
    vq = torch.empty_like(kq)

    def attn_kv_q4(i):
        nh.prefill_bf16(q, k, v, out, Hq, Hkv, D, k_pool=kq, v_pool=vq, block_table=tab,
                        block_tokens=bt, kv_dtype=nh.KV_Q4_20B)

    # the row-wise quantiser alone on the chunk's K rows as f32 (65536 rows of 128)
    kf = k.float().contiguous()
    kqf = torch.empty((n * Hkv, rbq), dtype=torch.uint8, device="cuda")

    def quant(i):
        nh.q4_quantize(kf, n * Hkv, D, kqf)

    reps = max(20, steps)
    settle(attn_kv, torch)
    ms_kv = timed(attn_kv, reps, max(2, warmup // 5), torch)
    us = event_mean(attn, reps, torch) * 1e3
    pct = event_pcts(attn, reps, torch)
    us_kv = event_mean(attn_kv, reps, torch) * 1e3
    pct_kv = event_pcts(attn_kv, reps, torch)
    us_kv_q4 = event_mean(attn_kv_q4, reps, torch) * 1e3
    us_quant = event_mean(quant, reps, torch) * 1e3
    attn(0)
    torch.cuda.synchronize()

    def f32_of(x):  # bf16 tensor -> its exact f32 values on the host
        return (x.view(torch.int16).cpu().numpy().astype(np.uint16).astype(np.uint32) << 16).view(np.float32)

    SAMPLES["c5"] = {"q": f32_of(q), "k": f32_of(k), "v": f32_of(v), "out": out.cpu().numpy()}
    quant_bytes = n * Hkv * D * 4 + n * Hkv * rbq
    tf = flops / (us * 1e-6) / 1e12
    busy = _profile_value("prefill_c5_mfma_counters.txt", "mfma_busy_frac", "c5")
    return {"us_with_kv_write": us_kv, "us_with_kv_write_p10_p50_p90": _us3(pct_kv),
            "us_with_kv_write_q4": us_kv_q4,
            "tflops_with_kv_write_q4": flops / (us_kv_q4 * 1e-6) / 1e12,
            "q4_quantize_65536x128": {"us": us_quant, "bytes": quant_bytes,
                                      "gbs": quant_bytes / (us_quant * 1e-6) / 1e9},
            "us_with_kv_write_wall": ms_kv * 1e3,
            "tflops_with_kv_write": flops / (us_kv * 1e-6) / 1e12,
            "mfma_frac_with_kv_write": flops / (us_kv * 1e-6) / 1e12 / BF16_PEAK_TFLOPS,
            "us_prefill_call": us, "us_prefill_call_p10_p50_p90": _us3(pct), "reps": reps,
            "prefill_call": "the attention kernel (which also checks V's binary16 range; one launch)",
            "flops": flops, "tflops": tf, "mfma_frac": tf / BF16_PEAK_TFLOPS,
            "kv_write_bytes": 2 * n * Hkv * D * (2 + 4),
            "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                         "traffic": None, "mfma_busy_frac_counters": busy}}


def _smi_sample():
    """Socket power (W) and the mean graphics clock over the XCDs (MHz), from
    a read-only `amd-smi metric -p -c --json`; None where unavailable."""
    try:
        r = subprocess.run(["amd-smi", "metric", "-p", "-c", "--json"], capture_output=True,
                           text=True, timeout=30)
        d = json.loads(r.stdout)
        g = (d["gpu_data"] if isinstance(d, dict) else d)[0]
        pw = g.get("power", {}).get("socket_power", {}).get("value")
        clks = [v["clk"]["value"] for k, v in g.get("clock", {}).items()
                if k.startswith("gfx_") and isinstance(v, dict) and isinstance(v.get("clk"), dict)
                and isinstance(v["clk"].get("value"), (int, float))]
        return (float(pw) if isinstance(pw, (int, float)) else None,
                float(np.mean(clks)) if clks else None)
    except Exception:  # no tool or an unexpected format: the sample is missing
        return None, None


def bench_c5_sustained(nh, torch, seconds, seed=0):
    """C5's prefill call back to back for `seconds` on the workload's N(0,1)
    inputs, then on all-zero inputs of the same shape (the same instructions
    with almost no data toggling), sampling socket power and graphics clock
    over the second half of each run: under this load the package power cap,
    not the instruction schedule, sets the clock."""
    n, Hq, Hkv, D = 8192, 32, 8, 128
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn((n, Hq, D), generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn((n, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((n, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
    out = torch.empty((n, Hq, D), device="cuda")
    flops = 4 * Hq * D * n * (n + 1) / 2
    res = {}
    for kind in ("randn", "zeros"):
        if kind == "zeros":
            q.zero_()
            k.zero_()
            v.zero_()
        st = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        samples, calls = [], 0
        stop = threading.Event()
        t0 = time.perf_counter()

        def sampler():  # off the issuing thread, so the GPU's queue never drains
            while not stop.wait(0.25):
                if time.perf_counter() - t0 > seconds / 2:
                    samples.append(_smi_sample())

        th = threading.Thread(target=sampler, daemon=True)
        th.start()
        e0.record(st)
        while time.perf_counter() - t0 < seconds:
            for _ in range(20):
                nh.prefill_bf16(q, k, v, out, Hq, Hkv, D)
            calls += 20
            torch.cuda.synchronize()
        e1.record(st)
        torch.cuda.synchronize()
        stop.set()
        th.join()
        us = e0.elapsed_time(e1) * 1e3 / calls
        pw = [x[0] for x in samples if x[0] is not None]
        mhz = [x[1] for x in samples if x[1] is not None]
        res[kind] = {"us_per_call": round(us, 1), "calls": calls,
                     "tflops": round(flops / (us * 1e-6) / 1e12, 1),
                     "mfma_frac": round(flops / (us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4),
                     "socket_power_w": round(float(np.mean(pw)), 1) if pw else None,
                     "gfx_clock_mhz": round(float(np.mean(mhz)), 1) if mhz else None,
                     "samples": len(samples)}
    return res


def cpu_baseline_c5(seed=0, n_rows=256, sample=None):
    """The reference's prefill: one decode call per row (executor.rs:132-137),
    timed on n_rows rows spread over the 8192 and scaled by attended keys."""
    import oracle
    import workloads as W

    n, hq, hkv, d = 8192, 32, 8, 128
    if sample is not None:  # the GPU run's own bf16 inputs, as their f32 values
        qb, kb, vb = sample["q"], sample["k"], sample["v"]
        origin = "the GPU run's own bf16 q, k, v, copied from HBM"
    else:
        q, k, v = W.prefill_inputs(n, hq, hkv, d, seed=seed)
        qb, kb, vb = W.bf16_round(q), W.bf16_round(k), W.bf16_round(v)
        origin = "a seeded draw of the same shapes, rounded to bf16"
    lay = oracle.token_major_layout(np.ascontiguousarray(kb), np.ascontiguousarray(vb), hkv, d)
    rows = np.linspace(0, n - 1, n_rows).astype(np.int32)
    thr = _cores()
    qf = np.ascontiguousarray(qb.reshape(n, -1))
    dt, runs = _cpu_time(lambda: oracle.attention_rows(qf, lay, rows, hq, hkv, d, threads=thr),
                         budget_s=3.0, max_calls=50)
    keys_sample = float((rows.astype(np.int64) + 1).sum())
    keys_all = n * (n + 1) / 2.0
    est = dt * keys_all / keys_sample
    flops = 4 * hq * d * keys_all
    out = {"value": flops / est / 1e12, "unit": "TFLOP/s (extrapolated)", "cores": thr,
           "kind": "port", "us_extrapolated": est * 1e6,
           "sample": (f"{runs} runs of {n_rows} evenly spaced rows, all 32 heads "
                      f"({dt * 1e3:.1f} ms; inputs: {origin}), scaled by attended keys to all "
                      f"8192 rows")}
    if sample is not None:
        ref = oracle.attention_rows(qf, lay, rows, hq, hkv, d, threads=thr).reshape(n, hq, d)
        out.update(_err(sample["out"][rows], ref[rows]))
    return out


# ----------------------------------------------------------------------------
# other configs
# ----------------------------------------------------------------------------

def bench_c1(nh, torch, steps, warmup):
    import workloads as W

    q, k, v = (torch.from_numpy(x).cuda() for x in W.c1_contiguous(seed=0))
    out = torch.empty_like(q)
    scores = torch.empty(32 * 128, device="cuda")

    def call(i):
        nh.attention_node(q, k, v, out, 32, 4, 128, 64, 128, scores=scores)

    settle(call, torch)
    ms = timed(call, steps * 10, warmup, torch)
    us = event_mean(call, steps * 4, torch) * 1e3
    pct = event_pcts(call, max(steps, 20), torch)
    # algorithmic bytes: K and V of 4 kv heads x 128 positions x 64 f32 (262144)
    # + q and out (2 x 32 x 64 x 4) = 278528; at 8 TB/s that is 0.035 us, so
    # the call is bound by launch and dependent-access latency, not by HBM
    nbytes = 278528
    rl = hbm_roofline(nbytes, us, pmc_traffic("c1"))
    rl.update({"kernel": "decode_kernel<64,f32,contiguous> (the Attention node, one launch)",
               "bytes_per_launch": nbytes, "launch_us": round(us, 3),
               "ideal_us_at_peak": round(nbytes / (HBM_PEAK_GBS * 1e3), 4)})
    return {"us_per_layer": ms * 1e3, "call_us_event_mean": us, "call_us_p10_p50_p90": _us3(pct),
            "bytes_per_layer": nbytes, "roofline": rl}


def bench_abi(nh, torch, steps, warmup):
    """The project-ABI entry with no scratch argument (gpu_attention_device,
    fused_attention.cu:194-213: the reference allocates an n_heads*seq_len
    scores buffer per call; this library keeps one split-K buffer per
    stream, allocated by the first call) against nyion_attention_node given
    that scores buffer (ScratchBuffers::d_scores, swamp-gpu/src/lib.rs:290-331).  Contiguous f32 KV [Hkv][4096][64], 32/4
    heads, 40 rotated caches (336 MB, beyond the 256 MB Infinity Cache)."""
    Hq, Hkv, D, ctx, R = 32, 4, 64, 4096, 40
    g = torch.Generator(device="cuda").manual_seed(0)
    sets = [(torch.randn((Hkv, ctx, D), generator=g, device="cuda"),
             torch.randn((Hkv, ctx, D), generator=g, device="cuda")) for _ in range(R)]
    q = torch.randn((Hq, D), generator=g, device="cuda")
    out = torch.empty_like(q)
    scores = torch.empty(Hq * ctx, device="cuda")
    L = nh.load()
    # arguments resolved once: a call then costs only the C-ABI crossing
    dev_args = [(nh.ptr(q), nh.ptr(k), nh.ptr(v), nh.ptr(out), Hq, Hkv, ctx, D, ctx)
                for k, v in sets]
    node_args = [(nh.ptr(q), nh.ptr(k), nh.ptr(v), nh.ptr(scores), nh.ptr(out), Hq, Hkv, ctx, D,
                  ctx, nh.KV_F32, nh.stream_handle(None)) for k, v in sets]

    def device_call(i):
        if L.gpu_attention_device(*dev_args[i % R]) != 0:
            raise RuntimeError("gpu_attention_device failed")

    def node_call(i):
        if L.nyion_attention_node(*node_args[i % R]) != 0:
            nh.check(-1, "nyion_attention_node")

    bytes_call = 2 * Hkv * ctx * D * 4 + 2 * Hq * D * 4
    res = {"workload": "contiguous f32 KV, ctx 4096, 32/4 heads, D 64, cold",
           "bytes_per_call": bytes_call}
    for name, fn in (("gpu_attention_device", device_call), ("node_with_scores", node_call)):
        timed(fn, steps, warmup, torch)
        us = event_mean(fn, max(steps, 20) * 2, torch) * 1e3
        res[name] = {"call_us_event_mean": us, "call_us_p10_p50_p90": _us3(event_pcts(fn, max(steps, 20), torch)),
                     "gbs": bytes_call / (us * 1e-6) / 1e9}
    res["device_over_node"] = res["gpu_attention_device"]["call_us_event_mean"] / res["node_with_scores"]["call_us_event_mean"]
    return res


def bench_zone(nh, torch, steps, warmup):
    """Decode over a reference-shaped zone cache (32-token pages holding all
    22 layers, shuffled page order; the gather path) against the same rows
    through 16-token block tables (the aligned path): one layer, ctx 4096,
    32/4 heads, D 64, f32, 2 rotated copies (371 MB)."""
    Hq, Hkv, D, ctx, NL, R = 32, 4, 64, 4096, 22, 2
    n_pages = ctx // 32
    page_units = NL * Hkv * 32 * D
    g = torch.Generator(device="cuda").manual_seed(0)
    rng = np.random.default_rng(0)
    zone, paged = [], []
    for r in range(R):
        kz = torch.randn((n_pages * page_units,), generator=g, device="cuda")
        vz = torch.randn((n_pages * page_units,), generator=g, device="cuda")
        perm = rng.permutation(n_pages)
        bases = torch.from_numpy((perm * page_units).astype(np.int64)[None, :]).cuda()
        zone.append((kz, vz, bases))
        # layer 0 of the same rows as 16-token blocks: page p slot s -> block 2p + s // 16
        kp = kz.view(n_pages, NL, Hkv, 2, 16, D)[:, 0].permute(0, 2, 1, 3, 4).reshape(-1, Hkv, 16, D)
        vp = vz.view(n_pages, NL, Hkv, 2, 16, D)[:, 0].permute(0, 2, 1, 3, 4).reshape(-1, Hkv, 16, D)
        tab = torch.from_numpy(paged_tables(rng, 1, ctx // 16, ctx // 16)).cuda()
        kp2, vp2 = torch.empty_like(kp), torch.empty_like(vp)
        kp2[tab[0].long()] = kp.contiguous()
        vp2[tab[0].long()] = vp.contiguous()
        paged.append((kp2, vp2, tab))
    q = torch.randn((1, Hq, D), generator=g, device="cuda")
    ctx_t = torch.full((1,), ctx, dtype=torch.int32, device="cuda")
    out_z, out_p = torch.empty_like(q), torch.empty_like(q)
    ws = nh.alloc_workspace(nh.decode_workspace_size(1, Hq, Hkv, D, ctx))

    L = nh.load()
    zargs = [(nh.ptr(q), nh.ptr(kz), nh.ptr(vz), kz.numel(), nh.ptr(bases), n_pages, NL, 0,
              nh.ptr(ctx_t), None, 1, Hq, Hkv, D, nh.KV_F32, 0, 0, ctx, 0.0, nh.ptr(out_z),
              nh.ptr(ws), ws.numel(), nh.stream_handle(None)) for kz, vz, bases in zone]
    pcalls = [nh.prepare_paged_decode(q, kp, vp, tab, ctx_t, out_p, Hq, Hkv, D, 16, ctx, workspace=ws)
              for kp, vp, tab in paged]

    def zone_call(i):
        rc = L.nyion_zone_decode_attention(*zargs[i % R])
        if rc != 0:
            nh.check(rc, "nyion_zone_decode_attention")

    def paged_call(i):
        pcalls[i % R]()

    zone_call(0)
    paged_call(0)
    torch.cuda.synchronize()
    diff = float((out_z - out_p).abs().max())
    bytes_call = 2 * Hkv * ctx * D * 4 + 2 * Hq * D * 4
    res = {"workload": "f32 KV, ctx 4096, 32/4 heads, D 64, 22-layer zone pages", "bytes_per_call": bytes_call,
           "max_abs_zone_vs_paged": diff}
    for name, fn in (("zone", zone_call), ("paged16", paged_call)):
        timed(fn, steps, warmup, torch)
        us = event_mean(fn, max(steps, 20) * 2, torch) * 1e3
        res[name] = {"call_us_event_mean": us, "gbs": bytes_call / (us * 1e-6) / 1e9}
    res["zone_over_paged"] = res["zone"]["call_us_event_mean"] / res["paged16"]["call_us_event_mean"]
    return res


def _q4k_random(torch, rows, cols, seed):
    """Random Q4_K matrix on the device: uniform nibbles/scales, finite f16
    d = dmin in [5e-5, 5e-4]."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    nb = cols // 256
    w = torch.randint(0, 256, (rows, nb, 144), dtype=torch.uint8, device="cuda", generator=g)
    d = (torch.rand((rows, nb), device="cuda", generator=g) * 4.5e-4 + 5e-5).half()
    w[:, :, 0:2] = d.view(torch.uint8).view(rows, nb, 2)
    w[:, :, 2:4] = d.view(torch.uint8).view(rows, nb, 2)
    return w.view(rows, -1).contiguous()


def _q6k_random(torch, rows, cols, seed):
    """Random Q6_K matrix on the device: uniform ql/qh/scales, normal f16 d in
    [7e-5, 5e-4]."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    nb = cols // 256
    w = torch.randint(0, 256, (rows, nb, 210), dtype=torch.uint8, device="cuda", generator=g)
    d = (torch.rand((rows, nb), device="cuda", generator=g) * 4.3e-4 + 7e-5).half()
    w[:, :, 208:210] = d.view(torch.uint8).view(rows, nb, 2)
    return w.view(rows, -1).contiguous()


USE_GRAPHS = True


def _graph_us(torch, fn, reps):
    """Mean replay time of fn captured in a HIP graph (no host overhead);
    with --no-graph the same launches are issued directly."""
    if not USE_GRAPHS:
        fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) * 1e3 / reps
    gph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gph):
        fn()
    gph.replay()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        gph.replay()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) * 1e3 / reps


def bench_gemv(nh, torch, steps, warmup, cpu=True):
    """Q4_K weight GEMV (the projections either side of decode attention):
    the TinyLlama-1.1B decode step's 88 launches (per layer q/k/v in one
    launch, o, gate/up in one launch, down; 22 layers, 545 MB of weights, so
    the 256 MB MALL does not hold them) and Llama-3-8B-shaped gate/up
    (2 x 14336 x 4096, 66 MB per launch, 8 layers rotated), both replayed
    from HIP graphs."""
    H, F, KV, L = 2048, 5632, 256, 22
    lw = [{k: _q4k_random(torch, r, c, 7 * l + i) for i, (k, r, c) in enumerate(
        [("q", H, H), ("k", KV, H), ("v", KV, H), ("o", H, H), ("g", F, H), ("u", F, H), ("d", H, F)])}
        for l in range(L)]
    x = torch.randn(H, device="cuda")
    xf = torch.randn(F, device="cuda")
    o = {k: torch.empty(n, device="cuda") for k, n in
         dict(q=H, k=KV, v=KV, o=H, g=F, u=F, d=H).items()}
    step_bytes = sum(t.numel() for w in lw for t in w.values())

    def step():
        for w in lw:
            nh.gemv_q4k_multi([w["q"], w["k"], w["v"]], x, [o["q"], o["k"], o["v"]], H)
            nh.gemv_q4k(w["o"], x, o["o"], H, H)
            nh.gemv_q4k_multi([w["g"], w["u"]], x, [o["g"], o["u"]], H)
            nh.gemv_q4k(w["d"], xf, o["d"], H, F)

    reps = max(3, steps // 5)
    step_us = _graph_us(torch, step, reps)
    H8, F8, L8 = 4096, 14336, 8
    big = [(_q4k_random(torch, F8, H8, 100 + l), _q4k_random(torch, F8, H8, 200 + l)) for l in range(L8)]
    x8 = torch.randn(H8, device="cuda")
    og, ou = torch.empty(F8, device="cuda"), torch.empty(F8, device="cuda")

    def gateup():
        for gw, uw in big:
            nh.gemv_q4k_multi([gw, uw], x8, [og, ou], H8)

    gu_us = _graph_us(torch, gateup, reps) / L8
    gu_bytes = 2 * big[0][0].numel()
    res = {"timing": "graph replay" if USE_GRAPHS else "direct launches",
           "tinyllama_step_us": step_us, "tinyllama_step_bytes": step_bytes, "launches": 4 * L,
           "tinyllama_step_gbs": step_bytes / step_us / 1e3,
           "gateup_8b_us": gu_us, "gateup_8b_bytes": gu_bytes,
           "gateup_8b_gbs": gu_bytes / gu_us / 1e3,
           "gateup_8b_hbm_frac": gu_bytes / gu_us / 1e3 / HBM_PEAK_GBS}
    if cpu:
        import oracle

        wg = lw[0]["g"].cpu().numpy()
        xc = x.cpu().numpy()
        t0, n = time.perf_counter(), 0
        while time.perf_counter() - t0 < 2.0:
            oracle.gemv_q4k(wg, xc, F, H)
            n += 1
        dt = (time.perf_counter() - t0) / n
        res["cpu_oracle_gate_us"] = dt * 1e6
        res["cpu_oracle_threads"] = oracle.max_threads()
        res["cpu_oracle_gate_gbs"] = wg.size / dt / 1e9
    del lw, big
    torch.cuda.empty_cache()
    return res


def bench_gemv_q6k(nh, torch, steps, warmup, cpu=True):
    """Q6_K weight GEMV: the TinyLlama-1.1B output projection (32000 x 2048,
    53.8 MB; six copies rotated so that the 256 MB MALL does not hold them),
    and a Q4_K_M-style TinyLlama decode step through the spec list (per layer
    q/k/o/gate/up Q4_K, v/down Q6_K; one list per layer, launched as q+k,
    v, o, gate+up and down: 110 launches), both replayed from HIP graphs."""
    V, H, F, KV, L = 32000, 2048, 5632, 256, 22
    heads = [_q6k_random(torch, V, H, 300 + i) for i in range(6)]
    x = torch.randn(H, device="cuda")
    xf = torch.randn(F, device="cuda")
    logits = torch.empty(V, device="cuda")

    def lm_head():
        for w in heads:
            nh.gemv_q6k(w, x, logits, V, H)

    reps = max(3, steps // 5)
    head_us = _graph_us(torch, lm_head, reps) / len(heads)
    head_bytes = heads[0].numel()
    del heads
    lw = []
    for l in range(L):
        lw.append({"q": _q4k_random(torch, H, H, 7 * l), "k": _q4k_random(torch, KV, H, 7 * l + 1),
                   "v": _q6k_random(torch, KV, H, 7 * l + 2), "o": _q4k_random(torch, H, H, 7 * l + 3),
                   "g": _q4k_random(torch, F, H, 7 * l + 4), "u": _q4k_random(torch, F, H, 7 * l + 5),
                   "d": _q6k_random(torch, H, F, 7 * l + 6)})
    o = {k: torch.empty(n, device="cuda") for k, n in dict(q=H, k=KV, v=KV, o=H, g=F, u=F, d=H).items()}
    fmt = dict(q=144, k=144, v=210, o=144, g=144, u=144, d=210)
    rows = dict(q=H, k=KV, v=KV, o=H, g=F, u=F, d=H)
    xa = torch.randn(H, device="cuda")  # attention output, the o projection's input
    xm = torch.randn(H, device="cuda")  # post-attention hidden state, gate/up's input
    xin = dict(q=x, k=x, v=x, o=xa, g=xm, u=xm, d=xf)
    specs = [[(w[k], xin[k], o[k], rows[k], F if k == "d" else H, fmt[k]) for k in "qkvogud"]
             for w in lw]
    step_bytes = sum(t.numel() for w in lw for t in w.values())

    def step():
        for sp in specs:
            nh.gemv_specs(sp)

    step_us = _graph_us(torch, step, reps)
    res = {"timing": "graph replay" if USE_GRAPHS else "direct launches",
           "output_proj_us": head_us, "output_proj_bytes": head_bytes,
           "output_proj_gbs": head_bytes / head_us / 1e3,
           "output_proj_hbm_frac": head_bytes / head_us / 1e3 / HBM_PEAK_GBS,
           "q4km_step_us": step_us, "q4km_step_bytes": step_bytes, "launches": 5 * L,
           "q4km_step_gbs": step_bytes / step_us / 1e3}
    if cpu:
        import oracle

        n_rows = 2048  # a slice of the output projection's rows
        w0 = _q6k_random(torch, n_rows, H, 400).cpu().numpy()
        xc = x.cpu().numpy()
        t0, n = time.perf_counter(), 0
        while time.perf_counter() - t0 < 2.0:
            oracle.gemv_q6k(w0, xc, n_rows, H)
            n += 1
        dt = (time.perf_counter() - t0) / n
        res["cpu_oracle_rows"] = n_rows
        res["cpu_oracle_us"] = dt * 1e6
        res["cpu_oracle_threads"] = oracle.max_threads()
        res["cpu_oracle_gbs"] = w0.size / dt / 1e9
    del lw, specs
    torch.cuda.empty_cache()
    return res


def bench_kv_pool(nh, torch, steps, warmup):
    """Paged KV pool with host spill, TinyLlama geometry (22 layers, 4 kv heads,
    D=64, 16-token pages, f32: 704 KiB per page over all layers, K and V):
    cost of bringing a cold page back when the hot tier is full (one spill to
    pinned host memory plus one reload), and of creating a page."""
    layers, hkv, d, bt, hot, cold, pages = 22, 4, 64, 16, 64, 512, 512
    pool = nh.KvPool(layers, hkv, d, bt, nh.KV_F32, hot, cold, pages)
    page_bytes = 2 * layers * hkv * bt * d * 4
    n_create = 256
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for p in range(n_create):
        pool.ensure(p)
    torch.cuda.synchronize()
    create_us = (time.perf_counter() - t0) * 1e6 / n_create  # includes the spills past 64
    rng = np.random.default_rng(0)
    order = [int(p) for p in rng.integers(0, n_create - hot, max(32, steps))]
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st0 = pool.stats()
    s.record()
    t0 = time.perf_counter()
    for p in order:
        pool.ensure(p)
    e.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e6 / len(order)
    st1 = pool.stats()
    moves = (st1["evictions"] - st0["evictions"]) + (st1["reloads"] - st0["reloads"])
    gpu_us = s.elapsed_time(e) * 1e3
    res = {"page_bytes": page_bytes, "create_or_spill_us_wall": create_us,
           "cold_hit_us_wall": wall, "cold_hit_us_gpu": gpu_us / len(order),
           "page_moves": moves, "host_link_gbs": moves * page_bytes / gpu_us / 1e3}
    pool.close()
    return res


# ----------------------------------------------------------------------------

def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the attention path has no multi-GPU mode (each GPU "
              "would run its own sequences or kv heads with no exchange); run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    import torch

    import nyion_hip as nh

    nh.init(0)
    global USE_GRAPHS
    USE_GRAPHS = not args.no_graph
    # the Q6_K GEMV lines (outside the attention path's scope) run only when named
    only = set(filter(None, args.only.split(","))) or set(ALL) - {"gemv6"}
    steps, warmup = max(1, args.steps), max(0, args.warmup)
    res = {}
    if args.calib_copy:
        a = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        log("calibration copy: 3 x 512 MiB")
        del a, b
    if "c3" in only:
        log("64-sequence continuous batch (headline)")
        res["c3"] = bench_c3(nh, torch, steps, warmup)
        torch.cuda.empty_cache()
    if "c3h" in only:
        log("64-sequence continuous batch, binary16 KV")
        res["c3h"] = bench_c3(nh, torch, steps, warmup, f16=True)
        torch.cuda.empty_cache()
    if "c3q" in only:
        log("64-sequence continuous batch, Q4-20B KV")
        res["c3q"] = bench_c3(nh, torch, steps, warmup, q4=True)
        torch.cuda.empty_cache()
    if "c2" in only:
        log("22-layer decode step, ctx 4096")
        res["c2"] = bench_c2(nh, torch, steps, warmup)
        torch.cuda.empty_cache()
    if "c2t" in only:
        log("22-layer decode step, tracked form (scores + importance)")
        res["c2_tracked"] = bench_c2_tracked(nh, torch, steps)
        torch.cuda.empty_cache()
    if "c1" in only:
        log("contiguous 128-position node")
        res["c1"] = bench_c1(nh, torch, steps, warmup)
    if "abi" in only:
        log("project ABI: gpu_attention_device vs the node with its scores buffer")
        res["abi_cliff"] = bench_abi(nh, torch, steps, warmup)
        torch.cuda.empty_cache()
    if "zone" in only:
        log("zone-geometry cache vs 16-token block tables")
        res["zone"] = bench_zone(nh, torch, steps, warmup)
        torch.cuda.empty_cache()
    if "c4" in only:
        log("Q4 KV, ctx 131072, window 4096 (cold: rotated tables)")
        res["c4"] = bench_c4(nh, torch, steps, warmup)
        torch.cuda.empty_cache()
    if "a5" in only:
        log("attention_sparse_q4 on zone pages, ctx 131072, window 4096 (cold)")
        res["a5"] = bench_a5(nh, torch, steps, warmup)
        torch.cuda.empty_cache()
    if "c5" in only:
        log("causal prefill N=8192 with paged KV write")
        res["c5"] = bench_c5(nh, torch, steps, warmup)
        if args.sustain > 0:
            log(f"causal prefill N=8192 sustained {args.sustain:.0f} s on N(0,1) and on zero inputs")
            res["c5"]["sustained"] = bench_c5_sustained(nh, torch, args.sustain)
        torch.cuda.empty_cache()
    if "pool" in only:
        log("paged KV pool: cold-page round trips over the host link")
        res["kv_pool"] = bench_kv_pool(nh, torch, steps, warmup)
    if "gemv" in only:
        log("Q4_K weight GEMV: TinyLlama decode-step projections, 8B-shaped gate/up")
        res["gemv_q4k"] = bench_gemv(nh, torch, steps, warmup, cpu=not args.no_cpu)
    if "gemv6" in only:
        log("Q6_K weight GEMV: TinyLlama output projection, Q4_K_M-style decode step")
        res["gemv_q6k"] = bench_gemv_q6k(nh, torch, steps, warmup, cpu=not args.no_cpu)
    cpu = None
    if not args.no_cpu:
        for key, fn in (("c1", cpu_baseline_c1), ("c2", cpu_baseline_c2), ("c4", cpu_baseline_c4),
                        ("a5", cpu_baseline_a5), ("c5", cpu_baseline_c5)):
            if key in res:
                log(f"CPU baseline (oracle) for {key}")
                res[key]["cpu_baseline"] = (fn(sample=SAMPLES[key]) if key in SAMPLES else fn())
        if "c3" in res:
            log("CPU baseline (oracle) on a sample of the headline batch")
            cpu = cpu_baseline_c3(sample=SAMPLES.get("c3"))

    c3 = res.get("c3")
    line = {
        "metric": METRIC,
        "value": round(c3["gbs_wall"], 2) if c3 else None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(c3["ms_per_call_wall"], 4) if c3 else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1); paged 16-token blocks, shuffled tables)",
        "config": {"workload": "decode-continuous-batch-64seq-ctx512-32768-paged16-f32",
                   "batch": 64, "n_heads": C3_HQ, "n_kv_heads": C3_HKV, "head_dim": C3_D,
                   "context": "uniform [512, 32768], numpy PCG64 seed 0",
                   "block_tokens": C3_BT, "parallelism": "single-gpu"},
    }
    if c3:
        line["us_per_layer"] = round(c3["us_per_layer"], 3)
        line["us_p10_p50_p90"] = c3["us_p10_p50_p90"]
        line["settle_calls"] = c3["settle_calls"]
        line["config"]["tokens"] = c3["tokens"]
        rl = dict(c3["roofline"])
        rl.update({"kernel": "decode_kernel<64,f32,aligned> (one launch per decode call)",
                   "bytes_per_launch": c3["bytes"], "launch_us": round(c3["us_per_layer"], 3)})
        line["roofline"] = rl
    if cpu:
        line["cpu_baseline"] = cpu
    line["configs"] = {k: v for k, v in res.items() if k != "c3"}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
