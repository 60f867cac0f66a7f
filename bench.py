"""Benchmark: batched decode attention of the Needle KV-cache path on one
MI355X (the headline workload: 4096 independent sequences, 8 heads x 64,
fp16 K/V, ragged lengths uniform in [213, 1024], one new token per sequence
through 8 layers).

A step = for each of 8 layers: KV append of the new token and single-token
attention (nda_step: the append kernel then the decode kernel at this batch
size), then pos += 1 (nda_advance); inputs are resident in HBM before the
timed region. Prints one JSON line.

    python bench.py [--steps K] [--warmup W] [--no-cpu]
"""
import argparse
import gc
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "esp32-needle-3_amd"))
sys.path.insert(0, os.path.join(REPO, "oracle"))

HBM_PEAK_GBS = 8000.0
B, H, D, LAYERS = 4096, 8, 64, 8
LMIN, LMAX = 213, 1024
SEED = 20261201


def committed_traffic():
    """HBM bytes per decode launch measured with rocprofv3 FETCH_SIZE and
    WRITE_SIZE on this same command, calibrated on a copy of known size, as
    recorded in the committed profile summary (None when absent)."""
    import re
    path = os.path.join(REPO, "profiles", "attend_kernel_decode_b4096_f16.md")
    try:
        m = re.search(r"traffic_bytes_per_launch:\s*(\d+)", open(path).read())
        return int(m.group(1)) if m else None
    except OSError:
        return None


def host_info():
    """ROCm version, host CPU model and the cores the CPU legs could use."""
    info = {"cpus": os.cpu_count()}
    try:
        info["rocm"] = open("/opt/rocm/.info/version").read().strip()
    except OSError:
        info["rocm"] = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                info["cpu_model"] = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return info


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_port_f16(lens_all, seconds, nthreads, nseq=128, seed_off=1):
    """The oracle's fp16 decode (the engine's attn_heads restated with fp16
    KV; the reference has no fp16 cache) on a bounded sample of sequences
    drawn from lens_all, split over nthreads threads by sequence as the
    engine's nd_parallel_rows seam splits rows (nd_quant.h:213-230).
    Returns (tokens/s through LAYERS layers, attention FLOP/s, sample)."""
    import ndoracle as O

    rng = np.random.default_rng(SEED + seed_off)
    S = nseq
    lens = np.ascontiguousarray(rng.choice(lens_all, S), np.uint32)
    koff = np.zeros(S, np.uint64)
    koff[1:] = np.cumsum(lens[:-1].astype(np.uint64) * H * D)
    tot = int(lens.sum()) * H * D
    kbase = rng.standard_normal(tot, dtype=np.float32).astype(np.float16).view(np.uint16)
    vbase = rng.standard_normal(tot, dtype=np.float32).astype(np.float16).view(np.uint16)
    q = rng.standard_normal(S * H * D, dtype=np.float32)
    kn = rng.standard_normal(S * H * D, dtype=np.float32)
    vn = rng.standard_normal(S * H * D, dtype=np.float32)
    out = np.zeros(S * H * D, np.float32)
    # one call = one decode token for S sequences on one layer
    O.decode_batch_f16(H, H, D, D, lens, kbase, vbase, koff, koff, q, kn, vn, None, out, nthreads)
    calls, t0 = 0, time.perf_counter()
    while True:
        O.decode_batch_f16(H, H, D, D, lens, kbase, vbase, koff, koff, q, kn, vn, None, out, nthreads)
        calls += 1
        el = time.perf_counter() - t0
        if el >= seconds and calls >= 2:
            break
    tok_s = calls * S / el / LAYERS
    flops = calls * float(lens.sum() + S) * H * 2 * (D + D) / el
    return tok_s, flops, "%d sequences (L mean %.0f) x %d layer-calls, %.1f s" % (S, lens.mean(), calls, el)


def cpu_reference_int8(lens_all, seconds, threads):
    """The reference engine's own store + attn_heads (oracle/_ref, compiled
    from its sources) on the same shapes in its own dtype (int8 KV + scales,
    MHA 8 x 64), one session per sequence. For each thread count in
    `threads`: 1 is the host build's serial rows_serial; more runs the
    sessions side by side on that many threads (the reference's attention
    path has no shared writable state). Caches hold random int8 codes; one
    round is one decode token (store + attend) per sequence on one layer.
    Timed in C with CLOCK_MONOTONIC. Returns {threads: baseline object}."""
    import ctypes as C
    import ndoracle as O
    if not O.have_ref():
        return None
    rng = np.random.default_rng(SEED + 2)
    S = max(64, 4 * max(threads))
    lens = rng.choice(lens_all, S)
    sess = []
    for L in lens:
        r = O.RefSession(1, H, H, D, D, int(L) + 1)
        k, v, ks, vs = r.cache()
        k[:] = rng.integers(-127, 128, k.shape, dtype=np.int8)
        v[:] = rng.integers(-127, 128, v.shape, dtype=np.int8)
        ks[:] = rng.uniform(0.01, 0.03, ks.shape).astype(np.float32)
        vs[:] = rng.uniform(0.01, 0.03, vs.shape).astype(np.float32)
        O.ref().ref_set_pos(r.m, int(L) - 1)
        sess.append(r)
    models = (C.c_void_p * S)(*[r.m for r in sess])
    q = rng.standard_normal(H * D).astype(np.float32)
    kn = rng.standard_normal(H * D).astype(np.float32)
    vn = rng.standard_normal(H * D).astype(np.float32)
    res = {}
    for nt in threads:
        out = np.zeros(nt * H * D, np.float32)
        args = (models, S, 0, q.ctypes.data, kn.ctypes.data, vn.ctypes.data, out.ctypes.data, H * D)
        one = O.ref().ref_attention_rounds(*args, 1, nt)
        rounds = max(2, int(seconds / max(one, 1e-6)))
        el = O.ref().ref_attention_rounds(*args, rounds, nt)
        res[nt] = {"value": round(rounds * S / el / LAYERS, 1), "unit": "tokens/s", "cores": nt,
                   "kind": "reference",
                   "sample": "%d sequences (L mean %.0f), int8 KV (the engine's dtype), %d layer-calls, %.1f s"
                             % (S, lens.mean(), rounds * S, el)}
    for r in sess:
        r.close()
    return res


def usable_cores():
    """Cores the CPU legs may use on this host: the process's CPU affinity,
    bounded by a cgroup CPU quota when one is set and by the thread share the
    host declares in OMP_NUM_THREADS when that is set. Returns (cores, how)."""
    n = len(os.sched_getaffinity(0))
    how = ["affinity %d" % n]
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            q = max(1, int(-(-int(quota) // int(period))))
            how.append("cgroup quota %d" % q)
            n = min(n, q)
    except (OSError, ValueError):
        pass
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        how.append("OMP_NUM_THREADS %s" % omp)
        n = min(n, int(omp))
    return n, ", ".join(how)


def median_of(fn, repeats=5):
    """fn() -> seconds of one run; one warm-up, then the median of `repeats`."""
    fn()
    ts = sorted(fn() for _ in range(repeats))
    return ts[len(ts) // 2], ts


def cpu_reference_prefill_int8(threads, S=256, layers=LAYERS, repeats=5):
    """The 256-token single-sequence prefill (8 layers, MHA 8 x 64) through
    the reference engine's own code (oracle/_ref): the prompt fed one token
    at a time, each token's store + attention() dispatch in every layer, the
    heads through nd_parallel_rows - serial for 1 thread, the harness's
    n-thread splitter in that seam otherwise (8 heads: at most 8 threads have
    work). Timed in C with CLOCK_MONOTONIC; median of `repeats` after one
    warm-up. Returns {threads: object} or None without the harness."""
    import ndoracle as O
    if not O.have_ref():
        return None
    rng = np.random.default_rng(SEED + 21)
    q, k, v = (rng.standard_normal((S, H * D)).astype(np.float32) for _ in range(3))
    out = np.zeros((S, H * D), np.float32)
    flops = layers * H * 2 * (D + D) * S * (S + 1) / 2
    res = {}
    for nt in threads:
        r = O.RefSession(layers, H, H, D, D, S)
        if nt > 1 and O.ref().ref_pool_start(nt) != 0:
            r.close()
            continue

        def one():
            O.ref().ref_reset(r.m)
            return O.ref().ref_prefill_rounds(r.m, S, q.ctypes.data, k.ctypes.data, v.ctypes.data, out.ctypes.data)
        try:
            t, ts = median_of(one, repeats)
        finally:
            if nt > 1:
                O.ref().ref_pool_stop()
        r.close()
        res[nt] = {"value": round(S / t, 1), "unit": "prompt tokens/s (8 layers)", "cores": nt,
                   "kind": "reference", "ms_per_prefill": round(t * 1e3, 2),
                   "attention_GFLOPs": round(flops / t / 1e9, 3),
                   "sample": "the whole workload: 1 sequence x %d tokens x %d layers, int8 KV; median of %d "
                             "(%.1f-%.1f ms)" % (S, layers, repeats, ts[0] * 1e3, ts[-1] * 1e3)}
    return res


def cpu_port_prefill_f16(pre, ntok, nthreads, seed_off, repeats=5):
    """Token-by-token causal prefill through the oracle's fp16 attention
    port (the engine's attn_heads with fp16 KV; one call stores the token's
    k/v and attends over everything before it, as the engine prefills a
    prompt): sequence s has pre[s] stored positions and takes ntok[s] new
    tokens; sequences split over nthreads threads as independent sessions.
    Each round is one token of every sequence still prefilling, timed around
    the attention calls (CLOCK_MONOTONIC); median of `repeats` after one
    warm-up. Returns (seconds, attention FLOPs, repeat times)."""
    import ndoracle as O
    rng = np.random.default_rng(SEED + seed_off)
    S = len(pre)
    tot = np.asarray(pre, np.int64) + np.asarray(ntok, np.int64)
    koff = np.zeros(S, np.uint64)
    koff[1:] = np.cumsum(tot[:-1] * H * D).astype(np.uint64)
    pool = rng.standard_normal(1 << 22, dtype=np.float32).astype(np.float16).view(np.uint16)
    n_el = int(tot.sum()) * H * D
    kbase = np.resize(pool, n_el)
    vbase = np.resize(pool[::-1], n_el)
    T = int(max(ntok))
    q = rng.standard_normal((T, S * H * D), dtype=np.float32)
    kn = rng.standard_normal((T, S * H * D), dtype=np.float32)
    vn = rng.standard_normal((T, S * H * D), dtype=np.float32)
    out = np.zeros(S * H * D, np.float32)
    rounds = []
    for t in range(T):
        act = [s for s in range(S) if ntok[s] > t]
        lens = np.array([pre[s] + t + 1 for s in act], np.uint32)
        sel = np.concatenate([np.arange(s * H * D, (s + 1) * H * D) for s in act])
        rounds.append((lens, koff[act], np.ascontiguousarray(q[t, sel]), np.ascontiguousarray(kn[t, sel]),
                       np.ascontiguousarray(vn[t, sel])))
    flops = float(sum(H * 2 * (D + D) * (int(pre[s]) * int(ntok[s]) + int(ntok[s]) * (int(ntok[s]) + 1) / 2)
                      for s in range(S)))

    def one():
        el = 0.0
        for lens, ko, qq, kk, vv in rounds:
            t0 = time.perf_counter()
            O.decode_batch_f16(H, H, D, D, lens, kbase, vbase, ko, ko, qq, kk, vv, None, out, nthreads)
            el += time.perf_counter() - t0
        return el
    t, ts = median_of(one, repeats)
    return t, flops, ts


def config2_leg(N, stream, S=256, layers=LAYERS, reps=10):
    """The single-sequence causal prefill (1 sequence x 256 tokens, 8 layers,
    MHA 8 x 64, int8 K/V, the engine's own dtype): nda_prefill per layer on
    an empty sequence, whole 8-layer prefills timed back to back. A latency
    workload (one work-group column per head), not a throughput one."""
    rng = np.random.default_rng(SEED + 21)
    ctx = N.Context(layers, H, H, D, D, S, kv_dtype=N.KV_INT8, max_seqs=1)
    q, k, v, out = (N.DevBuf(S * H * D * 4) for _ in range(4))
    for i, b in enumerate((q, k, v)):
        b.upload(rng.standard_normal((S, H * D)).astype(np.float32))

    def one():
        ctx.seq_reset(0)
        for li in range(layers):
            ctx.prefill(li, [S], q, k, v, out, stream=stream)
        ctx.advance(1, [0], S, stream=stream)
    one()
    ctx.sync(stream)
    t0 = time.perf_counter()
    for _ in range(reps):
        one()
    ctx.sync(stream)
    el = (time.perf_counter() - t0) / reps
    ctx.close()
    flops = layers * H * 2 * (D + D) * S * (S + 1) / 2
    return {"workload": "causal prefill: 1 sequence x %d tokens, %d layers, 8 heads x 64, int8 K/V" % (S, layers),
            "ms_per_prefill": round(el * 1e3, 3), "prompt_tokens_per_s": round(S / el, 1),
            "tflops": round(flops / el / 1e12, 4), "flop_per_prefill": flops}


def prefill_leg(N, stream, nseq=256, lmin=8192, lmax=32768, chunk=512, reps=3):
    """Long-context leg: nseq sequences with L ~ U[lmin, lmax] stored positions
    each take one decode token (append + split-KV attention over L+1
    positions, HBM-bound), then a `chunk`-token causal prefill (append + MFMA
    attention) on one layer. Prefill FLOPs count the unmasked causal pairs
    only: sum_s H * 2 * (dk + dv) * (chunk * L_s + chunk * (chunk + 1) / 2).
    Decode bytes: sum_s (L_s + 1) * H * (dk + dv) * 2 plus q, out and the
    appended row."""
    rng = np.random.default_rng(SEED + 5)
    lens = rng.integers(lmin, lmax + 1, nseq)
    P = 16
    window = lmax + chunk + 16
    need = int(sum((int(L) + chunk + P) // P for L in lens)) + 64
    ctx = N.Context(1, H, H, D, D, window, kv_dtype=N.KV_F16, max_seqs=nseq, page_size=P, max_pages=need)
    for b in range(nseq):
        ctx.seq_set_pos(b, int(lens[b]))         # the fill stores positions [0, pos)
    ctx.kv_fill_normal(nseq, seed=SEED + 6, stream=stream)
    T = nseq * chunk
    q, k, v, out = (N.DevBuf(T * H * D * 4) for _ in range(4))
    for i, buf in enumerate((q, k, v)):
        buf.fill_normal(T * H * D, 0, SEED + 70 + i, stream=stream)
    dec = decode_long(N, ctx, stream, lens, q, k, v, out, reps=10)
    ctx.advance(nseq, stream=stream)             # the decoded token stays; the chunk follows it
    lens = lens + 1
    ntok = np.full(nseq, chunk, np.uint32)
    ctx.prefill(0, ntok, q, k, v, out, stream=stream)       # warm-up
    ctx.sync(stream)
    ctx.prof_enable(True)
    ctx.prof_read(reset=True)
    t0 = time.perf_counter()
    for _ in range(reps):
        ctx.prefill(0, ntok, q, k, v, out, stream=stream)
    ctx.sync(stream)
    el = time.perf_counter() - t0
    ms, launches = ctx.prof_read(reset=True)
    ctx.prof_enable(False)
    flops = float(sum(H * 2 * (D + D) * (chunk * int(L) + chunk * (chunk + 1) / 2) for L in lens))
    pf_ms = ms[N.K_PREFILL] / max(1, launches[N.K_PREFILL])
    tflops = flops / (pf_ms * 1e-3) / 1e12
    # sampled parity: two rows of one sequence against the oracle
    import ndoracle as O
    qh = q.to_array(np.float32, (T, H * D))
    oh = out.to_array(np.float32, (T, H * D))
    worst = 0.0
    b = int(rng.integers(0, nseq))
    L = int(lens[b])
    kk, vv, _, _ = ctx.kv_read(0, b, 0, L + chunk)
    for t in (0, chunk - 1):
        kv = O.kv_view(kk, vv, None, None, H, L + chunk, 0, L + t, O.KV_F16)
        want = O.attend_view(kv, qh[b * chunk + t], None)
        worst = max(worst, float(np.abs(want - oh[b * chunk + t]).max()))
    ctx.close()
    return {"workload": "causal prefill chunk: %d sequences, %d new tokens each over L ~ U[%d,%d] "
                        "stored positions, 8 heads x 64, fp16 K/V, 1 layer (append + attention)"
                        % (nseq, chunk, lmin, lmax),
            "tflops": round(tflops, 1), "unit": "TFLOP/s", "bound": "mfma",
            "peak": 2500.0, "frac": round(tflops / 2500.0, 4),
            "kernel": "prefill_kernel<f16,64,64,rep1,W8>", "kernel_ms": round(pf_ms, 3),
            "flop_per_launch": flops, "append_ms": round(ms[N.K_APPEND] / max(1, launches[N.K_APPEND]), 4),
            "call_ms": round(el * 1e3 / reps, 3), "max_abs_delta_sampled": worst,
            "note": "unmasked causal FLOPs; the kernel issues 2x this on MFMA (fp16 hi+lo for Q and P)",
            "decode": dec}


def ceiling_leg(N, iters=200000):
    """Measured device ceilings (libndprobe, include/ndp.h), register-only
    loops with no memory traffic:
    - the dense fp16 MFMA rate: 4 independent v_mfma_f32_32x32x16_f16 chains
      per wave, at 1 and 2 waves per SIMD (the best is the ceiling);
    - the shader clock under that load, per wave from s_memtime cycles over
      s_memrealtime time;
    - SIMD cycles per wave64 v_exp_f32 and v_fma_f32 (8 independent chains);
    - MFMA with 2 or 4 independent exps issued after each MFMA by the same
      wave: whether the VALU work hides under the matrix pipe."""
    def mfma(bpc, wpb, nexp=0, n=iters):
        r = N.probe_run(N.PROBE_MFMA_F16, 4, nexp, bpc, wpb, n)
        wps = bpc * wpb / 4.0
        return {"waves_per_simd": wps, "tflops": round(r["flops"] / (r["ms"] * 1e-3) / 1e12, 1),
                "clock_ghz": round(r["clock_ghz"], 3), "ms": round(r["ms"], 3),
                "simd_cycles_per_mfma": round(r["cycles_per_iter"] / 4 / wps, 2)}

    def valu(kind, bpc=2, wpb=4, n=iters // 2):
        r = N.probe_run(kind, 0, 0, bpc, wpb, n)
        wps = bpc * wpb / 4.0
        return {"waves_per_simd": wps, "simd_cycles_per_inst": round(r["cycles_per_iter"] / 8 / wps, 2),
                "clock_ghz": round(r["clock_ghz"], 3),
                "ginst_per_s": round(r["valu_insts"] / (r["ms"] * 1e-3) / 1e9, 1)}

    runs = [mfma(1, 4), mfma(2, 4), mfma(1, 8)]
    best = max(runs, key=lambda x: x["tflops"])
    return {"workload": "device ceilings: register-only probe loops on every CU",
            "mfma_f16_dense_tflops": best["tflops"], "clock_ghz_under_mfma": best["clock_ghz"],
            "mfma_runs": runs,
            "exp_f32": valu(N.PROBE_VALU_EXP), "fma_f32": valu(N.PROBE_VALU_FMA),
            "mfma_plus_exp": {"2_per_mfma": mfma(2, 4, 2, iters // 2), "4_per_mfma": mfma(2, 4, 4, iters // 2)},
            "nominal_mfma_f16_tflops": 2500.0,
            "note": "FLOPs of v_mfma_f32_32x32x16_f16 = 2*32*32*16 per wave instruction; clock = s_memtime "
                    "cycles / s_memrealtime time (device wall-clock rate), averaged over all waves"}


def decode_long(N, ctx, stream, lens, q, k, v, out, reps):
    """One decode token per sequence at position L_s (append + attention over
    [0, L_s], split-KV at this batch), repeated `reps` times at the same
    position; timed per kernel with HIP events on `stream`."""
    nseq = len(lens)
    ctx.step(0, nseq, q, k, v, out, stream=stream)           # warm-up
    ctx.sync(stream)
    ctx.prof_enable(True)
    ctx.prof_read(reset=True)
    t0 = time.perf_counter()
    for _ in range(reps):
        ctx.step(0, nseq, q, k, v, out, stream=stream)
    ctx.sync(stream)
    el = time.perf_counter() - t0
    ms, launches = ctx.prof_read(reset=True)
    ctx.prof_enable(False)
    # per step; at this batch nda_step fuses the append into the attention launch
    att_ms, comb_ms, app_ms = (ms[kind] / reps for kind in (N.K_DECODE, N.K_COMBINE, N.K_APPEND))
    kv_bytes = float(sum((int(L) + 1) * H * (D + D) * 2 for L in lens))
    io_bytes = nseq * H * D * 4 * 2
    app_bytes = nseq * H * (D + D) * (4 + 2)
    import ndoracle as O
    qh = q.to_array(np.float32, (nseq, H * D))
    oh = out.to_array(np.float32, (nseq, H * D))
    worst = 0.0
    for b in (0, nseq - 1):
        L = int(lens[b])
        kk, vv, _, _ = ctx.kv_read(0, b, 0, L + 1)
        kv = O.kv_view(kk, vv, None, None, H, L + 1, 0, L, O.KV_F16)
        worst = max(worst, float(np.abs(O.attend_view(kv, qh[b], None) - oh[b]).max()))
    return {"workload": "long-context decode: %d sequences, 1 token each over L ~ U[%d,%d] + 1 "
                        "positions, 8 heads x 64, fp16 K/V, 1 layer (append + split-KV attention + merge)"
                        % (nseq, int(lens.min()), int(lens.max())),
            "attend_ms": round(att_ms, 4), "combine_ms": round(comb_ms, 4), "append_ms": round(app_ms, 4),
            "call_ms": round(el * 1e3 / reps, 4),
            "attend_GBps": round((kv_bytes + io_bytes) / (att_ms * 1e-3) / 1e9, 1),
            "step_GBps": round((kv_bytes + io_bytes + app_bytes) / ((att_ms + comb_ms + app_ms) * 1e-3) / 1e9, 1),
            "frac_attend": round((kv_bytes + io_bytes) / (att_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "bytes_per_launch": kv_bytes + io_bytes,
            "max_abs_delta_sampled": worst}


def shared_prefix_leg(N, stream, nseq=1024, npre=213, nmin=32, nmax=64, dsteps=64, layers=LAYERS):
    """Shared prefix: nseq sequences share one npre-token prefix (stored once per
    layer); each prefills n ~ U[nmin, nmax] new tokens causally, then decodes
    dsteps tokens, through `layers` layers. Unique bytes count the prefix once
    per layer; logical bytes count it once per sequence."""
    rng = np.random.default_rng(SEED + 9)
    n = rng.integers(nmin, nmax + 1, nseq)
    window = 384                                   # the engine's KV window
    ctx = N.Context(layers, H, H, D, D, window, kv_dtype=N.KV_F16, max_seqs=nseq + 1)
    builder = nseq
    T = max(npre, int(n.sum()))
    q, k, v, out = (N.DevBuf(T * H * D * 4) for _ in range(4))
    for i, buf in enumerate((q, k, v)):
        buf.fill_normal(T * H * D, 0, SEED + 90 + i, stream=stream)
    for li in range(layers):
        ctx.prefill(li, [npre], q, k, v, out, seq_ids=[builder], stream=stream)
    ctx.advance(1, [builder], npre, stream=stream)
    pid = ctx.prefix_build(builder, stream=stream)
    for b in range(nseq):
        ctx.seq_attach(b, pid, stream=stream)
    ctx.sync(stream)
    ctx.prof_enable(True)
    ctx.prof_read(reset=True)
    t0 = time.perf_counter()
    for li in range(layers):
        ctx.prefill(li, n, q, k, v, out, stream=stream)
    ctx.sync(stream)
    t_pf = time.perf_counter() - t0
    ms, launches = ctx.prof_read(reset=True)
    pf_ms = ms[N.K_PREFILL] / max(1, launches[N.K_PREFILL])
    for b in range(nseq):
        ctx.advance(1, [b], int(n[b]), stream=stream)
    ctx.sync(stream)
    pf_flops = float(sum(H * 2 * (D + D) * (npre * int(x) + int(x) * (int(x) + 1) / 2) for x in n))
    pf_unique = (npre + int(n.sum())) * 2048 + int(n.sum()) * H * D * 4 * 2   # K/V once + q, out
    # the dsteps decode steps timed with the per-kernel events off (each
    # event pair adds enqueue work to these host-bound steps), then the
    # per-kernel split from psteps further steps with them on
    ctx.prof_enable(False)
    t0 = time.perf_counter()
    for _ in range(dsteps):
        for li in range(layers):
            ctx.step(li, nseq, q, k, v, out, stream=stream)
        ctx.advance(nseq, None, 1, stream=stream)
    ctx.sync(stream)
    t_dec = time.perf_counter() - t0
    psteps = 8
    ctx.prof_enable(True)
    ctx.prof_read(reset=True)
    for _ in range(psteps):
        for li in range(layers):
            ctx.step(li, nseq, q, k, v, out, stream=stream)
        ctx.advance(nseq, None, 1, stream=stream)
    ctx.sync(stream)
    ms2, launches2 = ctx.prof_read(reset=True)
    ctx.prof_enable(False)
    # per layer and step: every decode launch (with a shared prefix, the
    # prefix pass and the own-positions pass, which stores the new row) and
    # the merge
    dec_ms = (ms2[N.K_DECODE] + ms2[N.K_COMBINE]) / (psteps * layers)
    # per profiled decode step: the prefix once + every sequence's own
    # positions (steps dsteps .. dsteps + psteps - 1)
    own = sum(int(x) + dsteps + s + 1 for x in n for s in range(psteps)) / psteps
    uniq = npre * 2048 + own * 2048 + nseq * H * D * 4 * 2
    logical = nseq * npre * 2048 + own * 2048 + nseq * H * D * 4 * 2
    import ndoracle as O
    qh = q.to_array(np.float32, (nseq, H * D))
    oh = out.to_array(np.float32, (nseq, H * D))
    worst = 0.0
    for b in (0, nseq - 1):
        pos = ctx.seq_state(b)[0] - 1
        kk, vv, _, _ = ctx.kv_read(layers - 1, b, 0, pos + 1)
        kv = O.kv_view(kk, vv, None, None, H, pos + 1, 0, pos, O.KV_F16)
        want = O.attend_runs(kv, np.arange(pos + 1), [npre, pos + 1 - npre], qh[b], None)
        worst = max(worst, float(np.abs(want - oh[b]).max()))
    for b in range(nseq + 1):
        ctx.seq_reset(b)
    ctx.prefix_free(pid)
    ctx.close()
    return {"workload": "shared prefix: %d sequences share one %d-token prefix (stored once per layer), "
                        "causal prefill of n ~ U[%d,%d] tokens each, then %d decode steps; %d layers, "
                        "8 heads x 64, fp16, window 384" % (nseq, npre, nmin, nmax, dsteps, layers),
            "prefill_kernel_ms": round(pf_ms, 4), "prefill_tflops": round(pf_flops / (pf_ms * 1e-3) / 1e12, 1),
            "prefill_unique_GBps": round(pf_unique / (pf_ms * 1e-3) / 1e9, 1),
            "prefill_wall_ms": round(t_pf * 1e3, 2),
            "decode_tokens_per_s": round(nseq * dsteps / t_dec, 1),
            "decode_kernel_ms": round(dec_ms, 4),
            "decode_kernel_note": "per layer step, from %d further steps with per-kernel events" % psteps,
            "decode_unique_GBps": round(uniq / (dec_ms * 1e-3) / 1e9, 1),
            "decode_logical_GBps": round(logical / (dec_ms * 1e-3) / 1e9, 1),
            "max_abs_delta_sampled": worst}


def engine_session_leg(N, steps=200):
    """The engine drop-in: one session through the C shim (nd_gpu_attention,
    host arrays in and out, as attention() would call it), MHA 8 x 64, int8
    KV, 213 pinned prefix positions + decode; mean latency per layer call,
    beside the reference's own store + attn_heads on the same session shape
    (oracle/_ref, one host thread)."""
    import ndoracle as O
    rng = np.random.default_rng(SEED + 11)
    geom = (1, H, H, D, D, 512)
    g = N.GpuSession(*geom)
    r = O.RefSession(*geom) if O.have_ref() else None
    toks = [[rng.standard_normal(H * D).astype(np.float32) for _ in range(4)] for _ in range(8)]
    for t in range(213):
        g.attention(0, *toks[t % 8])
        g.step_end()
        if r:
            r.attention(0, *toks[t % 8])
            r.step_end()
    g.snapshot()
    if r:
        r.snapshot()
    t0 = time.perf_counter()
    for t in range(steps):
        g.attention(0, *toks[t % 8])
        g.step_end()
    gpu_us = (time.perf_counter() - t0) / steps * 1e6
    ref_us = None
    if r:
        t0 = time.perf_counter()
        for t in range(steps):
            r.attention(0, *toks[t % 8])
            r.step_end()
        ref_us = (time.perf_counter() - t0) / steps * 1e6
        r.close()
    g.close()
    front_gpu_us, front_ref_us = engine_front_timing(N, O, geom, toks, steps)
    return {"workload": "one engine session through nd_gpu_attention (host arrays): MHA 8 x 64, int8 KV, "
                        "window 512, 213 pinned + %d decode positions" % steps,
            "gpu_us_per_layer_call": round(gpu_us, 1),
            "reference_cpu_us_per_layer_call": None if ref_us is None else round(ref_us, 1),
            "front_gpu_us_per_layer_call": round(front_gpu_us, 1),
            "front_reference_cpu_us_per_layer_call": None if front_ref_us is None else round(front_ref_us, 1),
            "note": "latency-bound (host<->device copies + 1 fused launch); throughput comes from batching. "
                    "front_*: raw projections through nd_gpu_attention_raw (3-tap convolution, head norm, "
                    "RoPE, store, attend) beside the reference's tap_projection + zcrms_heads + store + "
                    "attn_heads"}


def engine_front_timing(N, O, geom, toks, steps, taps=3, theta=10000.0):
    """Per-layer-call latency of the shim with the attention front, and of
    the reference engine's own front + attention on one host thread."""
    rng = np.random.default_rng(SEED + 12)
    L, nh, nkv, qk, vd, W = geom
    t = lambda dim: (rng.standard_normal((L, taps, dim)) * 0.5).astype(np.float32)
    fw = O.FrontWeights(t(nh * qk), t(nkv * qk), t(nkv * vd),
                        (rng.standard_normal((L, qk)) * 0.25).astype(np.float32),
                        (rng.standard_normal((L, qk)) * 0.25).astype(np.float32))
    g = N.GpuSession(*geom)
    g.front_init(taps, theta, fw)
    for i in range(213):
        g.attention(0, *toks[i % 8])
        g.step_end()
    g.snapshot()
    t0 = time.perf_counter()
    for i in range(steps):
        g.attention(0, *toks[i % 8])
        g.step_end()
    gpu_us = (time.perf_counter() - t0) / steps * 1e6
    g.close()
    if not O.have_ref():
        return gpu_us, None
    r = O.RefSession(*geom)
    r.front_init(taps, theta)
    for i in range(213):
        q, k, v = r.front(0, fw, *toks[i % 8][:3])
        r.attention(0, q, k, v, toks[i % 8][3])
        r.step_end()
    r.snapshot()
    t0 = time.perf_counter()
    for i in range(steps):
        q, k, v = r.front(0, fw, *toks[i % 8][:3])
        r.attention(0, q, k, v, toks[i % 8][3])
        r.step_end()
    ref_us = (time.perf_counter() - t0) / steps * 1e6
    r.close()
    return gpu_us, ref_us


def cq_tensor_synth(rng, out, inp, group=128, bits=2):
    """A synthetic CQ tensor in the archive's blob layout: random codes,
    positive fp16 norms, a sorted codebook scaled by 1/sqrt(group)."""
    in_pad = (inp + group - 1) // group * group
    packed = rng.integers(0, 256, out * in_pad * bits // 8, dtype=np.uint8)
    norms = rng.uniform(0.25, 2.0, (out, in_pad // group)).astype(np.float16)
    cb = (np.sort(rng.standard_normal(1 << bits)) / np.sqrt(group)).astype(np.float32)
    return np.concatenate([packed, norms.view(np.uint8).ravel()]), cb


def cq_leg(N, stream, rows=B, d_model=768, reps=20):
    """The attention block's CQ projections for a batch of rows, at the
    archive's shapes (12 q / 2 kv heads, qk 48, v 64, d_model 768, 2-bit,
    group 128): prepare x, then q/k/v/gate from it; prepare attn, then
    out_proj. FLOPs = 2 * rows * in * out per projection. Timed on both
    paths: the split-precision one (fp16 MFMA, three products per block:
    what the attention block calls use) and the fp32-MFMA one."""
    rng = np.random.default_rng(SEED + 31)
    shapes = {"q": (576, d_model), "k": (96, d_model), "v": (128, d_model), "gate": (768, d_model),
              "out": (d_model, 768)}
    ts, hosts = {}, {}
    for name, (o, i) in shapes.items():
        blob, cb = cq_tensor_synth(rng, o, i)
        ts[name] = N.CQ(o, i, 128, 2, blob, cb)
        hosts[name] = (o, i, blob, cb)
    x = N.DevBuf(rows * d_model * 4)
    x.fill_normal(rows * d_model, 0, SEED + 32, stream=stream)
    att = N.DevBuf(rows * 768 * 4)
    att.fill_normal(rows * 768, 0, SEED + 33, stream=stream)
    xh = N.DevBuf(max(rows * ts["q"].in_pad * 4, ts["q"].split_bytes(rows)))
    ah = N.DevBuf(max(rows * ts["out"].in_pad * 4, ts["out"].split_bytes(rows)))
    ys = {name: N.DevBuf(rows * o * 4) for name, (o, _) in shapes.items()}
    qkvg = [ts[n] for n in ("q", "k", "v", "gate")]
    yq = [ys[n] for n in ("q", "k", "v", "gate")]

    def block_fp32():
        ts["q"].prepare(rows, x, xh, stream)
        N.cq_gemm_many(qkvg, rows, xh, yq, stream)
        ts["out"].prepare(rows, att, ah, stream)
        ts["out"].gemm(rows, ah, ys["out"], stream)

    def block_split():
        ts["q"].prepare_split(rows, x, xh, stream)
        N.cq_gemm_split_many(qkvg, rows, xh, yq, stream)
        ts["out"].prepare_split(rows, att, ah, stream)
        ts["out"].gemm_split(rows, ah, ys["out"], stream)

    def timed(fn):
        fn()
        tm = N.Timer()
        tm.start(stream)
        for _ in range(reps):
            fn()
        tm.stop(stream)
        return tm.ms() / reps

    import ndoracle as O
    o_, i_, blob, cb = hosts["gate"]
    t = O.CQTensor(o_, i_, 128, 2, blob, np.concatenate([cb, np.zeros(24, np.float32)]))

    def sampled():
        N.device_sync()
        xr = x.to_array(np.float32, (rows, d_model))
        yr = ys["gate"].to_array(np.float32, (rows, 768))
        worst = 0.0
        for r in (0, rows - 1):
            want = O.cq_gemv_lut2(t, O.cq_prepare(t, xr[r]))
            worst = max(worst, float(np.abs(want - yr[r]).max() / (np.abs(want).max() + 1e-30)))
        return worst

    fp32_ms = timed(block_fp32)
    worst_fp32 = sampled()
    split_ms = timed(block_split)
    worst_split = sampled()
    # the q/k/v/gate launch alone, split path (x prepared above)
    ts["q"].prepare_split(rows, x, xh, stream)
    qkvg_ms = timed(lambda: N.cq_gemm_split_many(qkvg, rows, xh, yq, stream))
    flops = sum(2.0 * rows * o * i for o, i in shapes.values())
    qkvg_flops = 2.0 * rows * d_model * (576 + 96 + 128 + 768)
    ref_us = None
    if O.have_ref():
        R = O.ref()
        cb28 = np.concatenate([cb, np.zeros(24, np.float32)])
        xhr = O.cq_prepare(t, x.to_array(np.float32, (rows, d_model))[0])
        lut = np.zeros(t.in_pad // 2 * 16, np.float32)
        yv = np.zeros(o_, np.float32)
        t0 = time.perf_counter()
        n = 0
        while time.perf_counter() - t0 < 1.0:
            R.ref_cq_lut2(o_, i_, 128, t.blob.ctypes.data, cb28.ctypes.data, xhr.ctypes.data,
                          lut.ctypes.data, yv.ctypes.data)
            n += 1
        ref_us = (time.perf_counter() - t0) / n * 1e6
    for q in ts.values():
        q.close()
    qkvg_tf = qkvg_flops / (qkvg_ms * 1e-3) / 1e12
    return {"workload": "CQ projections of one attention block for %d rows: 2-bit, group 128, d_model %d; "
                        "q 576, k 96, v 128, gate 768 from one prepared x in one launch, out_proj 768 "
                        "from 768" % (rows, d_model),
            "block_ms": round(split_ms, 4), "block_tflops": round(flops / (split_ms * 1e-3) / 1e12, 1),
            "qkvg_gemm_ms": round(qkvg_ms, 4), "qkvg_gemm_tflops": round(qkvg_tf, 1),
            "mfma_issued_frac": round(3 * qkvg_tf / 2500.0, 4),
            "rows_per_s": round(rows / (split_ms * 1e-3), 1),
            "max_rel_delta_sampled": worst_split,
            "fp32_path": {"block_ms": round(fp32_ms, 4), "block_tflops": round(flops / (fp32_ms * 1e-3) / 1e12, 1),
                          "max_rel_delta_sampled": worst_fp32},
            "reference_cpu_us_per_row_gate": None if ref_us is None else round(ref_us, 1),
            "note": "split path: fp16 MFMA (v_mfma_f32_32x32x16_f16) on fp16 pairs, three products per block, "
                    "so the MFMA pipe issues 3x the algorithmic FLOPs (mfma_issued_frac is against 2.5 PF); "
                    "fp32 path: v_mfma_f32_32x32x2_f32"}


ENGINE_GEOM = (12, 2, 48, 64)      # q heads, kv heads, qk and v head dims of the archive
ENGINE_D_MODEL, ENGINE_WINDOW = 768, 384


def engine_block_ctx(N, rng, nseq, taps, theta):
    """A context at the archive's attention shapes with synthetic front
    weights and 2-bit CQ projections (group 128) registered for every layer."""
    nh, nkv, qk, vd = ENGINE_GEOM
    dm = ENGINE_D_MODEL
    ctx = N.Context(LAYERS, nh, nkv, qk, vd, ENGINE_WINDOW, kv_dtype=N.KV_INT8, max_seqs=nseq)
    ctx.front_init(taps, theta)
    cqs = []
    shapes = [(nh * qk, dm), (nkv * qk, dm), (nkv * vd, dm), (nh * vd, dm), (dm, nh * vd)]
    for li in range(LAYERS):
        t = lambda dim: (rng.standard_normal((taps, dim)) * 0.5).astype(np.float32)
        ctx.front_weights(li, t(nh * qk), t(nkv * qk), t(nkv * vd),
                          (rng.standard_normal(qk) * 0.25).astype(np.float32),
                          (rng.standard_normal(qk) * 0.25).astype(np.float32))
        layer = []
        for o, i in shapes:
            blob, cb = cq_tensor_synth(rng, o, i)
            layer.append(N.CQ(o, i, 128, 2, blob, cb))
        ctx.block_weights(li, *layer)
        cqs.append(layer)
    return ctx, cqs


def block_prefill_leg(N, stream, nseq=1024, npre=213, nmin=32, nmax=64, reps=3, taps=3, theta=10000.0):
    """The engine's request flow through whole attention blocks, layer-batched:
    one sequence primes the 213-token schema prefix (nda_prefill_block per
    layer), it is shared (nda_prefix_build), then nseq requests attach to it
    and each prefills n ~ U[nmin, nmax] prompt tokens: per layer ONE
    nda_prefill_block over all sum(n) tokens (projections over every row,
    the front per sequence chunk, store + causal attention with the gate,
    out_proj). Archive shapes, int8 KV, 8 layers. Timed: the 8 layer calls
    of one pass, with the profiling events off (best of reps passes after
    one warm-up pass); the attach before each pass is not."""
    rng = np.random.default_rng(SEED + 61)
    n = rng.integers(nmin, nmax + 1, nseq)
    ctx, cqs = engine_block_ctx(N, rng, nseq + 1, taps, theta)
    dm, builder = ENGINE_D_MODEL, nseq
    T = int(n.sum())
    x = [N.DevBuf(max(T, npre) * dm * 4) for _ in range(LAYERS)]
    y = N.DevBuf(max(T, npre) * dm * 4)
    for li in range(LAYERS):
        x[li].fill_normal(max(T, npre) * dm, 0, SEED + 62 + li, stream=stream)
    for li in range(LAYERS):
        ctx.prefill_block(li, 1, [npre], x[li], y, seq_ids=[builder], stream=stream)
    ctx.advance(1, [builder], npre, stream=stream)
    pid = ctx.prefix_build(builder, stream=stream)
    best = None
    # pass 0 is a warm-up (the library sizes its buffers for 1024 sequences
    # and loads this work-group size's kernels on it), then `reps` timed
    # passes, then one more with the profiling events on for the split
    for rep in range(reps + 2):
        for b in range(nseq):
            ctx.seq_attach(b, pid, stream=stream)
        ctx.sync(stream)
        prof = rep == reps + 1
        if prof:
            ctx.prof_enable(True)
            ctx.prof_read(reset=True)
        # the enqueue is host time of the library's calls: no garbage
        # collection of the interpreter's heap (which the earlier legs grow)
        # inside it
        gc.collect()
        gc.disable()
        t0 = time.perf_counter()
        for li in range(LAYERS):
            ctx.prefill_block(li, nseq, n, x[li], y, stream=stream)
        enq = time.perf_counter() - t0
        ctx.sync(stream)
        el = time.perf_counter() - t0
        gc.enable()
        if prof:
            kms, _ = ctx.prof_read(reset=True)
            ctx.prof_enable(False)
        elif rep > 0 and (best is None or el < best):
            best, best_enq = el, enq
    per_pass = {name: round(kms[k], 4) for name, k in
                (("projections_ms", N.K_PROJ), ("front_ms", N.K_FRONT), ("append_ms", N.K_APPEND),
                 ("prefill_ms", N.K_PREFILL))}
    nh, nkv, qk, vd = ENGINE_GEOM
    flops = float(sum(nh * 2 * (qk + vd) * (npre * int(t) + int(t) * (int(t) + 1) / 2) for t in n)) * LAYERS
    for b in range(nseq + 1):
        ctx.seq_reset(b)
    ctx.prefix_free(pid)
    ctx.close()
    for layer in cqs:
        for c in layer:
            c.close()
    return {"workload": "layer-batched prefill of the engine's attention() blocks: %d requests on one shared "
                        "%d-token prefix, n ~ U[%d,%d] prompt tokens each (%d rows per layer call), 12/2 heads, "
                        "qk 48, v 64, d_model 768, int8 KV, 2-bit CQ projections, 3 qkv taps, 8 layers"
                        % (nseq, npre, nmin, nmax, T),
            "prompt_tokens_per_s": round(T / best, 1), "ms_per_pass": round(best * 1e3, 3),
            "host_enqueue_ms": round(best_enq * 1e3, 3),
            "kernel_ms_per_pass": per_pass,
            "attention_tflops": round(flops / (kms[N.K_PREFILL] * 1e-3) / 1e12, 1),
            "note": "parity of the same path is held by tests/test_gpu_prefill_block.py (against the engine's "
                    "attention() stepped one token at a time)"}


def block_leg(N, stream, nseq=B, steps=5, warmup=2, taps=3, theta=10000.0):
    """The engine's whole attention() per layer for a batch of sequences at
    the archive's shapes: 12 q / 2 kv heads, qk 48, v 64, d_model 768,
    window 384, int8 KV (the engine's format), 2-bit CQ projections, 3 qkv
    taps; L ~ U[213, 383] stored positions; 8 layers. A step is 8 x
    nda_attention_block (prepare + q/k/v/gate, front + store, decode with
    the gate, prepare + out_proj), then pos += 1."""
    rng = np.random.default_rng(SEED + 41)
    lens = rng.integers(213, 384, nseq)
    ctx, cqs = engine_block_ctx(N, rng, nseq, taps, theta)
    dm, W = ENGINE_D_MODEL, ENGINE_WINDOW
    for b in range(nseq):
        ctx.seq_set_pos(b, int(lens[b]))
        ctx.seq_reserve(b, W)
    ctx.kv_fill_normal(nseq, seed=SEED + 42, stream=stream)
    x = [N.DevBuf(nseq * dm * 4) for _ in range(LAYERS)]
    y = [N.DevBuf(nseq * dm * 4) for _ in range(LAYERS)]
    for li in range(LAYERS):
        x[li].fill_normal(nseq * dm, 0, SEED + 43 + li, stream=stream)

    def step():
        for li in range(LAYERS):
            ctx.attention_block(li, nseq, x[li], y[li], stream=stream)
        ctx.advance(nseq, None, 1, stream=stream)

    for _ in range(warmup):
        step()
    ctx.sync(stream)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    ctx.sync(stream)
    el = time.perf_counter() - t0
    # the per-kernel split from as many further steps with the profiling
    # events on (each scope's event pair adds a gap between launches, so the
    # timed steps run without them)
    ctx.prof_enable(True)
    ctx.prof_read(reset=True)
    for _ in range(steps):
        step()
    ctx.sync(stream)
    ms, launches = ctx.prof_read(reset=True)
    ctx.prof_enable(False)
    per_step = {name: round(ms[k] / steps, 4) for name, k in
                (("projections_ms", N.K_PROJ), ("front_store_ms", N.K_FRONT), ("decode_ms", N.K_DECODE),
                 ("combine_ms", N.K_COMBINE))}
    # The same decode launches back to back, without the per-kernel events:
    # nda_decode over the 8 layers at the positions reached, on synthetic q
    # and gate (a decode call stores nothing, so repeats read the same cache)
    nh, nkv, qk, vd = ENGINE_GEOM
    qd, gd, od = N.DevBuf(nseq * nh * qk * 4), N.DevBuf(nseq * nh * vd * 4), N.DevBuf(nseq * nh * vd * 4)
    qd.fill_normal(nseq * nh * qk, 0, SEED + 44, stream=stream)
    gd.fill_normal(nseq * nh * vd, 0, SEED + 45, stream=stream)
    for li in range(LAYERS):
        ctx.decode(li, nseq, qd, od, gate=gd, stream=stream)
    tm = N.Timer()
    tm.start(stream)
    for _ in range(steps):
        for li in range(LAYERS):
            ctx.decode(li, nseq, qd, od, gate=gd, stream=stream)
    tm.stop(stream)
    b2b_s = tm.ms() * 1e-3 / (steps * LAYERS)
    for buf in (qd, gd, od):
        buf.free()
    ctx.close()
    for layer in cqs:
        for c in layer:
            c.close()
    # the decode's algorithmic bytes per layer launch: every visible slot's
    # int8 K and V rows and their two scales, for both kv-heads (profiled
    # steps: positions lens + warmup + steps + s, slots min(pos + 1, window)),
    # plus the fp32 q and gate read and the output written (12 heads, as the
    # headline decode counts q and out)
    vis = [np.minimum(lens + warmup + steps + s_ + 1, W) for s_ in range(steps)]
    kv_bytes = float(np.mean([v.sum() for v in vis])) * nkv * (qk + vd + 8)
    b2b_bytes = float(np.minimum(lens + warmup + 2 * steps + 1, W).sum()) * nkv * (qk + vd + 8)
    qgo_bytes = float(nseq) * nh * (qk + 2 * vd) * 4
    dec_bytes = kv_bytes + qgo_bytes
    dec_s = per_step["decode_ms"] * 1e-3 / LAYERS
    return {"workload": "the engine's attention() per layer for %d sequences: 12/2 heads, qk 48, v 64, d_model 768, "
                        "window 384, int8 KV, 2-bit CQ projections, 3 qkv taps, L ~ U[213,383], 8 layers" % nseq,
            "tokens_per_s": round(nseq * steps / el, 1), "ms_per_step": round(el * 1e3 / steps, 4),
            "kernel_ms_per_step": per_step,
            "decode": {"kernel": "decode_mfma_kernel<48,64,rep6>", "bytes_per_launch": round(dec_bytes),
                       "kv_bytes_per_launch": round(kv_bytes),
                       "GBps": round(dec_bytes / dec_s / 1e9, 1) if dec_s > 0 else None,
                       "frac": round(dec_bytes / dec_s / 8e12, 4) if dec_s > 0 else None, "bound": "hbm",
                       "back_to_back_ms": round(b2b_s * 1e3, 4),
                       "back_to_back_frac": round((b2b_bytes + qgo_bytes) / b2b_s / 8e12, 4),
                       "note": "frac: the in-step launches timed by per-kernel events (each pair adds a gap); "
                               "back_to_back: the 8 layers' decode calls alone, one event pair around "
                               "%d steps" % steps},
            "note": "parity of the same path is held by tests/test_gpu_block.py (the engine's own attention() "
                    "golden session replayed within 5e-6)"}


def front_leg(N, stream, steps=5, warmup=2, taps=3, theta=10000.0):
    """The headline decode with the attention front: per layer nda_attention
    takes RAW q/k/v projections (tap convolution over 3 taps, per-head
    ZC-RMSNorm + RoPE, KV store, decode), then pos += 1. The front kernel's
    algorithmic HBM bytes per row: raw q/k/v in, taps-1 history rows read, one
    written, normalised q out, the fp16 K/V row stored:
    4*dcol*(taps+1) + 4*dq + 2*(dk+dv) with dcol = dq+dk+dv."""
    rng = np.random.default_rng(SEED + 21)
    lens = rng.integers(LMIN, LMAX + 1, B)
    total = warmup + 2 * steps              # timed steps, then as many profiled ones
    P = 16
    window = LMAX + total + 16
    need = int(sum((int(L) + total + P - 1) // P for L in lens)) + 64
    ctx = N.Context(LAYERS, H, H, D, D, window, kv_dtype=N.KV_F16, max_seqs=B, page_size=P, max_pages=need)
    ctx.front_init(taps, theta)
    for li in range(LAYERS):
        ctx.front_weights(li, *(rng.standard_normal(shape).astype(np.float32) * np.float32(scale)
                                for shape, scale in (((taps, H * D), 0.5), ((taps, H * D), 0.5),
                                                     ((taps, H * D), 0.5), ((D,), 0.25), ((D,), 0.25))))
    for b in range(B):
        ctx.seq_set_pos(b, int(lens[b]) - 1)
        ctx.seq_reserve(b, total + 1)
    ctx.kv_fill_normal(B, seed=SEED + 22, stream=stream)
    q, kn, vn, out = ([N.DevBuf(B * H * D * 4) for _ in range(LAYERS)] for _ in range(4))
    for li in range(LAYERS):
        for j, buf in enumerate((q[li], kn[li], vn[li])):
            buf.fill_normal(B * H * D, 0, SEED + 100 * li + j, stream=stream)
    ctx.sync(stream)

    def step():
        for li in range(LAYERS):
            ctx.attention(li, B, q[li], kn[li], vn[li], out[li], stream=stream)
        ctx.advance(B, None, 1, stream=stream)

    for _ in range(warmup):
        step()
    ctx.sync(stream)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    ctx.sync(stream)
    el = time.perf_counter() - t0
    # the per-kernel split from as many further steps with the profiling
    # events on (each scope's event pair adds a gap between launches, so the
    # timed steps run without them)
    ctx.prof_enable(True)
    ctx.prof_read(reset=True)
    for _ in range(steps):
        step()
    ctx.sync(stream)
    ms, launches = ctx.prof_read(reset=True)
    ctx.prof_enable(False)
    dq = H * D
    dcol = 3 * dq
    row_bytes = 4 * dcol * (taps + 1) + 4 * dq + 2 * (2 * dq)
    front_ms = ms[N.K_FRONT] / max(1, launches[N.K_FRONT])
    gbs = B * row_bytes / (front_ms * 1e-3) / 1e9
    ctx.close()
    for bufs in (q, kn, vn, out):
        for bb in bufs:
            bb.free()
    return {"workload": "batched decode with the attention front: 4096 sequences, 8 heads x 64, fp16 K/V, "
                        "L ~ U[213,1024], raw q/k/v -> %d-tap convolution + head norm + RoPE + store + "
                        "attend, 8 layers" % taps,
            "tokens_per_s": round(B * steps / el, 1), "ms_per_step": round(el * 1e3 / steps, 4),
            "front_kernel_ms": round(front_ms, 4), "decode_kernel_ms": round(
                ms[N.K_DECODE] / max(1, launches[N.K_DECODE]), 4),
            "front_GBps": round(gbs, 1), "front_frac": round(gbs / HBM_PEAK_GBS, 4),
            "front_bytes_per_launch": B * row_bytes}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--split-chunk", type=int, default=0)
    ap.add_argument("--page-size", type=int, default=16)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--calib", action="store_true",
                    help="first run a 4 GiB device copy (known traffic, for counter calibration)")
    ap.add_argument("--leg", choices=["cq", "cq_prefill", "block", "block_prefill", "prefill", "front", "shared",
                                      "ceiling"],
                    help="run only this leg and print its JSON object (for profiling one kernel family)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this library has no multi-GPU path "
              "(decode would shard by sequence with no exchange between GPUs)", file=sys.stderr)
        sys.exit(2)

    import ndattn as N

    name, cus = N.device_info()
    log("device:", name, "CUs:", cus)
    if args.calib:
        nb = 4 << 30
        src, dst = N.DevBuf(nb), N.DevBuf(nb)
        src.fill_normal(nb // 4, 0, 1)
        for _ in range(3):
            N._check(N.lib().nda_d2d(dst.value, src.value, nb, None))
        N.device_sync()
        log("calibration copy: 3 x %d bytes read + written" % nb)
        src.free()
        dst.free()
    if args.leg:
        stream = N.vp()
        N._check(N.lib().nda_stream_create(N.C.byref(stream)))
        legs = {"cq": lambda: cq_leg(N, stream), "cq_prefill": lambda: cq_leg(N, stream, rows=49787, reps=5),
                "block": lambda: block_leg(N, stream), "block_prefill": lambda: block_prefill_leg(N, stream),
                "prefill": lambda: prefill_leg(N, stream), "front": lambda: front_leg(N, stream),
                "shared": lambda: shared_prefix_leg(N, stream), "ceiling": lambda: ceiling_leg(N)}
        print(json.dumps(legs[args.leg]()), flush=True)
        return
    rng = np.random.default_rng(SEED)
    lens = rng.integers(LMIN, LMAX + 1, B)          # positions attended at the first step
    total_steps = args.warmup + args.steps
    window = LMAX + total_steps + 16
    P = args.page_size
    need_pages = int(sum((int(L) + total_steps + P - 1) // P for L in lens)) + 64
    ctx = N.Context(LAYERS, H, H, D, D, window, kv_dtype=N.KV_F16, max_seqs=B, page_size=P,
                    max_pages=need_pages, split_chunk=args.split_chunk)
    log("pool GiB: %.1f" % (ctx.device_bytes / 2 ** 30))
    stream = N.vp()
    N._check(N.lib().nda_stream_create(N.C.byref(stream)))
    for b in range(B):
        ctx.seq_set_pos(b, int(lens[b]) - 1)
        ctx.seq_reserve(b, total_steps + 1)
    ctx.kv_fill_normal(B, seed=SEED, stream=stream)
    # per-layer q, new k/v, out: resident in HBM
    q = [N.DevBuf(B * H * D * 4) for _ in range(LAYERS)]
    kn = [N.DevBuf(B * H * D * 4) for _ in range(LAYERS)]
    vn = [N.DevBuf(B * H * D * 4) for _ in range(LAYERS)]
    out = [N.DevBuf(B * H * D * 4) for _ in range(LAYERS)]
    for li in range(LAYERS):
        q[li].fill_normal(B * H * D, 0, SEED + 10 * li + 1, stream=stream)
        kn[li].fill_normal(B * H * D, 0, SEED + 10 * li + 2, stream=stream)
        vn[li].fill_normal(B * H * D, 0, SEED + 10 * li + 3, stream=stream)
    ctx.sync(stream)

    def step():
        for li in range(LAYERS):
            ctx.step(li, B, q[li], kn[li], vn[li], out[li], stream=stream)   # append + decode
        ctx.advance(B, None, 1, stream=stream)

    for _ in range(args.warmup):
        step()
    ctx.sync(stream)
    N.device_sync()
    # algorithmic bytes of the timed steps: lengths grow by one per step
    base = lens + args.warmup
    attended = sum(int(base.sum()) + s * B for s in range(args.steps))   # positions read, per layer
    row = H * 2 * D * 2                                   # K + V bytes per position, all heads
    qo = B * H * D * 4 * 2                                # q read + out write per layer launch
    dec_bytes = attended * row + args.steps * qo          # per layer, all timed steps
    app_bytes = B * (2 * H * D * 4 + 2 * H * D * 2)       # read k,v fp32 + write fp16, per launch

    ctx.prof_enable(True)
    ctx.prof_read(reset=True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    ctx.sync(stream)
    N.device_sync()
    el = time.perf_counter() - t0
    ms, launches = ctx.prof_read(reset=True)
    ctx.prof_enable(False)

    ms_per_step = el * 1e3 / args.steps
    tok_s = B * args.steps / el
    dec_ms = ms[N.K_DECODE] / max(1, launches[N.K_DECODE])
    app_ms = ms[N.K_APPEND] / max(1, launches[N.K_APPEND])
    dec_bytes_per_launch = dec_bytes / args.steps
    achieved = dec_bytes_per_launch / (dec_ms * 1e-3) / 1e9
    step_bytes = LAYERS * (dec_bytes_per_launch + app_bytes)
    log("step %.3f ms | decode kernel %.3f ms (%d launches) %.0f GB/s | append %.4f ms | combine %d" %
        (ms_per_step, dec_ms, launches[N.K_DECODE], achieved, app_ms, launches[N.K_COMBINE]))

    # sampled parity of the last step against the oracle (not timed)
    import ndoracle as O
    worst = 0.0
    qh = q[LAYERS - 1].to_array(np.float32, (B, H * D))
    oh = out[LAYERS - 1].to_array(np.float32, (B, H * D))
    for b in rng.choice(B, 8, replace=False):
        pos = ctx.seq_state(int(b))[0] - 1            # the last decode attended [0, pos]
        k, v, _, _ = ctx.kv_read(LAYERS - 1, int(b), 0, pos + 1)
        kv = O.kv_view(k, v, None, None, H, pos + 1, 0, pos, O.KV_F16)
        want = O.attend_view(kv, qh[b], None)
        worst = max(worst, float(np.abs(want - oh[b]).max()))
    log("sampled max |delta| vs oracle: %.3g" % worst)

    ctx.close()
    for bufs in (q, kn, vn, out):
        for bb in bufs:
            bb.free()
    front = front_leg(N, stream)
    log("front: %.0f tok/s, step %.3f ms, front kernel %.4f ms (%.0f GB/s)" % (
        front["tokens_per_s"], front["ms_per_step"], front["front_kernel_ms"], front["front_GBps"]))
    block = block_leg(N, stream)
    log("block: %.0f tok/s, step %.3f ms, per step %s" % (block["tokens_per_s"], block["ms_per_step"],
                                                          block["kernel_ms_per_step"]))
    block_pf = None
    if not args.no_prefill:
        block_pf = block_prefill_leg(N, stream)
        log("block prefill: %.0f prompt tok/s, pass %.3f ms, per pass %s" % (
            block_pf["prompt_tokens_per_s"], block_pf["ms_per_pass"], block_pf["kernel_ms_per_pass"]))
    cq = cq_leg(N, stream)
    cq_pf = cq_leg(N, stream, rows=49787, reps=5)      # the row count of the block prefill leg
    log("cq: block %.4f ms (%.1f TFLOP/s; fp32 path %.4f ms), q/k/v/gate gemm %.4f ms (%.1f TFLOP/s), "
        "sampled rel delta %.3g" % (cq["block_ms"], cq["block_tflops"], cq["fp32_path"]["block_ms"],
                                    cq["qkvg_gemm_ms"], cq["qkvg_gemm_tflops"], cq["max_rel_delta_sampled"]))
    engine = engine_session_leg(N)
    log("engine session: GPU %.1f us per layer call, reference CPU %s us" % (
        engine["gpu_us_per_layer_call"], engine["reference_cpu_us_per_layer_call"]))
    shared = None
    if not args.no_prefill:
        shared = shared_prefix_leg(N, stream)
        log("shared prefix: prefill %.1f TFLOP/s (%.1f GB/s unique), decode %.0f tok/s, %.0f GB/s unique / "
            "%.0f GB/s logical, sampled max |delta| %.3g" % (
                shared["prefill_tflops"], shared["prefill_unique_GBps"], shared["decode_tokens_per_s"],
                shared["decode_unique_GBps"], shared["decode_logical_GBps"], shared["max_abs_delta_sampled"]))
    ceiling = ceiling_leg(N)
    log("ceiling: dense fp16 MFMA %.1f TFLOP/s at %.3f GHz; exp %.2f, fma %.2f SIMD cycles per wave instruction" % (
        ceiling["mfma_f16_dense_tflops"], ceiling["clock_ghz_under_mfma"],
        ceiling["exp_f32"]["simd_cycles_per_inst"], ceiling["fma_f32"]["simd_cycles_per_inst"]))
    prefill = None
    if not args.no_prefill:
        prefill = prefill_leg(N, stream)
        prefill["peak_measured"] = ceiling["mfma_f16_dense_tflops"]
        prefill["frac_measured"] = round(prefill["tflops"] / ceiling["mfma_f16_dense_tflops"], 4)
        log("prefill: %.1f TFLOP/s (%.3f of 2.5 PF, %.3f of the measured %.0f), kernel %.3f ms, sampled max "
            "|delta| %.3g" % (prefill["tflops"], prefill["frac"], prefill["frac_measured"], prefill["peak_measured"],
                              prefill["kernel_ms"], prefill["max_abs_delta_sampled"]))

    cfg2 = config2_leg(N, stream)
    log("config 2 prefill (1 x 256 tokens, 8 layers, int8): %.3f ms, %.0f prompt tok/s" % (
        cfg2["ms_per_prefill"], cfg2["prompt_tokens_per_s"]))

    cpu = cpu_1 = cpu_ref = cpu_long = cpu_long_1 = cpu_cfg = None
    if not args.no_cpu:
        ncores, cores_how = usable_cores()
        log("cpu legs: %d cores (%s)" % (ncores, cores_how))
        sec = args.cpu_seconds
        c_tok, _, sample = cpu_port_f16(lens, sec * 0.3, ncores)
        cpu = {"value": round(c_tok, 1), "unit": "tokens/s", "cores": ncores, "kind": "port",
               "sample": sample + ", fp16 KV, no gate, oracle attn_heads restatement"}
        c1, _, sample1 = cpu_port_f16(lens, sec * 0.2, 1, nseq=32)
        cpu_1 = {"value": round(c1, 1), "unit": "tokens/s", "cores": 1, "kind": "port",
                 "sample": sample1 + ", fp16 KV, no gate, oracle attn_heads restatement"}
        log("cpu baseline (port, fp16): %.1f tok/s on %d threads, %.1f tok/s on 1" % (c_tok, ncores, c1))
        cpu_ref = cpu_reference_int8(lens, sec * 0.15, (1, ncores))
        if cpu_ref:
            cpu_ref = {"1": cpu_ref[1], str(ncores): cpu_ref[ncores]}
            log("cpu reference (int8): %.1f tok/s on 1 thread, %.1f on %d" % (
                cpu_ref["1"]["value"], cpu_ref[str(ncores)]["value"], ncores))
        # the long-context decode (8K-32K positions), a 16-sequence subsample
        rng_l = np.random.default_rng(SEED + 5)
        lt, lf, lsample = cpu_port_f16(rng_l.integers(8192, 32769, 256), sec * 0.2, ncores, nseq=max(16, ncores),
                                       seed_off=5)
        cpu_long = {"value": round(lt * LAYERS, 1), "unit": "tokens/s per layer", "cores": ncores,
                    "kind": "port", "attention_GFLOPs": round(lf / 1e9, 2),
                    "sample": lsample + ", fp16 KV, L ~ U[8192, 32768], one layer"}
        log("cpu long-context decode (port): %.1f tok/s per layer, %.1f GFLOP/s on %d threads" % (
            lt * LAYERS, lf / 1e9, ncores))
        lt1, lf1, lsample1 = cpu_port_f16(rng_l.integers(8192, 32769, 256), sec * 0.15, 1, nseq=2, seed_off=5)
        cpu_long_1 = {"value": round(lt1 * LAYERS, 1), "unit": "tokens/s per layer", "cores": 1,
                      "kind": "port", "attention_GFLOPs": round(lf1 / 1e9, 2),
                      "sample": lsample1 + ", fp16 KV, L ~ U[8192, 32768], one layer"}
        log("cpu long-context decode (port): %.1f tok/s per layer on 1 thread" % (lt1 * LAYERS))
        cpu_cfg = {"cores_available": ncores, "cores_source": cores_how}
        # config 2: the reference's own token-by-token prefill, int8
        nt2 = min(ncores, H)               # the seam splits 8 heads: more threads have no work
        c2 = cpu_reference_prefill_int8((1, nt2) if nt2 > 1 else (1,))
        if c2:
            cpu_cfg["config2_prefill_reference_int8"] = {str(k): v for k, v in c2.items()}
            log("cpu config 2 prefill (reference, int8): %s" % ", ".join(
                "%.1f ms on %d" % (v["ms_per_prefill"], k) for k, v in c2.items()))
        # config 4: suffix prefill after the shared 213-token prefix, subsamples
        rng4 = np.random.default_rng(SEED + 9)
        n4 = rng4.integers(32, 65, 1024)
        c4 = {}
        for nt, S in ((1, 16), (ncores, max(128, 8 * ncores))):
            t, f, ts = cpu_port_prefill_f16([213] * S, n4[:S], nt, seed_off=31)
            c4[str(nt)] = {"value": round(float(n4[:S].sum()) / t, 1), "unit": "prompt tokens/s per layer",
                           "cores": nt, "kind": "port", "attention_GFLOPs": round(f / t / 1e9, 3),
                           "sample": "the first %d of the 1024 sequences (n ~ U[32,64], %d tokens) after the "
                                     "213-token prefix, one layer, fp16 KV; median of 5 (%.3f-%.3f s)"
                                     % (S, int(n4[:S].sum()), ts[0], ts[-1])}
        cpu_cfg["config4_suffix_prefill_port_f16"] = c4
        log("cpu config 4 suffix prefill (port): %s" % ", ".join(
            "%.1f GFLOP/s on %s" % (v["attention_GFLOPs"], k) for k, v in c4.items()))
        # config 5: the 512-token chunk over 8K-32K stored positions, subsamples
        rng5 = np.random.default_rng(SEED + 5)
        L5 = rng5.integers(8192, 32769, 256) + 1
        c5 = {}
        for nt, S, Tk in ((1, 1, 8), (ncores, ncores, 8)):
            t, f, ts = cpu_port_prefill_f16(L5[:S], [Tk] * S, nt, seed_off=41)
            full = float(sum(H * 2 * (D + D) * (512 * int(L) + 512 * 513 / 2) for L in L5))
            c5[str(nt)] = {"value": round(f / t / 1e9, 3), "unit": "attention GFLOP/s",
                           "cores": nt, "kind": "port", "chunk_tokens_per_s": round(S * Tk / t, 2),
                           "full_chunk_s_estimate": round(full / (f / t), 1),
                           "sample": "the first %d tokens of the 512-token chunk of the first %d of the 256 "
                                     "sequences (L ~ U[8192,32768]), one layer, fp16 KV; median of 5 (%.3f-%.3f "
                                     "s); the full chunk scaled by its FLOPs" % (Tk, S, ts[0], ts[-1])}
        cpu_cfg["config5_chunk_prefill_port_f16"] = c5
        log("cpu config 5 chunk (port): %s" % ", ".join(
            "%.2f GFLOP/s on %s" % (v["value"], k) for k, v in c5.items()))

    res = {
        "metric": "decode attn tokens/s + HBM GB/s (% peak) at B=4096; prefill TFLOP/s",
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: K/V N(0,1) from a counter-based generator on device, q/k_new/v_new N(0,1)",
        "config": {"workload": "batched decode: 4096 sequences, 8 heads x 64, fp16 K/V, "
                               "L ~ U[213,1024], 1 token x 8 layers (append + attend)",
                   "global_batch": B, "layers": LAYERS, "heads": H, "head_dim": D,
                   "kv_len": [LMIN, LMAX], "page_size": P, "seed": SEED,
                   "step_GB": round(step_bytes / 1e9, 3),
                   "step_GBps": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 1)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": committed_traffic(),
                     "kernel": "attend_kernel<f16,64,64,rep1>", "kernel_ms": round(dec_ms, 4),
                     "bytes_per_launch": int(dec_bytes_per_launch)},
        "cpu_baseline": cpu,
        "cpu_baseline_1core": cpu_1,
        "cpu_reference_int8": cpu_ref,
        "cpu_long_context_decode": cpu_long,
        "cpu_long_context_decode_1core": cpu_long_1,
        "cpu_prefill_configs": cpu_cfg,
        "config2_prefill": cfg2,
        "prefill": prefill,
        "device_ceiling": ceiling,
        "engine_session": engine,
        "front": front,
        "cq_projections": cq,
        "cq_projections_prefill_rows": cq_pf,
        "attention_block": block,
        "attention_block_prefill": block_pf,
        "shared_prefix": shared,
        "max_abs_delta_sampled": worst,
        "device": name,
        "host": host_info(),
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
