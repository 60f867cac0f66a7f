"""The long-context and shared-prefix workloads at their own sizes on the GPU,
against the oracle (ndo_attend / ndo_attend_runs, the engine's attn_heads
restated, engine/src/nd_model.c:2105-2359, dispatch :2451-2483).

- Long context: fp16 K/V, 8 heads x 64, KV lengths from 8192 to 32768 (one
  sequence at exactly 32768), keys with 8-sigma outliers (a K row times 8,
  exact in fp16, with probability 1e-3 per position and head). One decode
  token through the split-KV attention and its merge, then a 512-token causal
  chunk on top. Every decode row is checked, and every chunk row of the
  32768- and 8192-key sequences.
- Shared prefix: 1024 sequences attached to one 213-token prefix per layer (8
  layers, as the workload has), causal suffixes of 32-64 tokens, then 64
  decode steps; sampled rows of the prefill and of every decode step are
  checked.
- The long-context workload at the size the benchmark times (256 sequences),
  and a short prefix with long own tails (the decode's shared-prefix pass
  must not be taken).

Bar: max |delta| <= 1e-3 (fp32 accumulate)."""
import os
import sys
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import ndoracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3
THREADS = 16        # oracle rows in parallel (ctypes calls release the GIL)


def nda():
    import ndattn
    return ndattn


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


def maxdiff(a, b):
    return float(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)).max())


def f16(x):
    return O.f32_to_f16_bits(x)


def outliers(rng, x, p=1e-3):
    """Rows [pos][head] of x multiplied by 8 with probability p each."""
    m = rng.random(x.shape[:2]) < p
    x[m] *= np.float32(8.0)
    return int(m.sum())


def test_long_context_decode_then_512_token_chunk():
    N = nda()
    nh, d, CH, W = 8, 64, 512, 33300
    rng = np.random.default_rng(5)
    lens = [32768, 8192, int(rng.integers(8193, 32768)), int(rng.integers(8193, 32768))]
    B = len(lens)
    say("long context: KV lengths", lens)
    ctx = N.Context(1, nh, nh, d, d, W, kv_dtype=O.KV_F16, max_seqs=B)
    n_out = 0
    for b, L in enumerate(lens):
        kf = rng.standard_normal((L - 1, nh, d)).astype(np.float32)
        n_out += outliers(rng, kf)
        vf = rng.standard_normal((L - 1, nh, d)).astype(np.float32)
        ctx.kv_write(0, b, 0, f16(kf), f16(vf))
        ctx.seq_set_pos(b, L - 1)
    del kf, vf
    # the decode token: stored at L-1 (append), then attends L positions
    q = rng.standard_normal((B, nh, d)).astype(np.float32)
    k = rng.standard_normal((B, nh, d)).astype(np.float32)
    n_out += outliers(rng, k)
    v = rng.standard_normal((B, nh, d)).astype(np.float32)
    g = rng.standard_normal((B, nh, d)).astype(np.float32)
    say("decode through split-KV;", n_out, "outlier key rows")
    dout = N.DevBuf(B * nh * d * 4)
    ctx.prof_enable(True)
    ctx.prof_read(reset=True)
    ctx.step(0, B, N.DevBuf.from_array(q), N.DevBuf.from_array(k), N.DevBuf.from_array(v), dout,
             gate=N.DevBuf.from_array(g))
    ctx.sync()
    _, launches = ctx.prof_read(reset=True)
    ctx.prof_enable(False)
    assert launches[N.K_COMBINE] > 0, "rows must be split and merged"
    got = dout.to_array(np.float32, (B, nh * d))
    worst_dec = 0.0
    for b, L in enumerate(lens):
        kk, vv, _, _ = ctx.kv_read(0, b, 0, L)
        view = O.kv_view(kk, vv, None, None, nh, L, 0, L - 1, O.KV_F16)
        worst_dec = max(worst_dec, maxdiff(got[b], O.attend_view(view, q[b].ravel(), g[b].ravel())))
    say("decode worst vs oracle", worst_dec)
    assert worst_dec <= TOL, worst_dec
    ctx.advance(B, None, 1)

    # the 512-token causal chunk at positions L .. L+511
    T = B * CH
    q = rng.standard_normal((T, nh, d)).astype(np.float32)
    k = rng.standard_normal((T, nh, d)).astype(np.float32)
    outliers(rng, k)
    v = rng.standard_normal((T, nh, d)).astype(np.float32)
    g = rng.standard_normal((T, nh, d)).astype(np.float32)
    say("512-token chunk on", B, "sequences")
    dout = N.DevBuf(T * nh * d * 4)
    ctx.prefill(0, [CH] * B, N.DevBuf.from_array(q), N.DevBuf.from_array(k), N.DevBuf.from_array(v), dout,
                gate=N.DevBuf.from_array(g))
    ctx.sync()
    got = dout.to_array(np.float32, (T, nh * d))
    worst = 0.0
    for b, L in enumerate(lens):
        end = L + CH
        kk, vv, _, _ = ctx.kv_read(0, b, 0, end)
        rows = range(CH) if b < 2 else sorted(rng.choice(CH, 32, replace=False))

        def one(t, b=b, L=L, kk=kk, vv=vv, end=end):
            view = O.kv_view(kk, vv, None, None, nh, end, 0, L + t, O.KV_F16)
            r = b * CH + t
            return maxdiff(got[r], O.attend_view(view, q[r].ravel(), g[r].ravel()))

        with ThreadPoolExecutor(THREADS) as ex:
            w = max(ex.map(one, rows))
        say("chunk rows checked", len(rows), "of sequence", b, "(L=%d): worst %.3g" % (L, w))
        worst = max(worst, w)
    assert worst <= TOL, worst
    ctx.close()


def test_shared_prefix_1024_sequences_64_decode_steps():
    N = nda()
    nh, d, B, npre, W, LAYERS, STEPS = 8, 64, 1024, 213, 384, 8, 64
    rng = np.random.default_rng(4)
    ctx = N.Context(LAYERS, nh, nh, d, d, W, kv_dtype=O.KV_F16, max_seqs=B + 1)
    say("shared prefix: building the 213-token prefix")
    for li in range(LAYERS):
        bufs = [N.DevBuf(npre * nh * d * 4) for _ in range(4)]
        for i, bb in enumerate(bufs[:3]):
            bb.fill_normal(npre * nh * d, 0, 1000 + 10 * li + i)
        ctx.prefill(li, [npre], bufs[0], bufs[1], bufs[2], bufs[3], seq_ids=[B])
    ctx.advance(1, [B], npre)
    pid = ctx.prefix_build(B)
    for b in range(B):
        ctx.seq_attach(b, pid)
    n = rng.integers(32, 65, B)
    T = int(n.sum())
    starts = np.concatenate([[0], np.cumsum(n)[:-1]])
    sample = sorted(int(x) for x in rng.choice(B, 12, replace=False))
    worst = 0.0

    def check(li, b, pos, qrow, grow, out_row):
        kk, vv, _, _ = ctx.kv_read(li, b, 0, pos + 1)
        view = O.kv_view(kk, vv, None, None, nh, pos + 1, 0, pos, O.KV_F16)
        want = O.attend_runs(view, np.arange(pos + 1), [npre, pos + 1 - npre], qrow, grow)
        return maxdiff(out_row, want)

    for li in range(LAYERS):
        say("suffix prefill, layer", li, "rows", T)
        dq, dk, dv, dg = (N.DevBuf(T * nh * d * 4) for _ in range(4))
        for i, bb in enumerate((dq, dk, dv, dg)):
            bb.fill_normal(T * nh * d, 0, 2000 + 10 * li + i)
        dout = N.DevBuf(T * nh * d * 4)
        ctx.prefill(li, n, dq, dk, dv, dout, gate=dg, seq_ids=list(range(B)))
        ctx.sync()
        q = dq.to_array(np.float32, (T, nh * d))
        g = dg.to_array(np.float32, (T, nh * d))
        got = dout.to_array(np.float32, (T, nh * d))
        for b in sample:
            for t in range(int(n[b])):
                r = int(starts[b]) + t
                worst = max(worst, check(li, b, npre + t, q[r], g[r], got[r]))
    say("suffix prefill worst", worst)
    for b in range(B):
        ctx.advance(1, [b], int(n[b]))

    dq, dk, dv, dout = (N.DevBuf(B * nh * d * 4) for _ in range(4))
    for step in range(STEPS):
        for li in range(LAYERS):
            for i, bb in enumerate((dq, dk, dv)):
                bb.fill_normal(B * nh * d, 0, 5000 + 100 * step + 10 * li + i)
            ctx.step(li, B, dq, dk, dv, dout)
            ctx.sync()
            q = dq.to_array(np.float32, (B, nh * d))
            got = dout.to_array(np.float32, (B, nh * d))
            assert np.isfinite(got).all()
            picks = sorted(int(x) for x in rng.choice(B, 3, replace=False))
            for b in picks:
                pos = ctx.seq_state(b)[0]
                worst = max(worst, check(li, b, pos, q[b], None, got[b]))
        ctx.advance(B, None, 1)
        if step % 16 == 15:
            say("decode step", step + 1, "worst so far", worst)
    assert worst <= TOL, worst
    for b in range(B):
        ctx.seq_reset(b)
    ctx.prefix_free(pid)
    ctx.close()


def test_short_prefix_long_tails_skip_the_prefix_pass():
    """1024 sequences on one 40-token prefix, each with 900-1400 positions of
    its own: rows span more than four prefix lengths, so the decode keeps
    the single VALU pass (one attention launch, no prefix pass, no merge)
    instead of cutting every row into prefix-sized chunks. Sampled rows meet
    the oracle."""
    N = nda()
    nh, d, W, B, npre = 8, 64, 1600, 1024, 40
    rng = np.random.default_rng(6)
    ctx = N.Context(1, nh, nh, d, d, W, kv_dtype=O.KV_F16, max_seqs=B + 1)
    bufs = [N.DevBuf(npre * nh * d * 4) for _ in range(4)]
    for i, bb in enumerate(bufs[:3]):
        bb.fill_normal(npre * nh * d, 0, 3000 + i)
    ctx.prefill(0, [npre], bufs[0], bufs[1], bufs[2], bufs[3], seq_ids=[B])
    ctx.advance(1, [B], npre)
    pid = ctx.prefix_build(B)
    own = rng.integers(900, 1401, B)
    for b in range(B):
        ctx.seq_attach(b, pid)
        ctx.seq_set_pos(b, npre + int(own[b]))
    ctx.kv_fill_normal(B, seed=3100)
    q, k, v, out = (N.DevBuf(B * nh * d * 4) for _ in range(4))
    for i, bb in enumerate((q, k, v)):
        bb.fill_normal(B * nh * d, 0, 3200 + i)
    ctx.sync()
    say("short prefix, long own tails: one decode step of", B, "sequences")
    ctx.prof_enable(True)
    ctx.prof_read(reset=True)
    ctx.step(0, B, q, k, v, out)
    ctx.sync()
    _, launches = ctx.prof_read(reset=True)
    ctx.prof_enable(False)
    assert launches[N.K_DECODE] == 1 and launches[N.K_COMBINE] == 0, launches
    qh = q.to_array(np.float32, (B, nh * d))
    got = out.to_array(np.float32, (B, nh * d))
    worst = 0.0
    for b in sorted(int(x) for x in rng.choice(B, 8, replace=False)):
        pos = ctx.seq_state(b)[0]
        kk, vv, _, _ = ctx.kv_read(0, b, 0, pos + 1)
        view = O.kv_view(kk, vv, None, None, nh, pos + 1, 0, pos, O.KV_F16)
        worst = max(worst, maxdiff(got[b], O.attend_view(view, qh[b])))
    say("worst vs oracle", worst)
    assert worst <= TOL
    for b in range(B + 1):
        ctx.seq_reset(b)
    ctx.prefix_free(pid)
    ctx.close()


def test_long_context_at_the_benchmarked_geometry():
    """The long-context workload at the size the benchmark times it: 256
    sequences with L ~ U[8192, 32768] stored positions (device-filled N(0,1)),
    a block of 8 K rows with 8-sigma outliers (times 8, exact in fp16) per
    sequence, one decode token (the split-KV plan of this batch and its merge),
    then a 512-token causal chunk over every sequence (this batch's prefill
    work order, longest items first over the eight XCD ranges). Decode rows
    and three chunk rows of 16 sequences are checked against the oracle."""
    N = nda()
    nh, d, CH, B, P = 8, 64, 512, 256, 16
    rng = np.random.default_rng(7)
    lens = rng.integers(8192, 32769, B)
    W = 32768 + CH + 16
    need = int(sum((int(L) + CH + P) // P for L in lens)) + 64
    ctx = N.Context(1, nh, nh, d, d, W, kv_dtype=O.KV_F16, max_seqs=B, page_size=P, max_pages=need)
    for b in range(B):
        ctx.seq_set_pos(b, int(lens[b]))
    ctx.kv_fill_normal(B, seed=8100)
    for b in range(B):
        p0 = int(rng.integers(0, int(lens[b]) - 8))
        kf = (rng.standard_normal((8, nh, d)) * 8.0).astype(np.float32)
        vf = rng.standard_normal((8, nh, d)).astype(np.float32)
        ctx.kv_write(0, b, p0, f16(kf), f16(vf))
    sample = sorted(int(x) for x in rng.choice(B, 16, replace=False))
    say("benchmarked long-context geometry: %d sequences, L %d..%d" % (B, lens.min(), lens.max()))
    q, k, v, g, out = (N.DevBuf(B * nh * d * 4) for _ in range(5))
    for i, bb in enumerate((q, k, v, g)):
        bb.fill_normal(B * nh * d, 0, 8200 + i)
    ctx.prof_enable(True)
    ctx.prof_read(reset=True)
    ctx.step(0, B, q, k, v, out, gate=g)
    ctx.sync()
    _, launches = ctx.prof_read(reset=True)
    ctx.prof_enable(False)
    assert launches[N.K_COMBINE] > 0, "the decode must split rows and merge them"
    qh, gh = q.to_array(np.float32, (B, nh * d)), g.to_array(np.float32, (B, nh * d))
    got = out.to_array(np.float32, (B, nh * d))
    worst = 0.0
    for b in sample:
        L = int(lens[b])
        kk, vv, _, _ = ctx.kv_read(0, b, 0, L + 1)
        view = O.kv_view(kk, vv, None, None, nh, L + 1, 0, L, O.KV_F16)
        worst = max(worst, maxdiff(got[b], O.attend_view(view, qh[b], gh[b])))
    say("decode, 16 sequences: worst vs oracle", worst)
    assert worst <= TOL, worst
    ctx.advance(B, None, 1)

    T = B * CH
    q, k, v, g, out = (N.DevBuf(T * nh * d * 4) for _ in range(5))
    for i, bb in enumerate((q, k, v, g)):
        bb.fill_normal(T * nh * d, 0, 8300 + i)
    say("512-token chunk on", B, "sequences")
    ctx.prefill(0, [CH] * B, q, k, v, out, gate=g)
    ctx.sync()
    qh, gh = q.to_array(np.float32, (T, nh * d)), g.to_array(np.float32, (T, nh * d))
    got = out.to_array(np.float32, (T, nh * d))
    worst = 0.0
    for b in sample:
        L = int(lens[b]) + 1
        kk, vv, _, _ = ctx.kv_read(0, b, 0, L + CH)
        for t in (0, 255, CH - 1):
            r = b * CH + t
            view = O.kv_view(kk, vv, None, None, nh, L + CH, 0, L + t, O.KV_F16)
            worst = max(worst, maxdiff(got[r], O.attend_view(view, qh[r], gh[r])))
    say("chunk, 16 sequences x 3 rows: worst vs oracle", worst)
    assert worst <= TOL, worst
    ctx.close()
