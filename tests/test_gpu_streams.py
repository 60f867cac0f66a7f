"""Calls on one context from two streams, alternating, with nothing
synchronised between them: each call rewrites the context's device tables
(sequence states, page tables, the GQA decode's longest-first row order) that
the previous call's kernels, queued on the other stream, may still read. The
context orders a call on a new stream after the work queued on the previous
one, so every step must still match the oracle (ndo_attend, the engine's
attn_heads restated, engine/src/nd_model.c:2105-2359; one session's calls are
serial in the engine, engine/include/nd_quant.h:221-228).

Engine shape (12 query / 2 kv heads, qk 48, v 64, int8 K/V, window 384), 600
sequences: the MFMA decode with its row order, rebuilt whenever sequence
state changes (every advance, and a reset-and-refill of 60 sequences in the
middle). Bar: max |delta| <= 1e-3."""
import ctypes as C
import sys

import numpy as np
import pytest

import ndoracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3


def nda():
    import ndattn
    return ndattn


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


def test_alternating_streams_match_the_oracle():
    N = nda()
    nh, nkv, qk, vd, W, L, B, STEPS = 12, 2, 48, 64, 384, 2, 600, 6
    rng = np.random.default_rng(71)
    streams = [N.vp(), N.vp()]
    for s in streams:
        N._check(N.lib().nda_stream_create(C.byref(s)))
    ctx = N.Context(L, nh, nkv, qk, vd, W, kv_dtype=O.KV_INT8, max_seqs=B)
    lens = rng.integers(100, 300, B)
    for b in range(B):
        ctx.seq_set_pos(b, int(lens[b]))
    ctx.kv_fill_normal(B, seed=7100, stream=streams[0])
    redone = sorted(int(x) for x in rng.choice(B, 60, replace=False))
    # per step and layer: q, k, v, gate inputs and the output, all kept
    bufs = [[[N.DevBuf(B * n * 4) for n in (nh * qk, nkv * qk, nkv * vd, nh * vd, nh * vd)] for _ in range(L)]
            for _ in range(STEPS)]
    pos_at = []                                # per step: every sequence's position
    redo_step = STEPS // 2
    for step in range(STEPS):
        st = streams[step % 2]
        if step == redo_step:
            # new positions and contents for some sequences, from this stream
            for b in redone:
                ctx.seq_reset(b)
                ctx.seq_set_pos(b, int(rng.integers(40, 320)))
            ctx.kv_fill_normal(len(redone), seq_ids=redone, seed=7200, stream=st)
        pos_at.append([ctx.seq_state(b)[0] for b in range(B)])
        for li in range(L):
            q, k, v, g, out = bufs[step][li]
            for i, (bb, n) in enumerate(((q, nh * qk), (k, nkv * qk), (v, nkv * vd), (g, nh * vd))):
                bb.fill_normal(B * n, 0, 7300 + 100 * step + 10 * li + i, stream=st)
            ctx.step(li, B, q, k, v, out, gate=g, stream=st)
        ctx.advance(B, None, 1, stream=st)
        say("step", step, "queued on stream", step % 2)
    for s in streams:
        ctx.sync(s)
    worst = 0.0
    for step in range(STEPS):
        for li in range(L):
            q, _, _, g, out = bufs[step][li]
            qh = q.to_array(np.float32, (B, nh * qk))
            gh = g.to_array(np.float32, (B, nh * vd))
            got = out.to_array(np.float32, (B, nh * vd))
            assert np.isfinite(got).all()
            picks = [int(x) for x in rng.choice(B, 10, replace=False)] + redone[:2]
            for b in picks:
                if b in redone and step < redo_step:
                    continue                   # its cache was replaced since
                pos = pos_at[step][b]
                kk, vv, ks, vs = ctx.kv_read(li, b, 0, pos + 1)
                view = O.kv_view(kk, vv, ks, vs, nh, pos + 1, 0, pos, O.KV_INT8)
                worst = max(worst, float(np.abs(got[b] - O.attend_view(view, qh[b], gh[b])).max()))
        say("step", step, "checked; worst so far", worst)
    assert worst <= TOL
    ctx.close()
    for s in streams:
        N._check(N.lib().nda_stream_destroy(s))
