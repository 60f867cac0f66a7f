"""GPU parity: libndattn (through its C ABI and the C engine shim) against the
oracle on identical inputs. Output tolerance max |delta| <= 1e-3 (fp32
accumulate, the bar the engine's attention is held to); stored int8 codes and
scales bit-exact."""
import os
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


def maxdiff(a, b):
    return float(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)).max())


# ------------------------------------------------------------ engine session

def replay(geom, script, seed, kv_dtype=O.KV_INT8, scale=1.0):
    """Same token stream through the oracle session and the GPU shim."""
    N = nda()
    rng = np.random.default_rng(seed)
    L, nh, nkv, qk, vd, W = geom
    o = O.OracleSession(*geom, kv_dtype=kv_dtype)
    g = N.GpuSession(*geom, kv_dtype=kv_dtype)
    worst = 0.0
    saved_o, saved_g = {}, {}
    outs = []
    for ev in script:
        if ev[0] == "tok":
            for li in range(L):
                q = (rng.standard_normal(nh * qk) * scale).astype(np.float32)
                k = (rng.standard_normal(nkv * qk) * scale).astype(np.float32)
                v = rng.standard_normal(nkv * vd).astype(np.float32)
                gt = rng.standard_normal(nh * vd).astype(np.float32) if ev[1] else None
                a = o.attention(li, q, k, v, gt)
                b = g.attention(li, q, k, v, gt)
                worst = max(worst, maxdiff(a, b))
                outs.append(b)
            o.step_end()
            g.step_end()
        elif ev[0] == "snap":
            assert o.snapshot() == 0 and g.snapshot() == 0
        elif ev[0] == "sink":
            o.set_sink(ev[1])
            g.set_sink(ev[1])
        elif ev[0] == "save":
            saved_o[ev[1]], saved_g[ev[1]] = o.prefix_save(), g.prefix_save()
            assert saved_o[ev[1]] and saved_g[ev[1]]
        elif ev[0] == "restore":
            assert o.prefix_restore(saved_o[ev[1]]) == 0
            assert g.prefix_restore(saved_g[ev[1]]) == 0
        elif ev[0] == "rewind":
            o.rewind()
            g.rewind()
        elif ev[0] == "reset":
            o.reset()
            g.reset()
        assert (g.pos, g.n_sink) == (o.pos, o.n_sink), ev
    return o, g, worst, outs


def check_cache(o, g, layers, positions):
    """GPU-stored codes and scales of every listed position == oracle's."""
    ctx = g.context()
    L, nh, nkv, qk, vd, W = o.geom
    ok, ov, oks, ovs = o.cache()
    for li in layers:
        for p in positions:
            sl = O.lib().ndo_kv_slot(W, o.n_sink, p)
            k, v, ks, vs = ctx.kv_read(li, 0, p, 1)
            assert np.array_equal(k[0], ok[li, sl]), (li, p)
            assert np.array_equal(v[0], ov[li, sl]), (li, p)
            if o.kv_dtype == O.KV_INT8:
                assert np.array_equal(ks[0].view(np.uint32), oks[li, sl].view(np.uint32)), (li, p)
                assert np.array_equal(vs[0].view(np.uint32), ovs[li, sl].view(np.uint32)), (li, p)


def test_prefix_213_plus_prompt_16_int8():
    """One layer, MHA 8x64, 213 pinned schema positions + 16 prompt tokens,
    int8 KV as the engine stores it."""
    say("int8 session 213 + 16 tokens")
    script = [("tok", True)] * 213 + [("snap",)] + [("tok", True)] * 16
    o, g, worst, _ = replay((1, 8, 8, 64, 64, 256), script, seed=1)
    assert worst <= TOL, worst
    check_cache(o, g, [0], range(229))


def test_engine_shapes_ring_wrap_int8():
    """The archive's geometry (12 q / 2 kv heads, qk 48, v 64, window 384)
    with 200 pinned positions and a ring that wraps."""
    say("engine shapes 460 tokens ring wrap")
    script = [("tok", True)] * 200 + [("snap",)] + [("tok", i % 4 != 0) for i in range(260)]
    o, g, worst, _ = replay((2, 12, 2, 48, 64, 384), script, seed=2, scale=2.0)
    assert worst <= TOL, worst
    check_cache(o, g, [0, 1], list(range(200)) + list(range(460 - 184, 460)))


def test_sliding_window_and_small_window():
    say("small windows")
    script = [("tok", True)] * 10 + [("sink", 10)] + [("tok", True)] * 150
    o, g, worst, _ = replay((1, 8, 2, 64, 64, 100), script, seed=3)
    assert worst <= TOL, worst
    script = [("tok", True)] * 5 + [("sink", 5)] + [("tok", True)] * 60
    o, g, worst, _ = replay((1, 4, 4, 64, 64, 40), script, seed=4)
    assert worst <= TOL, worst
    assert g.n_sink == 0


def test_prefix_switching_reproduces():
    """host/nd_ptest.c's flow: two prefixes restored alternately give
    identical outputs for the same next token."""
    say("prefix switching")
    N = nda()
    geom = (1, 12, 2, 48, 64, 384)
    rng = np.random.default_rng(5)
    L, nh, nkv, qk, vd, W = geom
    g = N.GpuSession(*geom)
    o = O.OracleSession(*geom)
    pre_g, pre_o, expect = [], [], []
    toks = [[rng.standard_normal(n).astype(np.float32) for n in (nh * qk, nkv * qk, nkv * vd, nh * vd)]
            for _ in range(5)]
    for i in range(2):
        g.reset()
        o.reset()
        for t in (toks[i], toks[i + 2]):
            g.attention(0, *t)
            o.attention(0, *t)
            g.step_end()
            o.step_end()
        assert g.snapshot() == 0 and o.snapshot() == 0
        pre_g.append(g.prefix_save())
        pre_o.append(o.prefix_save())
        expect.append(g.attention(0, *toks[4]))
        assert maxdiff(expect[-1], o.attention(0, *toks[4])) <= TOL
    for n in range(4):
        i = n % 2
        assert g.prefix_restore(pre_g[i]) == 0
        assert (g.pos, g.n_sink) == (2, 2)
        got = g.attention(0, *toks[4])
        assert np.array_equal(got.view(np.uint32), expect[i].view(np.uint32))
    for p in pre_g:
        g.prefix_free(p)


def test_rewind_and_long_outliers():
    say("rewind + outliers")
    script = ([("tok", True)] * 30 + [("snap",), ("save", 0)] + [("tok", True)] * 50 + [("rewind",)] +
              [("tok", True)] * 20 + [("restore", 0)] + [("tok", False)] * 10)
    o, g, worst, _ = replay((1, 12, 2, 48, 64, 384), script, seed=6, scale=3.0)
    assert worst <= TOL, worst


# ----------------------------------------------------------- batched decode

def _ragged_decode(kv_dtype, lens, window, seed, nh=8, nkv=8, qk=64, vd=64, split_chunk=0,
                   outlier_p=0.0, gated=True):
    N = nda()
    rng = np.random.default_rng(seed)
    B = len(lens)
    ctx = N.Context(1, nh, nkv, qk, vd, window, kv_dtype=kv_dtype, max_seqs=B, split_chunk=split_chunk)
    # history positions [0, L-1) written in stored format, new token appended
    hist = []
    for b, L in enumerate(lens):
        kf = rng.standard_normal((L - 1, nkv, qk)).astype(np.float32)
        if outlier_p:
            mask = rng.random((L - 1, nkv)) < outlier_p
            kf[mask] *= np.float32(8.0)
        vf = rng.standard_normal((L - 1, nkv, vd)).astype(np.float32)
        if kv_dtype == O.KV_F16:
            k, v, ks, vs = O.f32_to_f16_bits(kf), O.f32_to_f16_bits(vf), None, None
        else:
            k = np.zeros(kf.shape, np.int8)
            v = np.zeros(vf.shape, np.int8)
            ks = np.zeros((L - 1, nkv), np.float32)
            vs = np.zeros((L - 1, nkv), np.float32)
            for p in range(L - 1):
                for gg in range(nkv):
                    ks[p, gg] = O.lib().ndo_kv_quant_row(np.ascontiguousarray(kf[p, gg]), qk, k[p, gg])
                    vs[p, gg] = O.lib().ndo_kv_quant_row(np.ascontiguousarray(vf[p, gg]), vd, v[p, gg])
        if L > 1:
            ctx.kv_write(0, b, 0, k, v, ks, vs)
        ctx.seq_set_pos(b, L - 1)
        hist.append(L)
    q = rng.standard_normal((B, nh, qk)).astype(np.float32)
    kn = rng.standard_normal((B, nkv, qk)).astype(np.float32)
    vn = rng.standard_normal((B, nkv, vd)).astype(np.float32)
    gate = rng.standard_normal((B, nh, vd)).astype(np.float32) if gated else None
    dq, dk, dv = N.DevBuf.from_array(q), N.DevBuf.from_array(kn), N.DevBuf.from_array(vn)
    dg = N.DevBuf.from_array(gate) if gated else None
    dout = N.DevBuf(B * nh * vd * 4)
    ctx.step(0, B, dq, dk, dv, dout, gate=dg)
    ctx.sync()
    out = dout.to_array(np.float32, (B, nh, vd))
    worst = 0.0
    for b, L in enumerate(lens):
        k, v, ks, vs = ctx.kv_read(0, b, 0, L)
        kv = O.kv_view(k, v, ks if kv_dtype == O.KV_INT8 else None, vs if kv_dtype == O.KV_INT8 else None,
                       nh, L, 0, L - 1, kv_dtype)
        want = O.attend_view(kv, q[b].ravel(), None if gate is None else gate[b].ravel())
        worst = max(worst, maxdiff(out[b].ravel(), want))
        # the appended token was stored as the oracle stores it
        if kv_dtype == O.KV_F16:
            assert np.array_equal(k[L - 1], O.f32_to_f16_bits(kn[b]))
        else:
            for gg in range(nkv):
                c = np.zeros(qk, np.int8)
                sc = O.lib().ndo_kv_quant_row(np.ascontiguousarray(kn[b, gg]), qk, c)
                assert np.array_equal(c, k[L - 1, gg]) and np.float32(sc) == ks[L - 1, gg]
    return worst


@pytest.mark.parametrize("kv_dtype", [O.KV_F16, O.KV_INT8])
def test_batched_ragged_decode(kv_dtype):
    say("ragged decode dtype", kv_dtype)
    rng = np.random.default_rng(7)
    lens = [1, 2, 3, 15, 16, 17, 31, 64, 213, 229] + list(rng.integers(1, 1025, 22))
    worst = _ragged_decode(kv_dtype, lens, 1024, seed=8)
    assert worst <= TOL, worst


def test_gqa_decode_engine_shapes():
    say("gqa decode 12/2 48/64")
    lens = [1, 5, 100, 384, 383, 200]
    for dt in (O.KV_INT8, O.KV_F16):
        worst = _ragged_decode(dt, lens, 384, seed=9, nh=12, nkv=2, qk=48, vd=64)
        assert worst <= TOL, worst


def test_split_kv_long_context_with_outliers():
    """Split-KV with the LSE merge, lengths past the split size, 8-sigma keys."""
    say("split-kv long context")
    lens = [8192, 5000, 1025, 1024, 513, 7]
    worst = _ragged_decode(O.KV_F16, lens, 8192, seed=10, split_chunk=512, outlier_p=1e-3)
    assert worst <= TOL, worst


def test_no_gate_and_rep_variants():
    say("rep variants")
    for nh, nkv in ((8, 4), (8, 1), (16, 2), (6, 1)):
        worst = _ragged_decode(O.KV_F16, [3, 77, 300], 512, seed=nh * 10 + nkv, nh=nh, nkv=nkv, gated=False)
        assert worst <= TOL, (nh, nkv, worst)


# ------------------------------------------------------ prefill and prefixes

def test_causal_prefill_256_tokens_8_layers_int8():
    """8 layers x 256-token causal prefill through nda_prefill against the
    engine's token-by-token prefill; codes bit-exact."""
    say("prefill 8 layers x 256 tokens int8")
    N = nda()
    Lyr, nh, nkv, d, S = 8, 8, 8, 64, 256
    rng = np.random.default_rng(11)
    ctx = N.Context(Lyr, nh, nkv, d, d, S, kv_dtype=O.KV_INT8, max_seqs=1)
    o = O.OracleSession(Lyr, nh, nkv, d, d, S, O.KV_INT8)
    worst = 0.0
    for li in range(Lyr):
        q = rng.standard_normal((S, nh, d)).astype(np.float32)
        k = rng.standard_normal((S, nkv, d)).astype(np.float32)
        v = rng.standard_normal((S, nkv, d)).astype(np.float32)
        want = np.zeros((S, nh * d), np.float32)
        O.lib().ndo_prefill_tokens(O.C.byref(o.s), li, S, q.ctypes.data, k.ctypes.data, v.ctypes.data,
                                   None, want.ctypes.data)
        dq, dk, dv = N.DevBuf.from_array(q), N.DevBuf.from_array(k), N.DevBuf.from_array(v)
        dout = N.DevBuf(S * nh * d * 4)
        ctx.prefill(li, [S], dq, dk, dv, dout)
        ctx.sync()
        got = dout.to_array(np.float32, (S, nh * d))
        worst = max(worst, maxdiff(got, want))
        kk, vv, ks, vs = ctx.kv_read(li, 0, 0, S)
        ok, ov, oks, ovs = o.cache()
        assert np.array_equal(kk, ok[li]) and np.array_equal(vv, ov[li])
        assert np.array_equal(ks, oks[li]) and np.array_equal(vs, ovs[li])
    assert worst <= TOL, worst


def _views_for(ctx, li, seq, pos, nh, dtype):
    k, v, ks, vs = ctx.kv_read(li, seq, 0, pos + 1)
    if dtype == O.KV_F16:
        ks = vs = None
    return O.kv_view(k, v, ks, vs, nh, pos + 1, 0, pos, dtype), (k, v, ks, vs)


@pytest.mark.parametrize("kv_dtype", [O.KV_F16, O.KV_INT8])
def test_shared_prefix_prefill_then_decode(kv_dtype):
    """The shared-prefix flow at small batch: one 213-token prefix built once,
    shared by every sequence; ragged causal suffixes; decode steps."""
    say("shared prefix dtype", kv_dtype)
    N = nda()
    nh = nkv = 8
    d, W, B, npre = 64, 384, 12, 213
    rng = np.random.default_rng(12)
    ctx = N.Context(2, nh, nkv, d, d, W, kv_dtype=kv_dtype, max_seqs=B + 1)
    # build the prefix on sequence B by prefilling it
    for li in range(2):
        q = rng.standard_normal((npre, nh, d)).astype(np.float32)
        k = rng.standard_normal((npre, nkv, d)).astype(np.float32)
        v = rng.standard_normal((npre, nkv, d)).astype(np.float32)
        dout = N.DevBuf(npre * nh * d * 4)
        ctx.prefill(li, [npre], N.DevBuf.from_array(q), N.DevBuf.from_array(k), N.DevBuf.from_array(v),
                    dout, seq_ids=[B])
    ctx.advance(1, [B], npre)
    pid = ctx.prefix_build(B)
    for b in range(B):
        ctx.seq_attach(b, pid)
        assert ctx.seq_state(b) == (npre, npre, pid)
    with pytest.raises(N.NdaError):
        ctx.prefix_free(pid)       # attached: refused
    n = rng.integers(32, 65, B)
    worst = 0.0
    for li in range(2):
        T = int(n.sum())
        q = rng.standard_normal((T, nh, d)).astype(np.float32)
        k = rng.standard_normal((T, nkv, d)).astype(np.float32)
        v = rng.standard_normal((T, nkv, d)).astype(np.float32)
        g = rng.standard_normal((T, nh, d)).astype(np.float32)
        dout = N.DevBuf(T * nh * d * 4)
        ctx.prefill(li, n, N.DevBuf.from_array(q), N.DevBuf.from_array(k), N.DevBuf.from_array(v), dout,
                    gate=N.DevBuf.from_array(g), seq_ids=list(range(B)))
        ctx.sync()
        got = dout.to_array(np.float32, (T, nh * d))
        r = 0
        for b in range(B):
            view, keep = _views_for(ctx, li, b, npre + int(n[b]) - 1, nh, kv_dtype)
            for t in range(int(n[b])):
                pos = npre + t
                slots = np.arange(pos + 1)
                want = O.attend_runs(view, slots, [npre, pos + 1 - npre], q[r], g[r])
                worst = max(worst, maxdiff(got[r], want))
                r += 1
    for b in range(B):
        ctx.advance(1, [b], int(n[b]))
    for step in range(3):
        for li in range(2):
            q = rng.standard_normal((B, nh, d)).astype(np.float32)
            k = rng.standard_normal((B, nkv, d)).astype(np.float32)
            v = rng.standard_normal((B, nkv, d)).astype(np.float32)
            dout = N.DevBuf(B * nh * d * 4)
            ctx.step(li, B, N.DevBuf.from_array(q), N.DevBuf.from_array(k), N.DevBuf.from_array(v), dout)
            ctx.sync()
            got = dout.to_array(np.float32, (B, nh * d))
            for b in range(B):
                pos = ctx.seq_state(b)[0]
                view, keep = _views_for(ctx, li, b, pos, nh, kv_dtype)
                want = O.attend_runs(view, np.arange(pos + 1), [npre, pos + 1 - npre], q[b], None)
                worst = max(worst, maxdiff(got[b], want))
        ctx.advance(B, None, 1)
    assert worst <= TOL, worst
    for b in range(B):
        ctx.seq_reset(b)
    ctx.prefix_free(pid)


@pytest.mark.parametrize("kv_dtype,geom,npre,own_max,W,extra", [
    (O.KV_F16, (8, 8, 64, 64), 213, 40, 384, 0), (O.KV_INT8, (8, 8, 64, 64), 213, 40, 384, 0),
    (O.KV_F16, (8, 4, 64, 64), 213, 40, 384, 0), (O.KV_F16, (8, 8, 64, 64), 40, 100, 384, 0),
    (O.KV_INT8, (8, 8, 64, 64), 213, 64, 277, 30), (O.KV_F16, (8, 8, 64, 64), 100, 250, 384, 0),
    (O.KV_F16, (8, 2, 64, 64), 213, 40, 384, 0)])
def test_shared_prefix_decode_pass(kv_dtype, geom, npre, own_max, W, extra):
    """A decode batch whose sequences all share one prefix (at least 4
    (row, kv-head) units per CU) attends the prefix in one MFMA pass over all
    of them and their own positions on the VALU kernel, merged as split-KV
    chunks of the prefix's length. Rows of two chunks are merged by the
    own-positions pass; with a 40-slot prefix and up to 101 own positions
    other rows have up to four and go through the merge kernel. With a
    277-slot window (213 sinks, the 64-slot minimum ring) and 30 more decode
    steps first, the own ring wraps; with a 100-slot prefix and up to 250
    own positions, rows of three and four chunks go through the merge
    kernel. Rep 4 (2 kv-heads, 520 sequences for 4 units per CU) merges
    chunk 0 read at the epilogue rather than requested at the start. Every row against the
    oracle, gated and not; the pass is taken (two decode launches per call,
    the second storing the new row, no append launch, a merge launch only
    when some row has more than two chunks)."""
    nh, nkv, dk, dv = geom
    say("shared prefix decode pass", kv_dtype, geom, npre, own_max, W)
    N = nda()
    rng = np.random.default_rng(77 + nkv + npre + W)
    B = 264 if nkv >= 4 else 520
    ctx = N.Context(1, nh, nkv, dk, dv, W, kv_dtype=kv_dtype, max_seqs=B + 1)
    q = rng.standard_normal((npre, nh, dk)).astype(np.float32)
    k = rng.standard_normal((npre, nkv, dk)).astype(np.float32)
    v = rng.standard_normal((npre, nkv, dv)).astype(np.float32)
    dout = N.DevBuf(npre * nh * dv * 4)
    ctx.prefill(0, [npre], N.DevBuf.from_array(q), N.DevBuf.from_array(k), N.DevBuf.from_array(v), dout,
                seq_ids=[B])
    ctx.advance(1, [B], npre)
    pid = ctx.prefix_build(B)
    for b in range(B):
        ctx.seq_attach(b, pid)
    n = rng.integers(0, own_max + 1, B)
    ids = [b for b in range(B) if n[b] > 0]
    T = int(n.sum())
    q = rng.standard_normal((T, nh, dk)).astype(np.float32)
    k = rng.standard_normal((T, nkv, dk)).astype(np.float32)
    v = rng.standard_normal((T, nkv, dv)).astype(np.float32)
    dout = N.DevBuf(T * nh * dv * 4)
    ctx.prefill(0, [int(n[b]) for b in ids], N.DevBuf.from_array(q), N.DevBuf.from_array(k),
                N.DevBuf.from_array(v), dout, seq_ids=ids)
    for b in ids:
        ctx.advance(1, [b], int(n[b]))
    for _ in range(extra):
        x = [N.DevBuf.from_array(rng.standard_normal((B, d, e)).astype(np.float32))
             for d, e in ((nh, dk), (nkv, dk), (nkv, dv))]
        ctx.step(0, B, *x, N.DevBuf(B * nh * dv * 4))
        ctx.advance(B, None, 1)
    worst = 0.0
    for gated in (False, True):
        q = rng.standard_normal((B, nh, dk)).astype(np.float32)
        k = rng.standard_normal((B, nkv, dk)).astype(np.float32)
        v = rng.standard_normal((B, nkv, dv)).astype(np.float32)
        g = rng.standard_normal((B, nh, dv)).astype(np.float32) if gated else None
        dout = N.DevBuf(B * nh * dv * 4)
        ctx.sync()
        ctx.prof_enable(True)
        ctx.prof_read(reset=True)
        ctx.step(0, B, N.DevBuf.from_array(q), N.DevBuf.from_array(k), N.DevBuf.from_array(v), dout,
                 gate=N.DevBuf.from_array(g) if gated else None)
        ctx.sync()
        ms, launches = ctx.prof_read(reset=True)
        ctx.prof_enable(False)
        tot = max(npre + min(ctx.seq_state(b)[0] + 1 - npre, W - npre) for b in range(B))
        max_chunks = -(-tot // npre)
        assert launches[N.K_DECODE] == 2, list(launches)
        assert launches[N.K_APPEND] == 0, list(launches)
        assert launches[N.K_COMBINE] == (1 if max_chunks > 2 else 0), list(launches)
        got = dout.to_array(np.float32, (B, nh * dv))
        for b in range(B):
            pos = ctx.seq_state(b)[0]
            nown = min(pos + 1 - npre, W - npre)          # the ring's newest positions
            # the visible rows: the prefix, then the ring's positions
            parts = [ctx.kv_read(0, b, 0, npre), ctx.kv_read(0, b, pos + 1 - nown, nown)]
            k_, v_, ks_, vs_ = (np.concatenate([x[i] for x in parts]) for i in range(4))
            if kv_dtype == O.KV_F16:
                ks_ = vs_ = None
            view = O.kv_view(k_, v_, ks_, vs_, nh, npre + nown, 0, npre + nown - 1, kv_dtype)
            want = O.attend_runs(view, np.arange(npre + nown), [npre, nown], q[b], g[b] if gated else None)
            worst = max(worst, maxdiff(got[b], want))
        ctx.advance(B, None, 1)
    ctx.close()
    assert worst <= TOL, worst


def test_prefill_gqa_chunks_on_shared_prefix():
    """Prefill of several chunks on one shared prefix at the engine's GQA
    shape (12 q / 2 kv heads, qk 48, int8): a 100-token prefix (not a whole
    number of key tiles), a first and a second suffix chunk (own keys then
    include earlier suffix tokens), gated; then a call that mixes in a
    sequence without the prefix. Every output against the oracle's
    attention."""
    say("prefill gqa chunks on a shared prefix")
    N = nda()
    nh, nkv, qk, vd, W, B, npre = 12, 2, 48, 64, 384, 5, 100
    rng = np.random.default_rng(21)
    ctx = N.Context(1, nh, nkv, qk, vd, W, kv_dtype=O.KV_INT8, max_seqs=B + 2)

    def chunk(seq_ids, n, shared):
        T = int(sum(n))
        q = rng.standard_normal((T, nh, qk)).astype(np.float32)
        k = rng.standard_normal((T, nkv, qk)).astype(np.float32)
        v = rng.standard_normal((T, nkv, vd)).astype(np.float32)
        g = rng.standard_normal((T, nh, vd)).astype(np.float32)
        dout = N.DevBuf(T * nh * vd * 4)
        pos0 = [ctx.seq_state(b)[0] for b in seq_ids]
        ctx.prefill(0, n, N.DevBuf.from_array(q), N.DevBuf.from_array(k), N.DevBuf.from_array(v), dout,
                    gate=N.DevBuf.from_array(g), seq_ids=seq_ids)
        ctx.sync()
        got = dout.to_array(np.float32, (T, nh * vd))
        worst, r = 0.0, 0
        for b, nb, p0 in zip(seq_ids, n, pos0):
            view, keep = _views_for(ctx, 0, b, p0 + int(nb) - 1, nh, O.KV_INT8)
            for t in range(int(nb)):
                pos = p0 + t
                runs = [npre, pos + 1 - npre] if shared[b] else [pos + 1]
                want = O.attend_runs(view, np.arange(pos + 1), runs, q[r], g[r])
                worst = max(worst, maxdiff(got[r], want))
                r += 1
        for b, nb in zip(seq_ids, n):
            ctx.advance(1, [b], int(nb))
        return worst

    q = rng.standard_normal((npre, nh, qk)).astype(np.float32)
    k = rng.standard_normal((npre, nkv, qk)).astype(np.float32)
    v = rng.standard_normal((npre, nkv, vd)).astype(np.float32)
    ctx.prefill(0, [npre], N.DevBuf.from_array(q), N.DevBuf.from_array(k), N.DevBuf.from_array(v),
                N.DevBuf(npre * nh * vd * 4), seq_ids=[B])
    ctx.advance(1, [B], npre)
    pid = ctx.prefix_build(B)
    shared = {b: True for b in range(B)}
    shared[B + 1] = False
    for b in range(B):
        ctx.seq_attach(b, pid)
    worst = chunk(list(range(B)), [1, 17, 40, 33, 5], shared)          # first suffix chunks
    worst = max(worst, chunk([3, 0, 4], [70, 9, 1], shared))            # second chunks, out of order
    worst = max(worst, chunk([1, B + 1, 2], [6, 40, 12], shared))       # a sequence without the prefix
    say("prefill gqa chunks worst", worst)
    assert worst <= TOL, worst
    for b in range(B):
        ctx.seq_reset(b)
    ctx.prefix_free(pid)


def test_int8_store_edge_rows():
    """Exact .5 ties, zero rows, +-absmax, subnormal scales: codes and scales
    identical to the oracle's (which is pinned to the reference's store)."""
    say("int8 store edge rows")
    N = nda()
    rows = []
    rng = np.random.default_rng(13)
    rows.append(np.zeros(64, np.float32))
    rows.append(np.array([(i - 32) + 0.5 for i in range(64)], np.float32))
    rows.append(np.array([1e-38 * (i - 32) for i in range(64)], np.float32))
    rows.append((rng.standard_normal(64) * 1e-20).astype(np.float32))
    sc = np.float32(0.37)
    t = (rng.integers(-254, 255, 64) / 2.0).astype(np.float32)
    rows.append((t * sc).astype(np.float32))
    for _ in range(59):
        rows.append((rng.standard_normal(64) * 10 ** rng.uniform(-8, 8)).astype(np.float32))
    n = len(rows)
    ctx = N.Context(1, 1, 1, 64, 64, 128, kv_dtype=O.KV_INT8, max_seqs=n)
    kin = np.stack(rows).reshape(n, 1, 64)
    vin = kin[::-1].copy()
    ctx.kv_append(0, n, N.DevBuf.from_array(kin), N.DevBuf.from_array(vin))
    ctx.sync()
    for b in range(n):
        k, v, ks, vs = ctx.kv_read(0, b, 0, 1)
        for src, code, scl in ((kin[b, 0], k[0, 0], ks[0, 0]), (vin[b, 0], v[0, 0], vs[0, 0])):
            c = np.zeros(64, np.int8)
            s = O.lib().ndo_kv_quant_row(np.ascontiguousarray(src), 64, c)
            assert np.array_equal(c, code), b
            assert np.float32(s).view(np.uint32) == np.float32(scl).view(np.uint32), b


@pytest.mark.parametrize("geom,unaligned", [((8, 64, 64), False), ((2, 48, 64), False), ((3, 20, 36), False),
                                             ((8, 64, 64), True)])
def test_f16_store_rows(geom, unaligned):
    """fp16 K/V stores (nda_kv_append): every stored element is the fp32
    input rounded to nearest-even fp16, bit for bit, including values that
    round to the fp16 maximum, overflow to infinity, or go subnormal.
    Head dims that are multiples of 4 with 16-byte aligned inputs take the
    vector kernel, the rest (qk 20 / v 36 are multiples of 4; a k pointer
    4 bytes off alignment) the per-element one; rows in several pages, out
    of order."""
    nkv, dk, dv = geom
    say("f16 store rows", geom, unaligned)
    N = nda()
    rng = np.random.default_rng(17 + dk)
    n, W, steps = 300, 64, 3
    ctx = N.Context(1, nkv, nkv, dk, dv, W, kv_dtype=O.KV_F16, max_seqs=n)
    special = np.array([65504.0, 65519.9, 65520.0, -7e4, 6.1e-5, 6.0e-8, 2.9e-8, -3.0e-8, 0.0, -0.0,
                        1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], np.float32)
    ids = rng.permutation(n)[: n // 2].astype(np.uint32)
    for step in range(steps):
        kin = (rng.standard_normal((len(ids), nkv, dk)) * 10 ** rng.uniform(-6, 4, (len(ids), nkv, 1)))
        vin = (rng.standard_normal((len(ids), nkv, dv)) * 10 ** rng.uniform(-6, 4, (len(ids), nkv, 1)))
        kin, vin = kin.astype(np.float32), vin.astype(np.float32)
        kin.reshape(-1)[: len(special)] = special
        vin.reshape(-1)[-len(special):] = special
        kb = N.DevBuf.from_array(np.concatenate([np.zeros(1, np.float32), kin.reshape(-1)])) if unaligned \
            else N.DevBuf.from_array(kin)
        kptr = kb.value + 4 if unaligned else kb
        ctx.kv_append(0, len(ids), kptr, N.DevBuf.from_array(vin), seq_ids=list(ids))
        for b in ids:
            ctx.advance(1, [int(b)], 1)
        ctx.sync()
        with np.errstate(over="ignore"):             # the overflow to infinity is meant
            kh, vh = kin.astype(np.float16), vin.astype(np.float16)
        for j, b in enumerate(ids):
            k, v, _, _ = ctx.kv_read(0, int(b), step, 1)
            assert np.array_equal(k[0].view(np.uint16), kh[j].view(np.uint16)), (step, b)
            assert np.array_equal(v[0].view(np.uint16), vh[j].view(np.uint16)), (step, b)
    ctx.close()


# ------------------------------------------------------------ error handling

def test_error_paths():
    say("error paths")
    N = nda()
    ctx = N.Context(2, 4, 2, 64, 64, 64, kv_dtype=O.KV_F16, max_seqs=2, max_pages=5)
    z = N.DevBuf(1 << 16)
    with pytest.raises(N.NdaError) as e:
        ctx.decode(0, 1, z, z)                       # nothing stored yet
    assert e.value.code == -5
    with pytest.raises(N.NdaError) as e:
        ctx.kv_append(2, 1, z, z)                    # bad layer
    assert e.value.code == -1
    with pytest.raises(N.NdaError) as e:
        ctx.prefill(0, [65], z, z, z, z)              # would wrap the ring
    assert e.value.code == -4
    ctx.prefill(0, [64], z, z, z, z)                  # exactly the window: fine
    with pytest.raises(N.NdaError) as e:
        ctx.prefill(0, [64], z, z, z, z, seq_ids=[1])  # 4 more pages, 1 left
    assert e.value.code == -2
    assert ctx.seq_state(1)[0] == 0
    ctx.kv_append(0, 0, None, None)                   # empty batch
    ctx.decode(0, 0, None, None)
    with pytest.raises(N.NdaError):
        ctx.seq_attach(0, 3)                          # no such prefix
    with pytest.raises(N.NdaError):
        N.Context(1, 6, 4, 64, 64, 64)                 # heads not a multiple
    with pytest.raises(N.NdaError) as e:
        N.Context(1, 4, 4, 80, 64, 64)                 # no kernel for dk 80
    assert e.value.code == -6


# --------------------------------------------------- full-size sampled check

def test_decode_4096_ragged_sequences_one_layer_sampled():
    """The batched decode at full size on one layer (4096 ragged sequences, L in
    [213, 1024], fp16): the whole batch decodes, and 24 sampled sequences match
    the oracle; a second step after advance matches too."""
    say("decode 4096 ragged sequences, 1 layer")
    N = nda()
    B, nh, d, W = 4096, 8, 64, 1024
    rng = np.random.default_rng(14)
    lens = rng.integers(213, 1025, B)
    ctx = N.Context(1, nh, nh, d, d, W + 8, kv_dtype=O.KV_F16, max_seqs=B)
    for b in range(B):
        ctx.seq_set_pos(b, int(lens[b]) - 1)
        ctx.seq_reserve(b, 2)
    ctx.kv_fill_normal(B, seed=77)
    dq, dk, dv, dout = (N.DevBuf(B * nh * d * 4) for _ in range(4))
    for buf, s in ((dq, 1), (dk, 2), (dv, 3)):
        buf.fill_normal(B * nh * d, 0, s)
    sample = rng.choice(B, 24, replace=False)
    for step in range(2):
        ctx.step(0, B, dq, dk, dv, dout)
        ctx.sync()
        out = dout.to_array(np.float32, (B, nh * d))
        assert np.isfinite(out).all()
        q = dq.to_array(np.float32, (B, nh * d))
        for b in sample:
            pos = ctx.seq_state(int(b))[0]
            k, v, _, _ = ctx.kv_read(0, int(b), 0, pos + 1)
            kv = O.kv_view(k, v, None, None, nh, pos + 1, 0, pos, O.KV_F16)
            want = O.attend_view(kv, q[b], None)
            assert maxdiff(out[b], want) <= TOL, (step, b)
        ctx.advance(B, None, 1)


# ------------------------------------------------------- MFMA prefill kernel

def _prefill_case(kv_dtype, nh, nkv, qk, hist, ntok, seed, flags=0, outlier_p=0.0, gated=True):
    """Sequences with `hist[b]` stored positions prefill `ntok[b]` tokens in one
    call; every token's output against the oracle over positions [0, pos+t]."""
    N = nda()
    vd = 64
    rng = np.random.default_rng(seed)
    B = len(hist)
    W = max(h + n for h, n in zip(hist, ntok)) + 16
    ctx = N.Context(1, nh, nkv, qk, vd, W, kv_dtype=kv_dtype, max_seqs=B, flags=flags)
    for b, L in enumerate(hist):
        if L:
            kf = rng.standard_normal((L, nkv, qk)).astype(np.float32)
            if outlier_p:
                kf[rng.random((L, nkv)) < outlier_p] *= np.float32(8.0)
            vf = rng.standard_normal((L, nkv, vd)).astype(np.float32)
            if kv_dtype == O.KV_F16:
                ctx.kv_write(0, b, 0, O.f32_to_f16_bits(kf), O.f32_to_f16_bits(vf))
            else:
                k = np.zeros(kf.shape, np.int8)
                v = np.zeros(vf.shape, np.int8)
                ks = np.zeros((L, nkv), np.float32)
                vs = np.zeros((L, nkv), np.float32)
                for p in range(L):
                    for gg in range(nkv):
                        ks[p, gg] = O.lib().ndo_kv_quant_row(np.ascontiguousarray(kf[p, gg]), qk, k[p, gg])
                        vs[p, gg] = O.lib().ndo_kv_quant_row(np.ascontiguousarray(vf[p, gg]), vd, v[p, gg])
                ctx.kv_write(0, b, 0, k, v, ks, vs)
        ctx.seq_set_pos(b, L)
    T = int(sum(ntok))
    q = rng.standard_normal((T, nh, qk)).astype(np.float32)
    k = rng.standard_normal((T, nkv, qk)).astype(np.float32)
    v = rng.standard_normal((T, nkv, vd)).astype(np.float32)
    g = rng.standard_normal((T, nh, vd)).astype(np.float32) if gated else None
    dout = N.DevBuf(max(1, T) * nh * vd * 4)
    ctx.prefill(0, ntok, N.DevBuf.from_array(q), N.DevBuf.from_array(k), N.DevBuf.from_array(v), dout,
                gate=None if g is None else N.DevBuf.from_array(g))
    ctx.sync()
    got = dout.to_array(np.float32, (T, nh * vd))
    worst, r = 0.0, 0
    for b in range(B):
        n = int(ntok[b])
        if n == 0:
            continue
        end = hist[b] + n
        kk, vv, ks, vs = ctx.kv_read(0, b, 0, end)
        if kv_dtype == O.KV_F16:
            ks = vs = None
        for t in range(n):
            pos = hist[b] + t
            kv = O.kv_view(kk, vv, ks, vs, nh, end, 0, pos, kv_dtype)
            want = O.attend_view(kv, q[r].ravel(), None if g is None else g[r].ravel())
            worst = max(worst, maxdiff(got[r], want))
            r += 1
    return worst, got


@pytest.mark.parametrize("kv_dtype", [O.KV_F16, O.KV_INT8])
def test_prefill_mfma_ragged_batch(kv_dtype):
    """Row tiles with partial fills (1, 31, 32, 33, 64, 65, 129 tokens),
    existing history (0 to 700 positions), tile/diagonal boundaries."""
    say("prefill mfma ragged dtype", kv_dtype)
    hist = [0, 0, 5, 31, 100, 213, 700, 64, 1]
    ntok = [1, 129, 31, 32, 33, 64, 65, 200, 0]
    worst, _ = _prefill_case(kv_dtype, 8, 8, 64, hist, ntok, seed=21)
    assert worst <= TOL, worst


@pytest.mark.parametrize("kv_dtype", [O.KV_F16, O.KV_INT8])
def test_prefill_mfma_gqa_engine_shapes(kv_dtype):
    """12 query / 2 kv heads, qk 48: rows of a tile interleave the 6 heads."""
    say("prefill mfma gqa dtype", kv_dtype)
    worst, _ = _prefill_case(kv_dtype, 12, 2, 48, [0, 10, 213], [40, 7, 16], seed=22)
    assert worst <= TOL, worst


def test_prefill_mfma_rep_variants_and_no_gate():
    say("prefill mfma rep variants")
    for nh, nkv in ((8, 4), (8, 1), (16, 2)):
        worst, _ = _prefill_case(O.KV_F16, nh, nkv, 64, [3, 50], [20, 70], seed=nh + nkv, gated=False)
        assert worst <= TOL, (nh, nkv, worst)


def test_prefill_mfma_long_context_outliers():
    """A 512-token chunk over 4000 stored positions with 8-sigma keys."""
    say("prefill mfma long context")
    worst, _ = _prefill_case(O.KV_F16, 8, 8, 64, [4000], [512], seed=23, outlier_p=1e-3)
    assert worst <= TOL, worst


@pytest.mark.parametrize("hist,ntok", [([6000], [20]), ([8000], [40]), ([8000], [100])])
def test_prefill_small_groups_direct_and_staged_tiles(hist, ntok):
    """fp16 qk-64 chunks of at most 64 rows (2-wave groups) and 65-255 rows
    (4-wave groups) load their key tiles straight into LDS when the tile
    table fits the LDS their residency leaves (224 tiles at 2 waves), and
    stage them through registers without a table otherwise: 6000 + 20
    positions (189 tiles, direct), 8000 + 40 (252 tiles, staged), 8000 + 100
    at 4 waves (direct), with 8-sigma keys."""
    say("prefill small groups", hist, ntok)
    worst, _ = _prefill_case(O.KV_F16, 8, 8, 64, hist, ntok, seed=31 + ntok[0], outlier_p=1e-3)
    assert worst <= TOL, worst


def test_prefill_mfma_matches_valu_path():
    say("prefill mfma vs valu")
    hist, ntok = [17, 300], [90, 45]
    _, a = _prefill_case(O.KV_F16, 8, 8, 64, hist, ntok, seed=24)
    _, b = _prefill_case(O.KV_F16, 8, 8, 64, hist, ntok, seed=24, flags=1)
    assert maxdiff(a, b) <= 2e-6


@pytest.mark.parametrize("page_size", [32, 64])
def test_page_sizes_decode_and_prefill(page_size):
    """The paged layout at 32 and 64 positions per page: ragged decode,
    split-KV, shared-prefix prefill, against the oracle."""
    say("page size", page_size)
    N = nda()
    rng = np.random.default_rng(30 + page_size)
    nh = nkv = 8
    d, W = 64, 512
    for dt in (O.KV_F16, O.KV_INT8):
        ctx = N.Context(1, nh, nkv, d, d, W, kv_dtype=dt, max_seqs=5, page_size=page_size, split_chunk=128)
        # a 100-token prefix shared by 4 sequences, ragged suffixes, one decode step
        npre = 100
        q = rng.standard_normal((npre, nh, d)).astype(np.float32)
        k = rng.standard_normal((npre, nkv, d)).astype(np.float32)
        v = rng.standard_normal((npre, nkv, d)).astype(np.float32)
        dout = N.DevBuf(npre * nh * d * 4)
        ctx.prefill(0, [npre], N.DevBuf.from_array(q), N.DevBuf.from_array(k), N.DevBuf.from_array(v),
                    dout, seq_ids=[4])
        ctx.advance(1, [4], npre)
        pid = ctx.prefix_build(4)
        for b in range(4):
            ctx.seq_attach(b, pid)
        n = [1, 37, 64, 200]
        T = sum(n)
        q = rng.standard_normal((T, nh, d)).astype(np.float32)
        k = rng.standard_normal((T, nkv, d)).astype(np.float32)
        v = rng.standard_normal((T, nkv, d)).astype(np.float32)
        dout = N.DevBuf(T * nh * d * 4)
        ctx.prefill(0, n, N.DevBuf.from_array(q), N.DevBuf.from_array(k), N.DevBuf.from_array(v), dout,
                    seq_ids=[0, 1, 2, 3])
        ctx.sync()
        got = dout.to_array(np.float32, (T, nh * d))
        r, worst = 0, 0.0
        for b in range(4):
            view, keep = _views_for(ctx, 0, b, npre + n[b] - 1, nh, dt)
            for t in range(n[b]):
                pos = npre + t
                want = O.attend_runs(view, np.arange(pos + 1), [npre, pos + 1 - npre], q[r], None)
                worst = max(worst, maxdiff(got[r], want))
                r += 1
        for b in range(4):
            ctx.advance(1, [b], n[b])
        qd = rng.standard_normal((4, nh, d)).astype(np.float32)
        kd = rng.standard_normal((4, nkv, d)).astype(np.float32)
        vd = rng.standard_normal((4, nkv, d)).astype(np.float32)
        dout = N.DevBuf(4 * nh * d * 4)
        ctx.step(0, 4, N.DevBuf.from_array(qd), N.DevBuf.from_array(kd), N.DevBuf.from_array(vd), dout)
        ctx.sync()
        got = dout.to_array(np.float32, (4, nh * d))
        for b in range(4):
            pos = ctx.seq_state(b)[0]
            view, keep = _views_for(ctx, 0, b, pos, nh, dt)
            want = O.attend_runs(view, np.arange(pos + 1), [npre, pos + 1 - npre], qd[b], None)
            worst = max(worst, maxdiff(got[b], want))
        assert worst <= TOL, (dt, worst)


def _poison_free_pages(N, ctx, seqs, npages, page_size, window, nh, nkv, dk, dv):
    """Fill `npages` free pages with non-finite K/V through throwaway
    sequences (at most a window's pages each), then give them back: later
    owners find them there past their stored slots."""
    left = npages
    for seq in seqs:
        if left == 0:
            break
        take = min(left, window // page_size)
        left -= take
        n = take * page_size
        bad = np.full(n * nkv * max(dk, dv), np.nan, np.float32)
        bad[1::3] = np.inf
        q = N.DevBuf.from_array(np.zeros((n, nh, dk), np.float32))
        k = N.DevBuf.from_array(bad[:n * nkv * dk].reshape(n, nkv, dk))
        v = N.DevBuf.from_array(bad[:n * nkv * dv].reshape(n, nkv, dv))
        out = N.DevBuf(n * nh * dv * 4)
        ctx.prefill(0, [n], q, k, v, out, seq_ids=[seq])
        ctx.sync()
    assert left == 0
    for seq in seqs:
        ctx.seq_reset(seq)


@pytest.mark.parametrize("page_size", [16, 64])
@pytest.mark.parametrize("geom", [(8, 8, 64, 64), (12, 2, 48, 64)])
def test_prefill_segment_ends_over_stale_nonfinite_slots(page_size, geom):
    """Slots past a segment's end inside its last key tile (the prefix's
    partial tile, an own tile that ends early, a half tile wholly past the
    end) hold whatever their page held before. Here that is NaN / inf K/V
    left by an earlier owner: the outputs must still match the oracle on
    the stored slots. The pool holds exactly max_pages pages; the first
    poisoning takes all of them and the second every free one, so every
    slot these sequences do not store holds NaN or inf. Prefix of 200 =
    6*32 + 8 slots (at 16 slots a page, its partial tile's second half lies
    wholly past the end); suffixes of 20 and 45 tokens; then one decode
    step."""
    nh, nkv, dk, dv = geom
    say("stale slots", page_size, geom)
    N = nda()
    rng = np.random.default_rng(40 + page_size + nh)
    W, npre, n = 512, 200, [20, 45]
    per = (npre + page_size - 1) // page_size
    pages = 2 * per + sum((x + 1 + page_size - 1) // page_size for x in n) + 2
    for dt in (O.KV_F16, O.KV_INT8):
        ctx = N.Context(1, nh, nkv, dk, dv, W, kv_dtype=dt, max_seqs=4, page_size=page_size,
                        max_pages=pages)
        _poison_free_pages(N, ctx, [3, 0], pages, page_size, W, nh, nkv, dk, dv)
        q = rng.standard_normal((npre, nh, dk)).astype(np.float32)
        k = rng.standard_normal((npre, nkv, dk)).astype(np.float32)
        v = rng.standard_normal((npre, nkv, dv)).astype(np.float32)
        dout = N.DevBuf(npre * nh * dv * 4)
        ctx.prefill(0, [npre], N.DevBuf.from_array(q), N.DevBuf.from_array(k), N.DevBuf.from_array(v),
                    dout, seq_ids=[2])
        ctx.sync()
        got = dout.to_array(np.float32, (npre, nh * dv))
        view, keep = _views_for(ctx, 0, 2, npre - 1, nh, dt)
        worst = 0.0
        for t in (0, 31, 100, 191, 192, 199):
            want = O.attend_runs(view, np.arange(t + 1), [t + 1], q[t], None)
            worst = max(worst, maxdiff(got[t], want))
        ctx.advance(1, [2], npre)
        pid = ctx.prefix_build(2)
        ctx.seq_reset(2)
        _poison_free_pages(N, ctx, [3, 0], pages - per, page_size, W, nh, nkv, dk, dv)
        for b in range(2):
            ctx.seq_attach(b, pid)
        T = sum(n)
        q = rng.standard_normal((T, nh, dk)).astype(np.float32)
        k = rng.standard_normal((T, nkv, dk)).astype(np.float32)
        v = rng.standard_normal((T, nkv, dv)).astype(np.float32)
        dout = N.DevBuf(T * nh * dv * 4)
        ctx.prefill(0, n, N.DevBuf.from_array(q), N.DevBuf.from_array(k), N.DevBuf.from_array(v), dout,
                    seq_ids=[0, 1])
        ctx.sync()
        got = dout.to_array(np.float32, (T, nh * dv))
        assert np.isfinite(got).all(), dt
        r = 0
        for b in range(2):
            view, keep = _views_for(ctx, 0, b, npre + n[b] - 1, nh, dt)
            for t in range(n[b]):
                pos = npre + t
                want = O.attend_runs(view, np.arange(pos + 1), [npre, pos + 1 - npre], q[r], None)
                worst = max(worst, maxdiff(got[r], want))
                r += 1
        for b in range(2):
            ctx.advance(1, [b], n[b])
        qd = rng.standard_normal((2, nh, dk)).astype(np.float32)
        kd = rng.standard_normal((2, nkv, dk)).astype(np.float32)
        vd = rng.standard_normal((2, nkv, dv)).astype(np.float32)
        dout = N.DevBuf(2 * nh * dv * 4)
        ctx.step(0, 2, N.DevBuf.from_array(qd), N.DevBuf.from_array(kd), N.DevBuf.from_array(vd), dout)
        ctx.sync()
        got = dout.to_array(np.float32, (2, nh * dv))
        assert np.isfinite(got).all(), dt
        for b in range(2):
            pos = ctx.seq_state(b)[0]
            view, keep = _views_for(ctx, 0, b, pos, nh, dt)
            want = O.attend_runs(view, np.arange(pos + 1), [npre, pos + 1 - npre], qd[b], None)
            worst = max(worst, maxdiff(got[b], want))
        ctx.close()
        assert worst <= TOL, (dt, worst)
