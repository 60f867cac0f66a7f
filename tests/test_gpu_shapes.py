"""Every attention shape the engine defines, beyond the two with specialised
kernels: head dims that are multiples of 4 up to 64 (ND_KV_HD_CAP,
engine/include/nd_model.h:244) and 1-8 query heads per kv-head (ND_KV_REP_CAP,
:245), including odd groups (rep 3, 5, 7), qk 32 and qk 36 / 20 (whose last
4 dims the engine's qk_dot8 sums term by term). These run on the kernels
instantiated for dims padded to 64 with the true dims read at run time.

Against the oracle (pinned bit-exact to the reference for these shapes in
tests/test_oracle_ref.py): engine sessions through the C shim (fused store +
decode, sinks, ring wrap, snapshot / rewind, prefix save / restore) with
stored int8 codes bit-identical; batched ragged decode at the two-launch
size; split-KV with the merge; the VALU causal prefill. Bar: max |delta| <=
1e-3. Shapes the engine does not define are refused at creation."""
import sys

import numpy as np
import pytest

import ndoracle as O
from test_gpu_parity import check_cache, maxdiff, replay

pytestmark = pytest.mark.gpu

TOL = 1e-3

# (n_heads, n_kv_heads, qk_head_dim, v_head_dim)
SHAPES = [(6, 2, 32, 32), (10, 2, 36, 20), (7, 1, 64, 64), (8, 1, 20, 44), (4, 4, 16, 8), (3, 1, 48, 64),
          (16, 4, 64, 32)]


def nda():
    import ndattn
    return ndattn


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("shape", SHAPES)
def test_engine_session_int8(shape):
    nh, nkv, qk, vd = shape
    say("session int8", shape)
    W = 96
    script = ([("tok", True)] * 20 + [("sink", 12), ("snap",), ("save", 0)] +
              [("tok", i % 3 != 0) for i in range(90)] + [("restore", 0)] + [("tok", True)] * 5 +
              [("rewind",), ("tok", True)] * 3 + [("tok", True)] * 80)
    o, g, worst, _ = replay((2, nh, nkv, qk, vd, W), script, seed=nh * 100 + qk, scale=1.5)
    say("worst", worst)
    assert worst <= TOL, worst
    ns = o.n_sink          # the snapshot pins the positions it saved
    assert 0 < ns < W - 64
    check_cache(o, g, [0, 1], list(range(ns)) + list(range(o.pos - (W - ns), o.pos)))
    g.close()


@pytest.mark.parametrize("shape", SHAPES[:4])
def test_engine_session_f16(shape):
    nh, nkv, qk, vd = shape
    say("session f16", shape)
    script = [("tok", True)] * 40 + [("snap",)] + [("tok", True)] * 70
    o, g, worst, _ = replay((1, nh, nkv, qk, vd, 64), script, seed=nh + qk, kv_dtype=O.KV_F16)
    assert worst <= TOL, worst
    g.close()


@pytest.mark.parametrize("kv_dtype", [O.KV_INT8, O.KV_F16])
@pytest.mark.parametrize("shape", [(10, 2, 36, 20), (7, 1, 64, 64), (6, 2, 32, 32)])
def test_batched_decode_two_launch_size(kv_dtype, shape):
    """Enough (row, kv-head) units for the separate append launch: 4096
    rows' worth, ragged 40-600 positions, then a second step; sampled rows
    against the oracle, every appended row stored as the oracle stores it."""
    N = nda()
    nh, nkv, qk, vd = shape
    B = 4096 // nkv + 64
    say("batched decode", shape, "dtype", kv_dtype, "rows", B)
    rng = np.random.default_rng(qk + nh)
    lens = rng.integers(40, 601, B)
    ctx = N.Context(1, nh, nkv, qk, vd, 640, kv_dtype=kv_dtype, max_seqs=B)
    for b in range(B):
        ctx.seq_set_pos(b, int(lens[b]) - 1)
        ctx.seq_reserve(b, 2)
    ctx.kv_fill_normal(B, seed=5)
    dq, dk, dv, dg, dout = (N.DevBuf(B * nh * 64 * 4) for _ in range(5))
    for buf, sd, n in ((dq, 1, nh * qk), (dk, 2, nkv * qk), (dv, 3, nkv * vd), (dg, 4, nh * vd)):
        buf.fill_normal(B * n, 0, sd)
    sample = rng.choice(B, 16, replace=False)
    worst = 0.0
    for step in range(2):
        ctx.step(0, B, dq, dk, dv, dout, gate=dg)
        ctx.sync()
        out = dout.to_array(np.float32, (B, nh * vd))
        assert np.isfinite(out).all()
        q = dq.to_array(np.float32, (B, nh * qk))
        g = dg.to_array(np.float32, (B, nh * vd))
        kn = dk.to_array(np.float32, (B, nkv, qk))
        for b in sample:
            pos = ctx.seq_state(int(b))[0]
            k, v, ks, vs = ctx.kv_read(0, int(b), 0, pos + 1)
            if kv_dtype == O.KV_F16:
                ks = vs = None
                assert np.array_equal(k[pos], O.f32_to_f16_bits(kn[b]))
            else:
                for gg in range(nkv):
                    c = np.zeros(qk, np.int8)
                    sc = O.lib().ndo_kv_quant_row(np.ascontiguousarray(kn[b, gg]), qk, c)
                    assert np.array_equal(c, k[pos, gg]) and np.float32(sc) == ks[pos, gg]
            kv = O.kv_view(k, v, ks, vs, nh, pos + 1, 0, pos, kv_dtype)
            worst = max(worst, maxdiff(out[b], O.attend_view(kv, q[b], g[b])))
        ctx.advance(B, None, 1)
    say("worst", worst)
    assert worst <= TOL, worst
    ctx.close()


def _write_history(ctx, rng, b, L, nkv, qk, vd, kv_dtype):
    kf = rng.standard_normal((L, nkv, qk)).astype(np.float32)
    vf = rng.standard_normal((L, nkv, vd)).astype(np.float32)
    if kv_dtype == O.KV_F16:
        ctx.kv_write(0, b, 0, O.f32_to_f16_bits(kf), O.f32_to_f16_bits(vf))
        return
    k = np.zeros(kf.shape, np.int8)
    v = np.zeros(vf.shape, np.int8)
    ks = np.zeros((L, nkv), np.float32)
    vs = np.zeros((L, nkv), np.float32)
    for p in range(L):
        for gg in range(nkv):
            ks[p, gg] = O.lib().ndo_kv_quant_row(np.ascontiguousarray(kf[p, gg]), qk, k[p, gg])
            vs[p, gg] = O.lib().ndo_kv_quant_row(np.ascontiguousarray(vf[p, gg]), vd, v[p, gg])
    ctx.kv_write(0, b, 0, k, v, ks, vs)


@pytest.mark.parametrize("kv_dtype", [O.KV_INT8, O.KV_F16])
def test_split_kv_odd_shapes(kv_dtype):
    """Rows cut into 256-position chunks and merged (the merge reads v_hd at
    run time)."""
    N = nda()
    say("split-kv odd shapes", kv_dtype)
    for nh, nkv, qk, vd in ((10, 2, 36, 20), (7, 1, 64, 64)):
        rng = np.random.default_rng(qk * 3 + vd)
        lens = [1500, 700, 257, 256, 3]
        B = len(lens)
        ctx = N.Context(1, nh, nkv, qk, vd, 1600, kv_dtype=kv_dtype, max_seqs=B, split_chunk=256)
        for b, L in enumerate(lens):
            if L > 1:
                _write_history(ctx, rng, b, L - 1, nkv, qk, vd, kv_dtype)
            ctx.seq_set_pos(b, L - 1)
        q = rng.standard_normal((B, nh, qk)).astype(np.float32)
        k = rng.standard_normal((B, nkv, qk)).astype(np.float32)
        v = rng.standard_normal((B, nkv, vd)).astype(np.float32)
        g = rng.standard_normal((B, nh, vd)).astype(np.float32)
        dout = N.DevBuf(B * nh * vd * 4)
        ctx.prof_enable(True)
        ctx.prof_read(reset=True)
        ctx.step(0, B, N.DevBuf.from_array(q), N.DevBuf.from_array(k), N.DevBuf.from_array(v), dout,
                 gate=N.DevBuf.from_array(g))
        ctx.sync()
        assert ctx.prof_read(reset=True)[1][N.K_COMBINE] > 0
        ctx.prof_enable(False)
        out = dout.to_array(np.float32, (B, nh * vd))
        worst = 0.0
        for b, L in enumerate(lens):
            kk, vv, ks, vs = ctx.kv_read(0, b, 0, L)
            if kv_dtype == O.KV_F16:
                ks = vs = None
            kv = O.kv_view(kk, vv, ks, vs, nh, L, 0, L - 1, kv_dtype)
            worst = max(worst, maxdiff(out[b], O.attend_view(kv, q[b].ravel(), g[b].ravel())))
        say((nh, nkv, qk, vd), "worst", worst)
        assert worst <= TOL, worst
        ctx.close()


@pytest.mark.parametrize("kv_dtype", [O.KV_INT8, O.KV_F16])
@pytest.mark.parametrize("shape", [(6, 2, 32, 32), (10, 2, 36, 20), (8, 1, 20, 44)])
def test_causal_prefill_odd_shapes(kv_dtype, shape):
    """Ragged chunks over stored history, every output row against the oracle
    over positions [0, pos + t]."""
    N = nda()
    nh, nkv, qk, vd = shape
    say("prefill", shape, "dtype", kv_dtype)
    rng = np.random.default_rng(nh * 7 + qk)
    hist = [0, 5, 40, 130]
    ntok = [33, 1, 70, 17]
    B = len(hist)
    W = max(h + n for h, n in zip(hist, ntok)) + 8
    ctx = N.Context(1, nh, nkv, qk, vd, W, kv_dtype=kv_dtype, max_seqs=B)
    for b, L in enumerate(hist):
        if L:
            _write_history(ctx, rng, b, L, nkv, qk, vd, kv_dtype)
        ctx.seq_set_pos(b, L)
    T = int(sum(ntok))
    q = rng.standard_normal((T, nh, qk)).astype(np.float32)
    k = rng.standard_normal((T, nkv, qk)).astype(np.float32)
    v = rng.standard_normal((T, nkv, vd)).astype(np.float32)
    g = rng.standard_normal((T, nh, vd)).astype(np.float32)
    dout = N.DevBuf(T * nh * vd * 4)
    ctx.prefill(0, ntok, N.DevBuf.from_array(q), N.DevBuf.from_array(k), N.DevBuf.from_array(v), dout,
                gate=N.DevBuf.from_array(g))
    ctx.sync()
    got = dout.to_array(np.float32, (T, nh * vd))
    worst, r = 0.0, 0
    for b in range(B):
        end = hist[b] + ntok[b]
        kk, vv, ks, vs = ctx.kv_read(0, b, 0, end)
        if kv_dtype == O.KV_F16:
            ks = vs = None
        for t in range(ntok[b]):
            kv = O.kv_view(kk, vv, ks, vs, nh, end, 0, hist[b] + t, kv_dtype)
            worst = max(worst, maxdiff(got[r], O.attend_view(kv, q[r].ravel(), g[r].ravel())))
            r += 1
    say("worst", worst)
    assert worst <= TOL, worst
    ctx.close()


def test_undefined_shapes_refused():
    """Head dims that are not multiples of 4, above 64, or more than 8 query
    heads per kv-head: the engine's attn_heads does not define them."""
    N = nda()
    for nh, nkv, qk, vd in ((8, 8, 30, 64), (8, 8, 64, 62), (8, 8, 68, 64), (9, 1, 64, 64), (8, 8, 64, 0)):
        with pytest.raises(N.NdaError) as e:
            N.Context(1, nh, nkv, qk, vd, 64)
        assert e.value.code in (-1, -6), (nh, nkv, qk, vd, e.value.code)
    ctx = N.Context(1, 10, 2, 36, 20, 64)
    ctx.front_init(3, 10000.0)                 # every defined shape has a front
    ctx.close()
