"""GPU parity of the attention front (nda_front / nda_attention and the
shim's nd_gpu_attention_raw) against the oracle: the front's q/k/v rows and
the tap histories bit-exact, stored int8 codes and scales bit-exact,
attention outputs within max |delta| <= 1e-3; and the engine session replay
against the reference engine's own golden outputs. The shapes include odd
ones (qk 36 / v 20, 7 query heads on one kv-head, qk 16 / v 8) that run on
the front kernel with run-time dims; the oracle's front is pinned bit-exact
to the reference at those shapes in tests/test_oracle_front.py."""
import os
import sys

import numpy as np
import pytest

import ndoracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3
HERE = os.path.dirname(os.path.abspath(__file__))


def nda():
    import ndattn
    return ndattn


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def maxdiff(a, b):
    return float(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)).max())


def make_weights(rng, L, nh, nkv, qk, vd, taps):
    t = lambda dim: (rng.standard_normal((L, taps, dim)) * 0.5).astype(np.float32)
    return O.FrontWeights(t(nh * qk), t(nkv * qk), t(nkv * vd),
                          (rng.standard_normal((L, qk)) * 0.25).astype(np.float32),
                          (rng.standard_normal((L, qk)) * 0.25).astype(np.float32))


def front_ctx(N, L, nh, nkv, qk, vd, window, kv_dtype, nseq, taps, theta, fw, max_prefixes=8):
    ctx = N.Context(L, nh, nkv, qk, vd, window, kv_dtype=kv_dtype, max_seqs=nseq, max_prefixes=max_prefixes)
    ctx.front_init(taps, theta)
    for li in range(L):
        ctx.front_weights(li, *fw.arrays(li))
    return ctx


def oracle_sessions(nseq, geom, kv_dtype, taps, theta):
    out = []
    for _ in range(nseq):
        o = O.OracleSession(*geom, kv_dtype=kv_dtype)
        o.front_init(taps, theta)
        out.append(o)
    return out


@pytest.mark.parametrize("shape,kv_dtype,taps,theta", [
    ((8, 8, 64, 64), O.KV_F16, 3, 10000.0),
    ((12, 2, 48, 64), O.KV_INT8, 3, 10000.0),     # the archive's shapes
    ((8, 2, 64, 64), O.KV_INT8, 4, 1000000.0),
    ((16, 2, 64, 64), O.KV_F16, 1, 500000.0),
    # shapes on the kernel with run-time dims
    ((10, 2, 36, 20), O.KV_INT8, 3, 10000.0),
    ((7, 1, 64, 64), O.KV_F16, 2, 10000.0),
    ((8, 1, 20, 44), O.KV_INT8, 4, 1000000.0),
    ((4, 4, 16, 8), O.KV_F16, 1, 10000.0),
    ((16, 4, 64, 32), O.KV_INT8, 3, 10000.0),
    ((3, 1, 48, 64), O.KV_INT8, 3, 10000.0),
])
def test_front_rows_bit_exact(shape, kv_dtype, taps, theta):
    """nda_front, one token per sequence per call, sequences at different
    positions (some below taps-1, some far out): q/k/v rows and the live
    histories bit-identical to the oracle's front."""
    N = nda()
    nh, nkv, qk, vd = shape
    say("front rows", shape, kv_dtype, taps)
    rng = np.random.default_rng(11 + taps)
    L, W = 2, 512
    starts = [0, 1, 2, 7, 300, 4000]
    B = len(starts)
    fw = make_weights(rng, L, nh, nkv, qk, vd, taps)
    ctx = front_ctx(N, L, nh, nkv, qk, vd, W, kv_dtype, B, taps, theta, fw)
    orc = oracle_sessions(B, (L, nh, nkv, qk, vd, W), kv_dtype, taps, theta)
    for b, p in enumerate(starts):
        ctx.seq_set_pos(b, p)
        orc[b].s.pos = p
    dq, dk, dv = nh * qk, nkv * qk, nkv * vd
    bq, bk, bv = (N.DevBuf(B * d * 4) for d in (dq, dk, dv))
    oq, ok_, ov = (N.DevBuf(B * d * 4) for d in (dq, dk, dv))
    for step in range(taps + 3):
        for li in range(L):
            q = rng.standard_normal((B, dq)).astype(np.float32)
            k = rng.standard_normal((B, dk)).astype(np.float32)
            v = rng.standard_normal((B, dv)).astype(np.float32)
            if step == 1:
                k[2] *= np.float32(3e3)
            bq.upload(q), bk.upload(k), bv.upload(v)
            ctx.front(li, B, bq, bk, bv, oq, ok_, ov)
            ctx.sync()
            gq, gk, gv = oq.to_array(np.float32, (B, dq)), ok_.to_array(np.float32, (B, dk)), \
                ov.to_array(np.float32, (B, dv))
            for b in range(B):
                wq, wk, wv = orc[b].front(li, fw, q[b], k[b], v[b])
                assert np.array_equal(bits(gq[b]), bits(wq)), (step, li, b)
                assert np.array_equal(bits(gk[b]), bits(wk)), (step, li, b)
                assert np.array_equal(bits(gv[b]), bits(wv)), (step, li, b)
        ctx.advance(B)
        for o in orc:
            o.step_end()
    for b in range(B):
        want = np.concatenate([h.reshape(L, taps, -1) for h in orc[b].hist()], axis=2)
        assert np.array_equal(bits(ctx.front_hist(b)), bits(want)), b


@pytest.mark.parametrize("shape,kv_dtype", [((12, 2, 48, 64), O.KV_F16), ((12, 2, 48, 64), O.KV_INT8),
                                             ((10, 2, 36, 20), O.KV_INT8), ((7, 1, 64, 64), O.KV_F16)])
def test_front_multi_token_chunk(shape, kv_dtype):
    """nda_front over chunks of several tokens per sequence (a prefill chunk's
    front) equals the token-by-token oracle, including the history left for
    the next single-token call."""
    N = nda()
    say("front multi-token chunk", shape, kv_dtype)
    rng = np.random.default_rng(5)
    nh, nkv, qk, vd = shape
    L, W, taps, theta = 1, 256, 3, 10000.0
    n_tok = [5, 1, 9, 0, 3, 2]
    starts = [0, 4, 1, 8, 20, 0]
    B = len(n_tok)
    fw = make_weights(rng, L, nh, nkv, qk, vd, taps)
    ctx = front_ctx(N, L, nh, nkv, qk, vd, W, kv_dtype, B, taps, theta, fw)
    orc = oracle_sessions(B, (L, nh, nkv, qk, vd, W), kv_dtype, taps, theta)
    dq, dk, dv = nh * qk, nkv * qk, nkv * vd
    # sequences start at different positions with empty histories (a fresh
    # context), as the oracle sessions do
    for b, p in enumerate(starts):
        ctx.seq_set_pos(b, p)
        orc[b].s.pos = p
    T = sum(n_tok)
    for rnd in range(2):
        q = rng.standard_normal((T, dq)).astype(np.float32)
        k = rng.standard_normal((T, dk)).astype(np.float32)
        v = rng.standard_normal((T, dv)).astype(np.float32)
        bq, bk, bv = N.DevBuf.from_array(q), N.DevBuf.from_array(k), N.DevBuf.from_array(v)
        oq, ok_, ov = (N.DevBuf(max(1, T * d * 4)) for d in (dq, dk, dv))
        ctx.front(0, B, bq, bk, bv, oq, ok_, ov, n_tokens=n_tok)
        ctx.sync()
        gq, gk, gv = oq.to_array(np.float32, (T, dq)), ok_.to_array(np.float32, (T, dk)), \
            ov.to_array(np.float32, (T, dv))
        r = 0
        for b in range(B):
            for t in range(n_tok[b]):
                wq, wk, wv = orc[b].front(0, fw, q[r], k[r], v[r])
                assert np.array_equal(bits(gq[r]), bits(wq)), (rnd, b, t)
                assert np.array_equal(bits(gk[r]), bits(wk)), (rnd, b, t)
                assert np.array_equal(bits(gv[r]), bits(wv)), (rnd, b, t)
                orc[b].step_end()
                r += 1
        for b in range(B):
            if n_tok[b]:
                ctx.advance(1, seq_ids=[b], n=n_tok[b])
            want = np.concatenate([h.reshape(L, taps, -1) for h in orc[b].hist()], axis=2)
            assert np.array_equal(bits(ctx.front_hist(b)), bits(want)), (rnd, b)


@pytest.mark.parametrize("shape,kv_dtype", [((12, 2, 48, 64), O.KV_F16), ((12, 2, 48, 64), O.KV_INT8),
                                             ((8, 8, 64, 64), O.KV_F16)])
def test_front_multi_token_large_launch(shape, kv_dtype):
    """A multi-token front launch of at least 4096 (row, kv group) units runs
    two rows per work-group: bit-exact against the token-by-token oracle over
    an odd row count (the last work-group's second row is past the end),
    sequences of 0 and 1 tokens (pairs straddle sequences) and a second round
    reading the history the first one left."""
    N = nda()
    say("front multi-token large launch", shape, kv_dtype)
    rng = np.random.default_rng(17)
    nh, nkv, qk, vd = shape
    L, W, taps, theta = 1, 256, 3, 10000.0
    B = 48 if nkv == 2 else 16
    n_tok = [int(x) for x in rng.integers(20, 90, B)]
    n_tok[3], n_tok[7], n_tok[8] = 0, 1, 1
    if sum(n_tok) % 2 == 0:
        n_tok[0] += 1
    T = sum(n_tok)
    assert T * nkv >= 4096 and T % 2 == 1
    starts = [int(x) for x in rng.integers(0, 40, B)]
    fw = make_weights(rng, L, nh, nkv, qk, vd, taps)
    ctx = front_ctx(N, L, nh, nkv, qk, vd, W, kv_dtype, B, taps, theta, fw)
    orc = oracle_sessions(B, (L, nh, nkv, qk, vd, W), kv_dtype, taps, theta)
    dq, dk, dv = nh * qk, nkv * qk, nkv * vd
    for b, p in enumerate(starts):
        ctx.seq_set_pos(b, p)
        orc[b].s.pos = p
    for rnd in range(2):
        q = rng.standard_normal((T, dq)).astype(np.float32)
        k = rng.standard_normal((T, dk)).astype(np.float32)
        v = rng.standard_normal((T, dv)).astype(np.float32)
        bq, bk, bv = N.DevBuf.from_array(q), N.DevBuf.from_array(k), N.DevBuf.from_array(v)
        oq, ok_, ov = (N.DevBuf(T * d * 4) for d in (dq, dk, dv))
        ctx.front(0, B, bq, bk, bv, oq, ok_, ov, n_tokens=n_tok)
        ctx.sync()
        gq, gk, gv = oq.to_array(np.float32, (T, dq)), ok_.to_array(np.float32, (T, dk)), \
            ov.to_array(np.float32, (T, dv))
        r = 0
        for b in range(B):
            for t in range(n_tok[b]):
                wq, wk, wv = orc[b].front(0, fw, q[r], k[r], v[r])
                assert np.array_equal(bits(gq[r]), bits(wq)), (rnd, b, t)
                assert np.array_equal(bits(gk[r]), bits(wk)), (rnd, b, t)
                assert np.array_equal(bits(gv[r]), bits(wv)), (rnd, b, t)
                orc[b].step_end()
                r += 1
        for b in range(B):
            if n_tok[b]:
                ctx.advance(1, seq_ids=[b], n=n_tok[b])
            want = np.concatenate([h.reshape(L, taps, -1) for h in orc[b].hist()], axis=2)
            assert np.array_equal(bits(ctx.front_hist(b)), bits(want)), (rnd, b)


@pytest.mark.parametrize("shape,kv_dtype", [((8, 2, 64, 64), O.KV_INT8), ((8, 2, 64, 64), O.KV_F16),
                                             ((10, 2, 36, 20), O.KV_INT8), ((7, 1, 64, 64), O.KV_F16)])
def test_attention_batched_sessions(shape, kv_dtype):
    """nda_attention (front + store + decode) over a batch of sequences for
    many steps: outputs within tolerance of the oracle's engine step, stored
    codes / fp16 rows bit-exact; then a snapshot of one sequence shared by the
    others (prefix build + attach), decoding on, a rewind and a reset."""
    N = nda()
    say("attention batched", shape, kv_dtype)
    rng = np.random.default_rng(9)
    nh, nkv, qk, vd = shape
    L, W, taps, theta = 2, 96, 3, 10000.0
    B = 4
    geom = (L, nh, nkv, qk, vd, W)
    fw = make_weights(rng, L, nh, nkv, qk, vd, taps)
    ctx = front_ctx(N, L, nh, nkv, qk, vd, W, kv_dtype, B, taps, theta, fw)
    orc = oracle_sessions(B, geom, kv_dtype, taps, theta)
    dq, dk, dv, do = nh * qk, nkv * qk, nkv * vd, nh * vd
    bq, bk, bv, bg, bo = (N.DevBuf(B * d * 4) for d in (dq, dk, dv, do, do))
    worst = 0.0

    def step(ids):
        nonlocal worst
        n = len(ids)
        for li in range(L):
            q = rng.standard_normal((n, dq)).astype(np.float32)
            k = rng.standard_normal((n, dk)).astype(np.float32)
            v = rng.standard_normal((n, dv)).astype(np.float32)
            g = rng.standard_normal((n, do)).astype(np.float32)
            bq.upload(q), bk.upload(k), bv.upload(v), bg.upload(g)
            ctx.attention(li, n, bq, bk, bv, bo, gate=bg, seq_ids=ids)
            ctx.sync()
            got = bo.to_array(np.float32, (n, do))
            for i, b in enumerate(ids):
                fq, fk, fv = orc[b].front(li, fw, q[i], k[i], v[i])
                want = orc[b].attention(li, fq, fk, fv, g[i])
                worst = max(worst, maxdiff(got[i], want))
        ctx.advance(n, seq_ids=ids)
        for b in ids:
            orc[b].step_end()

    def check_state(b):
        s = orc[b]
        pos, n_sink, _ = ctx.seq_state(b)
        assert (pos, n_sink) == (s.pos, s.n_sink), b
        want = np.concatenate([h.reshape(L, taps, -1) for h in s.hist()], axis=2)
        assert np.array_equal(bits(ctx.front_hist(b)), bits(want)), b
        ok, ov, oks, ovs = s.cache()
        lo = s.pos - (W - s.n_sink) + 1 if s.pos >= W else 0     # oldest ring position kept
        for li in range(L):
            for p in list(range(min(s.n_sink, s.pos))) + list(range(max(lo, s.n_sink), s.pos)):
                sl = O.lib().ndo_kv_slot(W, s.n_sink, p)
                k, v, ks, vs = ctx.kv_read(li, b, p, 1)
                assert np.array_equal(k[0], ok[li, sl]) and np.array_equal(v[0], ov[li, sl]), (b, li, p)
                if kv_dtype == O.KV_INT8:
                    assert np.array_equal(bits(ks[0]), bits(oks[li, sl])), (b, li, p)

    ids = list(range(B))
    for _ in range(12):
        step(ids)
    for b in ids:
        check_state(b)
    # sequence 0 becomes a shared prefix: snapshot (build + attach), others attach
    pid = ctx.prefix_build(0)
    for b in ids:
        ctx.seq_attach(b, pid)
    assert orc[0].snapshot() == 0
    # the other oracle sessions take sequence 0's snapshot state, as a restore
    # of sequence 0's saved prefix would give them
    for b in ids[1:]:
        _copy_oracle_state(orc[0], orc[b], geom, kv_dtype, taps)
    for _ in range(100):         # past the window: the ring wraps behind the pinned prefix
        step(ids)
    for b in ids:
        check_state(b)
    ctx.seq_rewind(2)
    orc[2].rewind()
    ctx.seq_reset(3)
    orc[3].reset()
    for _ in range(5):
        step(ids)
    for b in ids:
        check_state(b)
    say("attention batched worst", worst)
    assert worst <= TOL, worst


def _copy_oracle_state(src, dst, geom, kv_dtype, taps):
    """dst := src (KV arrays, scales, histories, snapshot, pos/sink)."""
    import ctypes as C
    L, nh, nkv, qk, vd, W = geom
    es = 1 if kv_dtype == O.KV_INT8 else 2
    sizes = {"k_cache": L * W * nkv * qk * es, "v_cache": L * W * nkv * vd * es,
             "k_scale": L * W * nkv * 4, "v_scale": L * W * nkv * 4}
    dcols = {"q": nh * qk, "k": nkv * qk, "v": nkv * vd}
    for x in "qkv":
        sizes[x + "_hist"] = sizes["snap_" + x + "_hist"] = L * taps * dcols[x] * 4
    for name, n in sizes.items():
        C.memmove(getattr(dst.s, name), getattr(src.s, name), n)
    for f in ("pos", "n_sink", "has_snap", "snap_pos"):
        setattr(dst.s, f, getattr(src.s, f))


def test_shim_front_session_against_reference_golden():
    """The engine drop-in with the front (nd_gpu_attention_raw) replays the
    golden script that the reference engine's own code produced
    (tests/golden: front_engine, 12/2 heads, qk 48, 3 taps, snapshot /
    rewind / prefix switching): outputs within tolerance of the reference's,
    the stored cache's checksums and the tap histories identical."""
    N = nda()
    sys.path.insert(0, os.path.join(HERE, "golden"))
    from gen_golden import SESSIONS, front_weights  # noqa: E402
    from detgen import Stream  # noqa: E402
    G = np.load(os.path.join(HERE, "golden", "golden.npz"))
    spec = SESSIONS["front_engine"]
    say("shim front golden replay")
    L, nh, nkv, qk, vd, W = spec["geom"]
    taps, theta = spec["front"]
    g = N.GpuSession(L, nh, nkv, qk, vd, W, kv_dtype=N.KV_INT8)
    fw = front_weights(spec)
    g.front_init(taps, theta, fw)
    st = Stream(spec["seed"])
    outs, saved = [], {}
    for ev in spec["script"]:
        if ev[0] == "tok":
            for li in range(L):
                q, k, v = st.take(nh * qk), st.take(nkv * qk), st.take(nkv * vd)
                gt = st.take(nh * vd) if ev[1] else None
                outs.append(g.attention(li, q, k, v, gt))
            g.step_end()
        elif ev[0] == "snap":
            assert g.snapshot() == 0
        elif ev[0] == "save":
            saved[ev[1]] = g.prefix_save()
            assert saved[ev[1]]
        elif ev[0] == "restore":
            assert g.prefix_restore(saved[ev[1]]) == 0
        elif ev[0] == "reset":
            g.reset()
        elif ev[0] == "rewind":
            g.rewind()
    want = G["sess_front_engine"]
    got = np.stack(outs)
    assert got.shape == want.shape
    worst = maxdiff(got, want)
    say("shim front golden worst", worst)
    assert worst <= TOL, worst
    # live histories of the session equal the reference's live histories
    ctx = g.context()
    ref_live = G["sess_front_engine_hist"][: G["sess_front_engine_hist"].size // 2]
    dcol = nh * qk + nkv * (qk + vd)
    live = ctx.front_hist(0)                      # [L][taps][dcol] as q | k | v
    parts = [live[:, :, :nh * qk], live[:, :, nh * qk:nh * qk + nkv * qk], live[:, :, nh * qk + nkv * qk:]]
    assert live.shape == (L, taps, dcol)
    assert np.array_equal(bits(np.concatenate([p.ravel() for p in parts])), bits(ref_live))
    for p in saved.values():
        g.prefix_free(p)
    g.close()


def test_front_error_paths():
    N = nda()
    say("front error paths")
    rng = np.random.default_rng(2)
    ctx = N.Context(2, 8, 8, 64, 64, 64, kv_dtype=N.KV_F16, max_seqs=4)
    buf = N.DevBuf(4 * 512 * 4)
    with pytest.raises(N.NdaError) as e:
        ctx.front(0, 1, buf, buf, buf, buf, buf, buf)
    assert e.value.code == -5                 # not initialised
    ctx.front_init(3, 10000.0, max_pos=100)
    with pytest.raises(N.NdaError) as e:
        ctx.front_init(3, 10000.0)
    assert e.value.code == -5
    with pytest.raises(N.NdaError) as e:
        ctx.front(0, 1, buf, buf, buf, buf, buf, buf)
    assert e.value.code == -5                 # no weights for layer 0
    fw = make_weights(rng, 2, 8, 8, 64, 64, 3)
    ctx.front_weights(0, *fw.arrays(0))
    with pytest.raises(N.NdaError) as e:
        ctx.front(0, 2, buf, buf, buf, buf, buf, buf, seq_ids=[1, 1])
    assert e.value.code == -1                 # a sequence twice
    ctx.seq_set_pos(0, 99)
    with pytest.raises(N.NdaError) as e:
        ctx.front(0, 1, buf, buf, buf, buf, buf, buf, n_tokens=[2])
    assert e.value.code == -4                 # beyond the rotary table
    ctx.front(0, 1, buf, buf, buf, buf, buf, buf, n_tokens=[1])
    ctx.sync()
    bad = N.Context(1, 8, 8, 64, 64, 64, kv_dtype=N.KV_F16, max_seqs=1)
    with pytest.raises(N.NdaError) as e:
        bad.front_init(0, 10000.0)
    assert e.value.code == -1
