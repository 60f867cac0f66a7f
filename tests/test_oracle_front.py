"""The oracle's attention front (tap convolution, per-head ZC-RMSNorm, RoPE;
engine/src/nd_model.c:2413-2424) pinned two ways: bit-exact against the
reference's own tap_projection / zcrms_heads compiled from its sources (live,
where the harness is built), and against what the mathematics fixes (one-hot
taps, the causal truncation, the norm's closed form, rotation invariants,
float64 trigonometry)."""
import numpy as np
import pytest

import ndoracle as O
from detgen import Stream


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def ulps(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


def weights(seed, L, nh, nkv, qk, vd, taps):
    st = Stream(seed)
    shape = lambda dim: st.take(L * taps * dim).reshape(L, taps, dim) * np.float32(0.5)
    return O.FrontWeights(shape(nh * qk), shape(nkv * qk), shape(nkv * vd),
                          st.take(L * qk).reshape(L, qk) * np.float32(0.25),
                          st.take(L * qk).reshape(L, qk) * np.float32(0.25))


# ------------------------------------------------------------- reference

@pytest.mark.skipif(not O.have_ref(), reason="reference harness not built")
@pytest.mark.parametrize("geom,taps,theta", [
    ((2, 12, 2, 48, 64, 64), 3, 10000.0),     # the archive's shapes
    ((1, 8, 8, 64, 64, 64), 1, 10000.0),      # one tap: w0 * x
    ((1, 8, 2, 64, 64, 64), 2, 500000.0),     # GQA 4
    ((1, 16, 2, 64, 64, 64), 4, 1000000.0),   # GQA 8, 4 taps
    ((1, 6, 3, 48, 64, 64), 5, 10000.0),
    ((1, 10, 2, 36, 20, 64), 3, 10000.0),    # odd dims: qk 36 (9 rotary pairs per half)
    ((1, 7, 1, 64, 64, 64), 2, 10000.0),     # 7 query heads on one kv-head
    ((1, 8, 1, 20, 44, 64), 4, 1000000.0),
    ((1, 4, 4, 16, 8, 64), 1, 10000.0),
])
def test_front_matches_reference(geom, taps, theta):
    L, nh, nkv, qk, vd, W = geom
    o = O.OracleSession(*geom)
    r = O.RefSession(*geom)
    o.front_init(taps, theta)
    r.front_init(taps, theta)
    fw = weights(31 + taps, L, nh, nkv, qk, vd, taps)
    st = Stream(977 + taps)
    for step in range(3 * taps + 7):
        for li in range(L):
            q, k, v = st.take(nh * qk), st.take(nkv * qk), st.take(nkv * vd)
            if step == 5:
                k = k * np.float32(1e4)          # large rows: the norm's range
            got = o.front(li, fw, q, k, v)
            want = r.front(li, fw, q, k, v)
            for g, w in zip(got, want):
                assert np.array_equal(bits(g), bits(w)), (step, li)
        o.step_end()
        r.step_end()
    for g, w in zip(o.hist(), r.hist()):
        assert np.array_equal(bits(g), bits(w))


@pytest.mark.skipif(not O.have_ref(), reason="reference harness not built")
def test_front_large_positions_match_reference():
    """Positions far from 0 (large rotary angles), set directly."""
    geom = (1, 8, 8, 64, 64, 64)
    o = O.OracleSession(*geom)
    r = O.RefSession(*geom)
    o.front_init(3, 10000.0)
    r.front_init(3, 10000.0)
    fw = weights(5, 1, 8, 8, 64, 64, 3)
    st = Stream(4242)
    for pos in (1000, 1001, 1002, 32767, 65535, 200000):
        o.s.pos = pos
        O.ref().ref_set_pos(r.m, pos)
        q, k, v = st.take(512), st.take(512), st.take(512)
        for g, w in zip(o.front(0, fw, q, k, v), r.front(0, fw, q, k, v)):
            assert np.array_equal(bits(g), bits(w)), pos


# ---------------------------------------------------------- mathematics

def test_rope_tables_against_float64():
    for qk, theta in ((64, 10000.0), (48, 10000.0), (64, 1000000.0)):
        inv = O.rope_inv(theta, qk)
        exact = 1.0 / np.power(np.float64(theta), np.float32(np.arange(0, qk, 2, dtype=np.float32) / np.float32(qk)).astype(np.float64))
        assert ulps(inv, exact.astype(np.float32)).max() <= 2
        assert inv[0] == np.float32(1.0)
        for pos in (0, 1, 7, 213, 1023, 32768, 65535):
            cs, sn = O.rope_row(inv, qk, pos)
            ang = (np.float32(pos) * inv).astype(np.float64)       # the rounded float argument
            assert ulps(cs, np.cos(ang).astype(np.float32)).max() <= 1
            assert ulps(sn, np.sin(ang).astype(np.float32)).max() <= 1
            if pos == 0:
                assert np.all(cs == 1.0) and np.all(sn == 0.0)


def test_tap_conv_one_hot_is_a_delay():
    """w = e_j (all columns) gives the raw projection j positions back, exactly,
    and 0 before the sequence start; the history slot pos % taps takes the raw row."""
    taps, dim = 4, 10
    st = Stream(3)
    raws = [st.take(dim) for _ in range(12)]
    for j in range(taps):
        w = np.zeros((taps, dim), np.float32)
        w[j] = 1.0
        hist = np.zeros((taps, dim), np.float32)
        for pos, x in enumerate(raws):
            out, hist = O.tap_conv(x, hist, w, pos)
            assert np.array_equal(hist[pos % taps], x)
            want = raws[pos - j] if pos >= j else np.zeros(dim, np.float32)
            assert np.array_equal(bits(out), bits(want + np.float32(0.0)))


def test_tap_conv_against_float64_sum():
    taps, dim = 3, 257
    st = Stream(9)
    w = st.take(taps * dim).reshape(taps, dim)
    hist = np.zeros((taps, dim), np.float32)
    raws = [st.take(dim) for _ in range(6)]
    for pos, x in enumerate(raws):
        out, hist = O.tap_conv(x, hist, w, pos)
        want = sum(w[j].astype(np.float64) * raws[pos - j] for j in range(min(taps, pos + 1)))
        assert np.allclose(out, want, rtol=1e-6, atol=1e-6)


def test_zcrms_closed_form():
    """s = 0 and the identity rotation: x / rms(x) per head; s scales by (1+s)."""
    st = Stream(17)
    for nh, dim in ((3, 64), (2, 48), (1, 7)):
        x = st.take(nh * dim).reshape(nh, dim) * np.float32(3.0)
        half = dim // 2
        one, zero = np.ones(half, np.float32), np.zeros(half, np.float32)
        got = O.zcrms_heads(x, np.zeros(dim, np.float32), one, zero)
        x64 = x.astype(np.float64)
        want = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6)
        assert np.allclose(got, want, rtol=2e-6, atol=1e-7)
        s = st.take(dim) * np.float32(0.3)
        got_s = O.zcrms_heads(x, s, one, zero)
        assert np.allclose(got_s, want * (1.0 + s.astype(np.float64)), rtol=4e-6, atol=1e-6)


def test_zcrms_rotation_invariants():
    """RoPE rotates each (i, i+half) pair by the same angle: pair norms are kept,
    the angle between q and k pairs rotated at one position is kept, and a
    quarter turn maps (a, b) to (-b, a)."""
    st = Stream(23)
    dim, half = 64, 32
    x = st.take(2 * dim).reshape(2, dim)
    s = np.zeros(dim, np.float32)
    ang = st.take(half) * np.float32(2.0)
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    base = O.zcrms_heads(x, s, np.ones(half, np.float32), np.zeros(half, np.float32)).astype(np.float64)
    rot = O.zcrms_heads(x, s, cs, sn).astype(np.float64)
    n0 = base[:, :half] ** 2 + base[:, half:] ** 2
    n1 = rot[:, :half] ** 2 + rot[:, half:] ** 2
    assert np.allclose(n0, n1, rtol=1e-5)
    dot0 = base[0, :half] * base[1, :half] + base[0, half:] * base[1, half:]
    dot1 = rot[0, :half] * rot[1, :half] + rot[0, half:] * rot[1, half:]
    assert np.allclose(dot0, dot1, rtol=1e-4, atol=1e-5)
    q = O.zcrms_heads(x, s, np.zeros(half, np.float32), np.ones(half, np.float32))
    b32 = base.astype(np.float32)
    assert np.array_equal(q[:, :half], -b32[:, half:]) and np.array_equal(q[:, half:], b32[:, :half])


def test_front_session_history_and_rewind():
    """The session front keeps per-layer histories: two layers do not mix,
    a rewind restores the snapshot's histories, a reset zeroes them."""
    geom = (2, 4, 2, 64, 64, 64)
    o = O.OracleSession(*geom)
    o.front_init(3, 10000.0)
    fw = weights(77, 2, 4, 2, 64, 64, 3)
    st = Stream(78)
    for _ in range(4):
        for li in range(2):
            o.front(li, fw, st.take(256), st.take(128), st.take(128))
        o.step_end()
    h0 = o.hist()
    assert not np.array_equal(h0[0][0], h0[0][1])
    assert o.snapshot() == 0
    for _ in range(2):
        o.front(0, fw, st.take(256), st.take(128), st.take(128))
        o.step_end()
    assert not np.array_equal(o.hist()[0], h0[0])
    o.rewind()
    for a, b in zip(o.hist(), h0):
        assert np.array_equal(a, b)
    assert o.pos == 4
    o.reset()
    assert all(not h.any() for h in o.hist())
