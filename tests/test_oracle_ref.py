"""The oracle against the reference engine's code compiled from its own
sources (oracle/_ref/libndref.so), live, on many more inputs than the
committed fixture holds. Skipped where that harness was not built."""
import ctypes as C

import numpy as np
import pytest

import ndoracle as O

pytestmark = pytest.mark.skipif(not O.have_ref(), reason="reference harness not built")


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_kv_slot_and_sink_clamp_exhaustive():
    R, L = O.ref(), O.lib()
    for window in (1, 2, 3, 17, 64, 65, 100, 384):
        for n in range(0, window + 70):
            assert L.ndo_clamp_sink(window, n) == R.ref_clamp_sink(window, n)
        for n_sink in range(0, window, max(1, window // 7)):
            for p in range(0, 3 * window + 5):
                assert L.ndo_kv_slot(window, n_sink, p) == R.ref_kv_slot(window, n_sink, p)


def test_kv_slot_closed_form():
    """Brute force: a ring of window-n_sink slots after n_sink fixed ones."""
    L = O.lib()
    for window, n_sink in ((10, 3), (384, 213), (7, 0)):
        ring = {}
        for p in range(5 * window):
            s = L.ndo_kv_slot(window, n_sink, p)
            assert 0 <= s < window
            if p < n_sink:
                assert s == p
            else:
                assert s >= n_sink
                ring[s] = p
        assert len(ring) == window - n_sink


def test_exp_matches_reference_dense():
    R, L = O.ref(), O.lib()
    rng = np.random.default_rng(5)
    xs = np.concatenate([rng.uniform(-90, 90, 20000), rng.normal(0, 3, 20000)]).astype(np.float32)
    for x in xs:
        assert np.float32(L.ndo_expf(float(x))).view(np.uint32) == np.float32(R.ref_expf(float(x))).view(np.uint32)
    r0, r1 = C.c_float(), C.c_float()
    for i in range(0, 2000, 2):
        R.ref_expf_pair(float(xs[i]), float(xs[i + 1]), C.byref(r0), C.byref(r1))
        assert np.float32(r0.value) == np.float32(L.ndo_expf(float(xs[i])))
        assert np.float32(r1.value) == np.float32(L.ndo_expf(float(xs[i + 1])))


def test_exp_accuracy_bound():
    """Against float64 exp: ~3e-6 relative near 0 (the truncated coefficients of nd_quant.h:93-117; the header says ~1e-7), growing
    with |x| through the rounded x*log2(e). A wrong coefficient or rounding
    step is off by >1e-4 and fails this."""
    L = O.lib()
    for lo, hi, bound in ((-1, 1, 5e-6), (-10, 0, 5e-6), (-87, 87, 1e-5)):
        xs = np.linspace(lo, hi, 20001).astype(np.float32)
        got = np.array([L.ndo_expf(float(x)) for x in xs], np.float64)
        rel = np.abs(got / np.exp(xs.astype(np.float64)) - 1)
        assert rel.max() < bound, (lo, hi, rel.max())
    assert L.ndo_expf(100.0) == np.float32(3.4028235e38) and L.ndo_expf(-100.0) == 0.0


def test_sigmoid_pair_matches_scalar_and_reference():
    R, L = O.ref(), O.lib()
    rng = np.random.default_rng(6)
    y0, y1 = C.c_float(), C.c_float()
    xs = rng.normal(0, 6, 4000).astype(np.float32)
    for i in range(0, xs.size, 2):
        R.ref_sigmoid_pair(float(xs[i]), float(xs[i + 1]), C.byref(y0), C.byref(y1))
        assert np.float32(y0.value) == np.float32(L.ndo_sigmoid(float(xs[i])))
        assert np.float32(y1.value) == np.float32(L.ndo_sigmoid(float(xs[i + 1])))


def test_kv_store_division_form_equals_reference_markstein():
    """The oracle divides; the reference uses a residual (Markstein) form it
    documents as equal to the divide. Check on random rows and on quotients
    sitting exactly on .5 ties and within an ulp of them."""
    R, L = O.ref(), O.lib()
    rng = np.random.default_rng(7)
    for trial in range(3000):
        n = 64
        if trial % 3 == 0:
            x = rng.normal(0, 10 ** rng.uniform(-6, 6), n).astype(np.float32)
        elif trial % 3 == 1:
            sc = np.float32(rng.uniform(1e-3, 10))
            t = (rng.integers(-254, 255, n) / 2.0).astype(np.float32)
            x = (t * sc).astype(np.float32)
            x = np.nextafter(x, x + rng.choice([-1, 0, 1], n).astype(np.float32)).astype(np.float32)
        else:
            x = rng.standard_normal(n).astype(np.float32)
            x[rng.integers(0, n)] = 0.0
        scale = np.float32(np.abs(x).max()) / np.float32(127.0)
        if scale == 0:
            scale = np.float32(1.0)
        a = np.zeros(n, np.int8)
        b = np.zeros(n, np.int8)
        L.ndo_kv_store_int8(a, np.ascontiguousarray(x), n, float(scale))
        R.ref_kv_store_int8(b, np.ascontiguousarray(x), n, float(scale))
        assert np.array_equal(a, b), trial


def _run_pair(geom, kv_steps, events, seed):
    rng = np.random.default_rng(seed)
    L, nh, nkv, qk, vd, W = geom
    o, r = O.OracleSession(*geom), O.RefSession(*geom)
    saved_o, saved_r = {}, {}
    for ev in events(kv_steps):
        if ev[0] == "tok":
            for li in range(L):
                q = rng.standard_normal(nh * qk).astype(np.float32) * np.float32(ev[2])
                k = rng.standard_normal(nkv * qk).astype(np.float32) * np.float32(ev[2])
                v = rng.standard_normal(nkv * vd).astype(np.float32)
                g = rng.standard_normal(nh * vd).astype(np.float32) if ev[1] else None
                a = o.attention(li, q, k, v, g)
                b = r.attention(li, q, k, v, g)
                assert np.array_equal(bits(a), bits(b))
            o.step_end()
            r.step_end()
        elif ev[0] == "snap":
            assert o.snapshot() == r.snapshot() == 0
        elif ev[0] == "sink":
            o.set_sink(ev[1])
            r.set_sink(ev[1])
        elif ev[0] == "save":
            saved_o[ev[1]], saved_r[ev[1]] = o.prefix_save(), r.prefix_save()
            assert bool(saved_o[ev[1]]) == bool(saved_r[ev[1]])
        elif ev[0] == "restore":
            assert o.prefix_restore(saved_o[ev[1]]) == r.prefix_restore(saved_r[ev[1]])
        elif ev[0] == "rewind":
            o.rewind()
            r.rewind()
        elif ev[0] == "reset":
            o.reset()
            r.reset()
        assert (o.pos, o.n_sink) == (r.pos, r.n_sink)
    for a, b in zip(o.cache(), r.cache()):
        assert np.array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8))


# MHA 8x64, the archive's 12/2 qk48, GQA 2/3/5/7/8, and head dims the engine
# allows besides (multiples of 4 up to ND_KV_HD_CAP 64: qk 32, qk 36 and 20,
# whose last 4 columns qk_dot8 sums one term at a time, v 20 and 32)
@pytest.mark.parametrize("geom", [(1, 8, 8, 64, 64, 300), (2, 12, 2, 48, 64, 384), (1, 6, 3, 48, 64, 90),
                                  (1, 16, 2, 64, 64, 200), (1, 3, 1, 64, 64, 64), (1, 10, 2, 32, 32, 150),
                                  (1, 14, 2, 36, 20, 120), (1, 4, 2, 20, 64, 100), (1, 5, 1, 64, 16, 80)])
def test_sessions_bit_exact(geom):
    def ev(n):
        out = [("tok", True, 1.0)] * 40 + [("snap",)] + [("tok", i % 2 == 0, 1.0 + (i % 5)) for i in range(n)]
        return out
    _run_pair(geom, 400, ev, seed=geom[1] * 7 + geom[5])


def test_prefix_switching_bit_exact():
    """nd_ptest's flow (host/nd_ptest.c:25-41) plus rewinds and long outliers."""
    def ev(_):
        return ([("reset",), ("tok", True, 1.0), ("tok", True, 1.0), ("snap",), ("save", 0), ("tok", True, 1.0),
                 ("reset",), ("tok", True, 1.0)] + [("tok", True, 3.0)] * 30 + [("snap",), ("save", 1)] +
                [("tok", True, 1.0)] * 5 + [("restore", 0), ("tok", True, 1.0), ("rewind",), ("tok", False, 8.0),
                                            ("restore", 1)] + [("tok", True, 2.0)] * 400 + [("rewind",), ("tok", True, 1.0)])
    _run_pair((1, 12, 2, 48, 64, 384), 0, ev, seed=99)


def test_prefill_timer_on_the_row_seam_bit_exact():
    """The CPU-baseline driver of the reference (ref_prefill_rounds: a prompt
    fed one token at a time through every layer, the heads dispatched through
    nd_parallel_rows) gives the same rows serially and on a 4-thread splitter
    installed in the engine's seam (disjoint head ranges, the contract of
    engine/include/nd_quant.h:213-230), and both equal the oracle's replay of
    the same tokens."""
    L, nh, S = 2, 8, 40
    rng = np.random.default_rng(8)
    q = rng.standard_normal((S, nh * 64)).astype(np.float32)
    k = rng.standard_normal((S, nh * 64)).astype(np.float32)
    v = rng.standard_normal((S, nh * 64)).astype(np.float32)
    outs = []
    for threads in (1, 4):
        r = O.RefSession(L, nh, nh, 64, 64, 64)
        out = np.zeros((S, nh * 64), np.float32)
        if threads > 1:
            assert O.ref().ref_pool_start(threads) == 0
        try:
            t = O.ref().ref_prefill_rounds(r.m, S, q.ctypes.data, k.ctypes.data, v.ctypes.data, out.ctypes.data)
        finally:
            if threads > 1:
                O.ref().ref_pool_stop()
        assert t > 0 and r.pos == S
        outs.append(out)
        r.close()
    assert np.array_equal(bits(outs[0]), bits(outs[1]))
    o = O.OracleSession(L, nh, nh, 64, 64, 64)
    for t in range(S):
        for li in range(L):
            got = o.attention(li, q[t], k[t], v[t], None)
        o.step_end()
        assert np.array_equal(bits(got), bits(outs[0][t])), t
