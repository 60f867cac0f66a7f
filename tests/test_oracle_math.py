"""The oracle against what the mathematics fixes: float64 textbook attention,
closed-form special cases, invariances. Covers the fp16 mode too, for which
the reference has no code path."""
import numpy as np
import pytest

import ndoracle as O


def make_view(rng, nh, nkv, qk, vd, L, dtype, scale_k=1.0):
    kf = (rng.standard_normal((L, nkv, qk)) * scale_k).astype(np.float32)
    vf = rng.standard_normal((L, nkv, vd)).astype(np.float32)
    if dtype == O.KV_F16:
        k, v, ks, vs = O.f32_to_f16_bits(kf), O.f32_to_f16_bits(vf), None, None
    else:
        k = np.zeros((L, nkv, qk), np.int8)
        v = np.zeros((L, nkv, vd), np.int8)
        ks = np.zeros((L, nkv), np.float32)
        vs = np.zeros((L, nkv), np.float32)
        for p in range(L):
            for g in range(nkv):
                ks[p, g] = O.lib().ndo_kv_quant_row(np.ascontiguousarray(kf[p, g]), qk, k[p, g])
                vs[p, g] = O.lib().ndo_kv_quant_row(np.ascontiguousarray(vf[p, g]), vd, v[p, g])
    return k, v, ks, vs


@pytest.mark.parametrize("dtype", [O.KV_INT8, O.KV_F16])
@pytest.mark.parametrize("geom", [(8, 8, 64, 64), (12, 2, 48, 64), (4, 1, 64, 64)])
def test_attend_matches_float64_textbook(dtype, geom):
    rng = np.random.default_rng(1)
    nh, nkv, qk, vd = geom
    L = 229
    k, v, ks, vs = make_view(rng, nh, nkv, qk, vd, L, dtype, scale_k=2.0)
    kv = O.kv_view(k, v, ks, vs, nh, L, 0, L - 1, dtype)
    q = rng.standard_normal(nh * qk).astype(np.float32)
    g = rng.standard_normal(nh * vd).astype(np.float32)
    got = O.attend_view(kv, q, g)
    want = O.attend_f64(kv, np.arange(L), q, g)
    assert np.abs(got - want).max() < 2e-6


def test_special_cases_closed_form():
    rng = np.random.default_rng(2)
    nh, nkv, qk, vd = 4, 2, 64, 64
    # L = 1: out = v * sigmoid(g), exactly the dequantised row
    k, v, ks, vs = make_view(rng, nh, nkv, qk, vd, 1, O.KV_F16)
    kv = O.kv_view(k, v, ks, vs, nh, 1, 0, 0, O.KV_F16)
    q = rng.standard_normal(nh * qk).astype(np.float32)
    got = O.attend_view(kv, q, None).reshape(nh, vd)
    vrow = v.astype(np.uint16).view(np.float16).astype(np.float32)[0]
    for h in range(nh):
        assert np.array_equal(got[h], vrow[h // 2])
    # identical keys: mean of V
    L = 37
    k, v, ks, vs = make_view(rng, nh, nkv, qk, vd, L, O.KV_F16)
    k[:] = k[0]
    kv = O.kv_view(k, v, ks, vs, nh, L, 0, L - 1, O.KV_F16)
    got = O.attend_view(kv, q, None).reshape(nh, vd)
    vv = v.view(np.float16).astype(np.float64)
    for h in range(nh):
        assert np.allclose(got[h], vv[:, h // 2].mean(0), atol=1e-6)
    # one dominant key: that V row
    k, v, ks, vs = make_view(rng, nh, nkv, qk, vd, L, O.KV_F16)
    qd = np.ones(nh * qk, np.float32)
    k[:] = O.f32_to_f16_bits(np.zeros((L, nkv, qk), np.float32))
    k[11] = O.f32_to_f16_bits(np.full((nkv, qk), 20.0, np.float32))
    kv = O.kv_view(k, v, ks, vs, nh, L, 0, L - 1, O.KV_F16)
    got = O.attend_view(kv, qd, None).reshape(nh, vd)
    vv = v.view(np.float16).astype(np.float32)
    for h in range(nh):
        assert np.allclose(got[h], vv[11, h // 2], atol=1e-6)


def test_shift_invariance_and_gate_zero():
    """Adding a constant to every score changes nothing (a key component
    along q does that); sigmoid(0) = 0.5 halves the output exactly."""
    rng = np.random.default_rng(3)
    nh = nkv = 2
    qk = vd = 64
    L = 50
    k, v, ks, vs = make_view(rng, nh, nkv, qk, vd, L, O.KV_F16)
    kv = O.kv_view(k, v, ks, vs, nh, L, 0, L - 1, O.KV_F16)
    q = rng.standard_normal(nh * qk).astype(np.float32)
    a = O.attend_view(kv, q, None)
    b = O.attend_view(kv, q, np.zeros(nh * vd, np.float32))
    assert np.array_equal(b, a * np.float32(0.5))
    want = O.attend_f64(kv, np.arange(L), q, None)
    kf = k.view(np.float16).astype(np.float32)
    qh = q.reshape(nh, qk)
    for h in range(nh):
        kf[:, h] += qh[h] / np.dot(qh[h], qh[h]) * 3.0
    k2 = O.f32_to_f16_bits(kf)
    kv2 = O.kv_view(k2, v, ks, vs, nh, L, 0, L - 1, O.KV_F16)
    want2 = O.attend_f64(kv2, np.arange(L), q, None)
    # f16 rounding of the shifted keys moves scores by ~1e-3 at most
    assert np.abs(want2 - want).max() < 5e-3


def test_sink_ring_equals_explicit_positions():
    """Sinks + wrapped ring visit exactly the sink positions and the last
    window-n_sink positions (nd_model.c:2451-2477), in that order."""
    rng = np.random.default_rng(4)
    nh, nkv, qk, vd, W = 4, 2, 48, 64, 80
    S = O.OracleSession(1, nh, nkv, qk, vd, W, O.KV_INT8)
    hist_k, hist_v = [], []
    for p in range(300):
        if p == 10:
            S.set_sink(10)
        k = rng.standard_normal(nkv * qk).astype(np.float32)
        v = rng.standard_normal(nkv * vd).astype(np.float32)
        S.kv_store(0, k, v)
        hist_k.append(k)
        hist_v.append(v)
        S.step_end()
    S.s.pos = 299
    kk, vv, kss, vss = S.cache()
    q = rng.standard_normal(nh * qk).astype(np.float32)
    got = S.attend(0, q, None)
    n_sink = S.n_sink
    assert n_sink == 10
    positions = list(range(10)) + list(range(300 - (W - 10), 300))
    slots = [O.lib().ndo_kv_slot(W, 10, p) for p in positions]
    kv = O.kv_view(kk[0], vv[0], kss[0], vss[0], nh, W, 10, 299, O.KV_INT8)
    want = O.attend_runs(kv, slots, [10, len(slots) - 10], q, None)
    assert np.array_equal(got, want)
    # and the dequantised rows are the ones stored for those positions
    for p, s in zip(positions, slots):
        for g in range(nkv):
            deq = kk[0, s, g].astype(np.float32) * kss[0, s, g]
            assert np.abs(deq - hist_k[p][g * qk:(g + 1) * qk]).max() <= kss[0, s, g] * 0.5 + 1e-7


def test_f16_conversion_round_trip():
    rng = np.random.default_rng(8)
    x = np.concatenate([rng.standard_normal(5000) * 10, rng.standard_normal(1000) * 1e-6,
                        [65504, 65520, -65519, 6e-8, 3e-8, 0.0]]).astype(np.float32)
    mine = np.array([O.lib().ndo_f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(mine, O.f32_to_f16_bits(x))
    back = np.array([O.lib().ndo_f16_to_f32(int(h)) for h in mine], np.float32)
    assert np.array_equal(back, mine.view(np.float16).astype(np.float32))
