"""The oracle's CQ projection kernels (engine/src/nd_quant.c) pinned
bit-exact against the reference's own nd_fwht, nd_cq_prepare,
nd_cq_gemv_prepared, nd_cq_lut_build and nd_cq_gemv_lut2 (live, where the
harness is built) and against what the mathematics fixes: H.H = n.I, a
delta's transform, orthonormality, and the float64 matvec with the
explicitly dequantised weights (cb[idx] * norm) @ H."""
import numpy as np
import pytest
from scipy.linalg import hadamard

import ndoracle as O
from detgen import Stream, det_normal, make_cq_tensor as make_tensor


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


SHAPES = [(24, 256, 128, 2), (17, 200, 64, 2), (9, 300, 128, 4), (13, 96, 32, 3),
          (31, 512, 128, 3), (8, 130, 64, 4)]


@pytest.mark.skipif(not O.have_ref(), reason="reference harness not built")
@pytest.mark.parametrize("shape", SHAPES)
def test_cq_matches_reference(shape):
    out, inp, group, b = shape
    R = O.ref()
    t = make_tensor(sum(shape), out, inp, group, b, special_norms=True)
    st = Stream(out * 7 + inp)
    for trial in range(3):
        x = st.take(inp) * np.float32(4.0 if trial == 2 else 1.0)
        xh = O.cq_prepare(t, x)
        xr = np.zeros(t.in_pad, np.float32)
        R.ref_cq_prepare(inp, group, x.ctypes.data, xr.ctypes.data)
        assert np.array_equal(bits(xh), bits(xr))
        y = O.cq_gemv(t, xh)
        yr = np.zeros(out, np.float32)
        R.ref_cq_gemv(out, inp, group, b, t.blob.ctypes.data, t.codebook.ctypes.data, xh.ctypes.data,
                      yr.ctypes.data)
        assert np.array_equal(bits(y), bits(yr)), trial
        if b == 2:
            y2 = O.cq_gemv_lut2(t, xh)
            lut = np.zeros(t.in_pad // 2 * 16, np.float32)
            y2r = np.zeros(out, np.float32)
            R.ref_cq_lut2(out, inp, group, t.blob.ctypes.data, t.codebook.ctypes.data, xh.ctypes.data,
                          lut.ctypes.data, y2r.ctypes.data)
            assert np.array_equal(bits(y2), bits(y2r)), trial


@pytest.mark.skipif(not O.have_ref(), reason="reference harness not built")
def test_fwht_matches_reference():
    R = O.ref()
    for n in (1, 2, 4, 8, 64, 128, 256):
        x = det_normal(n, n)
        a, b = x.copy(), x.copy()
        O.lib().ndo_fwht(a.ctypes.data, n)
        R.ref_fwht(b.ctypes.data, n)
        assert np.array_equal(bits(a), bits(b)), n


def test_fwht_closed_forms():
    for n in (2, 8, 128):
        # integers: exact; applying twice multiplies by n
        x = (np.arange(n) % 7 - 3).astype(np.float32)
        y = x.copy()
        O.lib().ndo_fwht(y.ctypes.data, n)
        assert np.array_equal(y, (hadamard(n) @ x.astype(np.int64)).astype(np.float32))
        O.lib().ndo_fwht(y.ctypes.data, n)
        assert np.array_equal(y, x * n)
        d = np.zeros(n, np.float32)
        d[0] = 1.0
        O.lib().ndo_fwht(d.ctypes.data, n)
        assert np.all(d == 1.0)


def test_prepare_is_orthonormal_per_group():
    t = make_tensor(3, 4, 300, 128, 2)
    x = det_normal(9, 300)
    xh = O.cq_prepare(t, x).astype(np.float64)
    xp = np.zeros(t.in_pad)
    xp[:300] = x
    H = hadamard(128) / np.sqrt(128.0)
    want = np.concatenate([H @ xp[g * 128:(g + 1) * 128] for g in range(t.in_pad // 128)])
    assert np.allclose(xh, want, rtol=1e-6, atol=1e-6)
    assert np.isclose(np.linalg.norm(xh), np.linalg.norm(x), rtol=1e-6)


@pytest.mark.parametrize("shape", SHAPES)
def test_gemv_against_float64_dequantised(shape):
    """y = W x with W rebuilt explicitly: per group (cb[idx] * norm) @ H."""
    out, inp, group, b = shape
    t = make_tensor(sum(shape) + 5, out, inp, group, b)
    x = det_normal(out + 3, inp)
    H = hadamard(group) / np.sqrt(float(group))
    cb = t.cb().astype(np.float64)
    codes, nrm = t.codes(), t.norms().astype(np.float64)
    W = np.zeros((out, t.in_pad))
    for g in range(t.in_pad // group):
        sl = slice(g * group, (g + 1) * group)
        W[:, sl] = (cb[codes[:, sl]] * nrm[:, g:g + 1]) @ H
    want = W[:, :inp] @ x.astype(np.float64)
    xh = O.cq_prepare(t, x)
    y = O.cq_gemv(t, xh)
    scale = np.abs(W[:, :inp]) @ np.abs(x.astype(np.float64)) + 1e-30
    assert np.all(np.abs(y - want) <= 1e-5 * scale + 1e-7)
    if b == 2:
        y2 = O.cq_gemv_lut2(t, xh)
        assert np.all(np.abs(y2 - want) <= 1e-5 * scale + 1e-7)


def test_codes_decode_lsb_first():
    """The bitstream reader: index k of a row occupies bits [k*bits, (k+1)*bits)."""
    t = make_tensor(1, 2, 64, 32, 3)
    row = t.blob[: t.rowbytes]
    bitstream = int.from_bytes(row.tobytes(), "little")
    want = [(bitstream >> (3 * k)) & 7 for k in range(64)]
    assert list(t.codes()[0]) == want


def test_golden_cq_vectors():
    """The committed reference outputs (tests/golden/golden.npz, written by
    the reference's own nd_cq_gemv_prepared / nd_cq_gemv_lut2)."""
    import os
    G = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz"))
    for i, shape in enumerate(G["cq_shapes"]):
        out, inp, group, b = (int(v) for v in shape)
        blob = G["cq_blob_%d" % i]
        t = O.CQTensor(out, inp, group, b, blob, G["cq_cb_%d" % i])
        xh = O.cq_prepare(t, G["cq_x_%d" % i])
        assert np.array_equal(bits(xh), bits(G["cq_xh_%d" % i]))
        assert np.array_equal(bits(O.cq_gemv(t, xh)), bits(G["cq_y_%d" % i]))
        if b == 2:
            assert np.array_equal(bits(O.cq_gemv_lut2(t, xh)), bits(G["cq_y2_%d" % i]))
