"""GPU parity of the CQ projections (nda_cq_prepare / nda_cq_gemm) against
the oracle (itself bit-exact to the reference's nd_cq_prepare and
nd_cq_gemv_prepared / nd_cq_gemv_lut2): the prepared rows bit-exact, the
matvec outputs within fp32 reassociation of the engine's, bounded as
|y - y_ref| <= 1e-5 * sum|w x| + 1e-6 per output; and the reference's own
golden outputs."""
import os
import sys

import numpy as np
import pytest

import ndoracle as O
from detgen import det_normal, make_cq_tensor

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def nda():
    import ndattn
    return ndattn


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def abs_scale(t, x):
    """sum_k |w[o][k]| |x[k]| per output, float64: the reassociation bound."""
    from scipy.linalg import hadamard
    H = hadamard(t.group) / np.sqrt(float(t.group))
    cb = t.cb().astype(np.float64)
    codes, nrm = t.codes(), t.norms().astype(np.float64)
    W = np.zeros((t.out, t.in_pad))
    for g in range(t.in_pad // t.group):
        sl = slice(g * t.group, (g + 1) * t.group)
        W[:, sl] = (cb[codes[:, sl]] * nrm[:, g:g + 1]) @ H
    return np.abs(W[:, :t.inp]) @ np.abs(x.astype(np.float64)).T


def run(t, x):
    N = nda()
    rows = x.shape[0]
    q = N.CQ(t.out, t.inp, t.group, t.bits, t.blob, t.cb())
    dx = N.DevBuf.from_array(x)
    dxh = N.DevBuf(max(1, rows) * q.in_pad * 4)
    dy = N.DevBuf(max(1, rows) * t.out * 4)
    q.prepare(rows, dx, dxh)
    q.gemm(rows, dxh, dy)
    N.device_sync()
    xh = dxh.to_array(np.float32, (rows, q.in_pad))
    y = dy.to_array(np.float32, (rows, t.out))
    q.close()
    return xh, y


@pytest.mark.parametrize("shape,rows", [
    ((64, 512, 128, 2), 64),      # one full tile
    ((576, 768, 128, 2), 70),     # the archive's q_proj shape (12 x 48 from d_model 768), ragged rows
    ((100, 200, 64, 4), 33),      # padding, partial output tile
    ((13, 96, 32, 3), 5),         # 3-bit straddling fields, group below the tile width
    ((130, 1024, 256, 2), 129),
    ((768, 576, 128, 2), 3),      # out_proj shape, few rows
])
def test_cq_prepare_and_gemm(shape, rows):
    out, inp, group, b = shape
    say("cq", shape, rows)
    t = make_cq_tensor(out + inp + group + b, out, inp, group, b, special_norms=True)
    x = np.stack([det_normal(1000 + r, inp) for r in range(rows)]) * np.float32(3.0)
    xh, y = run(t, x)
    sc = abs_scale(t, x)
    worst = 0.0
    for r in range(rows):
        want_xh = O.cq_prepare(t, x[r])
        assert np.array_equal(bits(xh[r]), bits(want_xh)), r
        want = O.cq_gemv_lut2(t, want_xh) if b == 2 else O.cq_gemv(t, want_xh)
        err = np.abs(y[r].astype(np.float64) - want)
        assert np.all(err <= 1e-5 * sc[:, r] + 1e-6), (r, float(err.max()))
        worst = max(worst, float(err.max()))
    say("cq worst", worst)


def test_cq_gemm_many_matches_single_launches():
    """q/k/v/gate of the archive's shapes in one launch equal four launches
    bit for bit (the same tiles, the same order of operations)."""
    N = nda()
    say("cq gemm many")
    shapes = [576, 96, 128, 768]
    rows, inp = 70, 768
    ts = [make_cq_tensor(700 + i, o, inp, 128, 2) for i, o in enumerate(shapes)]
    qs = [N.CQ(o, inp, 128, 2, t.blob, t.cb()) for o, t in zip(shapes, ts)]
    x = np.stack([det_normal(50 + r, inp) for r in range(rows)])
    dx = N.DevBuf.from_array(x)
    dxh = N.DevBuf(rows * qs[0].in_pad * 4)
    qs[0].prepare(rows, dx, dxh)
    one = [N.DevBuf(rows * o * 4) for o in shapes]
    many = [N.DevBuf(rows * o * 4) for o in shapes]
    for q, y in zip(qs, one):
        q.gemm(rows, dxh, y)
    N.cq_gemm_many(qs, rows, dxh, many)
    N.device_sync()
    for o, a, b in zip(shapes, one, many):
        assert np.array_equal(a.to_array(np.uint32, (rows, o)), b.to_array(np.uint32, (rows, o)))
    bad = N.CQ(64, 512, 128, 2, make_cq_tensor(9, 64, 512, 128, 2).blob, ts[0].cb())
    with pytest.raises(N.NdaError):
        N.cq_gemm_many([qs[0], bad], rows, dxh, many[:2])     # another reduction length
    for q in qs + [bad]:
        q.close()


def test_cq_golden_reference_outputs():
    """The reference's own outputs for the committed CQ vectors."""
    G = np.load(os.path.join(HERE, "golden", "golden.npz"))
    say("cq golden")
    for i, shape in enumerate(G["cq_shapes"]):
        out, inp, group, b = (int(v) for v in shape)
        t = O.CQTensor(out, inp, group, b, G["cq_blob_%d" % i], G["cq_cb_%d" % i])
        x = G["cq_x_%d" % i][None, :]
        xh, y = run(t, x)
        assert np.array_equal(bits(xh[0]), bits(G["cq_xh_%d" % i]))
        ref = G["cq_y2_%d" % i] if b == 2 else G["cq_y_%d" % i]
        sc = abs_scale(t, x)[:, 0]
        assert np.all(np.abs(y[0].astype(np.float64) - ref) <= 1e-5 * sc + 1e-6)


@pytest.mark.parametrize("shapes,inp,group,rows", [
    ([576, 96, 128, 768], 768, 128, 5),       # the archive's q/k/v/gate from d_model 768
    ([768], 576, 128, 3),                     # its out_proj
    ([360, 72, 40, 200], 256, 128, 64),       # 10 q / 2 kv heads, qk 36, v 20; 64 rows
    ([256], 200, 128, 2),                     # out_proj over 200 inputs (padded to 256)
    ([300, 17], 2048, 256, 4),                # the largest table (in_pad 2048)
    ([33], 100, 16, 9),                       # group 16, padded
    ([70, 70], 96, 32, 1),
])
def test_cq_lut2_bit_exact(shapes, inp, group, rows):
    """nda_cq_gemv_lut2: every output bit-identical to the engine's
    nd_cq_gemv_lut2 (the oracle's restatement, pinned bit-exact to the
    reference), special norms (subnormal, negative, zero) included."""
    N = nda()
    say("cq lut2", shapes, inp, group, rows)
    ts = [make_cq_tensor(900 + 7 * i + inp, o, inp, group, 2, special_norms=True) for i, o in enumerate(shapes)]
    qs = [N.CQ(o, inp, group, 2, t.blob, t.cb()) for o, t in zip(shapes, ts)]
    x = np.stack([det_normal(300 + r, inp) for r in range(rows)]) * np.float32(2.5)
    dx = N.DevBuf.from_array(x)
    dxh = N.DevBuf(rows * qs[0].in_pad * 4)
    qs[0].prepare(rows, dx, dxh)
    ys = [N.DevBuf(rows * o * 4) for o in shapes]
    N.cq_gemv_lut2(qs, rows, dxh, ys)
    N.device_sync()
    xh = dxh.to_array(np.float32, (rows, qs[0].in_pad))
    for t, o, y in zip(ts, shapes, ys):
        got = y.to_array(np.float32, (rows, o))
        for r in range(rows):
            want = O.cq_gemv_lut2(t, xh[r])
            assert np.array_equal(bits(got[r]), bits(want)), (o, r)
    for q in qs:
        q.close()


def test_cq_lut2_golden_and_refusals():
    """The reference's own nd_cq_gemv_lut2 outputs for the committed 2-bit
    vectors, bit for bit; widths and table sizes the kernel does not take
    are refused with NDA_ERR_UNSUPPORTED."""
    N = nda()
    say("cq lut2 golden")
    G = np.load(os.path.join(HERE, "golden", "golden.npz"))
    seen = 0
    for i, shape in enumerate(G["cq_shapes"]):
        out, inp, group, b = (int(v) for v in shape)
        if b != 2:
            continue
        q = N.CQ(out, inp, group, b, G["cq_blob_%d" % i], G["cq_cb_%d" % i])
        if q.in_pad > 2048:
            q.close()
            continue
        dxh = N.DevBuf.from_array(G["cq_xh_%d" % i][None, :].astype(np.float32))
        dy = N.DevBuf(out * 4)
        N.cq_gemv_lut2([q], 1, dxh, [dy])
        N.device_sync()
        assert np.array_equal(bits(dy.to_array(np.float32, (1, out))[0]), bits(G["cq_y2_%d" % i])), i
        seen += 1
        q.close()
    assert seen > 0
    t3 = make_cq_tensor(5, 16, 64, 32, 3)
    q3 = N.CQ(16, 64, 32, 3, t3.blob, t3.cb())
    t4 = make_cq_tensor(6, 8, 4096, 128, 2)
    q4 = N.CQ(8, 4096, 128, 2, t4.blob, t4.cb())
    buf = N.DevBuf(4096 * 4 * 2)
    for q in (q3, q4):
        with pytest.raises(N.NdaError) as e:
            N.cq_gemv_lut2([q], 1, buf, [buf])
        assert e.value.code == -6
        q.close()


def test_cq_error_paths():
    N = nda()
    say("cq errors")
    t = make_cq_tensor(5, 8, 64, 32, 2)
    with pytest.raises(N.NdaError) as e:
        N.CQ(8, 64, 48, 2, t.blob, t.cb())           # group not a power of two
    assert e.value.code == -6
    with pytest.raises(N.NdaError) as e:
        N.CQ(8, 64, 32, 5, t.blob, t.cb())           # bits
    assert e.value.code == -6
    q = N.CQ(8, 64, 32, 2, t.blob, t.cb())
    buf = N.DevBuf(4096)
    with pytest.raises(N.NdaError) as e:
        q.prepare(1, buf.value + 4, buf)             # misaligned
    assert e.value.code == -1
    q.close()


# ------------------------------------------------ split-precision path

def run_split(t, x):
    N = nda()
    rows = x.shape[0]
    q = N.CQ(t.out, t.inp, t.group, t.bits, t.blob, t.cb())
    dx = N.DevBuf.from_array(x)
    dxs = N.DevBuf(max(16, q.split_bytes(rows)))
    dy = N.DevBuf(max(1, rows) * t.out * 4)
    q.prepare_split(rows, dx, dxs)
    q.gemm_split(rows, dxs, dy)
    N.device_sync()
    P = q.in_pad
    rp = (rows + 31) // 32 * 32
    raw = dxs.to_array(np.uint8, (q.split_bytes(rows),))
    blk = raw[:rp * P * 4].view(np.float16)
    # operand order: [row/32][col/16][plane][lane = row%32 + 32 (col%16/8)][col%8]
    r, c = np.meshgrid(np.arange(rows), np.arange(P), indexing="ij")
    lane = r % 32 + 32 * ((c % 16) // 8)
    base = ((r // 32) * (P // 16) + c // 16) * 2
    hi = blk[((base + 0) * 64 + lane) * 8 + c % 8]
    lo = blk[((base + 1) * 64 + lane) * 8 + c % 8]
    e = raw[rp * P * 4:].view(np.int32)
    y = dy.to_array(np.float32, (rows, t.out))
    q.close()
    return hi, lo, e, y


@pytest.mark.parametrize("shape,rows,scale", [
    ((576, 768, 128, 2), 70, 3.0),     # q_proj of the archive, ragged rows
    ((768, 768, 128, 2), 300, 1.0),    # gate / out_proj, several row tiles
    ((100, 200, 64, 2), 33, 1e-4),     # padding, partial tiles, small activations
    ((130, 1024, 256, 2), 129, 5e3),   # large activations
    ((40, 96, 32, 2), 5, 1.0),         # the smallest group the path takes (LDS prepare)
    ((64, 1024, 1024, 2), 37, 1.0),    # register prepare, stages across column blocks
    ((72, 1536, 512, 2), 45, 1.0),     # the widest row of the register prepare
    ((48, 2300, 128, 2), 9, 1.0),      # past it: the LDS prepare
])
def test_cq_split_prepare_and_gemm(shape, rows, scale):
    """The split form holds the engine's prepared row times 2^e exactly to
    2^-22, the row's largest |value| in [2^14, 2^15); the GEMM is within the
    fp32 reassociation bound of the engine's matvec."""
    out, inp, group, b = shape
    say("cq split", shape, rows, scale)
    t = make_cq_tensor(out + inp + group + 7, out, inp, group, b, special_norms=True)
    x = np.stack([det_normal(2000 + r, inp) for r in range(rows)]) * np.float32(scale)
    x[rows // 2] = 0.0                                   # a zero row: exponent 0, zero output
    hi, lo, e, y = run_split(t, x)
    sc = abs_scale(t, x)
    worst = 0.0
    for r in range(rows):
        want_xh = O.cq_prepare(t, x[r]).astype(np.float64)
        v = want_xh * 2.0 ** int(e[r])
        pair = hi[r].astype(np.float64) + lo[r].astype(np.float64)
        assert np.all(np.abs(pair - v) <= 2.0 ** -22 * np.abs(v).max() + 1e-30), r
        # exactly: hi the fp16 rounding of the scaled engine value, lo that of the rest
        v32 = v.astype(np.float32)
        assert np.array_equal(v32.astype(np.float64), v), r       # the scaling is exact
        want_hi = v32.astype(np.float16)
        want_lo = (v32 - want_hi.astype(np.float32)).astype(np.float16)
        assert np.array_equal(hi[r].view(np.uint16), want_hi.view(np.uint16)), r
        assert np.array_equal(lo[r].view(np.uint16), want_lo.view(np.uint16)), r
        m = np.abs(v).max()
        assert (m == 0 and e[r] == 0) or 2 ** 14 <= m < 2 ** 15, (r, m, e[r])
        want = O.cq_gemv_lut2(t, O.cq_prepare(t, x[r]))
        err = np.abs(y[r].astype(np.float64) - want)
        assert np.all(err <= 1e-5 * sc[:, r] + 1e-6 * max(1.0, scale)), (r, float(err.max()))
        worst = max(worst, float((err / (sc[:, r] + 1e-30)).max()))
    assert np.all(y[rows // 2] == 0.0)
    say("cq split worst relative to sum|w x|", worst)


def test_cq_split_many_matches_single_and_rejects():
    """q/k/v/gate in one launch equal four launches bit for bit; widths and
    groups the path does not take are refused."""
    N = nda()
    say("cq split many")
    shapes = [576, 96, 128, 768]
    rows, inp = 150, 768
    ts = [make_cq_tensor(800 + i, o, inp, 128, 2) for i, o in enumerate(shapes)]
    qs = [N.CQ(o, inp, 128, 2, t.blob, t.cb()) for o, t in zip(shapes, ts)]
    x = np.stack([det_normal(60 + r, inp) for r in range(rows)])
    dx = N.DevBuf.from_array(x)
    dxs = N.DevBuf(qs[0].split_bytes(rows))
    qs[0].prepare_split(rows, dx, dxs)
    one = [N.DevBuf(rows * o * 4) for o in shapes]
    many = [N.DevBuf(rows * o * 4) for o in shapes]
    for q, y in zip(qs, one):
        q.gemm_split(rows, dxs, y)
    N.cq_gemm_split_many(qs, rows, dxs, many)
    N.device_sync()
    for o, a, b in zip(shapes, one, many):
        assert np.array_equal(a.to_array(np.uint32, (rows, o)), b.to_array(np.uint32, (rows, o)))
    t4 = make_cq_tensor(9, 64, 512, 128, 4)
    q4 = N.CQ(64, 512, 128, 4, t4.blob, t4.cb())
    buf = N.DevBuf(q4.split_bytes(4) + 64)
    with pytest.raises(N.NdaError) as e:
        q4.gemm_split(4, buf, buf)                   # 4-bit: not this path
    assert e.value.code == -6
    t16 = make_cq_tensor(10, 8, 64, 16, 2)
    q16 = N.CQ(8, 64, 16, 2, t16.blob, t16.cb())
    with pytest.raises(N.NdaError) as e:
        q16.prepare_split(1, buf, buf)               # group 16
    assert e.value.code == -6
    for q in qs + [q4, q16]:
        q.close()


def test_cq_split_persistent_walks_and_column_scales():
    """q/k/v/gate over 6181 rows: 49 row tiles x 13 output tiles = 637 items
    for the 512 persistent work-groups, so a work-group walks two items
    (across tensors and row tiles, the next item's loads issued during the
    last step of the one before). The launch equals the four single-tensor
    launches (under 512 items each: one item per work-group) bit for bit,
    and sampled rows are within the reassociation bound of the oracle.
    Columns 5-7 of q probe the per-column scaling: all norms zero (exponent
    0, output exactly 0), the fp16 maximum beside subnormal norms, and all
    norms subnormal."""
    N = nda()
    say("cq split persistent walks")
    shapes = [576, 96, 128, 768]
    rows, inp, group = 6181, 768, 128
    ts = [make_cq_tensor(900 + i, o, inp, group, 2, special_norms=True) for i, o in enumerate(shapes)]
    t = ts[0]
    ng = inp // group
    pb = t.out * inp // 4
    blob = np.array(t.blob, copy=True)
    nrm = blob[pb:].view(np.float16).reshape(t.out, ng)
    nrm[5, :] = 0.0
    nrm[6, :] = np.float16(6e-8)                     # the smallest fp16 subnormal
    nrm[6, 2] = np.float16(65504.0)
    nrm[7, :] = np.float16(-6e-8)
    ts[0] = O.CQTensor(t.out, inp, group, 2, blob, t.cb())
    qs = [N.CQ(o, inp, group, 2, tt.blob, tt.cb()) for o, tt in zip(shapes, ts)]
    x = np.stack([det_normal(7000 + r, inp) for r in range(rows)])
    dx = N.DevBuf.from_array(x)
    dxs = N.DevBuf(qs[0].split_bytes(rows))
    qs[0].prepare_split(rows, dx, dxs)
    one = [N.DevBuf(rows * o * 4) for o in shapes]
    many = [N.DevBuf(rows * o * 4) for o in shapes]
    for q, y in zip(qs, one):
        q.gemm_split(rows, dxs, y)
    N.cq_gemm_split_many(qs, rows, dxs, many)
    N.device_sync()
    sample = sorted(set(list(range(0, rows, 193)) + [rows - 37, rows - 2, rows - 1]))
    for i, (o, a, b) in enumerate(zip(shapes, one, many)):
        ya = a.to_array(np.uint32, (rows, o))
        assert np.array_equal(ya, b.to_array(np.uint32, (rows, o))), shapes[i]
        y = ya.view(np.float32)
        if i == 0:
            assert np.all(y[:, 5] == 0.0)
        sc = abs_scale(ts[i], x[sample])
        for j, r in enumerate(sample):
            want = O.cq_gemv_lut2(ts[i], O.cq_prepare(ts[i], x[r]))
            err = np.abs(y[r].astype(np.float64) - want)
            assert np.all(err <= 1e-5 * sc[:, j] + 1e-6), (shapes[i], r, float(err.max()))
    for q in qs:
        q.close()
