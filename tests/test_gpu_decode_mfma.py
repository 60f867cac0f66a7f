"""GPU parity of the MFMA decode of GQA groups: int8 K/V with 4 or more query
heads per kv-head, which nda_decode runs on decode_mfma_kernel (one wave per
row and pair of kv-heads, or per row and kv-head for odd kv-head counts; the
heads as MFMA columns). Each case stores the cache an
engine session at that position holds (the sinks and the ring's latest
positions, written through nda_kv_write), decodes once, and compares the
outputs with the oracle's attention over the same slots (ndo_attend, the
engine's attn_heads restated, engine/src/nd_model.c:2105-2359) and with the
VALU decode kernel on the same cache (NDA_FLAG_DECODE_VALU). Bar: max |delta|
<= 1e-3 against the oracle (fp32 accumulate); the two kernels differ only in
summation order. Every case lists at least 8 rows of 2 kv-heads (16 work
items), the smallest launch the MFMA route takes."""
import sys

import numpy as np
import pytest

import ndoracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3
KERNELS_TOL = 1e-4      # MFMA against VALU decode: reassociation only


def nda():
    import ndattn
    return ndattn


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


def _quant(rows):
    """int8 codes and scales of fp32 rows [n][d], as the engine stores them."""
    codes = np.zeros(rows.shape, np.int8)
    sc = np.zeros(rows.shape[0], np.float32)
    for i in range(rows.shape[0]):
        sc[i] = O.lib().ndo_kv_quant_row(np.ascontiguousarray(rows[i]), rows.shape[1], codes[i])
    return codes, sc


class Cache:
    """Slot arrays of one sequence [window][nkv][hd] in the engine's layout."""

    def __init__(self, rng, W, nkv, qk, vd):
        self.k = np.zeros((W, nkv, qk), np.int8)
        self.v = np.zeros((W, nkv, vd), np.int8)
        self.ks = np.zeros((W, nkv), np.float32)
        self.vs = np.zeros((W, nkv), np.float32)
        self.rng, self.nkv, self.qk, self.vd = rng, nkv, qk, vd

    def row(self, slot, outlier=False):
        """Fresh stored row at a slot; returns (k, v, ks, vs) for kv_write."""
        kf = self.rng.standard_normal((self.nkv, self.qk)).astype(np.float32)
        if outlier:
            kf *= np.float32(6.0)
        vf = self.rng.standard_normal((self.nkv, self.vd)).astype(np.float32)
        k, ks = _quant(kf)
        v, vs = _quant(vf)
        self.k[slot], self.v[slot], self.ks[slot], self.vs[slot] = k, v, ks, vs
        return k[None], v[None], ks[None], vs[None]


def _visible_positions(pos, n_sink, W):
    """Positions an engine session at `pos` still holds: sinks and the ring."""
    sinks = list(range(min(n_sink, pos + 1)))
    lo = max(n_sink, pos + 1 - (W - n_sink))
    return sinks + list(range(lo, pos + 1))


def _run(nh, nkv, qk, W, specs, seed, gated=True, order=None, prefix=0, outlier_p=0.0, page_size=16):
    """specs: (pos, n_sink) per sequence; with prefix > 0 every sequence is
    attached to a prefix of `prefix` sink positions built on an extra
    sequence, so its (pos, n_sink) is (pos, prefix). Returns the worst
    |delta| against the oracle for the MFMA and VALU kernels and between them."""
    N = nda()
    vd = 64
    rng = np.random.default_rng(seed)
    B = len(specs)
    ids = list(range(B)) if order is None else list(order)
    caches = [Cache(rng, W, nkv, qk, vd) for _ in range(B)]
    pre = Cache(rng, W, nkv, qk, vd)
    writes = []                                     # (seq, pos, rows) in order
    if prefix:
        for p in range(prefix):
            writes.append((B, p, pre.row(p)))
        for c in caches:
            c.k[:prefix], c.v[:prefix], c.ks[:prefix], c.vs[:prefix] = pre.k[:prefix], pre.v[:prefix], \
                pre.ks[:prefix], pre.vs[:prefix]
    for b, (pos, ns) in enumerate(specs):
        ns = prefix if prefix else ns
        for p in _visible_positions(pos, ns, W):
            if prefix and p < prefix:
                continue
            sl = O.lib().ndo_kv_slot(W, ns, p)
            writes.append((b, p, caches[b].row(sl, outlier=rng.random() < outlier_p)))
    n = len(ids)
    q = rng.standard_normal((n, nh, qk)).astype(np.float32)
    gate = rng.standard_normal((n, nh, vd)).astype(np.float32) if gated else None

    outs = []
    for flags in (0, N.FLAG_DECODE_VALU):
        ctx = N.Context(1, nh, nkv, qk, vd, W, kv_dtype=N.KV_INT8, max_seqs=B + 1, flags=flags,
                        page_size=page_size)
        if prefix:
            ctx.seq_set_sink(B, prefix)
        else:
            for b, (pos, ns) in enumerate(specs):
                if ns:
                    ctx.seq_set_sink(b, ns)
        pid = None
        for b, p, (k, v, ks, vs) in writes:
            if prefix and b < B and pid is None:
                ctx.seq_set_pos(B, prefix)
                pid = ctx.prefix_build(B)
                for bb in range(B):
                    ctx.seq_attach(bb, pid)
            ctx.kv_write(0, b, p, k, v, ks, vs)
        for b, (pos, _) in enumerate(specs):
            ctx.seq_set_pos(b, pos)
        dq = N.DevBuf.from_array(q)
        dg = N.DevBuf.from_array(gate) if gated else None
        dout = N.DevBuf(n * nh * vd * 4)
        ctx.decode(0, n, dq, dout, gate=dg, seq_ids=ids)
        ctx.sync()
        outs.append(dout.to_array(np.float32, (n, nh, vd)))
        ctx.close()
    worst = [0.0, 0.0]
    for i, b in enumerate(ids):
        pos, ns = specs[b]
        ns = prefix if prefix else min(ns, max(0, W - 64))
        c = caches[b]
        kv = O.kv_view(c.k, c.v, c.ks, c.vs, nh, W, ns, pos, O.KV_INT8)
        want = O.attend_view(kv, q[i].ravel(), None if gate is None else gate[i].ravel())
        for j in range(2):
            worst[j] = max(worst[j], float(np.abs(outs[j][i].ravel().astype(np.float64) - want).max()))
    between = float(np.abs(outs[0].astype(np.float64) - outs[1]).max())
    return worst[0], worst[1], between


# (pos, n_sink): 1 key, the 32-key tile edges, the engine's 213 + 16, a full
# 384-slot window, wrapped rings with and without sinks
SPECS = [(0, 0), (1, 0), (30, 0), (31, 0), (32, 0), (62, 0), (63, 0), (64, 0), (212, 0), (228, 0),
         (382, 0), (383, 0), (500, 0), (700, 4), (1000, 64), (391, 31)]


@pytest.mark.parametrize("nh,nkv,qk", [(12, 2, 48), (8, 2, 64), (16, 2, 64), (12, 2, 64), (8, 1, 64), (16, 4, 64),
                                       (24, 4, 48), (12, 3, 64), (18, 3, 48)])
def test_decode_mfma_gqa_ragged_ring(nh, nkv, qk):
    say("decode mfma", nh, nkv, qk)
    order = list(range(len(SPECS)))[::-1]       # rows listed out of order
    mf, va, between = _run(nh, nkv, qk, 384, SPECS, seed=nh * 100 + qk, order=order)
    say("worst vs oracle: mfma", mf, "valu", va, "between", between)
    assert mf <= TOL and va <= TOL, (mf, va)
    assert between <= KERNELS_TOL, between


def test_decode_mfma_ungated_outliers_subset():
    """No gate, 6-sigma keys (the lazy running max moves), a subset of rows
    (8 of 10, enough work items for the MFMA route)."""
    say("decode mfma ungated outliers")
    specs = [(100, 0), (383, 0), (450, 8), (40, 0), (257, 0), (0, 0), (95, 0), (31, 0), (700, 16), (33, 0)]
    mf, va, between = _run(12, 2, 48, 384, specs, seed=77, gated=False, order=[3, 0, 4, 9, 7, 1, 8, 2],
                           outlier_p=0.05)
    say("worst vs oracle: mfma", mf, "valu", va, "between", between)
    assert mf <= TOL and va <= TOL, (mf, va)
    assert between <= KERNELS_TOL, between


def test_decode_mfma_shared_prefix():
    """Sequences attached to a 213-position prefix (slots 0-212 from the
    prefix's pages, the prefix / own boundary inside a 32-key tile), own rings
    from empty to wrapped."""
    say("decode mfma shared prefix")
    specs = [(213, 0), (214, 0), (229, 0), (244, 0), (245, 0), (383, 0), (384, 0), (600, 0)]
    mf, va, between = _run(12, 2, 48, 384, specs, seed=91, prefix=213)
    say("worst vs oracle: mfma", mf, "valu", va, "between", between)
    assert mf <= TOL and va <= TOL, (mf, va)
    assert between <= KERNELS_TOL, between


@pytest.mark.parametrize("page_size", [32, 64])
@pytest.mark.parametrize("nh,nkv,qk", [(12, 2, 48), (8, 2, 64)])
def test_decode_mfma_page_sizes(nh, nkv, qk, page_size):
    """Pages of 32 and 64 slots: a tile's halves share a page and its K rows,
    V rows and scales are separate runs (the 16-slot pages of the other
    cases are read as one run per kv-head block); rings, sinks and a shared
    prefix whose end falls inside a page."""
    say("decode mfma pages", page_size, nh, nkv, qk)
    mf, va, between = _run(nh, nkv, qk, 384, SPECS, seed=page_size + qk, page_size=page_size)
    assert mf <= TOL and va <= TOL and between <= KERNELS_TOL, (mf, va, between)
    specs = [(213, 0), (229, 0), (245, 0), (600, 0)]
    mf, va, between = _run(nh, nkv, qk, 384, specs + specs, seed=page_size + 3, prefix=213, page_size=page_size)
    assert mf <= TOL and va <= TOL and between <= KERNELS_TOL, (mf, va, between)


def test_decode_mfma_ordered_batch():
    """A batch large enough for the longest-first work order of the GQA
    decode: 2048 sequences x 2 kv-heads at the engine's shape (12 q heads,
    qk 48, int8), lengths 1-700 over a 384-slot window (short rows and
    wrapped rings), a synthetic cache. Three decode steps through nda_step
    (new rows stored, positions advanced between steps, so the order is
    rebuilt), two layers each (the order reused), and before the last
    advance a listed subset through nda_decode (rows in call order, no work
    order). Every output against the VALU kernel on a context fed the same
    (1e-4), and sampled rows against the oracle over the cache as stored
    (1e-3)."""
    say("decode mfma ordered batch")
    N = nda()
    nh, nkv, qk, vd, W, B, L, steps = 12, 2, 48, 64, 384, 2048, 2, 3
    rng = np.random.default_rng(91)
    lens = rng.integers(0, 700, B)
    calls = [[tuple(rng.standard_normal((B, h, d)).astype(np.float32)
                    for h, d in ((nh, qk), (nkv, qk), (nkv, vd), (nh, vd))) for li in range(L)]
             for step in range(steps)]
    sub = sorted(rng.choice(B, 300, replace=False).tolist(), key=lambda x: -lens[x])
    q_sub = rng.standard_normal((len(sub), nh, qk)).astype(np.float32)
    sample = [int(b) for b in rng.choice(B, 12, replace=False)]
    outs = {}
    worst = 0.0
    for flags in (0, N.FLAG_DECODE_VALU):
        ctx = N.Context(L, nh, nkv, qk, vd, W, kv_dtype=N.KV_INT8, max_seqs=B, flags=flags)
        for b in range(B):
            ctx.seq_set_pos(b, int(lens[b]))
            ctx.seq_reserve(b, W)
        ctx.kv_fill_normal(B, seed=92)
        res = []
        for step in range(steps):
            for li in range(L):
                q, k, v, g = calls[step][li]
                dout = N.DevBuf(B * nh * vd * 4)
                ctx.step(li, B, N.DevBuf.from_array(q), N.DevBuf.from_array(k), N.DevBuf.from_array(v), dout,
                         gate=N.DevBuf.from_array(g))
                ctx.sync()
                got = dout.to_array(np.float32, (B, nh * vd))
                res.append(got)
                if flags == 0:
                    for b in sample:
                        pos = ctx.seq_state(b)[0]
                        n = min(pos + 1, W)
                        kk, vv, ks, vs = ctx.kv_read(li, b, pos + 1 - n, n)
                        view = O.kv_view(kk, vv, ks, vs, nh, n, 0, n - 1, O.KV_INT8)
                        want = O.attend_runs(view, np.arange(n), [n], q[b], g[b])
                        worst = max(worst, float(np.abs(got[b].astype(np.float64) - want).max()))
            if step == steps - 1:
                dout = N.DevBuf(len(sub) * nh * vd * 4)
                ctx.decode(0, len(sub), N.DevBuf.from_array(q_sub), dout, seq_ids=sub)
                ctx.sync()
                res.append(dout.to_array(np.float32, (len(sub), nh * vd)))
            ctx.advance(B, None, 1)
        outs[flags] = res
        ctx.close()
    between = max(float(np.abs(a.astype(np.float64) - b).max()) for a, b in zip(outs[0], outs[N.FLAG_DECODE_VALU]))
    say("ordered batch worst vs oracle", worst, "mfma vs valu", between)
    assert worst <= TOL, worst
    assert between <= KERNELS_TOL, between
