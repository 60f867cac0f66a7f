"""nda_decode_noalloc - nda_decode with its scratch (the launch's sequence ids
and the split-KV partials) in a static per-GPU device array instead of
context buffers grown by hipMalloc - against nda_decode on the same cache and
inputs. The two run the same kernels, so the bar is bit-identical outputs, on
two calls in a row, the second smaller; sampled rows also meet the oracle
(ndo_attend, the engine's attn_heads restated) within 1e-3. A call whose
scratch would not fit is refused with NDA_ERR_RANGE and writes nothing."""
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


def _context(N, lens, nh, nkv, qk, kv_dtype, seed, **kw):
    """One layer; every sequence holds positions [0, L] (L filled with
    synthetic N(0,1) values, position L stored by an append)."""
    B = len(lens)
    ctx = N.Context(1, nh, nkv, qk, 64, int(max(lens)) + 16, kv_dtype=kv_dtype, max_seqs=B, **kw)
    for b in range(B):
        ctx.seq_set_pos(b, int(lens[b]))
    ctx.kv_fill_normal(B, seed=seed)
    dk, dv = N.DevBuf(B * nkv * qk * 4), N.DevBuf(B * nkv * 64 * 4)
    dk.fill_normal(B * nkv * qk, 0, seed + 1)
    dv.fill_normal(B * nkv * 64, 0, seed + 2)
    ctx.kv_append(0, B, dk, dv)
    ctx.sync()
    return ctx


def _sentinel(N, n):
    d = N.DevBuf(n * 4)
    N._check(N.lib().nda_memset(d.value, 0xFF, n * 4))      # NaN everywhere
    return d


def _both(N, ctx, nseq, ids, q, gate, nh):
    """nda_decode then nda_decode_noalloc on the same inputs; returns both
    outputs and the profiled launch counts of each call."""
    outs, launches = [], []
    for noalloc in (False, True):
        d = _sentinel(N, nseq * nh * 64)
        ctx.prof_enable(True)
        ctx.prof_read(reset=True)
        (ctx.decode_noalloc if noalloc else ctx.decode)(0, nseq, q, d, gate=gate, seq_ids=ids)
        ctx.sync()
        launches.append(ctx.prof_read(reset=True)[1])
        ctx.prof_enable(False)
        outs.append(d.to_array(np.float32, (nseq, nh, 64)))
    return outs, launches


def _oracle_rows(ctx, rows, ids, q, gate, out, nh, kv_dtype):
    worst = 0.0
    for i in rows:
        b = int(ids[i]) if ids is not None else i
        pos = ctx.seq_state(b)[0]
        k, v, ks, vs = ctx.kv_read(0, b, 0, pos + 1)
        if kv_dtype == O.KV_F16:
            ks = vs = None
        kv = O.kv_view(k, v, ks, vs, nh, pos + 1, 0, pos, kv_dtype)
        want = O.attend_view(kv, q[i].ravel(), None if gate is None else gate[i].ravel())
        worst = max(worst, float(np.abs(out[i].ravel().astype(np.float64) - want).max()))
    return worst


def test_noalloc_split_kv_matches_decode_twice():
    """fp16 8 x 64, 48 sequences of 3000-8192 positions: 384 (row, head)
    units leave rows cut into chunks of 1024 positions, so the partials and
    the merge run in the static scratch. Then 12 of the sequences, listed out
    of order."""
    N = nda()
    nh = 8
    rng = np.random.default_rng(31)
    lens = rng.integers(3000, 8193, 48)
    ctx = _context(N, lens, nh, nh, 64, O.KV_F16, seed=501)
    for nseq, ids in ((48, None), (12, [int(x) for x in rng.permutation(48)[:12]])):
        say("noalloc split-KV", nseq, "rows")
        qh = rng.standard_normal((nseq, nh, 64)).astype(np.float32)
        gh = rng.standard_normal((nseq, nh, 64)).astype(np.float32)
        q, g = N.DevBuf.from_array(qh), N.DevBuf.from_array(gh)
        (ref, got), (lr, lg) = _both(N, ctx, nseq, ids, q, g, nh)
        assert lr[N.K_COMBINE] > 0, "the case must take the split-KV path"
        assert sum(lg) == 0, "nda_decode_noalloc records no profiling events"
        assert np.isfinite(ref).all()
        assert np.array_equal(ref, got)
        w = _oracle_rows(ctx, range(0, nseq, max(1, nseq // 4)), ids, qh, gh, got, nh, O.KV_F16)
        say("worst vs oracle", w)
        assert w <= TOL
    ctx.close()


def test_noalloc_gqa_mfma_matches_decode_twice():
    """int8 12/2 heads, qk 48 (the engine's shape, MFMA decode): ids in the
    scratch, no partials. 32 rows, then 16 listed out of order."""
    N = nda()
    nh, nkv, qk = 12, 2, 48
    rng = np.random.default_rng(32)
    lens = rng.integers(213, 384, 32)
    ctx = _context(N, lens, nh, nkv, qk, O.KV_INT8, seed=601)
    for nseq, ids in ((32, None), (16, [int(x) for x in rng.permutation(32)[:16]])):
        say("noalloc gqa", nseq, "rows")
        qh = rng.standard_normal((nseq, nh, qk)).astype(np.float32)
        gh = rng.standard_normal((nseq, nh, 64)).astype(np.float32)
        q, g = N.DevBuf.from_array(qh), N.DevBuf.from_array(gh)
        (ref, got), _ = _both(N, ctx, nseq, ids, q, g, nh)
        assert np.isfinite(ref).all()
        assert np.array_equal(ref, got)
        w = _oracle_rows(ctx, range(0, nseq, 5), ids, qh, gh, got, nh, O.KV_INT8)
        say("worst vs oracle", w)
        assert w <= TOL
    ctx.close()


def test_noalloc_refuses_scratch_overflow():
    """A fixed 64-position split over 16 rows of 32768 positions needs
    16 * 8 * 513 * 66 * 4 B = 17.3 MB of partials, more than the 16 MiB
    scratch: NDA_ERR_RANGE, the output untouched; a smaller call after it
    still matches nda_decode."""
    N = nda()
    nh = 8
    lens = np.full(16, 32767)
    ctx = _context(N, lens, nh, nh, 64, O.KV_F16, seed=701, split_chunk=64)
    q = N.DevBuf(16 * nh * 64 * 4)
    q.fill_normal(16 * nh * 64, 0, 9)
    d = _sentinel(N, 16 * nh * 64)
    with pytest.raises(N.NdaError) as e:
        ctx.decode_noalloc(0, 16, q, d)
    assert e.value.code == -4
    ctx.sync()
    assert np.isnan(d.to_array(np.float32, (16, nh, 64))).all()
    say("overflow refused; 2 rows after it")
    (ref, got), _ = _both(N, ctx, 2, [5, 3], q, None, nh)
    assert np.isfinite(ref).all() and np.array_equal(ref, got)
    ctx.close()


def test_noalloc_allocates_nothing(allocator):
    """A fresh context; with every device allocation refused through the
    allocator seam, nda_decode_noalloc over listed sequences (ids in the
    scratch) whose rows are split (partials in the scratch) succeeds twice,
    the second call smaller, and the allocator sees no request at all. The
    outputs then meet the oracle."""
    N = nda()
    nh = 8
    rng = np.random.default_rng(33)
    lens = rng.integers(3000, 8193, 48)
    ctx = _context(N, lens, nh, nh, 64, O.KV_F16, seed=801)
    calls = [(48, [int(x) for x in rng.permutation(48)]), (12, [int(x) for x in rng.permutation(48)[:12]])]
    inputs = []
    for nseq, ids in calls:
        qh = rng.standard_normal((nseq, nh, 64)).astype(np.float32)
        inputs.append((qh, N.DevBuf.from_array(qh), N.DevBuf(nseq * nh * 64 * 4)))
    ctx.sync()
    say("noalloc with every allocation refused")
    allocator.seen = 0
    allocator.armed = True
    try:
        for (nseq, ids), (_, q, d) in zip(calls, inputs):
            ctx.decode_noalloc(0, nseq, q, d, seq_ids=ids)
        ctx.sync()
    finally:
        allocator.armed = False
    assert allocator.seen == 0, "nda_decode_noalloc asked the allocator for memory"
    for (nseq, ids), (qh, _, d) in zip(calls, inputs):
        got = d.to_array(np.float32, (nseq, nh, 64))
        assert np.isfinite(got).all()
        w = _oracle_rows(ctx, range(0, nseq, max(1, nseq // 4)), ids, qh, None, got, nh, O.KV_F16)
        say(nseq, "rows: worst vs oracle", w)
        assert w <= TOL
    ctx.close()


def test_noalloc_on_a_shared_prefix_batch():
    """1024 sequences on one 213-token prefix: nda_decode attends the prefix
    in one pass for the batch, nda_decode_noalloc row by row; the two agree
    within fp32 reassociation and both meet the oracle."""
    N = nda()
    nh, d, W, B, npre = 8, 64, 384, 1024, 213
    rng = np.random.default_rng(34)
    ctx = N.Context(1, nh, nh, d, d, W, kv_dtype=O.KV_F16, max_seqs=B + 1)
    bufs = [N.DevBuf(npre * nh * d * 4) for _ in range(4)]
    for i, bb in enumerate(bufs[:3]):
        bb.fill_normal(npre * nh * d, 0, 90 + i)
    ctx.prefill(0, [npre], bufs[0], bufs[1], bufs[2], bufs[3], seq_ids=[B])
    ctx.advance(1, [B], npre)
    pid = ctx.prefix_build(B)
    n = rng.integers(1, 40, B)
    for b in range(B):
        ctx.seq_attach(b, pid)
    T = int(n.sum())
    pb = [N.DevBuf(T * nh * d * 4) for _ in range(4)]
    for i, bb in enumerate(pb[:3]):
        bb.fill_normal(T * nh * d, 0, 95 + i)
    ctx.prefill(0, n, pb[0], pb[1], pb[2], pb[3])
    for b in range(B):
        ctx.advance(1, [b], int(n[b]))
    k = N.DevBuf(B * nh * d * 4)
    k.fill_normal(B * nh * d, 0, 99)
    ctx.kv_append(0, B, k, k)
    ctx.sync()
    qh = rng.standard_normal((B, nh, d)).astype(np.float32)
    q = N.DevBuf.from_array(qh)
    say("shared prefix: decode (prefix pass) and decode_noalloc")
    (ref, got), (lr, lg) = _both(N, ctx, B, None, q, None, nh)
    assert lr[N.K_DECODE] == 2, "nda_decode must take the shared-prefix pass here"
    assert np.isfinite(ref).all() and np.isfinite(got).all()
    diff = float(np.abs(ref - got).max())
    say("decode vs decode_noalloc", diff)
    assert diff <= 1e-4
    w = _oracle_rows(ctx, (0, 311, B - 1), None, qh, None, got, nh, O.KV_F16)
    say("worst vs oracle", w)
    assert w <= TOL
    for b in range(B + 1):
        ctx.seq_reset(b)
    ctx.prefix_free(pid)
    ctx.close()
