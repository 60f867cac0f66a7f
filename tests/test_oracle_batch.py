"""The oracle's threaded fp16 batch decode (ndo_decode_batch_f16, the CPU
baseline's composition of per-sequence stores and attention) against what
pins it independently: each sequence's output against float64 textbook
softmax attention over the same fp16 cache, the stored new token against
numpy's fp16 rounding at slot len-1, and the result independent of the
thread count."""
import numpy as np

import ndoracle as O


def _batch(rng, lens, nh, d, nthreads):
    S = len(lens)
    lens = np.ascontiguousarray(lens, np.uint32)
    off = np.zeros(S, np.uint64)
    off[1:] = np.cumsum(lens[:-1].astype(np.uint64) * nh * d)
    tot = int(lens.sum()) * nh * d
    kb = rng.standard_normal(tot).astype(np.float16).view(np.uint16)
    vb = rng.standard_normal(tot).astype(np.float16).view(np.uint16)
    q = rng.standard_normal(S * nh * d).astype(np.float32)
    kn = rng.standard_normal(S * nh * d).astype(np.float32)
    vn = rng.standard_normal(S * nh * d).astype(np.float32)
    out = np.zeros(S * nh * d, np.float32)
    O.decode_batch_f16(nh, nh, d, d, lens, kb, vb, off, off, q, kn, vn, None, out, nthreads)
    return lens, off, kb, vb, q, kn, vn, out


def test_batch_decode_against_float64_attention():
    rng = np.random.default_rng(3)
    nh, d = 8, 64
    lens = [1, 2, 3, 17, 64, 213, 229, 700]
    lens, off, kb, vb, q, kn, vn, out = _batch(rng, lens, nh, d, 4)
    for b, L in enumerate(lens):
        K = kb[int(off[b]):int(off[b]) + int(L) * nh * d].view(np.float16).astype(np.float64).reshape(L, nh, d)
        V = vb[int(off[b]):int(off[b]) + int(L) * nh * d].view(np.float16).astype(np.float64).reshape(L, nh, d)
        # the new token was stored at slot L-1, rounded to nearest even
        assert np.array_equal(K[L - 1].astype(np.float16), kn[b * nh * d:(b + 1) * nh * d].reshape(nh, d)
                              .astype(np.float16))
        assert np.array_equal(V[L - 1].astype(np.float16), vn[b * nh * d:(b + 1) * nh * d].reshape(nh, d)
                              .astype(np.float16))
        qb = q[b * nh * d:(b + 1) * nh * d].reshape(nh, d).astype(np.float64)
        for h in range(nh):
            s = K[:, h, :] @ qb[h] / np.sqrt(d)
            w = np.exp(s - s.max())
            want = (w / w.sum()) @ V[:, h, :]
            got = out[(b * nh + h) * d:(b * nh + h + 1) * d]
            assert np.abs(got - want).max() <= 2e-6 * max(1.0, np.abs(want).max()), (b, h)


def test_batch_decode_thread_count_invariant():
    rng = np.random.default_rng(5)
    lens = list(rng.integers(1, 400, 33))
    outs = []
    for nt in (1, 3, 16):
        outs.append(_batch(np.random.default_rng(9), lens, 8, 64, nt)[-1])
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
