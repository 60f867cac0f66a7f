"""GPU parity of the layer-batched block prefill (nda_prefill_block: CQ
projections over the chunk, the front over each sequence's tokens, the KV
store and causal attention with the gate, out_proj) against the oracle's
block stepped one token at a time, which is bit-exact to the engine's own
attention() (the engine prefills by repeated nd_model_step_hidden,
esp32/main/main.c:233-234, :312-315). Same bar as the decode block: outputs
within 1e-3 relative to the call's output scale, stored int8 codes within
one step where the projections' fp32 reassociation moves a value across a
rounding boundary (counted, at most 0.01%; these cases see one or two in
~10^5)."""
import sys

import numpy as np
import pytest

import ndoracle as O
from detgen import make_block_weights

pytestmark = pytest.mark.gpu

TOL = 1e-3


def nda():
    import ndattn
    return ndattn


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


def rel_err(got, want):
    return float(np.abs(got.astype(np.float64) - want).max()) / max(1.0, float(np.abs(want).max()))


class Rig:
    """One context and one oracle session per sequence over the same weights."""

    def __init__(self, kv_dtype, B, L=2, nh=12, nkv=2, qk=48, vd=64, W=128, dm=256, taps=3,
                 theta=10000.0, seed=0):
        N = nda()
        from test_gpu_block import cq_objects
        from test_oracle_block import front_weights
        self.N, self.kv_dtype, self.B = N, kv_dtype, B
        self.geom = (L, nh, nkv, qk, vd, W)
        self.L, self.W, self.dm, self.taps = L, W, dm, taps
        self.fw = front_weights(seed + 77, L, nh, nkv, qk, vd, taps)
        self.bw = make_block_weights(seed + 78, L, nh, nkv, qk, vd, dm)
        self.ctx = N.Context(L, nh, nkv, qk, vd, W, kv_dtype=kv_dtype, max_seqs=B)
        self.ctx.front_init(taps, theta)
        self.cqs = [cq_objects(N, self.bw, li, nh, nkv, qk, vd) for li in range(L)]
        for li in range(L):
            self.ctx.front_weights(li, *self.fw.arrays(li))
            self.ctx.block_weights(li, *self.cqs[li])
        self.orc = []
        for _ in range(B):
            o = O.OracleSession(L, nh, nkv, qk, vd, W, kv_dtype=kv_dtype)
            o.front_init(taps, theta)
            self.orc.append(o)
        self.rng = np.random.default_rng(seed + 5)
        self.worst = 0.0

    def chunk(self, ids, n_tokens):
        """Every layer takes each sequence's whole chunk in one call; the
        oracle steps the same tokens one at a time through all layers."""
        N, dm = self.N, self.dm
        T = int(sum(n_tokens))
        x = self.rng.standard_normal((self.L, T, dm)).astype(np.float32)
        got = np.zeros((self.L, T, dm), np.float32)
        bx, bo = N.DevBuf(max(1, T) * dm * 4), N.DevBuf(max(1, T) * dm * 4)
        for li in range(self.L):
            bx.upload(x[li])
            self.ctx.prefill_block(li, len(ids), n_tokens, bx, bo, seq_ids=ids)
            self.ctx.sync()
            got[li] = bo.to_array(np.float32, (T, dm))
        r0 = 0
        for b, n in zip(ids, n_tokens):
            for t in range(n):
                for li in range(self.L):
                    want = self.orc[b].attention_block(li, self.fw, self.bw, x[li, r0 + t])
                    self.worst = max(self.worst, rel_err(got[li, r0 + t], want))
                self.orc[b].step_end()
            r0 += n
        for b, n in zip(ids, n_tokens):
            if n:
                self.ctx.advance(1, seq_ids=[b], n=n)

    def decode(self, ids):
        N, dm = self.N, self.dm
        n = len(ids)
        bx, bo = N.DevBuf(n * dm * 4), N.DevBuf(n * dm * 4)
        for li in range(self.L):
            x = self.rng.standard_normal((n, dm)).astype(np.float32)
            bx.upload(x)
            self.ctx.attention_block(li, n, bx, bo, seq_ids=ids)
            self.ctx.sync()
            got = bo.to_array(np.float32, (n, dm))
            for i, b in enumerate(ids):
                want = self.orc[b].attention_block(li, self.fw, self.bw, x[i])
                self.worst = max(self.worst, rel_err(got[i], want))
        self.ctx.advance(n, seq_ids=ids)
        for b in ids:
            self.orc[b].step_end()

    def check_cache(self, b):
        """Stored rows against the oracle's: int8 codes within one step
        (returns the flips and the codes compared), fp16 rows within the
        projections' reassociation; scales within 1e-5 relative."""
        s = self.orc[b]
        pos, n_sink, _ = self.ctx.seq_state(b)
        assert (pos, n_sink) == (s.pos, s.n_sink), b
        ok, ov, oks, ovs = s.cache()
        lo = s.pos - (self.W - s.n_sink) + 1 if s.pos >= self.W else 0
        flips = codes = 0
        for li in range(self.L):
            seen_ring = False
            for p in list(range(min(s.n_sink, s.pos))) + list(range(max(lo, s.n_sink), s.pos)):
                sl = O.lib().ndo_kv_slot(self.W, s.n_sink, p)
                try:
                    k, v, ks, vs = self.ctx.kv_read(li, b, p, 1)
                except self.N.NdaError as e:
                    # after a rewind, the oldest ring positions before the
                    # snapshot may have been overwritten by later tokens (the
                    # engine's rewind restores no KV): only those are refused
                    assert e.code == -4 and p >= s.n_sink and not seen_ring, (b, li, p)
                    continue
                seen_ring |= p >= s.n_sink
                for g_, w_ in ((k[0], ok[li, sl]), (v[0], ov[li, sl])):
                    if self.kv_dtype == O.KV_INT8:
                        d = np.abs(g_.astype(np.int32) - w_.astype(np.int32))
                        assert d.max() <= 1, (b, li, p)
                        flips += int((d != 0).sum())
                        codes += d.size
                    else:
                        gv = g_.view(np.float16).astype(np.float64)
                        wv = w_.view(np.float16).astype(np.float64)
                        # within one fp16 step (2^-10 relative) of the oracle's row
                        assert np.all(np.abs(gv - wv) <= 2.0 ** -10 * np.maximum(1.0, np.abs(wv))), (b, li, p)
                if self.kv_dtype == O.KV_INT8:
                    for g_, w_ in ((ks[0], oks[li, sl]), (vs[0], ovs[li, sl])):
                        assert np.all(np.abs(g_ - w_) <= 1e-5 * np.abs(w_) + 1e-30), (b, li, p)
        return flips, codes

    def close(self):
        for layer in self.cqs:
            for c in layer:
                c.close()


@pytest.mark.parametrize("shape,kv_dtype", [((12, 2, 48, 64), O.KV_INT8), ((12, 2, 48, 64), O.KV_F16),
                                             ((10, 2, 36, 20), O.KV_INT8), ((8, 1, 20, 44), O.KV_F16)])
def test_prefill_block_ragged_chunks(shape, kv_dtype):
    """Sequences at different positions prefill ragged chunks (1 to 70
    tokens) in one call per layer, then decode on through the block; at the
    engine's shape and at two shapes whose front has run-time dims."""
    say("prefill block ragged", shape, kv_dtype)
    nh, nkv, qk, vd = shape
    R = Rig(kv_dtype, B=5, nh=nh, nkv=nkv, qk=qk, vd=vd)
    R.decode([1, 3])                     # two sequences start a few tokens in
    R.decode([1, 3])
    R.decode([3])
    R.chunk([0, 1, 2, 3, 4], [1, 17, 70, 33, 5])
    for _ in range(3):
        R.decode([0, 1, 2, 3, 4])
    R.chunk([4, 0], [40, 9])             # a second chunk, listed out of order
    for _ in range(2):
        R.decode([0, 1, 2, 3, 4])
    flips = codes = 0
    for b in range(5):
        f, c = R.check_cache(b)
        flips, codes = flips + f, codes + c
    say("prefill block worst (relative)", R.worst, "code flips", flips, "of", codes)
    assert R.worst <= TOL, R.worst
    assert flips <= max(1, codes // 10000), (flips, codes)
    R.close()


def test_prefill_block_shared_prefix_flow():
    """The engine's request flow: a prefix primed in one chunk on sequence 0,
    saved and shared (nda_prefix_build + attach; the oracle sessions take
    sequence 0's snapshot, as its prefix restore would give them), a suffix
    chunk per request, decode past the window so the ring wraps behind the
    pinned prefix, a rewind to the prefix and a second suffix."""
    sys.path.insert(0, __import__("os").path.dirname(__file__))
    from test_gpu_front import _copy_oracle_state
    say("prefill block shared prefix")
    B = 4
    R = Rig(O.KV_INT8, B=B, W=96, seed=11)
    R.chunk([0], [37])
    pid = R.ctx.prefix_build(0)
    for b in range(B):
        R.ctx.seq_attach(b, pid)
    assert R.orc[0].snapshot() == 0
    for b in range(1, B):
        _copy_oracle_state(R.orc[0], R.orc[b], R.geom, O.KV_INT8, R.taps)
    R.chunk([0, 1, 2, 3], [12, 30, 1, 45])
    for _ in range(60):                  # past the window of 96
        R.decode([0, 1, 2, 3])
    R.ctx.seq_rewind(2)
    R.orc[2].rewind()
    R.chunk([2], [20])
    R.decode([0, 1, 2, 3])
    flips = codes = 0
    for b in range(B):
        f, c = R.check_cache(b)
        flips, codes = flips + f, codes + c
        h = R.ctx.front_hist(b)
        want = np.concatenate([x.reshape(R.L, R.taps, -1) for x in R.orc[b].hist()], axis=2)
        assert np.all(np.abs(h - want) <= 1e-4 * np.maximum(1.0, np.abs(want))), b
    say("prefill block prefix worst (relative)", R.worst, "code flips", flips, "of", codes)
    assert R.worst <= TOL, R.worst
    assert flips <= max(1, codes // 10000), (flips, codes)
    R.close()


def test_prefill_block_rejects_without_changing_state():
    N = nda()
    say("prefill block errors")
    R = Rig(O.KV_INT8, B=2, W=64, seed=3)
    R.chunk([0], [10])
    h0, st0 = R.ctx.front_hist(0), R.ctx.seq_state(0)
    T = 60
    bx, bo = N.DevBuf(T * R.dm * 4), N.DevBuf(T * R.dm * 4)
    with pytest.raises(N.NdaError) as e:
        R.ctx.prefill_block(0, 1, [55], bx, bo, seq_ids=[0])       # 10 + 55 > 64: would wrap
    assert e.value.code == -4
    with pytest.raises(N.NdaError) as e:
        R.ctx.prefill_block(0, 1, [4], bx.value + 4, bo, seq_ids=[0])   # misaligned
    assert e.value.code == -1
    with pytest.raises(N.NdaError) as e:
        R.ctx.prefill_block(0, 2, [2, 2], bx, bo, seq_ids=[1, 1])     # listed twice
    assert e.value.code == -1
    assert np.array_equal(R.ctx.front_hist(0), h0) and R.ctx.seq_state(0) == st0
    R.ctx.prefill_block(0, 1, [0], bx, bo, seq_ids=[1])               # an empty chunk: nothing to do
    bare = N.Context(1, 12, 2, 48, 64, 64, kv_dtype=N.KV_INT8, max_seqs=1)
    with pytest.raises(N.NdaError) as e:
        bare.prefill_block(0, 1, [3], bx, bo)                        # no projection weights
    assert e.value.code == -5
    R.chunk([0, 1], [54, 3])             # the rejected chunks left the state usable
    say("prefill block errors worst", R.worst)
    assert R.worst <= TOL
    R.close()
