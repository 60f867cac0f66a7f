"""GPU parity of the whole attention block (nda_attention_block and the
shim's nd_gpu_attention_block: CQ projections, front, store, attention with
the gate, out_proj) against the oracle's block, which is bit-exact to the
engine's own attention(). A decode step's projections (at most 64 rows)
follow the engine's own LUT order, so q/k/v and the stored int8 codes are
the engine's bit for bit (checked: no code differs); outputs are held to
max |delta| <= 1e-3, relative to the call's largest output where that
exceeds 1 (out_proj sums hundreds of terms)."""
import os
import sys

import numpy as np
import pytest

import ndoracle as O
from detgen import Stream, make_block_weights

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
TOL = 1e-3


def nda():
    import ndattn
    return ndattn


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


def cq_objects(N, bw, li, nh, nkv, qk, vd):
    outs = [nh * qk, nkv * qk, nkv * vd, nh * vd, bw.d_model]
    ins = [bw.d_model] * 4 + [nh * vd]
    return [N.CQ(outs[t], ins[t], bw.group, 2, bw.blobs[li][t], bw.codebook[:4]) for t in range(5)]


def test_shim_block_replays_engine_golden():
    """The engine drop-in for attention() as a whole replays the golden
    session the engine's own attention() produced."""
    N = nda()
    sys.path.insert(0, HERE)
    from test_oracle_block import BLOCK, front_weights
    say("shim block golden")
    G = np.load(os.path.join(HERE, "golden", "golden.npz"))
    L, nh, nkv, qk, vd, W = BLOCK["geom"]
    g = N.GpuSession(*BLOCK["geom"], kv_dtype=N.KV_INT8)
    fw = front_weights(BLOCK["seed"] + 1, L, nh, nkv, qk, vd, BLOCK["taps"])
    g.front_init(BLOCK["taps"], BLOCK["theta"], fw)
    bw = make_block_weights(BLOCK["seed"] + 2, L, nh, nkv, qk, vd, BLOCK["d_model"])
    cqs = [cq_objects(N, bw, li, nh, nkv, qk, vd) for li in range(L)]
    for li in range(L):
        g.block_weights(li, *cqs[li])
    st = Stream(BLOCK["seed"])
    outs, saved = [], {}
    for ev in BLOCK["script"]:
        if ev[0] == "tok":
            for li in range(L):
                outs.append(g.attention_block(li, st.take(BLOCK["d_model"])))
            g.step_end()
        elif ev[0] == "snap":
            assert g.snapshot() == 0
        elif ev[0] == "save":
            saved[ev[1]] = g.prefix_save()
        elif ev[0] == "restore":
            assert g.prefix_restore(saved[ev[1]]) == 0
        elif ev[0] == "rewind":
            g.rewind()
        elif ev[0] == "reset":
            g.reset()
    got, want = np.stack(outs), G["block_out"]
    worst = float(np.abs(got.astype(np.float64) - want).max())
    say("shim block worst", worst, "max |out|", float(np.abs(want).max()))
    assert worst <= TOL, worst
    for p in saved.values():
        g.prefix_free(p)
    g.close()
    for layer in cqs:
        for c in layer:
            c.close()


@pytest.mark.parametrize("shape,kv_dtype", [((12, 2, 48, 64), O.KV_INT8), ((12, 2, 48, 64), O.KV_F16),
                                             ((10, 2, 36, 20), O.KV_INT8), ((7, 1, 64, 64), O.KV_F16)])
def test_block_batched(shape, kv_dtype):
    """nda_attention_block for a batch of sequences at different positions,
    many steps, against one oracle session per sequence; at the engine's
    shape and at two shapes whose front has run-time dims."""
    N = nda()
    sys.path.insert(0, HERE)
    from test_oracle_block import front_weights
    say("block batched", shape, kv_dtype)
    nh, nkv, qk, vd = shape
    L, W, dm, taps, theta = 2, 96, 768, 3, 10000.0
    B = 6
    fw = front_weights(77, L, nh, nkv, qk, vd, taps)
    bw = make_block_weights(78, L, nh, nkv, qk, vd, dm)
    ctx = N.Context(L, nh, nkv, qk, vd, W, kv_dtype=kv_dtype, max_seqs=B)
    ctx.front_init(taps, theta)
    cqs = [cq_objects(N, bw, li, nh, nkv, qk, vd) for li in range(L)]
    for li in range(L):
        ctx.front_weights(li, *fw.arrays(li))
        ctx.block_weights(li, *cqs[li])
    orc = []
    for _ in range(B):
        o = O.OracleSession(L, nh, nkv, qk, vd, W, kv_dtype=kv_dtype)
        o.front_init(taps, theta)
        orc.append(o)
    rng = np.random.default_rng(3)
    bx, bo = N.DevBuf(B * dm * 4), N.DevBuf(B * dm * 4)
    worst, flips, codes, sc_rel = 0.0, 0, 0, 0.0
    for step in range(40):
        ids = [b for b in range(B) if step >= 3 * b]       # sequences join at different steps
        n = len(ids)
        for li in range(L):
            x = rng.standard_normal((n, dm)).astype(np.float32)
            bx.upload(x)
            ctx.attention_block(li, n, bx, bo, seq_ids=ids)
            ctx.sync()
            got = bo.to_array(np.float32, (n, dm))
            for i, b in enumerate(ids):
                want = orc[b].attention_block(li, fw, bw, x[i])
                # relative to the call's output scale: out_proj sums 768 terms
                rel = np.abs(got[i].astype(np.float64) - want).max() / max(1.0, float(np.abs(want).max()))
                worst = max(worst, float(rel))
        ctx.advance(n, seq_ids=ids)
        for b in ids:
            orc[b].step_end()
    for b in range(B):
        pos = orc[b].pos
        ok, ov, oks, ovs = orc[b].cache()
        for li in range(L):
            k, v, ks, vs = ctx.kv_read(li, b, max(0, pos - W + 1), min(pos, W))
            for j, p in enumerate(range(max(0, pos - W + 1), pos)):
                sl = O.lib().ndo_kv_slot(W, 0, p)
                if kv_dtype == O.KV_INT8:
                    for got_c, want_c in ((k[j], ok[li, sl]), (v[j], ov[li, sl])):
                        d = np.abs(got_c.astype(np.int32) - want_c.astype(np.int32))
                        assert d.max() <= 1, (b, li, p)
                        flips += int((d != 0).sum())
                        codes += d.size
                    # scales: absmax / 127 of the engine's rows
                    for got_s, want_s in ((ks[j], oks[li, sl]), (vs[j], ovs[li, sl])):
                        rel = np.abs(got_s.astype(np.float64) - want_s) / np.abs(want_s.astype(np.float64))
                        sc_rel = max(sc_rel, float(rel.max()))
                else:   # fp16 rows: the engine's values rounded to fp16, bit for bit
                    for got_r, want_r in ((k[j], ok[li, sl]), (v[j], ov[li, sl])):
                        assert np.array_equal(got_r.view(np.uint16), want_r.view(np.uint16)), (b, li, p)
    say("block batched worst (relative)", worst, "code flips", flips, "of", codes, "scale rel", sc_rel)
    assert worst <= TOL, worst
    assert flips == 0, (flips, codes)        # the engine's projections, bit for bit
    assert sc_rel == 0.0, sc_rel
    for layer in cqs:
        for c in layer:
            c.close()
