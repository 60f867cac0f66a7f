"""The oracle's whole attention block (ndo_attention_block: CQ projections,
the front, the int8 store, attn_heads with the gate, out_proj) bit-exact
against the engine's own attention() (engine/src/nd_model.c:2382-2502),
driven through the reference harness over sessions with snapshot, rewind
and prefix restore; and against the committed golden outputs."""
import os

import numpy as np
import pytest

import ndoracle as O
from detgen import Stream, make_block_weights

HERE = os.path.dirname(os.path.abspath(__file__))


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def front_weights(seed, L, nh, nkv, qk, vd, taps):
    st = Stream(seed)
    shape = lambda dim: st.take(L * taps * dim).reshape(L, taps, dim) * np.float32(0.5)
    return O.FrontWeights(shape(nh * qk), shape(nkv * qk), shape(nkv * vd),
                          st.take(L * qk).reshape(L, qk) * np.float32(0.25),
                          st.take(L * qk).reshape(L, qk) * np.float32(0.25))


BLOCK = dict(geom=(2, 12, 2, 48, 64, 64), d_model=256, taps=3, theta=10000.0, seed=901,
             script=[("tok",)] * 20 + [("snap",), ("save", 0)] + [("tok",)] * 50 + [("rewind",)] +
                    [("tok",)] * 3 + [("reset",)] + [("tok",)] * 4 + [("restore", 0)] + [("tok",)] * 3)


# an odd shape: qk 36 / v 20, 5 query heads per kv-head, out_proj over 200 inputs
BLOCK_ODD = dict(BLOCK, geom=(2, 10, 2, 36, 20, 64), seed=907)


def replay_block(S, spec):
    L, nh, nkv, qk, vd, W = spec["geom"]
    S.front_init(spec["taps"], spec["theta"])
    fw = front_weights(spec["seed"] + 1, L, nh, nkv, qk, vd, spec["taps"])
    bw = make_block_weights(spec["seed"] + 2, L, nh, nkv, qk, vd, spec["d_model"])
    if isinstance(S, O.RefSession):
        S.block_setup(bw)
    st = Stream(spec["seed"])
    outs, saved = [], {}
    for ev in spec["script"]:
        if ev[0] == "tok":
            for li in range(L):
                outs.append(S.attention_block(li, fw, bw, st.take(spec["d_model"])))
            S.step_end()
        elif ev[0] == "snap":
            assert S.snapshot() == 0
        elif ev[0] == "save":
            saved[ev[1]] = S.prefix_save()
        elif ev[0] == "restore":
            assert S.prefix_restore(saved[ev[1]]) == 0
        elif ev[0] == "rewind":
            S.rewind()
        elif ev[0] == "reset":
            S.reset()
    return np.stack(outs), saved


@pytest.mark.skipif(not O.have_ref(), reason="reference harness not built")
@pytest.mark.parametrize("spec", [BLOCK, BLOCK_ODD], ids=["12x2_48_64", "10x2_36_20"])
def test_block_matches_engine_attention(spec):
    o = O.OracleSession(*spec["geom"])
    r = O.RefSession(*spec["geom"])
    a, sa = replay_block(o, spec)
    b, sb = replay_block(r, spec)
    assert np.array_equal(bits(a), bits(b))
    for x, y in zip(o.cache(), r.cache()):
        assert np.array_equal(np.asarray(x), np.asarray(y))
    for x, y in zip(o.hist(), r.hist()):
        assert np.array_equal(bits(x), bits(y))
    for p in sa.values():
        O.lib().ndo_prefix_free(p)
    for p in sb.values():
        O.ref().ref_prefix_free(p)


def test_block_golden():
    G = np.load(os.path.join(HERE, "golden", "golden.npz"))
    o = O.OracleSession(*BLOCK["geom"])
    a, sa = replay_block(o, BLOCK)
    for p in sa.values():
        O.lib().ndo_prefix_free(p)
    assert np.array_equal(bits(a), bits(G["block_out"]))
