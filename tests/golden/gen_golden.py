"""Writes tests/golden/golden.npz from the reference engine's own attention
code (oracle/_ref/libndref.so, compiled by oracle/ref.mk from the reference
sources). Run where the reference tree exists (/root/reference):

    make -C oracle && python tests/golden/gen_golden.py

Inputs are integer-derived (detgen.py), so the fixture stores seeds and
outputs only. The exp_pairs vectors take their inputs from the reference's
own fixture esp32/main/exp_pairs.h (1024 real softmax argument pairs),
read here as data.
"""
import os
import re
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle"))
sys.path.insert(0, HERE)
import ctypes as C  # noqa: E402

import ndoracle as O  # noqa: E402
from detgen import Stream, det_normal  # noqa: E402

REF = os.environ.get("REF", "/root/reference")

# Session scripts. Each event: ("tok", gated) store+attend one token on every
# layer then pos++, ("snap",), ("sink", n), ("save", slot), ("restore", slot),
# ("reset",), ("rewind",). Outputs are recorded for the token steps listed in `record`.
SESSIONS = {
    # one layer, MHA 8x64, 213-token pinned prefix + 16 prompt tokens
    "cfg1": dict(geom=(1, 8, 8, 64, 64, 256), seed=101,
                 script=[("tok", True)] * 213 + [("snap",)] + [("tok", True)] * 16,
                 record=list(range(213, 229))),
    # the archive's shapes: 12 q / 2 kv heads, qk 48, v 64, window 384, ring wraps
    "engine": dict(geom=(2, 12, 2, 48, 64, 384), seed=202,
                   script=[("tok", True)] * 200 + [("snap",)] + [("tok", True)] * 260,
                   record=list(range(0, 460, 23)) + [459]),
    # GQA rep 4, tiny window with 10 sinks: many wraps, one ungated token in 3
    "wrap": dict(geom=(1, 8, 2, 64, 64, 100), seed=303,
                 script=[("tok", True)] * 10 + [("sink", 10)] +
                        [("tok", i % 3 != 0) for i in range(250)],
                 record=list(range(0, 260, 13)) + [259]),
    # window <= 64: the sink clamp pins nothing; plain sliding window
    "small": dict(geom=(1, 4, 4, 64, 64, 40), seed=404,
                  script=[("tok", True)] * 5 + [("sink", 5)] + [("tok", True)] * 60,
                  record=list(range(0, 65, 8)) + [64]),
    # nd_ptest's flow: two 2-token prefixes restored alternately
    "ptest": dict(geom=(1, 12, 2, 48, 64, 384), seed=505,
                  script=[("reset",), ("tok", True), ("tok", True), ("snap",), ("save", 0), ("tok", True),
                          ("reset",), ("tok", True), ("tok", True), ("snap",), ("save", 1), ("tok", True),
                          ("restore", 0), ("tok", True), ("restore", 1), ("tok", True),
                          ("restore", 0), ("tok", True), ("restore", 1), ("tok", True)],
                  record="all"),
    # 8 heads x 64 on 2 layers: causal prefill of 256 tokens, window 256
    "prefill": dict(geom=(2, 8, 8, 64, 64, 256), seed=606,
                    script=[("tok", True)] * 256, record=list(range(0, 256, 17)) + [255]),
    # with the attention front (tap convolution + head norm + RoPE on raw
    # projections): the archive's shapes, 3 taps, snapshot / rewind / prefix
    # switching, which must carry the tap histories along
    "front_engine": dict(geom=(2, 12, 2, 48, 64, 384), seed=707, front=(3, 10000.0),
                         script=[("tok", True)] * 30 + [("snap",), ("save", 0)] + [("tok", True)] * 5 +
                                [("rewind",)] + [("tok", True)] * 3 +
                                [("reset",)] + [("tok", True)] * 7 + [("snap",), ("save", 1)] +
                                [("tok", True)] * 2 + [("restore", 0)] + [("tok", True)] * 2 +
                                [("restore", 1)] + [("tok", True)] * 2,
                         record="all"),
    # MHA 8x64 with 4 taps and theta 1e6 past a ring wrap, at large positions
    "front_cfg": dict(geom=(1, 8, 8, 64, 64, 128), seed=808, front=(4, 1000000.0),
                      script=[("tok", True)] * 20 + [("sink", 20)] + [("tok", i % 4 != 0) for i in range(200)],
                      record=list(range(0, 220, 7)) + [219]),
}


def front_weights(spec):
    """Per-layer tap weights [L][taps][dim] and norm scales [L][qk_hd]."""
    L, nh, nkv, qk, vd, W = spec["geom"]
    taps = spec["front"][0]
    st = Stream(spec["seed"] + 1)
    shape = lambda dim: st.take(L * taps * dim).reshape(L, taps, dim) * np.float32(0.5)
    return O.FrontWeights(shape(nh * qk), shape(nkv * qk), shape(nkv * vd),
                          st.take(L * qk).reshape(L, qk) * np.float32(0.25),
                          st.take(L * qk).reshape(L, qk) * np.float32(0.25))


def run_session(S, spec):
    """Replays a script on an OracleSession or a RefSession; with a `front`
    entry the raw q/k/v go through the attention front first."""
    L, nh, nkv, qk, vd, W = spec["geom"]
    st = Stream(spec["seed"])
    outs, saved = [], {}
    ntok = 0
    rec = spec["record"]
    fw = None
    if "front" in spec:
        S.front_init(*spec["front"])
        fw = front_weights(spec)
    for ev in spec["script"]:
        if ev[0] == "tok":
            for li in range(L):
                q = st.take(nh * qk)
                k = st.take(nkv * qk)
                v = st.take(nkv * vd)
                g = st.take(nh * vd) if ev[1] else None
                if fw is not None:
                    q, k, v = S.front(li, fw, q, k, v)
                o = S.attention(li, q, k, v, g)
                if rec == "all" or ntok in rec:
                    outs.append(o.copy())
            S.step_end()
            ntok += 1
        elif ev[0] == "snap":
            assert S.snapshot() == 0
        elif ev[0] == "sink":
            S.set_sink(ev[1])
        elif ev[0] == "save":
            saved[ev[1]] = S.prefix_save()
            assert saved[ev[1]]
        elif ev[0] == "restore":
            assert S.prefix_restore(saved[ev[1]]) == 0
        elif ev[0] == "reset":
            S.reset()
        elif ev[0] == "rewind":
            S.rewind()
    return np.stack(outs), saved


def hist_blob(S):
    """Live and snapshot tap histories, flattened (float32)."""
    return np.concatenate([h.ravel() for h in S.hist(False) + S.hist(True)]).astype(np.float32)


def exp_pairs_inputs():
    text = open(os.path.join(REF, "esp32/main/exp_pairs.h")).read()
    body = text[text.index("{", text.index("kb_exp_pairs")) + 1: text.index("};")]
    vals = [float(x.rstrip("f")) for x in re.findall(r"-?\d+\.?\d*(?:e-?\d+)?f", body)]
    return np.array(vals, np.float32)


def main():
    R = O.ref()
    out = {}
    # exp on the reference's captured softmax arguments, paired form
    xp = exp_pairs_inputs()
    assert xp.size == 2048, xp.size
    r0, r1 = C.c_float(), C.c_float()
    ep = np.zeros_like(xp)
    for i in range(0, xp.size, 2):
        R.ref_expf_pair(float(xp[i]), float(xp[i + 1]), C.byref(r0), C.byref(r1))
        ep[i], ep[i + 1] = r0.value, r1.value
    out["exp_pairs_in"], out["exp_pairs_out"] = xp, ep
    # exp / sigmoid over a sweep including the clamps and rounding boundaries
    xs = np.concatenate([np.linspace(-100, 100, 4001, dtype=np.float32),
                         np.array([-88.0, 88.0, -88.00001, 88.00001, 0.0, -0.0, 0.5, -0.5,
                                   0.34657359, -0.34657359, 1e-30, -1e-30], np.float32),
                         det_normal(7, 2000) * 8]).astype(np.float32)
    out["exp_in"] = xs
    out["exp_out"] = np.array([R.ref_expf(float(x)) for x in xs], np.float32)
    out["sig_out"] = np.array([R.ref_sigmoid(float(x)) for x in xs], np.float32)
    # int8 store: random rows, exact ties, zero rows, +-absmax, tiny values
    rows = [det_normal(11, 64), det_normal(12, 48) * 1000, np.zeros(64, np.float32),
            np.array([127 * 0.5 + 0.5 * i for i in range(64)], np.float32) / 127,
            np.array([(i - 32) + 0.5 for i in range(64)], np.float32),
            np.array([1e-38 * (i - 32) for i in range(64)], np.float32),
            det_normal(13, 64) * 1e-20]
    codes, scales = [], []
    for r in rows:
        r = np.ascontiguousarray(r, np.float32)
        amax = float(np.max(np.abs(r)))
        sc = np.float32(amax) / np.float32(127.0) if amax > 0 else np.float32(1.0)
        d = np.zeros(r.size, np.int8)
        R.ref_kv_store_int8(d, r, r.size, float(sc))
        codes.append(np.pad(d, (0, 64 - d.size)))
        scales.append(sc)
    out["store_rows"] = np.stack([np.pad(r, (0, 64 - r.size)) for r in rows]).astype(np.float32)
    out["store_len"] = np.array([r.size for r in rows], np.int32)
    out["store_codes"] = np.stack(codes)
    out["store_scales"] = np.array(scales, np.float32)
    # attention sessions on the reference
    for name, spec in SESSIONS.items():
        S = O.RefSession(*spec["geom"])
        o, saved = run_session(S, spec)
        out["sess_" + name] = o.astype(np.float32)
        k, v, ks, vs = S.cache()
        out["sess_" + name + "_kvsum"] = np.array(
            [int(k.astype(np.int64).sum()), int(v.astype(np.int64).sum()),
             int(np.abs(k.astype(np.int64)).sum()), int(np.abs(v.astype(np.int64)).sum())], np.int64)
        if "front" in spec:
            out["sess_" + name + "_hist"] = hist_blob(S)
        for p in saved.values():
            O.ref().ref_prefix_free(p)
        S.close()
    # CQ projections: the reference's prepare, generic matvec and 2-bit table path
    from detgen import make_cq_tensor
    cq_shapes = [(24, 256, 128, 2), (9, 300, 128, 4), (13, 96, 32, 3)]
    out["cq_shapes"] = np.array(cq_shapes, np.int32)
    for i, (o, n, g, b) in enumerate(cq_shapes):
        t = make_cq_tensor(100 + i, o, n, g, b, special_norms=True)
        x = det_normal(200 + i, n)
        xh = np.zeros(t.in_pad, np.float32)
        R.ref_cq_prepare(n, g, x.ctypes.data, xh.ctypes.data)
        y = np.zeros(o, np.float32)
        R.ref_cq_gemv(o, n, g, b, t.blob.ctypes.data, t.codebook.ctypes.data, xh.ctypes.data, y.ctypes.data)
        out["cq_blob_%d" % i], out["cq_cb_%d" % i], out["cq_x_%d" % i] = t.blob, t.codebook, x
        out["cq_xh_%d" % i], out["cq_y_%d" % i] = xh, y
        if b == 2:
            lut = np.zeros(t.in_pad // 2 * 16, np.float32)
            y2 = np.zeros(o, np.float32)
            R.ref_cq_lut2(o, n, g, t.blob.ctypes.data, t.codebook.ctypes.data, xh.ctypes.data,
                          lut.ctypes.data, y2.ctypes.data)
            out["cq_y2_%d" % i] = y2
    # the engine's whole attention() over a session (tests/test_oracle_block.py)
    sys.path.insert(0, os.path.dirname(HERE))
    from test_oracle_block import BLOCK, replay_block
    rs = O.RefSession(*BLOCK["geom"])
    bo, bsaved = replay_block(rs, BLOCK)
    out["block_out"] = bo.astype(np.float32)
    for p in bsaved.values():
        O.ref().ref_prefix_free(p)
    np.savez_compressed(os.path.join(HERE, "golden.npz"), **out)
    print("wrote", os.path.join(HERE, "golden.npz"), {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
