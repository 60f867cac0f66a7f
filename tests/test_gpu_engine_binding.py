"""The engine-side binding at build level: oracle/_ref/libndrefgpu.so is
compiled against the reference engine's own nd_model.h and nd_model.c with
the binding code an engine maintainer adds (one nd_gpu_attention call on the
engine's m->q, m->kbuf, m->vbuf, m->gate into m->attn in place of the store
and attn_heads dispatch of attention(), engine/src/nd_model.c:2426-2483; the
session entry points forwarded to their nd_gpu_* counterparts), and linked
against the package's libndhost.so and libndattn.so. One token stream with
snapshots, sinks, prefix save / restore, rewind and reset drives the
engine's CPU attention and the GPU drop-in through the same nd_model: every
output within 1e-3 of the engine's (fp32 accumulate), positions and sink
counts equal after every event. The whole attention() binding (front
weights and the archive's CQ tensors registered from the engine's own
nd_layer records, one nd_gpu_attention_block call) runs beside the engine's
attention() function itself. Skipped where the harness was not built (no
reference tree at build time)."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
SO = os.path.join(REPO, "oracle", "_ref", "libndrefgpu.so")
TOL = 1e-3

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(SO):
            pytest.skip("engine binding harness not built (oracle/_ref/libndrefgpu.so)")
        import ndattn
        ndattn.lib()                  # the package's libndattn.so, the one the harness links
        L = C.CDLL(SO)
        vp, u32, fp = C.c_void_p, C.c_uint32, C.POINTER(C.c_float)
        ip, up = C.POINTER(C.c_int), C.POINTER(C.c_uint32)
        L.eng_open.restype = vp
        L.eng_open.argtypes = [u32] * 6
        L.eng_close.argtypes = [vp]
        L.eng_attention.restype = C.c_int
        L.eng_attention.argtypes = [vp, u32, fp, fp, fp, fp, fp, fp]
        for n in ("eng_step_end", "eng_reset", "eng_rewind"):
            getattr(L, n).argtypes = [vp]
        L.eng_set_sink.argtypes = [vp, u32]
        L.eng_snapshot.argtypes = [vp, ip, ip]
        L.eng_prefix_save.restype = vp
        L.eng_prefix_save.argtypes = [vp]
        L.eng_prefix_restore.argtypes = [vp, vp, ip, ip]
        L.eng_prefix_free.argtypes = [vp]
        L.eng_state.argtypes = [vp, up, up, up, up]
        L.eng_front.restype = C.c_int
        L.eng_front.argtypes = [vp, u32, C.c_float]
        L.eng_block_setup.restype = C.c_int
        L.eng_block_setup.argtypes = [vp, u32, u32, vp, vp, vp]
        L.eng_attention_block.restype = C.c_int
        L.eng_attention_block.argtypes = [vp, u32, fp, fp, fp]
        _lib = L
    return _lib


def fptr(a):
    return a.ctypes.data_as(C.POINTER(C.c_float)) if a is not None else None


def state(L, e):
    v = [C.c_uint32() for _ in range(4)]
    L.eng_state(e, *[C.byref(x) for x in v])
    return tuple(x.value for x in v)


def run(geom, script, seed, scale=1.0, block=None):
    """block: (d_model, taps, theta, front weights, block weights, input
    stream) to drive the whole attention() instead of the store + dispatch."""
    L = lib()
    nl, nh, nkv, qk, vd, W = geom
    e = L.eng_open(*geom)
    assert e, "eng_open failed"
    rng = np.random.default_rng(seed)
    saved = {}
    worst = 0.0
    keep = []
    try:
        if block:
            d_model, taps, theta, fw, bw, st = block
            assert L.eng_front(e, taps, theta) == 0
            blobs = (C.c_void_p * (5 * nl))(*[b.ctypes.data for layer in bw.blobs for b in layer])
            front = (C.c_void_p * (5 * nl))(*[a.ctypes.data for li in range(nl) for a in fw.arrays(li)])
            keep += [blobs, front, fw, bw]
            assert L.eng_block_setup(e, d_model, bw.group, blobs, bw.codebook.ctypes.data, front) == 0
        for ev in script:
            if ev[0] == "tok" and block:
                for li in range(nl):
                    x = np.ascontiguousarray(st.take(d_model), np.float32)
                    co = np.zeros(d_model, np.float32)
                    go = np.zeros(d_model, np.float32)
                    rc = L.eng_attention_block(e, li, fptr(x), fptr(co), fptr(go))
                    assert rc == 0, rc
                    # out_proj sums hundreds of terms: relative to the call's
                    # largest output where that exceeds 1
                    scale_o = max(1.0, float(np.abs(co).max()))
                    worst = max(worst, float(np.abs(co.astype(np.float64) - go).max()) / scale_o)
                L.eng_step_end(e)
            elif ev[0] == "tok":
                for li in range(nl):
                    q = (rng.standard_normal(nh * qk) * scale).astype(np.float32)
                    k = (rng.standard_normal(nkv * qk) * scale).astype(np.float32)
                    v = rng.standard_normal(nkv * vd).astype(np.float32)
                    g = rng.standard_normal(nh * vd).astype(np.float32) if ev[1] else None
                    co = np.zeros(nh * vd, np.float32)
                    go = np.zeros(nh * vd, np.float32)
                    rc = L.eng_attention(e, li, fptr(q), fptr(k), fptr(v), fptr(g), fptr(co), fptr(go))
                    assert rc == 0, rc
                    worst = max(worst, float(np.abs(co.astype(np.float64) - go).max()))
                L.eng_step_end(e)
            elif ev[0] == "snap":
                a, b = C.c_int(), C.c_int()
                L.eng_snapshot(e, C.byref(a), C.byref(b))
                assert a.value == b.value == 0, (a.value, b.value)
            elif ev[0] == "sink":
                L.eng_set_sink(e, ev[1])
            elif ev[0] == "save":
                saved[ev[1]] = L.eng_prefix_save(e)
                assert saved[ev[1]]
            elif ev[0] == "restore":
                a, b = C.c_int(), C.c_int()
                L.eng_prefix_restore(e, saved[ev[1]], C.byref(a), C.byref(b))
                assert a.value == b.value == 0, (a.value, b.value)
            elif ev[0] == "rewind":
                L.eng_rewind(e)
            elif ev[0] == "reset":
                L.eng_reset(e)
            pc, sc, pg, sg = state(L, e)
            assert (pc, sc) == (pg, sg), (ev, pc, sc, pg, sg)
    finally:
        for p in saved.values():
            L.eng_prefix_free(p)
        L.eng_close(e)
    return worst


def test_engine_binding_gqa_ring_prefixes():
    """The engine's shape (12 q / 2 kv heads, qk 48, v 64), 2 layers, a
    128-slot window whose ring wraps: 10 sinks set at position 10, a
    20-token prefix saved and restored twice, a second snapshot and a rewind
    to it, reset; gated and ungated tokens."""
    print("[gpu-case] engine binding gqa", flush=True)
    script = ([("tok", True)] * 10 + [("sink", 10)] + [("tok", True)] * 10 + [("snap",), ("save", 0)] +
              [("tok", i % 3 != 0) for i in range(150)] + [("restore", 0)] + [("tok", True)] * 30 +
              [("snap",)] + [("tok", True)] * 10 + [("rewind",)] + [("tok", False)] * 12 +
              [("restore", 0)] + [("tok", True)] * 130 + [("reset",)] + [("tok", True)] * 5)
    worst = run((2, 12, 2, 48, 64, 128), script, seed=31, scale=2.0)
    print("[gpu-case] engine binding gqa worst", worst, flush=True)
    assert worst <= TOL, worst


@pytest.mark.parametrize("odd", [False, True], ids=["12x2_48_64", "10x2_36_20"])
def test_engine_binding_whole_attention(odd):
    """The engine's attention(m, li, xin, out) itself against its one-call
    GPU binding: 12 q / 2 kv heads, qk 48, v 64 (and 10 q / 2 kv heads, qk
    36, v 20, whose front has run-time dims), d_model 256, 3 taps, 2-bit CQ
    projections registered from the engine's nd_layer records, 2 layers;
    snapshot, prefix save, rewind, reset and restore."""
    print("[gpu-case] engine binding whole attention", "odd" if odd else "", flush=True)
    sys.path.insert(0, HERE)
    from detgen import Stream, make_block_weights
    from test_oracle_block import BLOCK, BLOCK_ODD, front_weights
    if odd:
        BLOCK = BLOCK_ODD
    nl, nh, nkv, qk, vd, W = BLOCK["geom"]
    fw = front_weights(BLOCK["seed"] + 1, nl, nh, nkv, qk, vd, BLOCK["taps"])
    bw = make_block_weights(BLOCK["seed"] + 2, nl, nh, nkv, qk, vd, BLOCK["d_model"])
    worst = run(BLOCK["geom"], BLOCK["script"], seed=33,
                block=(BLOCK["d_model"], BLOCK["taps"], BLOCK["theta"], fw, bw, Stream(BLOCK["seed"])))
    print("[gpu-case] engine binding whole attention worst", worst, flush=True)
    assert worst <= TOL, worst


def test_engine_binding_mha():
    """8 heads x 64 (rep 1), one layer, 128-slot window, 200 tokens (the
    ring wraps), gated then ungated."""
    print("[gpu-case] engine binding mha", flush=True)
    script = [("tok", True)] * 40 + [("tok", False)] * 160
    worst = run((1, 8, 8, 64, 64, 128), script, seed=32)
    print("[gpu-case] engine binding mha worst", worst, flush=True)
    assert worst <= TOL, worst
