"""ctypes bindings for the CPU oracle (oracle/_build/libndoracle.so) and the
reference harness (oracle/_ref/libndref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, the package smoke check and
bench.py's cpu_baseline leg, never by the product library.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "_build", "libndoracle.so")
REF_SO = os.path.join(HERE, "_ref", "libndref.so")

KV_INT8, KV_F16 = 0, 1

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")


class KVView(C.Structure):
    _fields_ = [("nh", C.c_uint32), ("nkv", C.c_uint32), ("qk_hd", C.c_uint32),
                ("v_hd", C.c_uint32), ("window", C.c_uint32), ("n_sink", C.c_uint32),
                ("pos", C.c_uint32), ("kv_dtype", C.c_int),
                ("k", C.c_void_p), ("v", C.c_void_p),
                ("k_scale", C.c_void_p), ("v_scale", C.c_void_p)]


class Session(C.Structure):
    _fields_ = [("n_layers", C.c_uint32), ("nh", C.c_uint32), ("nkv", C.c_uint32),
                ("qk_hd", C.c_uint32), ("v_hd", C.c_uint32), ("window", C.c_uint32),
                ("kv_dtype", C.c_int), ("pos", C.c_uint32), ("n_sink", C.c_uint32),
                ("has_snap", C.c_int), ("snap_pos", C.c_uint32),
                ("k_cache", C.c_void_p), ("v_cache", C.c_void_p),
                ("k_scale", C.c_void_p), ("v_scale", C.c_void_p),
                ("taps", C.c_uint32),
                ("q_hist", C.c_void_p), ("k_hist", C.c_void_p), ("v_hist", C.c_void_p),
                ("snap_q_hist", C.c_void_p), ("snap_k_hist", C.c_void_p), ("snap_v_hist", C.c_void_p),
                ("rope_inv", C.c_void_p)]


class FrontW(C.Structure):
    _fields_ = [("tap_q", C.c_void_p), ("tap_k", C.c_void_p), ("tap_v", C.c_void_p),
                ("norm_q", C.c_void_p), ("norm_k", C.c_void_p)]


class BlockW(C.Structure):
    _fields_ = [("blob", C.c_void_p * 5), ("cb2", C.c_void_p), ("d_model", C.c_uint32),
                ("group", C.c_uint32)]


class BatchF16(C.Structure):
    _fields_ = [("nseq", C.c_uint32), ("nh", C.c_uint32), ("nkv", C.c_uint32),
                ("qk_hd", C.c_uint32), ("v_hd", C.c_uint32),
                ("len", C.c_void_p), ("koff", C.c_void_p), ("voff", C.c_void_p),
                ("kbase", C.c_void_p), ("vbase", C.c_void_p),
                ("q", C.c_void_p), ("k_new", C.c_void_p), ("v_new", C.c_void_p),
                ("gate", C.c_void_p), ("out", C.c_void_p)]


def _ptr(a):
    return None if a is None else a.ctypes.data


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError("oracle not built: run `make -C oracle oracle`")
        L = C.CDLL(ORACLE_SO)
        L.ndo_kv_slot.restype = C.c_uint32
        L.ndo_kv_slot.argtypes = [C.c_uint32] * 3
        L.ndo_clamp_sink.restype = C.c_uint32
        L.ndo_clamp_sink.argtypes = [C.c_uint32] * 2
        L.ndo_expf.restype = C.c_float
        L.ndo_expf.argtypes = [C.c_float]
        L.ndo_sigmoid.restype = C.c_float
        L.ndo_sigmoid.argtypes = [C.c_float]
        L.ndo_f32_to_f16.restype = C.c_uint16
        L.ndo_f32_to_f16.argtypes = [C.c_float]
        L.ndo_f16_to_f32.restype = C.c_float
        L.ndo_f16_to_f32.argtypes = [C.c_uint16]
        L.ndo_kv_quant_row.restype = C.c_float
        L.ndo_kv_quant_row.argtypes = [_f32p, C.c_uint32, _i8p]
        L.ndo_kv_store_int8.restype = None
        L.ndo_kv_store_int8.argtypes = [_i8p, _f32p, C.c_uint32, C.c_float]
        L.ndo_attend.argtypes = [C.POINTER(KVView), C.c_void_p, C.c_void_p, C.c_void_p]
        L.ndo_attend_runs.argtypes = [C.POINTER(KVView), C.c_void_p, C.c_void_p, C.c_uint32,
                                      C.c_void_p, C.c_void_p, C.c_void_p]
        L.ndo_attend_f64.argtypes = [C.POINTER(KVView), C.c_void_p, C.c_uint32, C.c_void_p,
                                     C.c_void_p, C.c_void_p]
        L.ndo_session_init.restype = C.c_int
        L.ndo_session_init.argtypes = [C.POINTER(Session)] + [C.c_uint32] * 6 + [C.c_int]
        for n in ("ndo_session_free", "ndo_reset", "ndo_rewind", "ndo_step_end"):
            getattr(L, n).argtypes = [C.POINTER(Session)]
            getattr(L, n).restype = None
        L.ndo_set_sink.argtypes = [C.POINTER(Session), C.c_uint32]
        L.ndo_snapshot.argtypes = [C.POINTER(Session)]
        L.ndo_snapshot.restype = C.c_int
        L.ndo_prefix_save.argtypes = [C.POINTER(Session)]
        L.ndo_prefix_save.restype = C.c_void_p
        L.ndo_prefix_restore.argtypes = [C.POINTER(Session), C.c_void_p]
        L.ndo_prefix_restore.restype = C.c_int
        L.ndo_prefix_free.argtypes = [C.c_void_p]
        L.ndo_attention.argtypes = [C.POINTER(Session), C.c_uint32] + [C.c_void_p] * 5
        L.ndo_kv_store.argtypes = [C.POINTER(Session), C.c_uint32, C.c_void_p, C.c_void_p]
        L.ndo_attend_session.argtypes = [C.POINTER(Session), C.c_uint32] + [C.c_void_p] * 3
        L.ndo_prefill_tokens.argtypes = [C.POINTER(Session), C.c_uint32, C.c_uint32] + [C.c_void_p] * 5
        L.ndo_decode_batch_f16.argtypes = [C.POINTER(BatchF16), C.c_int]
        L.ndo_decode_batch_f16.restype = C.c_int
        L.ndo_rope_inv.argtypes = [C.c_float, C.c_uint32, C.c_void_p]
        L.ndo_rope_row.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p]
        L.ndo_tap_conv.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32]
        L.ndo_zcrms_heads.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p,
                                      C.c_void_p]
        L.ndo_session_front.argtypes = [C.POINTER(Session), C.c_uint32, C.c_float]
        L.ndo_session_front.restype = C.c_int
        L.ndo_front.argtypes = [C.POINTER(Session), C.c_uint32, C.POINTER(FrontW)] + [C.c_void_p] * 3
        L.ndo_attention_block.restype = C.c_int
        L.ndo_attention_block.argtypes = [C.POINTER(Session), C.c_uint32, C.POINTER(FrontW),
                                          C.POINTER(BlockW), C.c_void_p, C.c_void_p]
        L.ndo_cq_in_pad.restype = C.c_uint32
        L.ndo_cq_in_pad.argtypes = [C.c_uint32, C.c_uint32]
        L.ndo_fwht.argtypes = [C.c_void_p, C.c_uint32]
        L.ndo_cq_prepare.argtypes = [C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p]
        L.ndo_cq_gemv.argtypes = [C.c_uint32] * 4 + [C.c_void_p] * 4
        L.ndo_cq_lut_build.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p]
        L.ndo_cq_gemv_lut2.argtypes = [C.c_uint32] * 3 + [C.c_void_p] * 3
        _lib = L
    return _lib


def have_ref():
    return os.path.exists(REF_SO)


def ref():
    global _ref
    if _ref is None:
        if not have_ref():
            raise RuntimeError("reference harness not built (oracle/_ref/libndref.so)")
        R = C.CDLL(REF_SO)
        R.ref_kv_slot.restype = C.c_uint32
        R.ref_kv_slot.argtypes = [C.c_uint32] * 3
        R.ref_clamp_sink.restype = C.c_uint32
        R.ref_clamp_sink.argtypes = [C.c_uint32] * 2
        R.ref_expf.restype = C.c_float
        R.ref_expf.argtypes = [C.c_float]
        R.ref_sigmoid.restype = C.c_float
        R.ref_sigmoid.argtypes = [C.c_float]
        R.ref_expf_pair.argtypes = [C.c_float, C.c_float, C.POINTER(C.c_float), C.POINTER(C.c_float)]
        R.ref_sigmoid_pair.argtypes = [C.c_float, C.c_float, C.POINTER(C.c_float), C.POINTER(C.c_float)]
        R.ref_kv_store_int8.argtypes = [_i8p, _f32p, C.c_uint32, C.c_float]
        R.ref_session_new.restype = C.c_void_p
        R.ref_session_new.argtypes = [C.c_uint32] * 6
        for n in ("ref_session_free", "ref_reset", "ref_rewind", "ref_step_end", "ref_prefix_free"):
            getattr(R, n).argtypes = [C.c_void_p]
            getattr(R, n).restype = None
        R.ref_set_sink.argtypes = [C.c_void_p, C.c_uint32]
        R.ref_set_pos.argtypes = [C.c_void_p, C.c_uint32]
        R.ref_snapshot.argtypes = [C.c_void_p]
        R.ref_snapshot.restype = C.c_int
        R.ref_prefix_save.argtypes = [C.c_void_p]
        R.ref_prefix_save.restype = C.c_void_p
        R.ref_prefix_restore.argtypes = [C.c_void_p, C.c_void_p]
        R.ref_prefix_restore.restype = C.c_int
        R.ref_pos.argtypes = [C.c_void_p]
        R.ref_pos.restype = C.c_uint32
        R.ref_n_sink.argtypes = [C.c_void_p]
        R.ref_n_sink.restype = C.c_uint32
        R.ref_cache.argtypes = [C.c_void_p] + [C.POINTER(C.c_void_p)] * 4
        R.ref_kv_store.argtypes = [C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p]
        R.ref_attend.argtypes = [C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p]
        R.ref_attention.argtypes = [C.c_void_p, C.c_uint32] + [C.c_void_p] * 5
        R.ref_session_front.argtypes = [C.c_void_p, C.c_uint32, C.c_float]
        R.ref_session_front.restype = C.c_int
        R.ref_front.argtypes = [C.c_void_p, C.c_uint32] + [C.c_void_p] * 8
        R.ref_hist.argtypes = [C.c_void_p, C.c_int] + [C.POINTER(C.c_void_p)] * 3
        R.ref_fwht.argtypes = [C.c_void_p, C.c_uint32]
        R.ref_cq_prepare.argtypes = [C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p]
        R.ref_cq_gemv.argtypes = [C.c_uint32] * 4 + [C.c_void_p] * 4
        R.ref_cq_lut2.argtypes = [C.c_uint32] * 3 + [C.c_void_p] * 5
        R.ref_block_setup.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p]
        R.ref_block_setup.restype = C.c_int
        R.ref_attention_block.argtypes = [C.c_void_p, C.c_uint32] + [C.c_void_p] * 7
        R.ref_attention_rounds.restype = C.c_double
        R.ref_attention_rounds.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32] + [C.c_void_p] * 4 + \
            [C.c_uint32] * 3
        R.ref_pool_start.restype = C.c_int
        R.ref_pool_start.argtypes = [C.c_int]
        R.ref_pool_stop.argtypes = []
        R.ref_prefill_rounds.restype = C.c_double
        R.ref_prefill_rounds.argtypes = [C.c_void_p, C.c_uint32] + [C.c_void_p] * 4
        _ref = R
    return _ref


# ------------------------------------------------------------------ helpers

def f32_to_f16_bits(x):
    """fp32 -> fp16 bit patterns, round to nearest even (numpy's cast is RNE)."""
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


class OracleSession:
    """One engine session's KV state, restated (nd_model.h:132-148)."""

    def __init__(self, n_layers, nh, nkv, qk_hd, v_hd, window, kv_dtype=KV_INT8):
        self.s = Session()
        rc = lib().ndo_session_init(C.byref(self.s), n_layers, nh, nkv, qk_hd, v_hd, window, kv_dtype)
        if rc:
            raise ValueError("ndo_session_init failed: %d" % rc)
        self.geom = (n_layers, nh, nkv, qk_hd, v_hd, window)
        self.kv_dtype = kv_dtype

    def close(self):
        if self.s is not None:
            lib().ndo_session_free(C.byref(self.s))
            self.s = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def pos(self):
        return self.s.pos

    @property
    def n_sink(self):
        return self.s.n_sink

    def reset(self):
        lib().ndo_reset(C.byref(self.s))

    def set_sink(self, n):
        lib().ndo_set_sink(C.byref(self.s), n)

    def snapshot(self):
        return lib().ndo_snapshot(C.byref(self.s))

    def rewind(self):
        lib().ndo_rewind(C.byref(self.s))

    def prefix_save(self):
        return lib().ndo_prefix_save(C.byref(self.s))

    def prefix_restore(self, p):
        return lib().ndo_prefix_restore(C.byref(self.s), p)

    def step_end(self):
        lib().ndo_step_end(C.byref(self.s))

    def attention(self, li, q, k, v, gate=None):
        L, nh, nkv, qk, vd, W = self.geom
        out = np.zeros(nh * vd, np.float32)
        q = np.ascontiguousarray(q, np.float32)
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        g = None if gate is None else np.ascontiguousarray(gate, np.float32)
        lib().ndo_attention(C.byref(self.s), li, _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(out))
        return out

    def kv_store(self, li, k, v):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        lib().ndo_kv_store(C.byref(self.s), li, _ptr(k), _ptr(v))

    def attend(self, li, q, gate=None):
        L, nh, nkv, qk, vd, W = self.geom
        out = np.zeros(nh * vd, np.float32)
        q = np.ascontiguousarray(q, np.float32)
        g = None if gate is None else np.ascontiguousarray(gate, np.float32)
        lib().ndo_attend_session(C.byref(self.s), li, _ptr(q), _ptr(g), _ptr(out))
        return out

    def front_init(self, taps, rope_theta):
        rc = lib().ndo_session_front(C.byref(self.s), taps, rope_theta)
        if rc:
            raise ValueError("ndo_session_front failed: %d" % rc)

    def front(self, li, w, q, k, v):
        """The attention front at the current position: returns (q, k, v)
        after tap convolution, head norm and RoPE; w = FrontWeights."""
        q = np.array(q, np.float32)
        k = np.array(k, np.float32)
        v = np.array(v, np.float32)
        lib().ndo_front(C.byref(self.s), li, C.byref(w.struct(li)), _ptr(q), _ptr(k), _ptr(v))
        return q, k, v

    def hist(self, snap=False):
        """(q, k, v) tap histories [layer][tap][dim] (copies)."""
        L, nh, nkv, qk, vd, W = self.geom
        T = self.s.taps
        out = []
        for ptr, dim in ((self.s.snap_q_hist if snap else self.s.q_hist, nh * qk),
                         (self.s.snap_k_hist if snap else self.s.k_hist, nkv * qk),
                         (self.s.snap_v_hist if snap else self.s.v_hist, nkv * vd)):
            a = np.ctypeslib.as_array((C.c_float * (L * T * dim)).from_address(ptr))
            out.append(a.reshape(L, T, dim).copy())
        return tuple(out)

    def cache(self):
        """(k, v, k_scale, v_scale) numpy views [layer][window][nkv][hd]."""
        L, nh, nkv, qk, vd, W = self.geom
        dt = np.int8 if self.kv_dtype == KV_INT8 else np.uint16
        es = np.dtype(dt).itemsize
        k = np.ctypeslib.as_array((C.c_byte * (L * W * nkv * qk * es)).from_address(self.s.k_cache))
        v = np.ctypeslib.as_array((C.c_byte * (L * W * nkv * vd * es)).from_address(self.s.v_cache))
        ks = np.ctypeslib.as_array((C.c_float * (L * W * nkv)).from_address(self.s.k_scale))
        vs = np.ctypeslib.as_array((C.c_float * (L * W * nkv)).from_address(self.s.v_scale))
        return (k.view(dt).reshape(L, W, nkv, qk), v.view(dt).reshape(L, W, nkv, vd),
                ks.reshape(L, W, nkv), vs.reshape(L, W, nkv))


class RefSession:
    """The reference engine's own KV/attention code on one hand-built nd_model."""

    def __init__(self, n_layers, nh, nkv, qk_hd, v_hd, window):
        self.m = ref().ref_session_new(n_layers, nh, nkv, qk_hd, v_hd, window)
        self.geom = (n_layers, nh, nkv, qk_hd, v_hd, window)

    def close(self):
        if self.m:
            ref().ref_session_free(self.m)
            self.m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def pos(self):
        return ref().ref_pos(self.m)

    @property
    def n_sink(self):
        return ref().ref_n_sink(self.m)

    def reset(self):
        ref().ref_reset(self.m)

    def set_sink(self, n):
        ref().ref_set_sink(self.m, n)

    def snapshot(self):
        return ref().ref_snapshot(self.m)

    def rewind(self):
        ref().ref_rewind(self.m)

    def prefix_save(self):
        return ref().ref_prefix_save(self.m)

    def prefix_restore(self, p):
        return ref().ref_prefix_restore(self.m, p)

    def step_end(self):
        ref().ref_step_end(self.m)

    def attention(self, li, q, k, v, gate=None):
        L, nh, nkv, qk, vd, W = self.geom
        out = np.zeros(nh * vd, np.float32)
        q = np.ascontiguousarray(q, np.float32)
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        g = None if gate is None else np.ascontiguousarray(gate, np.float32)
        ref().ref_attention(self.m, li, _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(out))
        return out

    def front_init(self, taps, rope_theta):
        if ref().ref_session_front(self.m, taps, rope_theta):
            raise ValueError("ref_session_front failed")
        self.taps = taps

    def front(self, li, w, q, k, v):
        q = np.array(q, np.float32)
        k = np.array(k, np.float32)
        v = np.array(v, np.float32)
        a = w.arrays(li)
        ref().ref_front(self.m, li, *(_ptr(x) for x in a), _ptr(q), _ptr(k), _ptr(v))
        return q, k, v

    def hist(self, snap=False):
        L, nh, nkv, qk, vd, W = self.geom
        T = self.taps
        ptrs = [C.c_void_p() for _ in range(3)]
        ref().ref_hist(self.m, 1 if snap else 0, *(C.byref(p) for p in ptrs))
        out = []
        for p, dim in zip(ptrs, (nh * qk, nkv * qk, nkv * vd)):
            if not p.value:     # no snapshot taken yet: the engine has not allocated it
                out.append(np.zeros((L, T, dim), np.float32))
                continue
            a = np.ctypeslib.as_array((C.c_float * (L * T * dim)).from_address(p.value))
            out.append(a.reshape(L, T, dim).copy())
        return tuple(out)

    def cache(self):
        L, nh, nkv, qk, vd, W = self.geom
        k, v, ks, vs = C.c_void_p(), C.c_void_p(), C.c_void_p(), C.c_void_p()
        ref().ref_cache(self.m, C.byref(k), C.byref(v), C.byref(ks), C.byref(vs))
        kk = np.ctypeslib.as_array((C.c_int8 * (L * W * nkv * qk)).from_address(k.value))
        vv = np.ctypeslib.as_array((C.c_int8 * (L * W * nkv * vd)).from_address(v.value))
        kss = np.ctypeslib.as_array((C.c_float * (L * W * nkv)).from_address(ks.value))
        vss = np.ctypeslib.as_array((C.c_float * (L * W * nkv)).from_address(vs.value))
        return (kk.reshape(L, W, nkv, qk), vv.reshape(L, W, nkv, vd),
                kss.reshape(L, W, nkv), vss.reshape(L, W, nkv))


def kv_view(k, v, k_scale, v_scale, nh, window, n_sink, pos, kv_dtype):
    """A KVView over numpy arrays [window][nkv][hd] (kept alive by the caller)."""
    kv = KVView()
    kv.nh = nh
    kv.nkv = k.shape[1]
    kv.qk_hd = k.shape[2]
    kv.v_hd = v.shape[2]
    kv.window = window
    kv.n_sink = n_sink
    kv.pos = pos
    kv.kv_dtype = kv_dtype
    kv.k = k.ctypes.data
    kv.v = v.ctypes.data
    kv.k_scale = None if k_scale is None else k_scale.ctypes.data
    kv.v_scale = None if v_scale is None else v_scale.ctypes.data
    return kv


def attend_view(kv, q, gate=None):
    out = np.zeros(kv.nh * kv.v_hd, np.float32)
    q = np.ascontiguousarray(q, np.float32)
    g = None if gate is None else np.ascontiguousarray(gate, np.float32)
    lib().ndo_attend(C.byref(kv), _ptr(q), _ptr(g), _ptr(out))
    return out


def attend_runs(kv, slots, run_len, q, gate=None):
    out = np.zeros(kv.nh * kv.v_hd, np.float32)
    slots = np.ascontiguousarray(slots, np.uint32)
    run_len = np.ascontiguousarray(run_len, np.uint32)
    q = np.ascontiguousarray(q, np.float32)
    g = None if gate is None else np.ascontiguousarray(gate, np.float32)
    lib().ndo_attend_runs(C.byref(kv), _ptr(slots), _ptr(run_len), len(run_len), _ptr(q), _ptr(g), _ptr(out))
    return out


def attend_f64(kv, slots, q, gate=None):
    out = np.zeros(kv.nh * kv.v_hd, np.float64)
    slots = np.ascontiguousarray(slots, np.uint32)
    q = np.ascontiguousarray(q, np.float32)
    g = None if gate is None else np.ascontiguousarray(gate, np.float32)
    lib().ndo_attend_f64(C.byref(kv), _ptr(slots), len(slots), _ptr(q), _ptr(g), _ptr(out))
    return out


def decode_batch_f16(nh, nkv, qk_hd, v_hd, lens, kbase, vbase, koff, voff, q, k_new, v_new,
                     gate, out, nthreads):
    b = BatchF16()
    b.nseq = len(lens)
    b.nh, b.nkv, b.qk_hd, b.v_hd = nh, nkv, qk_hd, v_hd
    keep = [np.ascontiguousarray(lens, np.uint32), np.ascontiguousarray(koff, np.uint64),
            np.ascontiguousarray(voff, np.uint64)]
    b.len, b.koff, b.voff = (a.ctypes.data for a in keep)
    b.kbase, b.vbase = kbase.ctypes.data, vbase.ctypes.data
    b.q, b.k_new, b.v_new = q.ctypes.data, k_new.ctypes.data, v_new.ctypes.data
    b.gate = None if gate is None else gate.ctypes.data
    b.out = out.ctypes.data
    rc = lib().ndo_decode_batch_f16(C.byref(b), nthreads)
    del keep
    return rc


# ------------------------------------------------------------ attention front

class FrontWeights:
    """Per-layer front weights: tap_q/tap_k/tap_v [L][taps][dim] and
    norm_q/norm_k [L][qk_hd] (float32, kept alive here)."""

    def __init__(self, tap_q, tap_k, tap_v, norm_q, norm_k):
        self.tap_q, self.tap_k, self.tap_v, self.norm_q, self.norm_k = (
            np.ascontiguousarray(a, np.float32) for a in (tap_q, tap_k, tap_v, norm_q, norm_k))
        self.taps = self.tap_q.shape[1]

    def arrays(self, li):
        return (self.tap_q[li], self.tap_k[li], self.tap_v[li], self.norm_q[li], self.norm_k[li])

    def struct(self, li):
        w = FrontW()
        w.tap_q, w.tap_k, w.tap_v, w.norm_q, w.norm_k = (a.ctypes.data for a in self.arrays(li))
        return w


def rope_inv(theta, qk_hd):
    inv = np.zeros(qk_hd // 2 + 1, np.float32)
    lib().ndo_rope_inv(theta, qk_hd, _ptr(inv))
    return inv[:qk_hd // 2]


def rope_row(inv, qk_hd, pos):
    inv = np.ascontiguousarray(inv, np.float32)
    cs = np.zeros(qk_hd // 2 + 1, np.float32)
    sn = np.zeros(qk_hd // 2 + 1, np.float32)
    lib().ndo_rope_row(_ptr(inv), qk_hd, pos, _ptr(cs), _ptr(sn))
    return cs[:qk_hd // 2], sn[:qk_hd // 2]


def tap_conv(proj, hist, w, pos):
    """One projection's tap convolution; returns (out, new_hist)."""
    proj = np.array(proj, np.float32)
    hist = np.array(hist, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    taps, dim = hist.shape
    lib().ndo_tap_conv(_ptr(proj), _ptr(hist), _ptr(w), taps, pos, dim)
    return proj, hist


def zcrms_heads(x, s, cs, sn):
    """x [nheads][dim] -> normed + rotated copy."""
    x = np.array(x, np.float32)
    s, cs, sn = (np.ascontiguousarray(a, np.float32) for a in (s, cs, sn))
    lib().ndo_zcrms_heads(_ptr(x), x.shape[0], x.shape[1], _ptr(s), _ptr(cs), _ptr(sn))
    return x


# ----------------------------------------------------------- CQ projections

class CQTensor:
    """A CQ tensor as the archive stores it: blob = packed rows
    [out][in_pad*bits/8] then fp16 norms [out][in_pad/group] (little-endian);
    codebook = the archive's 28 floats cb2 | cb3 | cb4."""

    def __init__(self, out, inp, group, bits, blob, codebook):
        self.out, self.inp, self.group, self.bits = out, inp, group, bits
        self.blob = np.ascontiguousarray(blob, np.uint8)
        self.codebook = np.ascontiguousarray(codebook, np.float32)
        self.in_pad = (inp + group - 1) // group * group
        self.rowbytes = self.in_pad * bits // 8
        assert self.blob.size == out * self.rowbytes + out * (self.in_pad // group) * 2

    def cb(self):
        off = {2: 0, 3: 4, 4: 12}[self.bits]
        return self.codebook[off:off + (1 << self.bits)]

    def codes(self):
        """Index matrix [out][in_pad] decoded from the LSB-first bitstream."""
        rows = self.blob[: self.out * self.rowbytes].reshape(self.out, self.rowbytes)
        bitsarr = np.unpackbits(rows, axis=1, bitorder="little").reshape(self.out, self.in_pad, self.bits)
        return (bitsarr * (1 << np.arange(self.bits))).sum(axis=2)

    def norms(self):
        nb = self.blob[self.out * self.rowbytes:]
        return nb.view(np.float16).astype(np.float32).reshape(self.out, self.in_pad // self.group)


def cq_prepare(t, x):
    x = np.ascontiguousarray(x, np.float32)
    xh = np.zeros(t.in_pad, np.float32)
    lib().ndo_cq_prepare(t.inp, t.group, _ptr(x), _ptr(xh))
    return xh


def cq_gemv(t, xh):
    xh = np.ascontiguousarray(xh, np.float32)
    y = np.zeros(t.out, np.float32)
    cb = np.ascontiguousarray(t.cb())
    lib().ndo_cq_gemv(t.out, t.inp, t.group, t.bits, _ptr(t.blob), _ptr(cb), _ptr(xh), _ptr(y))
    return y


def cq_gemv_lut2(t, xh):
    xh = np.ascontiguousarray(xh, np.float32)
    lut = np.zeros(t.in_pad // 2 * 16, np.float32)
    y = np.zeros(t.out, np.float32)
    cb = np.ascontiguousarray(t.cb())
    lib().ndo_cq_lut_build(_ptr(cb), _ptr(xh), t.in_pad, _ptr(lut))
    lib().ndo_cq_gemv_lut2(t.out, t.inp, t.group, _ptr(t.blob), _ptr(lut), _ptr(y))
    return y


# ----------------------------------------------------- the whole attention block

class BlockWeights:
    """Per layer the five 2-bit CQ blobs (q, k, v, gate, out_proj) and the
    codebook (28 floats, cb2 first)."""

    def __init__(self, blobs, codebook, d_model, group):
        self.blobs = [[np.ascontiguousarray(b, np.uint8) for b in layer] for layer in blobs]
        self.codebook = np.ascontiguousarray(codebook, np.float32)
        self.d_model, self.group = d_model, group

    def struct(self, li):
        w = BlockW()
        for t in range(5):
            w.blob[t] = self.blobs[li][t].ctypes.data
        w.cb2 = self.codebook.ctypes.data
        w.d_model, w.group = self.d_model, self.group
        return w


def _block_oracle(self, li, fw, bw, xin):
    out = np.zeros(bw.d_model, np.float32)
    xin = np.ascontiguousarray(xin, np.float32)
    rc = lib().ndo_attention_block(C.byref(self.s), li, C.byref(fw.struct(li)), C.byref(bw.struct(li)),
                                   _ptr(xin), _ptr(out))
    if rc:
        raise ValueError("ndo_attention_block: %d" % rc)
    return out


OracleSession.attention_block = _block_oracle


def _block_setup_ref(self, bw):
    flat = [b for layer in bw.blobs for b in layer]
    arr = (C.c_void_p * len(flat))(*[b.ctypes.data for b in flat])
    self._bw = bw
    if ref().ref_block_setup(self.m, bw.d_model, bw.group, arr, bw.codebook.ctypes.data):
        raise ValueError("ref_block_setup failed")


def _block_ref(self, li, fw, bw, xin):
    out = np.zeros(bw.d_model, np.float32)
    xin = np.ascontiguousarray(xin, np.float32)
    ref().ref_attention_block(self.m, li, *(_ptr(x) for x in fw.arrays(li)), _ptr(xin), _ptr(out))
    return out


RefSession.block_setup = _block_setup_ref
RefSession.attention_block = _block_ref
