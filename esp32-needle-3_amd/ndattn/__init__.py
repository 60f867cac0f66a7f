"""Python (ctypes) view of libndattn's C ABI (include/nda.h) and of the C
engine shim libndhost (include/nd_attn_gpu.h).

The product is the C ABI; this module is the binding the tests and bench.py
drive it through. There is no fallback: if the HIP library is not built, or no
GPU is present, every compute call raises.
"""
import ctypes as C
import os

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# The in-tree build is the only library this module loads.
LIB_PATH = os.path.join(PKG_DIR, "libndattn.so")
HOST_LIB_PATH = os.path.join(PKG_DIR, "libndhost.so")
PROBE_LIB_PATH = os.path.join(PKG_DIR, "libndprobe.so")

NDA_OK = 0
ERRORS = {-1: "NDA_ERR_ARG", -2: "NDA_ERR_NOMEM", -3: "NDA_ERR_HIP", -4: "NDA_ERR_RANGE",
          -5: "NDA_ERR_STATE", -6: "NDA_ERR_UNSUPPORTED", -7: "NDA_ERR_NODEV"}
KV_INT8, KV_F16 = 0, 1
FLAG_PREFILL_VALU, FLAG_DECODE_VALU = 1, 2   # nda_config.flags (include/nda.h)
K_APPEND, K_DECODE, K_COMBINE, K_PREFILL, K_FRONT, K_PROJ = 0, 1, 2, 3, 4, 5
K_COUNT = 6
FLAG_PREFILL_VALU = 1

# Every symbol include/nda.h declares (checked by the CPU test suite).
ABI_SYMBOLS = [
    "nda_create", "nda_destroy", "nda_last_error", "nda_device_bytes",
    "nda_seq_reset", "nda_seq_set_sink", "nda_seq_state", "nda_seq_set_pos",
    "nda_seq_reserve", "nda_advance",
    "nda_prefix_build", "nda_seq_attach", "nda_seq_rewind", "nda_prefix_free",
    "nda_kv_append", "nda_decode", "nda_decode_noalloc", "nda_step", "nda_prefill", "nda_sync",
    "nda_kv_read", "nda_kv_write", "nda_kv_fill_normal",
    "nda_set_allocator", "nda_dev_alloc", "nda_dev_free", "nda_h2d", "nda_d2h", "nda_d2d", "nda_memset", "nda_fill_normal",
    "nda_host_alloc", "nda_host_free", "nda_h2d_async", "nda_d2h_async",
    "nda_stream_create", "nda_stream_destroy", "nda_device_sync", "nda_device_info",
    "nda_prof_enable", "nda_prof_read",
    "nda_front_init", "nda_front_weights", "nda_front", "nda_attention", "nda_front_hist",
    "nda_cq_create", "nda_cq_destroy", "nda_cq_in_pad", "nda_cq_prepare", "nda_cq_gemm", "nda_cq_gemm_many",
    "nda_cq_split_bytes", "nda_cq_prepare_split", "nda_cq_gemm_split", "nda_cq_gemm_split_many",
    "nda_cq_gemv_lut2",
    "nda_event_create", "nda_event_destroy", "nda_event_record", "nda_event_elapsed",
    "nda_block_weights", "nda_attention_block", "nda_prefill_block",
]
HOST_SYMBOLS = [
    "nd_gpu_open", "nd_gpu_close", "nd_gpu_reset", "nd_gpu_set_sink", "nd_gpu_snapshot",
    "nd_gpu_rewind", "nd_gpu_prefix_save", "nd_gpu_prefix_restore", "nd_gpu_prefix_free",
    "nd_gpu_attention", "nd_gpu_step_end", "nd_gpu_pos", "nd_gpu_n_sink", "nd_gpu_ctx",
    "nd_gpu_front_init", "nd_gpu_front_weights", "nd_gpu_attention_raw",
    "nd_gpu_block_weights", "nd_gpu_attention_block",
]
PROBE_SYMBOLS = ["ndp_run"]
PROBE_MFMA_F16, PROBE_VALU_EXP, PROBE_VALU_FMA = 0, 1, 2   # include/ndp.h


class NdaError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("%s (%d): %s" % (ERRORS.get(code, "?"), code, msg))
        self.code = code


class Config(C.Structure):
    _fields_ = [("n_layers", C.c_uint32), ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32),
                ("qk_head_dim", C.c_uint32), ("v_head_dim", C.c_uint32), ("window", C.c_uint32),
                ("page_size", C.c_uint32), ("kv_dtype", C.c_uint32), ("max_seqs", C.c_uint32),
                ("max_prefixes", C.c_uint32), ("max_pages", C.c_uint64),
                ("split_chunk", C.c_uint32), ("flags", C.c_uint32)]


class FrontConfig(C.Structure):
    _fields_ = [("taps", C.c_uint32), ("rope_theta", C.c_float), ("max_pos", C.c_uint32)]


_lib = None
_host = None
vp, u32, u64, i32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int32


def lib():
    """Load libndattn.so (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("libndattn.so not built: run `make -C esp32-needle-3_amd`")
        L = C.CDLL(LIB_PATH)
        sig = {
            "nda_create": (C.c_int, [C.POINTER(Config), C.POINTER(vp)]),
            "nda_destroy": (None, [vp]),
            "nda_last_error": (C.c_char_p, [vp]),
            "nda_device_bytes": (u64, [vp]),
            "nda_seq_reset": (C.c_int, [vp, u32]),
            "nda_seq_set_sink": (C.c_int, [vp, u32, u32]),
            "nda_seq_state": (C.c_int, [vp, u32, C.POINTER(u32), C.POINTER(u32), C.POINTER(i32)]),
            "nda_seq_set_pos": (C.c_int, [vp, u32, u32]),
            "nda_seq_reserve": (C.c_int, [vp, u32, u32]),
            "nda_advance": (C.c_int, [vp, u32, vp, u32, vp]),
            "nda_prefix_build": (C.c_int, [vp, u32, C.POINTER(i32), vp]),
            "nda_seq_attach": (C.c_int, [vp, u32, i32, vp]),
            "nda_seq_rewind": (C.c_int, [vp, u32]),
            "nda_prefix_free": (C.c_int, [vp, i32]),
            "nda_kv_append": (C.c_int, [vp, u32, u32, vp, vp, vp, vp]),
            "nda_decode": (C.c_int, [vp, u32, u32, vp, vp, vp, vp, vp]),
            "nda_decode_noalloc": (C.c_int, [vp, u32, u32, vp, vp, vp, vp, vp]),
            "nda_step": (C.c_int, [vp, u32, u32, vp, vp, vp, vp, vp, vp, vp]),
            "nda_prefill": (C.c_int, [vp, u32, u32, vp, vp, vp, vp, vp, vp, vp, vp]),
            "nda_sync": (C.c_int, [vp, vp]),
            "nda_kv_read": (C.c_int, [vp, u32, u32, u32, u32, vp, vp, vp, vp]),
            "nda_kv_write": (C.c_int, [vp, u32, u32, u32, u32, vp, vp, vp, vp]),
            "nda_kv_fill_normal": (C.c_int, [vp, u32, vp, u64, vp]),
            "nda_set_allocator": (C.c_int, [vp, vp, vp]),
            "nda_dev_alloc": (C.c_int, [C.POINTER(vp), C.c_size_t]),
            "nda_dev_free": (C.c_int, [vp]),
            "nda_h2d": (C.c_int, [vp, vp, C.c_size_t]),
            "nda_d2h": (C.c_int, [vp, vp, C.c_size_t]),
            "nda_memset": (C.c_int, [vp, C.c_int, C.c_size_t]),
            "nda_d2d": (C.c_int, [vp, vp, C.c_size_t, vp]),
            "nda_host_alloc": (C.c_int, [C.POINTER(vp), C.c_size_t]),
            "nda_host_free": (C.c_int, [vp]),
            "nda_h2d_async": (C.c_int, [vp, vp, C.c_size_t, vp]),
            "nda_d2h_async": (C.c_int, [vp, vp, C.c_size_t, vp]),
            "nda_fill_normal": (C.c_int, [vp, u64, C.c_int, u64, C.c_float, vp]),
            "nda_stream_create": (C.c_int, [C.POINTER(vp)]),
            "nda_stream_destroy": (C.c_int, [vp]),
            "nda_device_sync": (C.c_int, []),
            "nda_device_info": (C.c_int, [C.c_char_p, C.c_size_t, C.POINTER(C.c_int)]),
            "nda_prof_enable": (C.c_int, [vp, C.c_int]),
            "nda_prof_read": (C.c_int, [vp, C.POINTER(C.c_double), C.POINTER(u64), C.c_int]),
            "nda_front_init": (C.c_int, [vp, C.POINTER(FrontConfig)]),
            "nda_front_weights": (C.c_int, [vp, u32, vp, vp, vp, vp, vp]),
            "nda_front": (C.c_int, [vp, u32, u32, vp, vp, vp, vp, vp, vp, vp, vp, vp]),
            "nda_attention": (C.c_int, [vp, u32, u32, vp, vp, vp, vp, vp, vp, vp]),
            "nda_front_hist": (C.c_int, [vp, u32, C.c_int, vp, vp]),
            "nda_cq_create": (C.c_int, [u32, u32, u32, u32, vp, vp, C.POINTER(vp)]),
            "nda_cq_destroy": (C.c_int, [vp]),
            "nda_cq_in_pad": (u32, [vp]),
            "nda_cq_prepare": (C.c_int, [vp, u32, vp, vp, vp]),
            "nda_cq_gemm": (C.c_int, [vp, u32, vp, vp, vp]),
            "nda_cq_gemm_many": (C.c_int, [vp, u32, u32, vp, vp, vp]),
            "nda_cq_split_bytes": (C.c_size_t, [vp, u32]),
            "nda_cq_prepare_split": (C.c_int, [vp, u32, vp, vp, vp]),
            "nda_cq_gemm_split": (C.c_int, [vp, u32, vp, vp, vp]),
            "nda_cq_gemm_split_many": (C.c_int, [vp, u32, u32, vp, vp, vp]),
            "nda_cq_gemv_lut2": (C.c_int, [vp, u32, u32, vp, vp, vp]),
            "nda_event_create": (C.c_int, [C.POINTER(vp)]),
            "nda_event_destroy": (C.c_int, [vp]),
            "nda_event_record": (C.c_int, [vp, vp]),
            "nda_event_elapsed": (C.c_int, [vp, vp, C.POINTER(C.c_float)]),
            "nda_block_weights": (C.c_int, [vp, u32, vp, vp, vp, vp, vp]),
            "nda_attention_block": (C.c_int, [vp, u32, u32, vp, vp, vp, vp]),
            "nda_prefill_block": (C.c_int, [vp, u32, u32, vp, vp, vp, vp, vp]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def host_lib():
    global _host
    if _host is None:
        lib()
        if not os.path.exists(HOST_LIB_PATH):
            raise RuntimeError("libndhost.so not built: run `make -C esp32-needle-3_amd`")
        H = C.CDLL(HOST_LIB_PATH)
        H.nd_gpu_open.restype = vp
        H.nd_gpu_open.argtypes = [u32] * 8
        for n in ("nd_gpu_close", "nd_gpu_reset", "nd_gpu_rewind", "nd_gpu_step_end", "nd_gpu_prefix_free"):
            getattr(H, n).restype = None
            getattr(H, n).argtypes = [vp]
        H.nd_gpu_set_sink.restype = None
        H.nd_gpu_set_sink.argtypes = [vp, u32]
        H.nd_gpu_snapshot.restype = C.c_int
        H.nd_gpu_snapshot.argtypes = [vp]
        H.nd_gpu_prefix_save.restype = vp
        H.nd_gpu_prefix_save.argtypes = [vp]
        H.nd_gpu_prefix_restore.restype = C.c_int
        H.nd_gpu_prefix_restore.argtypes = [vp, vp]
        H.nd_gpu_attention.restype = C.c_int
        H.nd_gpu_attention.argtypes = [vp, u32, vp, vp, vp, vp, vp]
        H.nd_gpu_pos.restype = u32
        H.nd_gpu_pos.argtypes = [vp]
        H.nd_gpu_n_sink.restype = u32
        H.nd_gpu_n_sink.argtypes = [vp]
        H.nd_gpu_ctx.restype = vp
        H.nd_gpu_ctx.argtypes = [vp]
        H.nd_gpu_front_init.restype = C.c_int
        H.nd_gpu_front_init.argtypes = [vp, u32, C.c_float, u32]
        H.nd_gpu_front_weights.restype = C.c_int
        H.nd_gpu_front_weights.argtypes = [vp, u32, vp, vp, vp, vp, vp]
        H.nd_gpu_attention_raw.restype = C.c_int
        H.nd_gpu_attention_raw.argtypes = [vp, u32, vp, vp, vp, vp, vp]
        H.nd_gpu_block_weights.restype = C.c_int
        H.nd_gpu_block_weights.argtypes = [vp, u32, vp, vp, vp, vp, vp]
        H.nd_gpu_attention_block.restype = C.c_int
        H.nd_gpu_attention_block.argtypes = [vp, u32, vp, u32, vp]
        _host = H
    return _host


def _check(rc, ctx=None):
    if rc != NDA_OK:
        msg = lib().nda_last_error(ctx).decode() if ctx else ""
        raise NdaError(rc, msg)


def device_info():
    name = C.create_string_buffer(256)
    cus = C.c_int(0)
    _check(lib().nda_device_info(name, 256, C.byref(cus)))
    return name.value.decode(), cus.value


def device_sync():
    _check(lib().nda_device_sync())


class DevBuf:
    """A device allocation owned by this object."""

    def __init__(self, nbytes):
        self.ptr = vp()
        self.nbytes = int(nbytes)
        _check(lib().nda_dev_alloc(C.byref(self.ptr), self.nbytes))

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        if a.nbytes:
            _check(lib().nda_h2d(b.ptr, a.ctypes.data, a.nbytes))
        return b

    def upload(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        _check(lib().nda_h2d(self.ptr, a.ctypes.data, a.nbytes))

    def to_array(self, dtype, shape):
        out = np.empty(shape, dtype)
        if out.nbytes:
            assert out.nbytes <= self.nbytes
            _check(lib().nda_d2h(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def fill_normal(self, n, dtype=0, seed=0, scale=1.0, stream=None):
        _check(lib().nda_fill_normal(self.ptr, n, dtype, seed, scale, stream))

    @property
    def value(self):
        return self.ptr.value

    def free(self):
        if self.ptr and self.ptr.value:
            lib().nda_dev_free(self.ptr)
            self.ptr = vp()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _ids(seq_ids):
    if seq_ids is None:
        return None, None
    a = np.ascontiguousarray(seq_ids, np.uint32)
    return a, a.ctypes.data


def _dp(x):
    """Device pointer of a DevBuf / int / None."""
    if x is None:
        return None
    if isinstance(x, DevBuf):
        return x.value
    return int(x)


class Context:
    """An nda_ctx: a paged KV pool for many sequences."""

    def __init__(self, n_layers, n_heads, n_kv_heads, qk_head_dim, v_head_dim, window,
                 kv_dtype=KV_INT8, max_seqs=1, page_size=16, max_prefixes=16, max_pages=0,
                 split_chunk=0, flags=0):
        cfg = Config(n_layers, n_heads, n_kv_heads, qk_head_dim, v_head_dim, window, page_size,
                     kv_dtype, max_seqs, max_prefixes, max_pages, split_chunk, flags)
        self.h = vp()
        self.owned = True
        _check(lib().nda_create(C.byref(cfg), C.byref(self.h)))
        self.cfg = cfg
        self._taps = 0

    @classmethod
    def borrow(cls, handle, cfg):
        """View of a context owned elsewhere (e.g. by the C shim): never destroyed here."""
        c = cls.__new__(cls)
        c.h = vp(handle)
        c.owned = False
        c.cfg = cfg
        c._taps = 0
        return c

    def close(self):
        if self.h and self.h.value and self.owned:
            lib().nda_destroy(self.h)
        self.h = vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _c(self, rc):
        _check(rc, self.h)

    @property
    def device_bytes(self):
        return lib().nda_device_bytes(self.h)

    def seq_state(self, seq):
        pos, ns, pf = u32(), u32(), i32()
        self._c(lib().nda_seq_state(self.h, seq, C.byref(pos), C.byref(ns), C.byref(pf)))
        return pos.value, ns.value, pf.value

    def seq_reset(self, seq):
        self._c(lib().nda_seq_reset(self.h, seq))

    def seq_set_sink(self, seq, n):
        self._c(lib().nda_seq_set_sink(self.h, seq, n))

    def seq_set_pos(self, seq, pos):
        self._c(lib().nda_seq_set_pos(self.h, seq, pos))

    def seq_reserve(self, seq, n):
        self._c(lib().nda_seq_reserve(self.h, seq, n))

    def advance(self, nseq, seq_ids=None, n=1, stream=None):
        keep, p = _ids(seq_ids)
        self._c(lib().nda_advance(self.h, nseq, p, n, stream))

    def prefix_build(self, seq, stream=None):
        pid = i32()
        self._c(lib().nda_prefix_build(self.h, seq, C.byref(pid), stream))
        return pid.value

    def seq_attach(self, seq, prefix_id, stream=None):
        self._c(lib().nda_seq_attach(self.h, seq, prefix_id, stream))

    def seq_rewind(self, seq):
        self._c(lib().nda_seq_rewind(self.h, seq))

    def prefix_free(self, prefix_id):
        self._c(lib().nda_prefix_free(self.h, prefix_id))

    def kv_append(self, layer, nseq, k, v, seq_ids=None, stream=None):
        keep, p = _ids(seq_ids)
        self._c(lib().nda_kv_append(self.h, layer, nseq, p, _dp(k), _dp(v), stream))

    def decode(self, layer, nseq, q, out, gate=None, seq_ids=None, stream=None):
        keep, p = _ids(seq_ids)
        self._c(lib().nda_decode(self.h, layer, nseq, p, _dp(q), _dp(gate), _dp(out), stream))

    def decode_noalloc(self, layer, nseq, q, out, gate=None, seq_ids=None, stream=None):
        """nda_decode_noalloc: nda_decode with its scratch in the GPU's static array."""
        keep, p = _ids(seq_ids)
        self._c(lib().nda_decode_noalloc(self.h, layer, nseq, p, _dp(q), _dp(gate), _dp(out), stream))

    def step(self, layer, nseq, q, k, v, out, gate=None, seq_ids=None, stream=None):
        keep, p = _ids(seq_ids)
        self._c(lib().nda_step(self.h, layer, nseq, p, _dp(q), _dp(k), _dp(v), _dp(gate), _dp(out),
                               stream))

    def prefill(self, layer, n_tokens, q, k, v, out, gate=None, seq_ids=None, stream=None):
        n = np.ascontiguousarray(n_tokens, np.uint32)
        keep, p = _ids(seq_ids)
        self._c(lib().nda_prefill(self.h, layer, len(n), p, n.ctypes.data, _dp(q), _dp(k), _dp(v),
                                  _dp(gate), _dp(out), stream))

    def sync(self, stream=None):
        self._c(lib().nda_sync(self.h, stream))

    def _kv_shapes(self, count):
        c = self.cfg
        dt = np.int8 if c.kv_dtype == KV_INT8 else np.uint16
        return (dt, (count, c.n_kv_heads, c.qk_head_dim), (count, c.n_kv_heads, c.v_head_dim),
                (count, c.n_kv_heads))

    def kv_read(self, layer, seq, p0, count):
        dt, ks, vs, ss = self._kv_shapes(count)
        k = np.zeros(ks, dt)
        v = np.zeros(vs, dt)
        ksc = np.zeros(ss, np.float32)
        vsc = np.zeros(ss, np.float32)
        self._c(lib().nda_kv_read(self.h, layer, seq, p0, count, k.ctypes.data, v.ctypes.data,
                                  ksc.ctypes.data, vsc.ctypes.data))
        return k, v, ksc, vsc

    def kv_write(self, layer, seq, p0, k, v, k_scale=None, v_scale=None):
        dt, _, _, _ = self._kv_shapes(0)
        k = np.ascontiguousarray(k, dt)
        v = np.ascontiguousarray(v, dt)
        count = k.shape[0]
        ks = None if k_scale is None else np.ascontiguousarray(k_scale, np.float32)
        vs = None if v_scale is None else np.ascontiguousarray(v_scale, np.float32)
        self._c(lib().nda_kv_write(self.h, layer, seq, p0, count, k.ctypes.data, v.ctypes.data,
                                   None if ks is None else ks.ctypes.data,
                                   None if vs is None else vs.ctypes.data))

    def kv_fill_normal(self, nseq, seed, seq_ids=None, stream=None):
        keep, p = _ids(seq_ids)
        self._c(lib().nda_kv_fill_normal(self.h, nseq, p, seed, stream))

    def prof_enable(self, on=True):
        self._c(lib().nda_prof_enable(self.h, 1 if on else 0))

    def front_init(self, taps, rope_theta, max_pos=0):
        fc = FrontConfig(taps, rope_theta, max_pos)
        self._c(lib().nda_front_init(self.h, C.byref(fc)))
        self._taps = taps

    def front_weights(self, layer, tap_q, tap_k, tap_v, norm_q, norm_k):
        """Host arrays: tap_* [taps][dim], norm_* [qk_head_dim]."""
        arrs = [np.ascontiguousarray(a, np.float32) for a in (tap_q, tap_k, tap_v, norm_q, norm_k)]
        self._c(lib().nda_front_weights(self.h, layer, *(a.ctypes.data for a in arrs)))

    def front(self, layer, nseq, q, k, v, q_out, k_out, v_out, n_tokens=None, seq_ids=None, stream=None):
        keep, p = _ids(seq_ids)
        n = None if n_tokens is None else np.ascontiguousarray(n_tokens, np.uint32)
        self._c(lib().nda_front(self.h, layer, nseq, p, None if n is None else n.ctypes.data,
                                _dp(q), _dp(k), _dp(v), _dp(q_out), _dp(k_out), _dp(v_out), stream))

    def attention(self, layer, nseq, q, k, v, out, gate=None, seq_ids=None, stream=None):
        keep, p = _ids(seq_ids)
        self._c(lib().nda_attention(self.h, layer, nseq, p, _dp(q), _dp(k), _dp(v), _dp(gate), _dp(out),
                                    stream))

    def block_weights(self, layer, q, k, v, gate, out_proj):
        """CQ objects for one layer (kept alive by the caller)."""
        self._c(lib().nda_block_weights(self.h, layer, q.h, k.h, v.h, gate.h, out_proj.h))

    def attention_block(self, layer, nseq, x, out, seq_ids=None, stream=None):
        keep, p = _ids(seq_ids)
        self._c(lib().nda_attention_block(self.h, layer, nseq, p, _dp(x), _dp(out), stream))

    def prefill_block(self, layer, nseq, n_tokens, x, out, seq_ids=None, stream=None):
        """x / out [sum(n_tokens)][d_model] device, packed token-major per sequence."""
        keep, p = _ids(seq_ids)
        n = np.ascontiguousarray(n_tokens, np.uint32)
        self._c(lib().nda_prefill_block(self.h, layer, nseq, p, n.ctypes.data, _dp(x), _dp(out), stream))

    def front_hist(self, seq, snap=False, stream=None):
        """One sequence's tap histories [n_layers][taps][dcol] (host copy)."""
        c = self.cfg
        dcol = c.n_heads * c.qk_head_dim + c.n_kv_heads * (c.qk_head_dim + c.v_head_dim)
        out = np.zeros((c.n_layers, self._taps, dcol), np.float32)
        self._c(lib().nda_front_hist(self.h, seq, 1 if snap else 0, out.ctypes.data, stream))
        return out

    def prof_read(self, reset=True):
        ms = (C.c_double * K_COUNT)()
        n = (u64 * K_COUNT)()
        self._c(lib().nda_prof_read(self.h, ms, n, 1 if reset else 0))
        return list(ms), list(n)


class GpuSession:
    """One engine session through the C shim (libndhost: nd_gpu_*)."""

    def __init__(self, n_layers, nh, nkv, qk_hd, v_hd, window, kv_dtype=KV_INT8, max_prefixes=8):
        self.m = host_lib().nd_gpu_open(n_layers, nh, nkv, qk_hd, v_hd, window, kv_dtype, max_prefixes)
        if not self.m:
            raise NdaError(-1, "nd_gpu_open failed")
        self.geom = (n_layers, nh, nkv, qk_hd, v_hd, window)
        self.kv_dtype = kv_dtype
        self.front_on = False
        self.taps = 0

    def context(self):
        """The session's nda_ctx (sequence 0), borrowed."""
        L, nh, nkv, qk, vd, W = self.geom
        c = Context.borrow(host_lib().nd_gpu_ctx(self.m),
                           Config(L, nh, nkv, qk, vd, W, 16, self.kv_dtype, 1, 0, 0, 0, 0))
        c._taps = self.taps
        return c

    def close(self):
        if self.m:
            host_lib().nd_gpu_close(self.m)
            self.m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def pos(self):
        return host_lib().nd_gpu_pos(self.m)

    @property
    def n_sink(self):
        return host_lib().nd_gpu_n_sink(self.m)

    def reset(self):
        host_lib().nd_gpu_reset(self.m)

    def set_sink(self, n):
        host_lib().nd_gpu_set_sink(self.m, n)

    def snapshot(self):
        return host_lib().nd_gpu_snapshot(self.m)

    def rewind(self):
        host_lib().nd_gpu_rewind(self.m)

    def prefix_save(self):
        return host_lib().nd_gpu_prefix_save(self.m)

    def prefix_restore(self, p):
        return host_lib().nd_gpu_prefix_restore(self.m, p)

    def prefix_free(self, p):
        host_lib().nd_gpu_prefix_free(p)

    def step_end(self):
        host_lib().nd_gpu_step_end(self.m)

    def attention(self, li, q, k, v, gate=None):
        L, nh, nkv, qk, vd, W = self.geom
        out = np.zeros(nh * vd, np.float32)
        q = np.ascontiguousarray(q, np.float32)
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        g = None if gate is None else np.ascontiguousarray(gate, np.float32)
        fn = host_lib().nd_gpu_attention_raw if self.front_on else host_lib().nd_gpu_attention
        rc = fn(self.m, li, q.ctypes.data, k.ctypes.data, v.ctypes.data,
                None if g is None else g.ctypes.data, out.ctypes.data)
        _check(rc)
        return out

    def block_weights(self, li, q, k, v, gate, out_proj):
        _check(host_lib().nd_gpu_block_weights(self.m, li, q.h, k.h, v.h, gate.h, out_proj.h))

    def attention_block(self, li, xin):
        xin = np.ascontiguousarray(xin, np.float32)
        out = np.zeros(xin.size, np.float32)
        _check(host_lib().nd_gpu_attention_block(self.m, li, xin.ctypes.data, xin.size, out.ctypes.data))
        return out

    def front_init(self, taps, rope_theta, weights, max_pos=0):
        """Enable the attention front; weights.arrays(li) gives one layer's
        (tap_q, tap_k, tap_v, norm_q, norm_k). attention() then takes raw
        projections."""
        _check(host_lib().nd_gpu_front_init(self.m, taps, rope_theta, max_pos))
        L = self.geom[0]
        self._front_keep = []
        for li in range(L):
            arrs = [np.ascontiguousarray(a, np.float32) for a in weights.arrays(li)]
            self._front_keep.append(arrs)
            _check(host_lib().nd_gpu_front_weights(self.m, li, *(a.ctypes.data for a in arrs)))
        self.front_on = True
        self.taps = taps


class CQ:
    """A CQ tensor on the device (nda_cq): the archive's blob + the codebook
    slice for its width (host arrays)."""

    def __init__(self, out, inp, group, bits, blob, codebook):
        blob = np.ascontiguousarray(blob, np.uint8)
        cb = np.ascontiguousarray(codebook, np.float32)
        self.h = vp()
        _check(lib().nda_cq_create(out, inp, group, bits, blob.ctypes.data, cb.ctypes.data, C.byref(self.h)))
        self.out, self.inp, self.group, self.bits = out, inp, group, bits
        self.in_pad = lib().nda_cq_in_pad(self.h)

    def prepare(self, rows, x, xh, stream=None):
        _check(lib().nda_cq_prepare(self.h, rows, _dp(x), _dp(xh), stream))

    def gemm(self, rows, xh, y, stream=None):
        _check(lib().nda_cq_gemm(self.h, rows, _dp(xh), _dp(y), stream))

    def split_bytes(self, rows):
        return lib().nda_cq_split_bytes(self.h, rows)

    def prepare_split(self, rows, x, xs, stream=None):
        _check(lib().nda_cq_prepare_split(self.h, rows, _dp(x), _dp(xs), stream))

    def gemm_split(self, rows, xs, y, stream=None):
        _check(lib().nda_cq_gemm_split(self.h, rows, _dp(xs), _dp(y), stream))

    def close(self):
        if self.h and self.h.value:
            lib().nda_cq_destroy(self.h)
        self.h = vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def cq_gemm_many(tensors, rows, xh, ys, stream=None):
    """One launch for tensors sharing a prepared activation: ys[i] = W_i . x."""
    n = len(tensors)
    th = (vp * n)(*[t.h for t in tensors])
    yp = (vp * n)(*[_dp(y) for y in ys])
    _check(lib().nda_cq_gemm_many(th, n, rows, _dp(xh), yp, stream))


def cq_gemm_split_many(tensors, rows, xs, ys, stream=None):
    """cq_gemm_many from the split-precision prepared form."""
    n = len(tensors)
    th = (vp * n)(*[t.h for t in tensors])
    yp = (vp * n)(*[_dp(y) for y in ys])
    _check(lib().nda_cq_gemm_split_many(th, n, rows, _dp(xs), yp, stream))


def cq_gemv_lut2(tensors, rows, xh, ys, stream=None):
    """The engine's own 2-bit LUT matvec (bit-identical) for tensors sharing
    a prepared activation (nda_cq_prepare's form): ys[i] = W_i . x."""
    n = len(tensors)
    th = (vp * n)(*[t.h for t in tensors])
    yp = (vp * n)(*[_dp(y) for y in ys])
    _check(lib().nda_cq_gemv_lut2(th, n, rows, _dp(xh), yp, stream))


class ProbeResult(C.Structure):
    _fields_ = [("ms", C.c_double), ("clock_ghz", C.c_double), ("cycles_per_iter", C.c_double),
                ("flops", C.c_double), ("valu_insts", C.c_double), ("waves", C.c_uint32),
                ("cus", C.c_uint32)]


_probe = None


def probe_lib():
    """Load libndprobe.so (include/ndp.h): the device-ceiling probe."""
    global _probe
    if _probe is None:
        if not os.path.exists(PROBE_LIB_PATH):
            raise RuntimeError("libndprobe.so not built: run `make -C esp32-needle-3_amd`")
        P = C.CDLL(PROBE_LIB_PATH)
        P.ndp_run.restype = C.c_int
        P.ndp_run.argtypes = [C.c_int] * 6 + [C.POINTER(ProbeResult)]
        _probe = P
    return _probe


def probe_run(kind, nacc=4, nexp=0, blocks_per_cu=2, waves_per_block=4, iters=100000):
    """One ndp_run launch; returns its ProbeResult fields as a dict."""
    r = ProbeResult()
    rc = probe_lib().ndp_run(kind, nacc, nexp, blocks_per_cu, waves_per_block, iters, C.byref(r))
    if rc != 0:
        raise NdaError(rc, "ndp_run(kind=%d)" % kind)
    return {f: getattr(r, f) for f, _ in ProbeResult._fields_}


class Timer:
    """Two HIP events on a stream: start(), stop(), ms()."""

    def __init__(self):
        self.a, self.b = vp(), vp()
        _check(lib().nda_event_create(C.byref(self.a)))
        _check(lib().nda_event_create(C.byref(self.b)))

    def start(self, stream=None):
        _check(lib().nda_event_record(self.a, stream))

    def stop(self, stream=None):
        _check(lib().nda_event_record(self.b, stream))

    def ms(self):
        f = C.c_float()
        _check(lib().nda_event_elapsed(self.a, self.b, C.byref(f)))
        return f.value
