"""ctypes bindings for the CPU checkers (test infrastructure only).

* ``Oracle``  -- oracle/libmoss_oracle.so, the C restatement (moss_oracle.c).
* ``RefCpu``  -- oracle/_ref/libmossref.so, the reference's own LLM-path sources
  compiled from the reference checkout by oracle/Makefile (present wherever it
  was built; it travels with the tree).
* ``RefDecoder`` -- the reference's audio codec decoder from the same library.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this.
"""
from __future__ import annotations

import ctypes as C
import os
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "libmoss_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libmossref.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(np.frombuffer(a, np.uint8) if isinstance(a, (bytes, bytearray)) else a, dtype=np.uint8)


class SampleParams(C.Structure):
    """mo_sample_params (moss_oracle.h) == SampleParams (csrc/include/moss/sampler.h:8-22)."""
    _fields_ = [("greedy", C.c_int), ("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float),
                ("repetition_penalty", C.c_float), ("end_greedy", C.c_int), ("min_frames", C.c_int),
                ("greedy_frames", C.c_int)]

    @classmethod
    def make(cls, greedy=True, temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0, end_greedy=True,
             min_frames=0, greedy_frames=0):
        return cls(int(greedy), temperature, top_k, top_p, repetition_penalty, int(end_greedy), min_frames,
                   greedy_frames)

    def ints(self):
        return np.array([self.greedy, self.top_k, self.end_greedy, self.min_frames, self.greedy_frames], np.int32)

    def floats(self):
        return np.array([self.temperature, self.top_p, self.repetition_penalty], np.float32)


class Oracle:
    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = self.lib = C.CDLL(path)
        L.mo_half_to_float.restype = C.c_float
        L.mo_half_to_float.argtypes = [C.c_uint16]
        L.mo_float_to_half.restype = C.c_uint16
        L.mo_float_to_half.argtypes = [C.c_float]
        L.mo_float_to_half_rne.restype = C.c_uint16
        L.mo_float_to_half_rne.argtypes = [C.c_float]
        L.mo_dequant_row_q8x4.argtypes = [_u8p, C.c_int, C.c_int, _f32p]
        L.mo_quantize_row_q8.argtypes = [_f32p, C.c_int, _i8p, _u16p, _f32p]
        for n in ("mo_row_dot_a16", "mo_row_dot_a16_scalar"):
            getattr(L, n).restype = C.c_float
            getattr(L, n).argtypes = [_u8p, C.c_int, C.c_int, _f32p]
        L.mo_row_dot_w8a8.restype = C.c_float
        L.mo_row_dot_w8a8.argtypes = [_u8p, C.c_int, C.c_int, _i8p, _f32p]
        L.mo_gemv_a16.argtypes = [_u8p, C.c_int, C.c_int, _f32p, _f32p]
        L.mo_gemm.argtypes = [_u8p, C.c_int, C.c_int, _f32p, C.c_int, _f32p, C.c_int]
        L.mo_gemm_w8a8_q.argtypes = [_u8p, C.c_int, C.c_int, _i8p, _f32p, C.c_int, _f32p]
        L.mo_gelu_new.restype = C.c_float
        L.mo_gelu_new.argtypes = [C.c_float]
        L.mo_layernorm.argtypes = [_f32p, _f32p, _f32p, _f32p]
        L.mo_rope_tables.argtypes = [C.c_int, _f32p, _f32p]
        L.mo_rope_apply.argtypes = [_f32p, C.c_int, _f32p, _f32p]
        L.mo_attention_core.argtypes = [_f32p, _f32p, C.c_int, C.c_int, _f32p, _f32p, _f32p]
        L.mo_rng_seed.argtypes = [C.c_void_p, C.c_uint64]
        L.mo_rng_next.restype = C.c_uint32
        L.mo_rng_next.argtypes = [C.c_void_p]
        L.mo_sample_token.restype = C.c_int
        L.mo_sample_token.argtypes = [_f32p, C.c_int, C.POINTER(SampleParams), C.c_void_p, C.c_int, C.c_void_p,
                                      C.c_void_p]
        L.mo_model_create.restype = C.c_void_p
        L.mo_model_create.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.c_char_p]
        L.mo_model_destroy.argtypes = [C.c_void_p]
        L.mo_model_set_kv_f16.argtypes = [C.c_void_p, C.c_int]
        L.mo_model_set_decode_a8.argtypes = [C.c_void_p, C.c_int]
        L.mo_model_reset.argtypes = [C.c_void_p]
        L.mo_model_position.restype = C.c_int
        L.mo_model_position.argtypes = [C.c_void_p]
        L.mo_model_hidden.restype = C.POINTER(C.c_float)
        L.mo_model_hidden.argtypes = [C.c_void_p]
        L.mo_model_set_hidden.argtypes = [C.c_void_p, _f32p]
        L.mo_model_kv_import.restype = C.c_int
        L.mo_model_kv_import.argtypes = [C.c_void_p, C.c_int, _f32p, _f32p]
        L.mo_model_kv_export.restype = C.c_int
        L.mo_model_kv_export.argtypes = [C.c_void_p, C.c_int, _f32p, _f32p]
        L.mo_model_embed_row.argtypes = [C.c_void_p, _i32p, _f32p]
        L.mo_model_global_step.argtypes = [C.c_void_p, _i32p]
        L.mo_model_local_reset.argtypes = [C.c_void_p]
        L.mo_model_local_step.argtypes = [C.c_void_p, _f32p, _f32p]
        L.mo_model_audio_logits.argtypes = [C.c_void_p, C.c_int, _f32p, _f32p]
        L.mo_model_assistant_logits.argtypes = [C.c_void_p, _f32p, _f32p]
        L.mo_model_prefill.argtypes = [C.c_void_p, _i32p, C.c_int, C.c_int, C.c_int]
        L.mo_model_generate.restype = C.c_int
        L.mo_model_generate.argtypes = [C.c_void_p, C.c_int, C.POINTER(SampleParams), C.c_uint64, C.c_void_p,
                                        C.c_int, _i32p, C.c_void_p, C.c_void_p]

    # -- scalar pieces
    def half_to_float(self, h):
        return self.lib.mo_half_to_float(int(h))

    def float_to_half(self, f):
        return self.lib.mo_float_to_half(float(f))

    def float_to_half_rne(self, f):
        return self.lib.mo_float_to_half_rne(float(f))

    def dequant_row(self, group, nb, k):
        out = np.empty(nb * 32, np.float32)
        self.lib.mo_dequant_row_q8x4(_u8(group), nb, k, out)
        return out

    def quantize_row(self, x):
        x = _f32(x)
        k = x.size
        q = np.empty(k, np.int8)
        dh = np.empty(k // 32, np.uint16)
        d = np.empty(k // 32, np.float32)
        self.lib.mo_quantize_row_q8(x, k, q, dh, d)
        return q, dh, d

    def gemv(self, w, rows, cols, x):
        y = np.empty(rows, np.float32)
        self.lib.mo_gemv_a16(_u8(w), rows, cols, _f32(x), y)
        return y

    def gemm(self, w, rows, cols, x, a16=True):
        x = _f32(x).reshape(-1, cols)
        y = np.empty((x.shape[0], rows), np.float32)
        self.lib.mo_gemm(_u8(w), rows, cols, x, x.shape[0], y, int(a16))
        return y

    def gemm_w8a8_q(self, w, rows, cols, q, d):
        """W8A8 product on given int8 activations q [m][cols] and block scales d [m][cols/32]."""
        q = np.ascontiguousarray(q, np.int8).reshape(-1, cols)
        d = _f32(d).reshape(q.shape[0], cols // 32)
        y = np.empty((q.shape[0], rows), np.float32)
        self.lib.mo_gemm_w8a8_q(_u8(w), rows, cols, q, d, q.shape[0], y)
        return y

    def row_dot_w8a8(self, group, nb, k, x):
        q, _, d = self.quantize_row(x)
        return self.lib.mo_row_dot_w8a8(_u8(group), nb, k, q, d)

    def layernorm(self, x, w, b):
        out = np.empty(768, np.float32)
        self.lib.mo_layernorm(_f32(x), _f32(w), _f32(b), out)
        return out

    def rope_tables(self, max_pos):
        c = np.empty((max_pos, 384), np.float32)
        s = np.empty((max_pos, 384), np.float32)
        self.lib.mo_rope_tables(max_pos, c, s)
        return c, s

    def rope_apply(self, vec, pos, cos_t, sin_t):
        v = _f32(vec).copy()
        self.lib.mo_rope_apply(v, pos, _f32(cos_t), _f32(sin_t))
        return v

    def attention(self, k_rows, v_rows, q):
        """k_rows, v_rows: [n][768] fp32; q: [768] -> out [768]."""
        k_rows, v_rows = _f32(k_rows), _f32(v_rows)
        n = k_rows.shape[0]
        out = np.empty(768, np.float32)
        scores = np.empty(max(n, 1), np.float32)
        self.lib.mo_attention_core(k_rows, v_rows, 768, n, _f32(q), out, scores)
        return out

    def rng_stream(self, seed, n):
        st = (C.c_uint32 * 4)()
        self.lib.mo_rng_seed(C.byref(st), seed)
        return np.array([self.lib.mo_rng_next(C.byref(st)) for _ in range(n)], np.uint32)

    def sample_token(self, logits, params: SampleParams, prev=None, seed=0, skip=0):
        logits = _f32(logits)
        st = (C.c_uint32 * 4)()
        self.lib.mo_rng_seed(C.byref(st), seed)
        for _ in range(skip):
            self.lib.mo_rng_next(C.byref(st))
        prev_a = np.ascontiguousarray(prev if prev is not None else np.zeros(0), dtype=np.int32)
        scratch = C.create_string_buffer(logits.size * 8)
        return self.lib.mo_sample_token(logits, logits.size, C.byref(params),
                                        prev_a.ctypes.data if prev_a.size else None, prev_a.size, C.byref(st),
                                        scratch)

    def model(self, blob: bytes, max_ctx: int = 768, kv_f16: bool = False, decode_a8: bool = False) -> "OracleModel":
        """decode_a8: decode GEMVs in W8A8 (the reference with MOSS_A16 unset), else W8A16."""
        return OracleModel(self, blob, max_ctx, kv_f16, decode_a8)


class OracleModel:
    def __init__(self, o: Oracle, blob: bytes, max_ctx: int, kv_f16: bool, decode_a8: bool = False):
        self.o, self.lib = o, o.lib
        self._blob = C.create_string_buffer(bytes(blob), len(blob))
        err = C.create_string_buffer(256)
        self.h = self.lib.mo_model_create(C.addressof(self._blob), len(blob), max_ctx, err)
        if not self.h:
            raise RuntimeError(err.value.decode())
        self.lib.mo_model_set_kv_f16(self.h, int(kv_f16))
        self.lib.mo_model_set_decode_a8(self.h, int(decode_a8))

    def __del__(self):
        if getattr(self, "h", None):
            self.lib.mo_model_destroy(self.h)
            self.h = None

    @property
    def position(self):
        return self.lib.mo_model_position(self.h)

    def hidden(self):
        return np.ctypeslib.as_array(self.lib.mo_model_hidden(self.h), (768,)).copy()

    def set_hidden(self, h):
        self.lib.mo_model_set_hidden(self.h, _f32(h))

    def kv_import(self, k, v):
        k, v = _f32(k), _f32(v)
        assert self.lib.mo_model_kv_import(self.h, k.shape[1], k, v) == 0

    def kv_export(self, n_pos):
        k = np.empty((12, n_pos, 768), np.float32)
        v = np.empty((12, n_pos, 768), np.float32)
        assert self.lib.mo_model_kv_export(self.h, n_pos, k, v) == 0
        return k, v

    def embed_row(self, row):
        out = np.empty(768, np.float32)
        self.lib.mo_model_embed_row(self.h, np.ascontiguousarray(row, np.int32), out)
        return out

    def global_step(self, row):
        self.lib.mo_model_global_step(self.h, np.ascontiguousarray(row, np.int32))

    def local_reset(self):
        self.lib.mo_model_local_reset(self.h)

    def local_step(self, x):
        out = np.empty(768, np.float32)
        self.lib.mo_model_local_step(self.h, _f32(x), out)
        return out

    def audio_logits(self, ch, h):
        out = np.empty(1024, np.float32)
        self.lib.mo_model_audio_logits(self.h, ch, _f32(h), out)
        return out

    def assistant_logits(self, h):
        out = np.empty(2, np.float32)
        self.lib.mo_model_assistant_logits(self.h, _f32(h), out)
        return out

    def prefill(self, rows, start=0, a16=False):
        rows = np.ascontiguousarray(rows, np.int32).reshape(-1, 17)
        self.lib.mo_model_prefill(self.h, rows, rows.shape[0], start, int(a16))

    def generate(self, max_frames, params: SampleParams, seed=0, forced=None, logits=False, gate=False):
        out = np.zeros((max_frames, 17), np.int32)
        fa = np.ascontiguousarray(forced, np.int32).reshape(-1, 17) if forced is not None else None
        ld = np.zeros((max_frames, 16, 1024), np.float32) if logits else None
        gd = np.zeros((max_frames, 4), np.float32) if gate else None
        n = self.lib.mo_model_generate(self.h, max_frames, C.byref(params), seed,
                                       fa.ctypes.data if fa is not None else None, 0 if fa is None else fa.shape[0],
                                       out, ld.ctypes.data if ld is not None else None,
                                       gd.ctypes.data if gd is not None else None)
        res = {"rows": out[:n]}
        if logits:
            res["logits"] = ld[:n]
        if gate:
            res["gate"] = gd[:n + 1 if n < max_frames else n]
        return res


class RefCpu:
    """The compiled reference (oracle/_ref/libmossref.so).  MOSS_A16 is fixed per
    process at the first GEMV (csrc/src/gemv.cpp:26-35); this binding sets it to
    ``decode`` on load, so gemv_par runs W8A16 and prefill runs W8A8 exactly as the
    reference release does.  ``act16_suspend`` toggles the decode mode."""

    def __init__(self, path: str = REF_SO, a16_mode: str = "decode"):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle ref` where the reference checkout exists")
        L = self.lib = C.CDLL(path)
        L.ref_set_a16_mode.argtypes = [C.c_char_p]
        L.ref_set_a16_mode(a16_mode.encode())
        L.ref_last_error.restype = C.c_char_p
        L.ref_act16_enabled.restype = C.c_int
        L.ref_act16_suspend.argtypes = [C.c_int]
        L.ref_half_to_float.restype = C.c_float
        L.ref_half_to_float.argtypes = [C.c_uint16]
        L.ref_float_to_half.restype = C.c_uint16
        L.ref_float_to_half.argtypes = [C.c_float]
        L.ref_quantize_row.argtypes = [_f32p, C.c_int, _i8p, _u16p, _f32p]
        L.ref_dequant_row_q8x4.argtypes = [_u8p, C.c_int, C.c_int, _f32p]
        for n in ("ref_row_dot_a16", "ref_row_dot_a16_scalar", "ref_row_dot_w8a8"):
            getattr(L, n).restype = C.c_float
            getattr(L, n).argtypes = [_u8p, C.c_int, C.c_int, _f32p]
        L.ref_pool_create.restype = C.c_void_p
        L.ref_pool_create.argtypes = [C.c_int, C.c_int]
        L.ref_pool_destroy.argtypes = [C.c_void_p]
        L.ref_gemv_par.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
        L.ref_gemv_par_median_us.restype = C.c_double
        L.ref_gemv_par_median_us.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                             C.c_int]
        L.ref_gemm_par.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_void_p]
        L.ref_attention_window.argtypes = [_f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _f32p, _f32p, C.c_int,
                                           C.c_int, _f32p, _f32p, C.c_int]
        L.ref_rng_stream.argtypes = [C.c_uint64, C.c_int, np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")]
        L.ref_sample_token.restype = C.c_int
        L.ref_sample_token.argtypes = [_f32p, C.c_int, _i32p, _f32p, C.c_void_p, C.c_int, C.c_uint64, C.c_int]
        L.ref_model_create.restype = C.c_void_p
        L.ref_model_create.argtypes = [C.c_int]
        L.ref_model_destroy.argtypes = [C.c_void_p]
        L.ref_model_load.restype = C.c_int
        L.ref_model_load.argtypes = [C.c_void_p, C.c_char_p]
        L.ref_model_reset.argtypes = [C.c_void_p]
        L.ref_model_position.restype = C.c_int
        L.ref_model_position.argtypes = [C.c_void_p]
        L.ref_model_hidden.argtypes = [C.c_void_p, _f32p]
        L.ref_model_prefill.argtypes = [C.c_void_p, _i32p, C.c_int, C.c_int]
        for n in ("ref_model_load_state",):
            getattr(L, n).restype = C.c_int
            getattr(L, n).argtypes = [C.c_void_p, C.c_char_p, _i32p, C.c_int, C.c_int]
        for n in ("ref_model_save_state", "ref_model_save_prefix", "ref_model_load_prefix"):
            getattr(L, n).restype = C.c_int
            getattr(L, n).argtypes = [C.c_void_p, C.c_char_p, _i32p, C.c_int]
        L.ref_model_snapshot_prefix.argtypes = [C.c_void_p]
        L.ref_model_restore_prefix.argtypes = [C.c_void_p]
        L.ref_model_set_logits_dump.argtypes = [C.c_void_p, C.c_char_p]
        L.ref_model_set_gate_dump.argtypes = [C.c_void_p, C.c_char_p]
        L.ref_model_generate.restype = C.c_int
        L.ref_model_generate.argtypes = [C.c_void_p, C.c_int, _i32p, _f32p, C.c_uint64, C.c_void_p, C.c_int, _i32p,
                                         C.c_void_p]

    def quantize_row(self, x):
        x = _f32(x)
        k = x.size
        q = np.empty(k, np.int8)
        dh = np.empty(k // 32, np.uint16)
        d = np.empty(k // 32, np.float32)
        self.lib.ref_quantize_row(x, k, q, dh, d)
        return q, dh, d

    def dequant_row(self, group, nb, k):
        out = np.empty(nb * 32, np.float32)
        self.lib.ref_dequant_row_q8x4(_u8(group), nb, k, out)
        return out

    def row_dot_a16(self, group, nb, k, x, scalar=False):
        f = self.lib.ref_row_dot_a16_scalar if scalar else self.lib.ref_row_dot_a16
        return f(_u8(group), nb, k, _f32(x))

    def row_dot_w8a8(self, group, nb, k, x):
        return self.lib.ref_row_dot_w8a8(_u8(group), nb, k, _f32(x))

    def pool(self, threads, k=768):
        return self.lib.ref_pool_create(threads, k)

    def gemv(self, w, rows, cols, x, threads=1, pool=None):
        w, x = _u8(w), _f32(x)
        y = np.empty(rows, np.float32)
        p = pool or self.lib.ref_pool_create(threads, cols)
        self.lib.ref_gemv_par(p, w.ctypes.data, rows, cols, x.ctypes.data, y.ctypes.data)
        if pool is None:
            self.lib.ref_pool_destroy(p)
        return y

    def gemv_median_us(self, w, rows, cols, x, threads=1, reps=1000):
        """Median time of one gemv_par call (reference thread pool of `threads`)."""
        w, x = _u8(w), _f32(x)
        y = np.empty(rows, np.float32)
        p = self.lib.ref_pool_create(threads, cols)
        us = self.lib.ref_gemv_par_median_us(p, w.ctypes.data, rows, cols, x.ctypes.data, y.ctypes.data, reps)
        self.lib.ref_pool_destroy(p)
        return us

    def gemm(self, w, rows, cols, x, threads=1):
        w, x = _u8(w), _f32(x).reshape(-1, cols)
        y = np.empty((x.shape[0], rows), np.float32)
        p = self.lib.ref_pool_create(threads, cols)
        self.lib.ref_gemm_par(p, w.ctypes.data, rows, cols, x.ctypes.data, x.shape[0], y.ctypes.data)
        self.lib.ref_pool_destroy(p)
        return y

    def attention_window(self, q_row, k_cache, v_cache, avx2=True):
        """Single query (t=1) over cache_n keys + the query row's own k/v (attn_avx2.cpp:93).
        q_row: [3*768] = q|k|v of the current position; k_cache/v_cache: [n][768]."""
        qkv = _f32(q_row).reshape(1, -1)
        kc, vc = _f32(k_cache), _f32(v_cache)
        n = kc.shape[0]
        out = np.empty(768, np.float32)
        scores = np.empty(n + 1, np.float32)
        self.lib.ref_attention_window(qkv, 1, 0, 1, 768, 12, kc if n else np.zeros((1, 768), np.float32),
                                      vc if n else np.zeros((1, 768), np.float32), n, 0, out, scores, int(avx2))
        return out

    def rng_stream(self, seed, n):
        out = np.empty(n, np.uint32)
        self.lib.ref_rng_stream(seed, n, out)
        return out

    def sample_token(self, logits, params: SampleParams, prev=None, seed=0, skip=0):
        prev_a = np.ascontiguousarray(prev if prev is not None else np.zeros(0), dtype=np.int32)
        logits = _f32(logits)
        return self.lib.ref_sample_token(logits, logits.size, params.ints(), params.floats(),
                                         prev_a.ctypes.data if prev_a.size else None, prev_a.size, seed, skip)

    def model(self, blob: bytes, threads: int = 1) -> "RefModel":
        return RefModel(self, blob, threads)


class RefModel:
    """Reference LlmModel loaded from a blob (written to a temp file: load() takes a path)."""

    def __init__(self, r: RefCpu, blob: bytes, threads: int):
        self.r, self.lib = r, r.lib
        self.h = self.lib.ref_model_create(threads)
        self.tmpdir = tempfile.mkdtemp(prefix="mossref_")
        self.path = os.path.join(self.tmpdir, "w.moss")
        with open(self.path, "wb") as f:
            f.write(blob)
        if self.lib.ref_model_load(self.h, self.path.encode()) != 0:
            raise RuntimeError(self.lib.ref_last_error().decode())

    def close(self):
        if getattr(self, "h", None):
            self.lib.ref_model_destroy(self.h)
            self.h = None
        if getattr(self, "path", None) and os.path.exists(self.path):
            os.remove(self.path)
            os.rmdir(self.tmpdir)
            self.path = None

    def __del__(self):
        self.close()

    @property
    def position(self):
        return self.lib.ref_model_position(self.h)

    def hidden(self):
        out = np.empty(768, np.float32)
        self.lib.ref_model_hidden(self.h, out)
        return out

    def prefill(self, rows, start=0):
        rows = np.ascontiguousarray(rows, np.int32).reshape(-1, 17)
        self.lib.ref_model_prefill(self.h, rows, rows.shape[0], start)

    def load_state(self, path, rows, ignore_fp=True):
        rows = np.ascontiguousarray(rows, np.int32).reshape(-1, 17)
        if self.lib.ref_model_load_state(self.h, path.encode(), rows, rows.shape[0], int(ignore_fp)) != 0:
            raise RuntimeError(self.lib.ref_last_error().decode())

    def save_state(self, path, rows):
        rows = np.ascontiguousarray(rows, np.int32).reshape(-1, 17)
        if self.lib.ref_model_save_state(self.h, path.encode(), rows, rows.shape[0]) != 0:
            raise RuntimeError(self.lib.ref_last_error().decode())

    def load_prefix(self, path, rows):
        rows = np.ascontiguousarray(rows, np.int32).reshape(-1, 17)
        if self.lib.ref_model_load_prefix(self.h, path.encode(), rows, rows.shape[0]) != 0:
            raise RuntimeError(self.lib.ref_last_error().decode())

    def generate(self, max_frames, params: SampleParams, seed=0, forced=None, timing=False, logits_path=None,
                 gate_path=None):
        out = np.zeros((max_frames, 17), np.int32)
        fa = np.ascontiguousarray(forced, np.int32).reshape(-1, 17) if forced is not None else None
        t = np.zeros((max_frames, 2), np.float64) if timing else None
        if logits_path:
            self.lib.ref_model_set_logits_dump(self.h, logits_path.encode())
        if gate_path:
            self.lib.ref_model_set_gate_dump(self.h, gate_path.encode())
        n = self.lib.ref_model_generate(self.h, max_frames, params.ints(), params.floats(), seed,
                                        fa.ctypes.data if fa is not None else None,
                                        0 if fa is None else fa.shape[0], out,
                                        t.ctypes.data if t is not None else None)
        res = {"rows": out[:n]}
        if timing:
            res["timing"] = t[:n]
        return res


class RefDecoder:
    """The reference AudioDecoder (decoder.h:15-36) from oracle/_ref/libmossref.so,
    loaded from a blob (written to a temp file: load() takes a path)."""

    def __init__(self, r: RefCpu, blob: bytes, threads: int = 1):
        L = self.lib = r.lib
        L.ref_dec_create.restype = C.c_void_p
        L.ref_dec_create.argtypes = [C.c_int]
        L.ref_dec_destroy.argtypes = [C.c_void_p]
        L.ref_dec_load.argtypes = [C.c_void_p, C.c_char_p]
        L.ref_dec_decode.argtypes = [C.c_void_p, _i32p, C.c_int, _f32p, C.c_int, C.POINTER(C.c_double)]
        L.ref_dec_reset_stream.argtypes = [C.c_void_p]
        L.ref_dec_decode_chunk.argtypes = [C.c_void_p, _i32p, C.c_int, _f32p, C.c_int]
        self.h = L.ref_dec_create(threads)
        self.tmpdir = tempfile.mkdtemp(prefix="mossdec_")
        self.path = os.path.join(self.tmpdir, "d.moss")
        with open(self.path, "wb") as f:
            f.write(blob)
        if L.ref_dec_load(self.h, self.path.encode()) != 0:
            raise RuntimeError(L.ref_last_error().decode())
        self.last_ms = 0.0

    def close(self):
        if getattr(self, "h", None):
            self.lib.ref_dec_destroy(self.h)
            self.h = None
        if getattr(self, "path", None) and os.path.exists(self.path):
            os.remove(self.path)
            os.rmdir(self.tmpdir)
            self.path = None

    def __del__(self):
        self.close()

    def decode(self, codes):
        """codes [16][frames] int32 -> samples [frames * 7680] (decoder.cpp:247)."""
        codes = np.ascontiguousarray(codes, np.int32)
        frames = codes.shape[1]
        out = np.empty(frames * 7680, np.float32)
        ms = C.c_double()
        n = self.lib.ref_dec_decode(self.h, codes, frames, out, out.size, C.byref(ms))
        if n < 0:
            raise RuntimeError("output buffer too small")
        self.last_ms = ms.value
        return out[:n]

    def reset_stream(self):
        self.lib.ref_dec_reset_stream(self.h)

    def decode_chunk(self, codes):
        """One streaming chunk (decoder.cpp:203), in order after reset_stream()."""
        codes = np.ascontiguousarray(codes, np.int32)
        out = np.empty(codes.shape[1] * 7680, np.float32)
        n = self.lib.ref_dec_decode_chunk(self.h, codes, codes.shape[1], out, out.size)
        if n < 0:
            raise RuntimeError("output buffer too small")
        return out[:n]
