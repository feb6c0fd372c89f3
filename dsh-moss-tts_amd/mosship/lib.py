"""ctypes binding of libmoss_hip.so (C ABI declared in include/moss_hip.h).

The library is the product: if it is missing this module raises instead of
falling back to anything else.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "libmoss_hip.so")

OK, EINVAL, EDEVICE, EFORMAT, EUNSUPPORTED, ESTATE = 0, 1, 2, 3, 4, 5
F32, F16 = 0, 1

# Quantiser capture (moss_hip_llm_capture): kinds and the per-step float offsets of a decode
# capture, as include/moss_hip.h declares them (name -> (offset, length)).
CAP_GLOBAL, CAP_LOCAL, CAP_PREFILL = 0, 1, 2
CAP_STEP = 17088
CAP = {"xin": (0, 768), "ln1": (768, 768), "ln1_q": (1536, 768), "ln1_d": (2304, 24), "qkv": (2328, 2304),
       "att": (4632, 768), "att_q": (5400, 768), "att_d": (6168, 24), "xm": (6192, 768), "ln2": (6960, 768),
       "ln2_q": (7728, 768), "ln2_d": (8496, 24), "h": (8520, 3072), "h_q": (11592, 3072), "h_d": (14664, 96),
       "xout": (14760, 768), "lnf": (15528, 768), "lnf_q": (16296, 768), "lnf_d": (17064, 24)}

EXPORTED = [
    "moss_hip_last_error", "moss_hip_abi_version",
    "moss_hip_llm_create", "moss_hip_llm_create_from_file", "moss_hip_llm_destroy", "moss_hip_llm_reset",
    "moss_hip_llm_position", "moss_hip_llm_get_hidden", "moss_hip_llm_set_hidden", "moss_hip_llm_prefill",
    "moss_hip_llm_global_step", "moss_hip_llm_generate", "moss_hip_llm_set_cancel_flag",
    "moss_hip_llm_snapshot_prefix", "moss_hip_llm_restore_prefix", "moss_hip_llm_prefix_pos",
    "moss_hip_llm_gate_rows", "moss_hip_llm_fallbacks", "moss_hip_fallbacks_total",
    "moss_hip_llm_kv_export", "moss_hip_llm_kv_import", "moss_hip_llm_capture", "moss_hip_llm_capture_read",
    "moss_hip_batch_create", "moss_hip_batch_destroy", "moss_hip_batch_set_stream", "moss_hip_batch_admit", "moss_hip_batch_get_hidden",
    "moss_hip_batch_position", "moss_hip_batch_kv_export", "moss_hip_batch_global_step", "moss_hip_batch_generate",
    "moss_hip_batch_capture", "moss_hip_batch_capture_read",
    "moss_hip_gemv_q8x4", "moss_hip_gemm_q8x4", "moss_hip_dequant_rows_q8x4", "moss_hip_attn_decode",
    "moss_hip_attn_decode_noalloc", "moss_hip_attn_paged",
    "moss_hip_quantize_rows", "moss_hip_gemm_q8x4_w8a8", "moss_hip_gemv_q8x4_w8a8",
    "moss_hip_codec_create", "moss_hip_codec_create_from_file", "moss_hip_codec_destroy",
    "moss_hip_codec_samples_per_frame", "moss_hip_codec_reset_stream", "moss_hip_codec_decode_chunk",
    "moss_hip_codec_decode", "moss_hip_codec_last_ms", "moss_hip_codec_stage_ms",
]


class MossHipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class Options(C.Structure):
    _fields_ = [("device", C.c_int), ("max_ctx", C.c_int), ("kv_dtype", C.c_int), ("use_graphs", C.c_int),
                ("prefill_a16", C.c_int), ("decode_kernels", C.c_int), ("decode_a8", C.c_int)]


class CodecOptions(C.Structure):
    """moss_hip_codec_options."""
    _fields_ = [("device", C.c_int), ("max_chunk_frames", C.c_int), ("contexts", C.c_int * 4), ("eager", C.c_int)]


class SampleParams(C.Structure):
    """moss_hip_sample_params == SampleParams (csrc/include/moss/sampler.h:8-22)."""
    _fields_ = [("greedy", C.c_int), ("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float),
                ("repetition_penalty", C.c_float), ("end_greedy", C.c_int), ("min_frames", C.c_int),
                ("greedy_frames", C.c_int)]

    @classmethod
    def make(cls, greedy=True, temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0, end_greedy=True,
             min_frames=0, greedy_frames=0):
        return cls(int(greedy), temperature, top_k, top_p, repetition_penalty, int(end_greedy), min_frames,
                   greedy_frames)


FRAME_CB = C.CFUNCTYPE(None, C.c_void_p, C.c_int, C.POINTER(C.c_int32))

_lib = None


def load(path: str = LIB_PATH) -> C.CDLL:
    """Load libmoss_hip.so (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with `make -C dsh-moss-tts_amd` (or __graft_entry__.build())")
    L = C.CDLL(path)
    vp, i32, f32p = C.c_void_p, C.c_int, C.POINTER(C.c_float)
    L.moss_hip_last_error.restype = C.c_char_p
    L.moss_hip_abi_version.restype = C.c_int
    L.moss_hip_llm_create.argtypes = [vp, C.c_size_t, C.POINTER(Options), C.POINTER(vp)]
    L.moss_hip_llm_create_from_file.argtypes = [C.c_char_p, C.POINTER(Options), C.POINTER(vp)]
    L.moss_hip_llm_destroy.argtypes = [vp]
    L.moss_hip_llm_destroy.restype = None
    for n in ("moss_hip_llm_reset", "moss_hip_llm_snapshot_prefix", "moss_hip_llm_restore_prefix"):
        getattr(L, n).argtypes = [vp]
    L.moss_hip_llm_position.argtypes = [vp]
    L.moss_hip_llm_prefix_pos.argtypes = [vp]
    L.moss_hip_llm_gate_rows.argtypes = [vp]
    L.moss_hip_llm_fallbacks.argtypes = [vp]
    L.moss_hip_llm_get_hidden.argtypes = [vp, vp]
    L.moss_hip_llm_set_hidden.argtypes = [vp, vp]
    L.moss_hip_llm_prefill.argtypes = [vp, vp, i32, i32]
    L.moss_hip_llm_global_step.argtypes = [vp, vp]
    L.moss_hip_llm_generate.argtypes = [vp, i32, C.POINTER(SampleParams), C.c_uint64, vp, i32, vp, C.POINTER(i32),
                                        vp, vp, vp, FRAME_CB, vp]
    L.moss_hip_llm_set_cancel_flag.argtypes = [vp, vp]
    L.moss_hip_llm_kv_export.argtypes = [vp, i32, vp, vp]
    L.moss_hip_llm_kv_import.argtypes = [vp, i32, vp, vp, vp]
    L.moss_hip_llm_capture.argtypes = [vp, i32]
    L.moss_hip_llm_capture_read.argtypes = [vp, i32, vp, C.c_size_t, C.POINTER(C.c_size_t)]
    L.moss_hip_gemv_q8x4.argtypes = [vp, i32, i32, vp, i32, vp, i32, vp]
    L.moss_hip_gemv_q8x4_w8a8.argtypes = [vp, i32, i32, vp, vp, vp]
    L.moss_hip_gemm_q8x4.argtypes = [vp, i32, i32, vp, i32, vp, vp]
    L.moss_hip_quantize_rows.argtypes = [vp, i32, i32, vp, vp, vp]
    L.moss_hip_gemm_q8x4_w8a8.argtypes = [vp, i32, i32, vp, vp, i32, vp, vp]
    L.moss_hip_batch_create.argtypes = [vp, i32, i32, i32, C.POINTER(vp)]
    L.moss_hip_batch_destroy.argtypes = [vp]
    L.moss_hip_batch_destroy.restype = None
    L.moss_hip_batch_set_stream.argtypes = [vp, i32, i32, vp, vp, vp]
    L.moss_hip_batch_admit.argtypes = [vp, i32, vp]
    L.moss_hip_batch_capture.argtypes = [vp, i32]
    L.moss_hip_batch_capture_read.argtypes = [vp, vp, C.c_size_t, C.POINTER(C.c_size_t)]
    L.moss_hip_batch_get_hidden.argtypes = [vp, i32, vp]
    L.moss_hip_batch_position.argtypes = [vp, i32]
    L.moss_hip_batch_kv_export.argtypes = [vp, i32, i32, vp, vp]
    L.moss_hip_batch_global_step.argtypes = [vp, i32, vp]
    L.moss_hip_batch_generate.argtypes = [vp, i32, i32, C.POINTER(SampleParams), vp, vp, vp, C.POINTER(C.c_double)]
    L.moss_hip_dequant_rows_q8x4.argtypes = [vp, i32, i32, vp, i32, vp, vp]
    L.moss_hip_attn_decode.argtypes = [vp, vp, vp, i32, i32, i32, i32, vp, i32, vp]
    L.moss_hip_attn_decode_noalloc.argtypes = [vp, vp, vp, i32, i32, i32, i32, vp, i32, vp]
    L.moss_hip_attn_paged.argtypes = [vp, vp, vp, i32, i32, vp, i32, i32, i32, vp, vp, i32, vp, i32, vp]
    L.moss_hip_codec_create.argtypes = [vp, C.c_size_t, C.POINTER(CodecOptions), C.POINTER(vp)]
    L.moss_hip_codec_create_from_file.argtypes = [C.c_char_p, C.POINTER(CodecOptions), C.POINTER(vp)]
    L.moss_hip_codec_destroy.argtypes = [vp]
    L.moss_hip_codec_destroy.restype = None
    L.moss_hip_codec_samples_per_frame.argtypes = [vp]
    L.moss_hip_codec_reset_stream.argtypes = [vp]
    L.moss_hip_codec_decode_chunk.argtypes = [vp, vp, i32, vp]
    L.moss_hip_codec_decode.argtypes = [vp, vp, i32, vp]
    L.moss_hip_codec_last_ms.argtypes = [vp]
    L.moss_hip_codec_last_ms.restype = C.c_double
    L.moss_hip_codec_stage_ms.argtypes = [vp, C.POINTER(C.c_double)]
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != OK:
        raise MossHipError(rc, load().moss_hip_last_error().decode(errors="replace"))


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- operators (torch device tensors)

def _stream(stream):
    if stream is not None:
        return C.c_void_p(stream)
    import torch
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def gemv_q8x4(w, rows: int, cols: int, x, y, stream=None) -> None:
    """y = W x on the device.  w: uint8 tensor (Q8_0_4X4), x/y: float32 or float16 tensors."""
    import torch
    dt = {torch.float32: F32, torch.float16: F16}
    check(load().moss_hip_gemv_q8x4(C.c_void_p(w.data_ptr()), rows, cols, C.c_void_p(x.data_ptr()), dt[x.dtype],
                                    C.c_void_p(y.data_ptr()), dt[y.dtype], _stream(stream)))


def gemv_q8x4_w8a8(w, rows: int, cols: int, x, y, stream=None) -> None:
    """y = W x with x quantised per 32-block (the reference's W8A8 gemv_par); x, y fp32."""
    check(load().moss_hip_gemv_q8x4_w8a8(C.c_void_p(w.data_ptr()), rows, cols, C.c_void_p(x.data_ptr()),
                                         C.c_void_p(y.data_ptr()), _stream(stream)))


def gemm_q8x4(w, rows: int, cols: int, x, m: int, y, stream=None) -> None:
    """Y[m][rows] = X[m][cols] W^T on the matrix cores (fp32 x / y device tensors)."""
    check(load().moss_hip_gemm_q8x4(C.c_void_p(w.data_ptr()), rows, cols, C.c_void_p(x.data_ptr()), m,
                                    C.c_void_p(y.data_ptr()), _stream(stream)))


def quantize_rows(x, m: int, cols: int, q, d, stream=None) -> None:
    """W8A8 activation quantisation: q[m][cols] int8, d[m][cols/32] fp32 (device tensors)."""
    check(load().moss_hip_quantize_rows(C.c_void_p(x.data_ptr()), m, cols, C.c_void_p(q.data_ptr()),
                                        C.c_void_p(d.data_ptr()), _stream(stream)))


def gemm_q8x4_w8a8(w, rows: int, cols: int, q, d, m: int, y, stream=None) -> None:
    """Y[m][rows] from int8 activations q and block scales d on the int8 matrix cores."""
    check(load().moss_hip_gemm_q8x4_w8a8(C.c_void_p(w.data_ptr()), rows, cols, C.c_void_p(q.data_ptr()),
                                         C.c_void_p(d.data_ptr()), m, C.c_void_p(y.data_ptr()), _stream(stream)))


def dequant_rows_q8x4(w, mat_rows: int, cols: int, rows_idx, out, stream=None) -> None:
    check(load().moss_hip_dequant_rows_q8x4(C.c_void_p(w.data_ptr()), mat_rows, cols, C.c_void_p(rows_idx.data_ptr()),
                                            rows_idx.numel(), C.c_void_p(out.data_ptr()), _stream(stream)))


def attn_decode(q, k_cache, v_cache, heads: int, ctx_stride: int, n_keys: int, out, stream=None,
                noalloc: bool = False) -> None:
    """moss_hip_attn_decode, or with noalloc=True moss_hip_attn_decode_noalloc (static scratch)."""
    import torch
    dt = {torch.float32: F32, torch.float16: F16}
    L = load()
    fn = L.moss_hip_attn_decode_noalloc if noalloc else L.moss_hip_attn_decode
    check(fn(C.c_void_p(q.data_ptr()), C.c_void_p(k_cache.data_ptr()), C.c_void_p(v_cache.data_ptr()),
             dt[k_cache.dtype], heads, ctx_stride, n_keys, C.c_void_p(out.data_ptr()), dt[out.dtype], _stream(stream)))


def attn_paged(q, k_pool, v_pool, heads: int, page_table, table_stride: int, page_size: int, row_pos, max_keys: int,
               out, row_stream=None, stream=None) -> None:
    """moss_hip_attn_paged: row r (stream row_stream[r], or r) attends its keys 0 .. row_pos[r]."""
    import torch
    dt = {torch.float32: F32, torch.float16: F16}
    L = load()
    rows = q.shape[0]
    check(L.moss_hip_attn_paged(C.c_void_p(q.data_ptr()), C.c_void_p(k_pool.data_ptr()), C.c_void_p(v_pool.data_ptr()),
                                dt[k_pool.dtype], heads, C.c_void_p(page_table.data_ptr()), table_stride, page_size,
                                rows, C.c_void_p(row_stream.data_ptr()) if row_stream is not None else None,
                                C.c_void_p(row_pos.data_ptr()), max_keys, C.c_void_p(out.data_ptr()), dt[out.dtype],
                                _stream(stream)))


# ---------------------------------------------------------------- model

class HipLLM:
    """Python view of the GPU LlmModel (moss_hip_llm_*)."""

    def __init__(self, blob: bytes, device: int = 0, max_ctx: int = 0, kv_fp32: bool = False, graphs: bool = True,
                 prefill_a16: bool = False, per_op: bool = False, decode_a8: bool = False):
        L = self.L = load()
        self._h = C.c_void_p()
        buf = np.frombuffer(blob, dtype=np.uint8)
        opt = Options(device, max_ctx, 1 if kv_fp32 else 0, 1 if graphs else 0, 1 if prefill_a16 else 0,
                      1 if per_op else 0, 1 if decode_a8 else 0)
        check(L.moss_hip_llm_create(_ptr(buf), buf.size, C.byref(opt), C.byref(self._h)))

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            self.L.moss_hip_llm_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        self.close()

    @property
    def position(self) -> int:
        return self.L.moss_hip_llm_position(self._h)

    @property
    def prefix_pos(self) -> int:
        return self.L.moss_hip_llm_prefix_pos(self._h)

    @property
    def fallbacks(self) -> int:
        """Fused decode launches redone on the per-operator path (moss_hip_llm_fallbacks)."""
        return self.L.moss_hip_llm_fallbacks(self._h)

    def reset(self):
        check(self.L.moss_hip_llm_reset(self._h))

    def hidden(self) -> np.ndarray:
        out = np.empty(768, np.float32)
        check(self.L.moss_hip_llm_get_hidden(self._h, _ptr(out)))
        return out

    def set_hidden(self, h):
        h = np.ascontiguousarray(h, np.float32)
        check(self.L.moss_hip_llm_set_hidden(self._h, _ptr(h)))

    def prefill(self, rows, start: int = 0):
        rows = np.ascontiguousarray(rows, np.int32).reshape(-1, 17)
        check(self.L.moss_hip_llm_prefill(self._h, _ptr(rows), rows.shape[0], start))

    def global_step(self, row):
        row = np.ascontiguousarray(row, np.int32).reshape(17)
        check(self.L.moss_hip_llm_global_step(self._h, _ptr(row)))

    def generate(self, max_frames: int, params: SampleParams | None = None, seed: int = 0, forced=None,
                 timing: bool = False, logits: bool = False, gate: bool = False, on_frame=None):
        params = params or SampleParams.make()
        out = np.zeros((max(max_frames, 1), 17), np.int32)
        fa = np.ascontiguousarray(forced, np.int32).reshape(-1, 17) if forced is not None else None
        t = np.zeros((max(max_frames, 1), 2), np.float64) if timing else None
        ld = np.zeros((max(max_frames, 1), 16, 1024), np.float32) if logits else None
        gd = np.zeros((max(max_frames, 1), 4), np.float32) if gate else None
        n = C.c_int(0)
        cb = FRAME_CB(lambda u, f, row: on_frame(f, np.ctypeslib.as_array(row, (17,)).copy())) if on_frame \
            else FRAME_CB()
        check(self.L.moss_hip_llm_generate(self._h, max_frames, C.byref(params), seed,
                                           _ptr(fa) if fa is not None else None, 0 if fa is None else fa.shape[0],
                                           _ptr(out), C.byref(n), _ptr(t) if t is not None else None,
                                           _ptr(ld) if ld is not None else None, _ptr(gd) if gd is not None else None,
                                           cb, None))
        res = {"rows": out[:n.value]}
        if timing:
            res["timing"] = t[:n.value]
        if logits:
            res["logits"] = ld[:n.value]
        if gate:
            res["gate"] = gd[:self.L.moss_hip_llm_gate_rows(self._h)]
        return res

    def set_cancel_flag(self, flag_array: np.ndarray | None):
        """flag_array: a 1-element uint8 numpy array kept alive by the caller (or None)."""
        self._cancel = flag_array
        check(self.L.moss_hip_llm_set_cancel_flag(self._h, _ptr(flag_array) if flag_array is not None else None))

    def snapshot_prefix(self):
        check(self.L.moss_hip_llm_snapshot_prefix(self._h))

    def restore_prefix(self):
        check(self.L.moss_hip_llm_restore_prefix(self._h))

    def capture(self, on: bool = True):
        """Quantiser capture (tests): W8A8 quantisers record their inputs and outputs."""
        check(self.L.moss_hip_llm_capture(self._h, 1 if on else 0))

    def capture_read(self, what: int) -> np.ndarray:
        """Raw bytes of the last capture of `what` (CAP_GLOBAL / CAP_LOCAL / CAP_PREFILL)."""
        n = C.c_size_t(0)
        check(self.L.moss_hip_llm_capture_read(self._h, what, None, 0, C.byref(n)))
        out = np.empty(n.value, np.uint8)
        check(self.L.moss_hip_llm_capture_read(self._h, what, _ptr(out), out.size, None))
        return out

    def capture_steps(self, what: int) -> list:
        """A decode capture as one dict per step (block or local position) of named float arrays."""
        raw = self.capture_read(what).view(np.float32).reshape(-1, CAP_STEP)
        return [{k: step[o:o + n].copy() for k, (o, n) in CAP.items()} for step in raw]

    def kv_export(self, n_pos: int):
        k = np.empty((12, n_pos, 768), np.float32)
        v = np.empty((12, n_pos, 768), np.float32)
        check(self.L.moss_hip_llm_kv_export(self._h, n_pos, _ptr(k), _ptr(v)))
        return k, v

    def kv_import(self, k, v, hidden=None):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        h = np.ascontiguousarray(hidden, np.float32) if hidden is not None else None
        check(self.L.moss_hip_llm_kv_import(self._h, k.shape[1], _ptr(k), _ptr(v), _ptr(h) if h is not None else None))


class HipBatch:
    """Python view of a moss_hip_batch (many streams decoded in lock-step)."""

    def __init__(self, model: HipLLM, max_streams: int, capacity: int, kv_fp32: bool = False):
        self.L = load()
        self.model = model  # keeps the weights alive
        self._h = C.c_void_p()
        check(self.L.moss_hip_batch_create(model._h, max_streams, capacity, 1 if kv_fp32 else 0, C.byref(self._h)))

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            self.L.moss_hip_batch_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        self.close()

    def set_stream(self, s: int, k, v, hidden):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        h = np.ascontiguousarray(hidden, np.float32)
        check(self.L.moss_hip_batch_set_stream(self._h, s, k.shape[1], _ptr(k), _ptr(v), _ptr(h)))

    def capture(self, on: bool = True):
        """Attention capture of a W8A8 batch (tests)."""
        check(self.L.moss_hip_batch_capture(self._h, 1 if on else 0))

    def capture_attention(self, max_streams: int) -> list:
        """The last frame's attention records: 29 dicts (12 global layers, local positions 0..16)
        of out [max_streams][768] fp32 and the raw int8 / scale operand (matrix-core order)."""
        n = C.c_size_t(0)
        check(self.L.moss_hip_batch_capture_read(self._h, None, 0, C.byref(n)))
        raw = np.empty(n.value, np.uint8)
        check(self.L.moss_hip_batch_capture_read(self._h, _ptr(raw), raw.size, None))
        s16 = (max_streams + 15) // 16 * 16
        per = 4 * max_streams * 768 + s16 * 768 + 4 * s16 * 24
        assert raw.size == 29 * per
        out = []
        for e in range(29):
            b = e * per
            out.append({"out": raw[b:b + 4 * max_streams * 768].view(np.float32).reshape(max_streams, 768),
                        "q": raw[b + 4 * max_streams * 768: b + 4 * max_streams * 768 + s16 * 768],
                        "d": raw[b + 4 * max_streams * 768 + s16 * 768: b + per]})
        return out

    def admit(self, s: int, model: HipLLM):
        """Stream s takes `model`'s state (K/V, hidden, position) device to device."""
        check(self.L.moss_hip_batch_admit(self._h, s, model._h))

    def position(self, s: int) -> int:
        return self.L.moss_hip_batch_position(self._h, s)

    def hidden(self, s: int) -> np.ndarray:
        out = np.empty(768, np.float32)
        check(self.L.moss_hip_batch_get_hidden(self._h, s, _ptr(out)))
        return out

    def kv_export(self, s: int, n_pos: int):
        k = np.empty((12, n_pos, 768), np.float32)
        v = np.empty((12, n_pos, 768), np.float32)
        check(self.L.moss_hip_batch_kv_export(self._h, s, n_pos, _ptr(k), _ptr(v)))
        return k, v

    def global_step(self, rows):
        rows = np.ascontiguousarray(rows, np.int32).reshape(-1, 17)
        check(self.L.moss_hip_batch_global_step(self._h, rows.shape[0], _ptr(rows)))

    def generate(self, n_streams: int, frames: int, params: SampleParams | None = None, seeds=None):
        params = params or SampleParams.make()
        out = np.zeros((max(frames, 1), n_streams, 17), np.int32)
        nf = np.zeros(n_streams, np.int32)
        ms = C.c_double(0.0)
        sd = None if seeds is None else np.ascontiguousarray(seeds, np.uint64).reshape(n_streams)
        check(self.L.moss_hip_batch_generate(self._h, n_streams, frames, C.byref(params),
                                             None if sd is None else _ptr(sd), _ptr(out), _ptr(nf), C.byref(ms)))
        return {"rows": out[:frames], "frames": nf, "ms": ms.value}


class HipCodec:
    """The GPU audio codec decoder (moss::AudioDecoder, csrc/include/moss/decoder.h:14-83).

    codes: int array [16][frames] (quantizer-major) in [0, 1024); results are float32 arrays
    of frames * samples_per_frame interleaved stereo samples."""

    def __init__(self, blob: bytes, max_chunk_frames: int = 0, contexts=(0, 0, 0, 0), eager: bool = False,
                 device: int = 0):
        L = load()
        o = CodecOptions(device, max_chunk_frames, (C.c_int * 4)(*contexts), int(eager))
        h = C.c_void_p()
        self._blob = np.frombuffer(blob, dtype=np.uint8)
        check(L.moss_hip_codec_create(_ptr(self._blob), len(blob), C.byref(o), C.byref(h)))
        self._h = h
        self.samples_per_frame = L.moss_hip_codec_samples_per_frame(h)

    def close(self):
        if getattr(self, "_h", None):
            load().moss_hip_codec_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def _run(self, fn, codes):
        c = np.ascontiguousarray(codes, dtype=np.int32)
        if c.ndim != 2 or c.shape[0] != 16:
            raise ValueError("codes must be [16][frames]")
        out = np.empty(c.shape[1] * self.samples_per_frame, np.float32)
        check(fn(self._h, _ptr(c), c.shape[1], _ptr(out)))
        return out

    def reset_stream(self) -> None:
        check(load().moss_hip_codec_reset_stream(self._h))

    def decode_chunk(self, codes) -> np.ndarray:
        return self._run(load().moss_hip_codec_decode_chunk, codes)

    def decode(self, codes) -> np.ndarray:
        return self._run(load().moss_hip_codec_decode, codes)

    @property
    def last_ms(self) -> float:
        return load().moss_hip_codec_last_ms(self._h)

    @property
    def stage_ms(self):
        out = (C.c_double * 4)()
        check(load().moss_hip_codec_stage_ms(self._h, out))
        return list(out)
