"""File formats of the MOSS-TTS-Nano LLM path, written from their published layout.

* ``.moss`` v1 weight container -- writer follows ``tools/export_weights.py:244-268``
  (``write_moss``) and the reader contract of ``csrc/src/weights.cpp:27-125``:
  16-byte header ``b"MOSW", u32 version=1, u32 n_tensors, u32 0``, then n 80-byte
  entries ``name[48], u8 dtype, u8 ndim, u16 0, u32 dims[3], u64 offset, u64 nbytes``,
  then the payload with every tensor aligned to 32 bytes.
* ``Q8_0_4X4`` matrices -- ``tools/export_weights.py:160-179`` (``pack_q8_4x4``):
  rows are taken in groups of 4; block b (32 columns) of a group is 136 bytes:
  4 fp16 scales (row k at byte 2k) followed by 4 x 32 int8 values (row k at 8+32k).
* Tensor list -- ``tools/export_weights.py:51-92`` (``build_specs``), 177 tensors.
* ``MOSSST1`` state file / ``MOSSPFX1`` prefix file -- ``csrc/src/llm.cpp:441-632``:
  40-byte header (magic[8], u32 version, u32 layers, u32 n_pos, u32 hidden,
  u64 rows_fp, u64 weights_fp) then, per layer, K[n_pos][768] and V[n_pos][768]
  fp32; the state file appends hidden[768] fp32.
* Fingerprints -- ``csrc/src/llm.cpp:407-439`` (FNV-1a 64 over row bytes; over
  the int64 file size plus the first 4 KiB of the weight file).

Synthetic weights (no checkpoint is available offline) follow the benchmark
definition: int8 ``q ~ U{-127..127}``, per-(row, 32-column block) fp16 scales
``|N(0, 0.02)| / 127``; LayerNorm w=1, b=0 (or randomised for tests), fp32 biases
``N(0, 0.02)``.  Everything is seeded through ``numpy.random.default_rng``.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np

HIDDEN, HEADS, HEAD_DIM, FF, VOCAB = 768, 12, 64, 3072, 16384
NVQ, CODEBOOK, AUDIO_PAD, SLOT, END = 16, 1024, 1024, 9, 7
MAX_CTX, LOCAL_LEN, LAYERS = 768, 17, 12

DT_F16, DT_Q8_0, DT_Q4_0, DT_F32, DT_Q8X4, DT_Q4X4 = 0, 1, 2, 3, 4, 5
DATA_ALIGN = 32  # payload alignment of every tensor (tools/export_weights.py:32,254)
BLOCK_BYTES = 136

_FNV_OFFSET = 1469598103934665603
_FNV_PRIME = 1099511628211
_MASK64 = (1 << 64) - 1


@dataclass(frozen=True)
class Spec:
    name: str
    kind: str  # "matrix" | "vector" | "embed"
    rows: int
    cols: int


def tensor_specs() -> list[Spec]:
    """The 177 tensors of the LLM file, in file order (export_weights.py:51-92)."""
    s = [Spec("wte", "embed", VOCAB, HIDDEN), Spec("lnf.w", "vector", 1, HIDDEN), Spec("lnf.b", "vector", 1, HIDDEN)]

    def layer(p: str) -> list[Spec]:
        return [
            Spec(p + "ln1.w", "vector", 1, HIDDEN), Spec(p + "ln1.b", "vector", 1, HIDDEN),
            Spec(p + "attn.w", "matrix", 3 * HIDDEN, HIDDEN), Spec(p + "attn.b", "vector", 1, 3 * HIDDEN),
            Spec(p + "proj.w", "matrix", HIDDEN, HIDDEN), Spec(p + "proj.b", "vector", 1, HIDDEN),
            Spec(p + "ln2.w", "vector", 1, HIDDEN), Spec(p + "ln2.b", "vector", 1, HIDDEN),
            Spec(p + "fc_in.w", "matrix", FF, HIDDEN), Spec(p + "fc_in.b", "vector", 1, FF),
            Spec(p + "fc_out.w", "matrix", HIDDEN, FF), Spec(p + "fc_out.b", "vector", 1, HIDDEN),
        ]

    for i in range(LAYERS):
        s += layer(f"g{i}.")
    s += [Spec(f"aemb.{ch}", "embed", CODEBOOK, HIDDEN) for ch in range(NVQ)]
    s += layer("local.")
    s += [Spec("local.lnf.w", "vector", 1, HIDDEN), Spec("local.lnf.b", "vector", 1, HIDDEN)]
    return s


# ------------------------------------------------------------------ 4x4 packing

def pack_q8x4(q: np.ndarray, d_f16: np.ndarray) -> np.ndarray:
    """int8 q[rows, K] and fp16 d[rows, K/32] -> Q8_0_4X4 bytes [rows/4, K/32*136]."""
    rows, k = q.shape
    if rows % 4 or k % 32:
        raise ValueError(f"Q8_0_4X4 needs rows % 4 == 0 and cols % 32 == 0, got {q.shape}")
    nb, groups = k // 32, rows // 4
    out = np.empty((groups, nb, BLOCK_BYTES), dtype=np.uint8)
    d_bytes = np.ascontiguousarray(d_f16.astype(np.float16)).view(np.uint8).reshape(groups, 4, nb, 2)
    out[:, :, 0:8] = d_bytes.transpose(0, 2, 1, 3).reshape(groups, nb, 8)
    q_bytes = np.ascontiguousarray(q.astype(np.int8)).view(np.uint8).reshape(groups, 4, nb, 32)
    out[:, :, 8:] = q_bytes.transpose(0, 2, 1, 3).reshape(groups, nb, 128)
    return out.reshape(groups, nb * BLOCK_BYTES)


def unpack_q8x4(packed: np.ndarray, rows: int, cols: int) -> tuple[np.ndarray, np.ndarray]:
    """Inverse of pack_q8x4: -> (int8 q[rows, cols], fp16 d[rows, cols/32])."""
    nb, groups = cols // 32, rows // 4
    blk = np.asarray(packed, dtype=np.uint8).reshape(groups, nb, BLOCK_BYTES)
    d = blk[:, :, 0:8].reshape(groups, nb, 4, 2).transpose(0, 2, 1, 3).copy().view(np.float16)
    q = blk[:, :, 8:].reshape(groups, nb, 4, 32).transpose(0, 2, 1, 3).copy().view(np.int8)
    return q.reshape(rows, cols), d.reshape(rows, nb)


def dequant_q8x4(packed: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Exact fp32 dequantisation w = fp32(d) * q (every product is exact in fp32)."""
    q, d = unpack_q8x4(packed, rows, cols)
    return (q.astype(np.float32).reshape(rows, cols // 32, 32) * d.astype(np.float32)[:, :, None]).reshape(rows, cols)


def synth_q8x4(rng: np.random.Generator, rows: int, cols: int, scale_sigma: float = 0.02) -> np.ndarray:
    """Random Q8_0_4X4 matrix: q ~ U{-127..127}, d = fp16(|N(0, sigma)| / 127)."""
    q = rng.integers(-127, 128, size=(rows, cols), dtype=np.int8)
    d = (np.abs(rng.standard_normal((rows, cols // 32), dtype=np.float32)) * scale_sigma / 127.0).astype(np.float16)
    return pack_q8x4(q, d)


# ------------------------------------------------------------------ .moss v1

def write_moss(entries: list[tuple[str, int, int, int, bytes]]) -> bytes:
    """entries: (name, dtype, rows, cols, payload) -> .moss v1 bytes."""
    header = b"MOSW" + struct.pack("<III", 1, len(entries), 0)
    data_start = 16 + 80 * len(entries)
    table = bytearray()
    payload = bytearray()
    for name, dtype, rows, cols, blob in entries:
        pad = (-(data_start + len(payload))) % DATA_ALIGN
        payload += b"\x00" * pad
        offset = data_start + len(payload)
        nb = name.encode("ascii")
        if len(nb) >= 48:
            raise ValueError(name)
        table += nb.ljust(48, b"\x00") + struct.pack("<BBH", dtype, 2, 0) + struct.pack("<III", rows, cols, 1)
        table += struct.pack("<QQ", offset, len(blob))
        payload += blob
    return bytes(header + table + payload)


def read_moss_index(blob: bytes) -> dict[str, tuple[int, int, int, int, int]]:
    """name -> (dtype, rows, cols, offset, nbytes); raises on a malformed blob."""
    if len(blob) < 16 or blob[:4] != b"MOSW":
        raise ValueError("not a .moss file")
    version, n, _ = struct.unpack_from("<III", blob, 4)
    if version != 1:
        raise ValueError(f"unsupported .moss version {version}")
    out = {}
    for i in range(n):
        base = 16 + 80 * i
        name = blob[base:base + 48].split(b"\x00", 1)[0].decode("ascii")
        dtype, ndim = blob[base + 48], blob[base + 49]
        d0, d1, d2 = struct.unpack_from("<III", blob, base + 52)
        off, nbytes = struct.unpack_from("<QQ", blob, base + 64)
        if off + nbytes > len(blob):
            raise ValueError(f"tensor out of range: {name}")
        if off % DATA_ALIGN:  # the exporter pads every tensor to it; the GPU loader requires it
            raise ValueError(f"tensor not {DATA_ALIGN}-byte aligned: {name}")
        out[name] = (dtype, d0, d1, off, nbytes)
    return out


def synth_model(seed: int = 1234, ln_random: bool = False, bias_sigma: float = 0.02,
                scale_sigma: float = 0.02, drop: str | None = None) -> bytes:
    """A seeded random-init .moss with the reference's exact tensor list and shapes.

    ``drop`` omits one tensor (to exercise the loader's missing-tensor error)."""
    rng = np.random.default_rng(seed)
    entries = []
    for s in tensor_specs():
        if s.name == drop:
            continue
        if s.kind == "vector":
            if s.name.endswith(("ln1.w", "ln2.w", "lnf.w")):
                v = (1.0 + 0.1 * rng.standard_normal(s.cols)).astype(np.float32) if ln_random else np.ones(s.cols, np.float32)
            elif s.name.endswith(("ln1.b", "ln2.b", "lnf.b")):
                v = (0.1 * rng.standard_normal(s.cols)).astype(np.float32) if ln_random else np.zeros(s.cols, np.float32)
            else:
                v = (bias_sigma * rng.standard_normal(s.cols)).astype(np.float32)
            entries.append((s.name, DT_F32, 1, s.cols, v.tobytes()))
        else:
            entries.append((s.name, DT_Q8X4, s.rows, s.cols, synth_q8x4(rng, s.rows, s.cols, scale_sigma).tobytes()))
    return write_moss(entries)


# ------------------------------------------------------------------ fingerprints & state

def fnv_bytes(h: int, data: bytes) -> int:
    for b in data:
        h = ((h ^ b) * _FNV_PRIME) & _MASK64
    return h


def fp_rows(rows: np.ndarray) -> int:
    """llm.cpp:419-423 -- FNV over the rows' int32 little-endian bytes."""
    r = np.ascontiguousarray(np.asarray(rows, dtype="<i4").reshape(-1, NVQ + 1))
    return fnv_bytes(_FNV_OFFSET, r.tobytes())


def fp_weights(blob: bytes) -> int:
    """llm.cpp:426-439 -- FNV over int64 file size then the first 4 KiB."""
    h = fnv_bytes(_FNV_OFFSET, struct.pack("<q", len(blob)))
    return fnv_bytes(h, blob[:4096])


STATE_MAGIC = b"MOSSST1\x00"
PREFIX_MAGIC = b"MOSSPFX1"


def write_state(k: np.ndarray, v: np.ndarray, hidden: np.ndarray | None, rows: np.ndarray, weights_fp: int,
                magic: bytes = STATE_MAGIC) -> bytes:
    """k, v: [12][n_pos][768] fp32 (reference layout); hidden [768] for a state file."""
    n_pos = k.shape[1]
    out = bytearray(magic + struct.pack("<IIII", 1, LAYERS, n_pos, HIDDEN) + struct.pack("<QQ", fp_rows(rows), weights_fp))
    for layer in range(LAYERS):
        out += np.ascontiguousarray(k[layer], dtype=np.float32).tobytes()
        out += np.ascontiguousarray(v[layer], dtype=np.float32).tobytes()
    if hidden is not None:
        out += np.ascontiguousarray(hidden, dtype=np.float32).tobytes()
    return bytes(out)


def read_state(blob: bytes, with_hidden: bool = True):
    """-> (magic, n_pos, rows_fp, weights_fp, k, v, hidden|None); raises on a bad file."""
    if len(blob) < 40:
        raise ValueError("state file too small")
    magic = blob[:8]
    version, layers, n_pos, hidden_n = struct.unpack_from("<IIII", blob, 8)
    rows_fp, weights_fp = struct.unpack_from("<QQ", blob, 24)
    if version != 1 or layers != LAYERS or hidden_n != HIDDEN or n_pos == 0 or n_pos > MAX_CTX:
        raise ValueError("bad state header")
    per = n_pos * HIDDEN * 4
    need = 40 + LAYERS * 2 * per + (HIDDEN * 4 if with_hidden else 0)
    if len(blob) < need:
        raise ValueError("state file truncated")
    k = np.empty((LAYERS, n_pos, HIDDEN), np.float32)
    v = np.empty((LAYERS, n_pos, HIDDEN), np.float32)
    off = 40
    for layer in range(LAYERS):
        k[layer] = np.frombuffer(blob, np.float32, n_pos * HIDDEN, off).reshape(n_pos, HIDDEN)
        off += per
        v[layer] = np.frombuffer(blob, np.float32, n_pos * HIDDEN, off).reshape(n_pos, HIDDEN)
        off += per
    hidden = np.frombuffer(blob, np.float32, HIDDEN, off).copy() if with_hidden else None
    return magic, n_pos, rows_fp, weights_fp, k, v, hidden


def text_rows(tokens: np.ndarray) -> np.ndarray:
    """Prompt rows [n][17] for text tokens: [tok, pad x16] (csrc/src/prompt.cpp:27-32)."""
    rows = np.full((len(tokens), NVQ + 1), AUDIO_PAD, dtype=np.int32)
    rows[:, 0] = tokens
    return rows
