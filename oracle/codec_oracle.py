"""Restatement of the MOSS audio codec decoder in numpy (float64).

TEST INFRASTRUCTURE ONLY: the checker of the codec decoder path.  Only tests/
(and bench.py's CPU leg) may use it.  Every step cites the reference source it
restates; the arithmetic is carried in float64, so against the reference (fp32
throughout) it agrees to fp32 rounding, not bit for bit.

Whole-utterance decode (decoder.cpp:247-281):
  x = quantize_front(codes)                           decoder.cpp:224-245
  for stage s (patch 4, 2, 2, 2; window 500, 800, 1200, 1600):
      x = patch(x, p)                                 decoder.cpp:73-87
      y = x W_in^T; 12 layers in total of             decoder.cpp:93-100
          y += ls1 * proj(attn(rope(LN1(y) W_qkv^T))) audio_layer.cpp:55-110
          y += ls2 * gelu(LN2(y) W_f1^T) W_f2^T
      x = y W_out^T
  samples = patch(x, 240)                             decoder.cpp:274
Streaming (decoder.cpp:203-221, 105-201): the same per chunk, RoPE at absolute
positions, each layer attending to its cached keys of earlier chunks (at most
`context` of them) plus the chunk's own, keys kept while 0 <= q_pos - k_pos < window.
"""
from __future__ import annotations

import numpy as np

import sys
import os

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "dsh-moss-tts_amd"))
from mosship.moss_format import DT_F16, DT_F32, read_moss_index  # noqa: E402
from mosship import codec_format as cf  # noqa: E402


def load(blob: bytes) -> dict[str, np.ndarray]:
    """Every tensor as float64 (fp16 matrices widened exactly)."""
    out = {}
    for name, (dt, rows, cols, off, nb) in read_moss_index(blob).items():
        raw = np.frombuffer(blob, dtype=np.uint8, count=nb, offset=off)
        if dt == DT_F32:
            a = raw.view(np.float32)
        elif dt == DT_F16:
            a = raw.view(np.float16)
        else:
            raise ValueError(f"{name}: dtype {dt} not handled by the codec oracle")
        a = a.astype(np.float64).reshape(rows, cols)
        out[name] = a[0] if rows == 1 else a
    return out


def quantize_front(w, codes):
    """decoder.cpp:224-245: z = sum_i (cb_i[code] W_i^T + b_i); x = z W_out^T + b."""
    t = codes.shape[1]
    z = np.zeros((t, cf.Z_DIM))
    for i in range(cf.NQ):
        emb = w[f"q{i}.cb"][codes[i]]                     # [t][8]
        z += emb @ w[f"q{i}.out.w"].T + w[f"q{i}.out.b"]
    return z @ w["q.out.w"].T + w["q.out.b"]


def patch(x, p):
    """decoder.cpp:73-87: [t][c] -> [t*p][c/p], out[ti*p + k][ci] = x[ti][ci*p + k]."""
    t, c = x.shape
    return x.reshape(t, c // p, p).transpose(0, 2, 1).reshape(t * p, c // p)


def layernorm(x, g, b):
    """audio_layer.cpp:17-28 (two-pass mean / variance, eps 1e-5)."""
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    return (x - mean) / np.sqrt(var + 1e-5) * g + b


def rope_tables(pos):
    """audio_layer.cpp:30-44: interleaved pairs (2i, 2i+1) of each 64-wide head, angle
    pos * exp(-ln(10000) * 2i / 64); the reference forms freq and angle in fp32."""
    i = np.arange(cf.HEAD_DIM // 2, dtype=np.float32)
    freq = np.exp(np.float32(-np.log(np.float32(10000.0))) * np.float32(2.0) * i / np.float32(cf.HEAD_DIM))
    ang = np.asarray(pos, np.float32)[:, None] * freq.astype(np.float32)[None, :]
    return np.cos(ang.astype(np.float64)), np.sin(ang.astype(np.float64))


def rope(x, cos, sin):
    """x [t][heads*64] rotated in place of each head's interleaved pairs."""
    t = x.shape[0]
    v = x.reshape(t, cf.HEADS, cf.HEAD_DIM // 2, 2)
    x0, x1 = v[..., 0], v[..., 1]
    c, s = cos[:, None, :], sin[:, None, :]
    return np.stack([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1).reshape(t, -1)


def gelu(x):
    """audio_layer.cpp:46: exact (erf) gelu."""
    from scipy.special import erf
    return 0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))


def attention(q, k, v, q_pos, k_pos, window):
    """Causal attention per head, key kept iff 0 <= q_pos - k_pos < window (window 0:
    no limit) -- attn_scalar.cpp:9-41 (whole decode) and :51-95 (streaming)."""
    out = np.empty_like(q)
    d = q_pos[:, None] - k_pos[None, :]
    keep = d >= 0
    if window > 0:
        keep &= d < window
    for h in range(cf.HEADS):
        sl = slice(h * cf.HEAD_DIM, (h + 1) * cf.HEAD_DIM)
        s = q[:, sl] @ k[:, sl].T / np.sqrt(cf.HEAD_DIM)
        s = np.where(keep, s, -np.inf)
        s = np.exp(s - s.max(axis=1, keepdims=True))
        s /= s.sum(axis=1, keepdims=True)
        out[:, sl] = s @ v[:, sl]
    return out


def layer(w, lp, y, pos, window, cache=None, context=0):
    """audio_layer.cpp:48-110 (cache None) or decoder.cpp:105-186 (streaming: cache is
    a dict with the layer's earlier keys/values and their positions, updated here)."""
    d = cf.D_MODEL
    qkv = layernorm(y, w[lp + "n1.w"], w[lp + "n1.b"]) @ w[lp + "attn.w"].T
    cos, sin = rope_tables(pos)
    q, k, v = rope(qkv[:, :d], cos, sin), rope(qkv[:, d:2 * d], cos, sin), qkv[:, 2 * d:]
    kp = pos
    if cache is not None:
        k = np.concatenate([cache["k"], k])
        v = np.concatenate([cache["v"], v])
        kp = np.concatenate([cache["pos"], pos])
    a = attention(q, k, v, pos, kp, window)
    if cache is not None:  # keep at most `context` keys (decoder.cpp:152-178)
        cache["k"], cache["v"], cache["pos"] = k[-context:], v[-context:], kp[-context:]
    y = y + w[lp + "ls1"] * (a @ w[lp + "proj.w"].T)
    f = gelu(layernorm(y, w[lp + "n2.w"], w[lp + "n2.b"]) @ w[lp + "f1.w"].T)
    return y + w[lp + "ls2"] * (f @ w[lp + "f2.w"].T)


def decode(blob_or_weights, codes, windows=cf.CONTEXTS):
    """codes [16][frames] -> samples [frames * 7680] (decoder.cpp:247-281); `windows`
    per stage (the reference's contexts; 0 = unlimited, for tests of the window)."""
    w = load(blob_or_weights) if isinstance(blob_or_weights, (bytes, bytearray)) else blob_or_weights
    x = quantize_front(w, np.asarray(codes))
    for s, p, nl, window in zip(cf.STAGES, cf.PATCHES, cf.LAYERS, windows):
        x = patch(x, p)
        y = x @ w[f"d{s}.in.w"].T
        pos = np.arange(y.shape[0])
        for n in range(nl):
            y = layer(w, f"d{s}.l{n}.", y, pos, window)
        x = y @ w[f"d{s}.out.w"].T
    return patch(x, cf.FINAL_PATCH).reshape(-1)


class Stream:
    """Streaming decode (decoder.cpp:100-221): chunks in order, state per stage/layer."""

    def __init__(self, blob_or_weights, contexts=cf.CONTEXTS):
        """`contexts`: per-stage windows (the reference's by default; others for tests of
        the window, as decode's `windows`)."""
        self.w = load(blob_or_weights) if isinstance(blob_or_weights, (bytes, bytearray)) else blob_or_weights
        self.contexts = tuple(contexts)
        self.offset = [0] * len(cf.STAGES)
        self.cache = [[{"k": np.zeros((0, cf.D_MODEL)), "v": np.zeros((0, cf.D_MODEL)),
                        "pos": np.zeros(0, np.int64)} for _ in range(nl)] for nl in cf.LAYERS]

    def chunk(self, codes):
        w = self.w
        x = quantize_front(w, np.asarray(codes))
        for si, (s, p, nl, context) in enumerate(zip(cf.STAGES, cf.PATCHES, cf.LAYERS, self.contexts)):
            x = patch(x, p)
            y = x @ w[f"d{s}.in.w"].T
            pos = self.offset[si] + np.arange(y.shape[0])
            for n in range(nl):
                y = layer(w, f"d{s}.l{n}.", y, pos, context, self.cache[si][n], context)
            self.offset[si] += y.shape[0]
            x = y @ w[f"d{s}.out.w"].T
        return patch(x, cf.FINAL_PATCH).reshape(-1)
