"""Tensor list and synthetic weights of the MOSS audio codec decoder (``.moss`` v1).

The tensor names and roles follow the reference loader ``csrc/src/decoder.cpp:26-68``
and the exporter ``tools/export_decoder.py:98-128``:

* ``q{i}.cb`` [1024, 8] fp32 codebook of quantizer i (16 of them), ``q{i}.out.w``
  [512, 8] fp32 and ``q{i}.out.b`` [512]: z = sum_i (cb_i[code_i] W_i^T + b_i);
* ``q.out.w`` [768, 512] and ``q.out.b`` [768]: the front end's output projection;
* four stages ``d1 d3 d5 d7`` (patch 4, 2, 2, 2; 4, 2, 2, 4 layers; d_model 256,
  4 heads x 64): ``d{s}.in.w`` [256, c_in / patch], ``d{s}.out.w`` [c_out, 256], and per
  layer ``attn.w`` [768, 256], ``proj.w`` [256, 256], ``f1.w`` [ffn, 256], ``f2.w``
  [256, ffn], LayerNorms ``n1`` / ``n2`` and per-channel layer scales ``ls1`` / ``ls2``;
* the last stage has 240 output channels: a final patch of 240 gives 7680 samples
  per frame (two interleaved channels of 3840).

The export keeps fp32 for vectors and for matrices whose column count is not a
multiple of 32 (``export_decoder.py:86``); the release file (``decoder_f16.moss``)
stores every other matrix as fp16.  The intermediate stage widths are not fixed
by the loader (it takes every shape from the file); the synthetic set uses 512.

Synthetic weights: N(0, 1/fan_in) matrices, N(0, 1) codebooks, layer scales
0.1 (or random), LayerNorm w = 1, b = 0 (or random).  Seeded.
"""
from __future__ import annotations

import numpy as np

from .moss_format import DT_F16, DT_F32, write_moss

D_MODEL, HEADS, HEAD_DIM = 256, 4, 64
NQ, CB_SIZE, CB_DIM, Z_DIM, Q_OUT = 16, 1024, 8, 512, 768
STAGES = (1, 3, 5, 7)
PATCHES = (4, 2, 2, 2)
LAYERS = (4, 2, 2, 4)
CONTEXTS = (500, 800, 1200, 1600)  # decoder.cpp:21 (ring windows, frames)
FINAL_PATCH = 240
SAMPLES_PER_FRAME = 4 * 2 * 2 * 2 * FINAL_PATCH  # 7680


def codec_specs(stage_out: tuple[int, ...] = (512, 512, 512, 240), ffn: int = 1024) -> list[tuple[str, int, int]]:
    """(name, rows, cols) of every tensor the decoder loads, vectors as rows = 1."""
    out = [("q.out.w", Q_OUT, Z_DIM), ("q.out.b", 1, Q_OUT)]
    for i in range(NQ):
        out += [(f"q{i}.cb", CB_SIZE, CB_DIM), (f"q{i}.out.w", Z_DIM, CB_DIM), (f"q{i}.out.b", 1, Z_DIM)]
    c = Q_OUT
    for s, p, nl, co in zip(STAGES, PATCHES, LAYERS, stage_out):
        if c % p:
            raise ValueError("stage input width must divide by the patch")
        out += [(f"d{s}.in.w", D_MODEL, c // p), (f"d{s}.out.w", co, D_MODEL)]
        for n in range(nl):
            lp = f"d{s}.l{n}."
            out += [(lp + "attn.w", 3 * D_MODEL, D_MODEL), (lp + "proj.w", D_MODEL, D_MODEL),
                    (lp + "f1.w", ffn, D_MODEL), (lp + "f2.w", D_MODEL, ffn)]
            out += [(lp + v, 1, D_MODEL) for v in ("n1.w", "n1.b", "n2.w", "n2.b", "ls1", "ls2")]
        c = co
    if c != FINAL_PATCH:
        raise ValueError("the last stage must have 240 output channels")
    return out


def synth_codec(seed: int = 7, dtype: int = DT_F16, ln_random: bool = False, ls: float = 0.1,
                stage_out: tuple[int, ...] = (512, 512, 512, 240), ffn: int = 1024) -> bytes:
    """A seeded random-init decoder ``.moss``; matrices with cols % 32 == 0 in `dtype`
    (DT_F16 as the release, or DT_F32), everything else fp32."""
    if dtype not in (DT_F16, DT_F32):
        raise ValueError("dtype must be DT_F16 or DT_F32")
    rng = np.random.default_rng(seed)
    entries = []
    for name, rows, cols in codec_specs(stage_out, ffn):
        if rows == 1:
            if name.endswith(".w") and (".n1." in name or ".n2." in name):
                v = 1.0 + 0.1 * rng.standard_normal(cols) if ln_random else np.ones(cols)
            elif name.endswith(".b") and (".n1." in name or ".n2." in name):
                v = 0.1 * rng.standard_normal(cols) if ln_random else np.zeros(cols)
            elif name.endswith(("ls1", "ls2")):
                v = ls * (1.0 + 0.5 * rng.standard_normal(cols)) if ln_random else np.full(cols, ls)
            else:
                v = 0.02 * rng.standard_normal(cols)
            entries.append((name, DT_F32, 1, cols, np.asarray(v, np.float32).tobytes()))
            continue
        if name.endswith(".cb"):
            m = rng.standard_normal((rows, cols))
        else:
            m = rng.standard_normal((rows, cols)) / np.sqrt(cols)
        m = m.astype(np.float32)
        if cols % 32 == 0 and dtype == DT_F16:
            entries.append((name, DT_F16, rows, cols, m.astype(np.float16).tobytes()))
        else:
            entries.append((name, DT_F32, rows, cols, m.tobytes()))
    return write_moss(entries)
