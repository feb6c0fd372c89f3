"""Writes the golden vectors under tests/golden/ by running the compiled reference.

The reference's LLM path has no fixtures of its own for Q8_0_4X4, W8A16,
attention or the frame loop (its csrc/tests/test_kernels.cpp computes an fp64
reference on the fly and never touches them).  So this script runs the
reference C++ itself -- compiled from its sources by oracle/Makefile into
oracle/_ref/libmossref.so -- on seeded inputs and stores inputs and outputs as
small .npz files.  The synthetic model is not stored: it is regenerated from its
seed by mosship.moss_format.synth_model, and its sha256 is recorded so a change
of generator is caught.

Usage:  make -C oracle && python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "dsh-moss-tts_amd"))

from mosship import moss_format as mf  # noqa: E402
from oracle import RefCpu, SampleParams  # noqa: E402

MODEL_SEED = 7


def save(name, **arrays):
    path = os.path.join(HERE, name)
    np.savez_compressed(path, **arrays)
    print(f"wrote {name} ({os.path.getsize(path)} bytes)")


def gemv_fixtures(r: RefCpu):
    rng = np.random.default_rng(101)
    for rows, cols in [(8, 768), (8, 3072), (16, 128)]:
        w = mf.synth_q8x4(rng, rows, cols)
        x = rng.standard_normal(cols).astype(np.float32)
        y = r.gemv(w, rows, cols, x, threads=1)
        nb = cols // 32
        deq = np.stack([r.dequant_row(w.reshape(rows // 4, -1)[i // 4], nb, i % 4) for i in range(rows)])
        w8a8 = np.array([r.row_dot_w8a8(w.reshape(rows // 4, -1)[i // 4], nb, i % 4, x) for i in range(rows)],
                        np.float32)
        xs = rng.standard_normal((3, cols)).astype(np.float32)
        gemm_a16 = r.gemm(w, rows, cols, xs, threads=1)  # MOSS_A16=decode, not suspended: A16
        r.lib.ref_act16_suspend(1)
        gemm_w8a8 = r.gemm(w, rows, cols, xs, threads=1)
        r.lib.ref_act16_suspend(0)
        save(f"gemv_r{rows}_k{cols}.npz", w=w, x=x, y=y, deq=deq, w8a8=w8a8, xs=xs, gemm_a16=gemm_a16,
             gemm_w8a8=gemm_w8a8)


def quant_fixture(r: RefCpu):
    rng = np.random.default_rng(202)
    x = rng.standard_normal(768).astype(np.float32) * 3.0
    x[0:32] = 0.0                                  # all-zero block: d = 0, id = 0
    x[32:64] = np.arange(32, dtype=np.float32) - 16.0  # amax 16 -> exact-ish grid
    x[64:96] = np.float32(1e-30) * rng.standard_normal(32).astype(np.float32)  # tiny values
    # values landing exactly on .5 after scaling: amax 127 -> id 1 -> ties to even
    x[96:128] = np.array([127.0] + [k + 0.5 for k in range(-15, 16)], np.float32)
    q, dh, d = r.quantize_row(x)
    halves = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    h2f = np.array([r.lib.ref_half_to_float(int(h)) for h in halves[::97]], np.float32)
    fvals = np.concatenate([rng.standard_normal(4000).astype(np.float32) * 1e3,
                            np.float32(2.0) ** np.arange(-30, 17, dtype=np.float32),
                            np.array([65504, 65519, 65520, 1e-8, 6.1e-5, 5.96e-8, 2.98e-8], np.float32)])
    f2h = np.array([r.lib.ref_float_to_half(float(v)) for v in fvals], np.uint16)
    save("quant_fp16.npz", x=x, q=q, dh=dh, d=d, halves=halves[::97], h2f=h2f, fvals=fvals, f2h=f2h)


def attention_fixture(r: RefCpu):
    rng = np.random.default_rng(303)
    out = {}
    for n in (0, 32, 130):  # keys in the cache; +1 for the query row's own k/v
        # fp16-representable inputs, stored as fp16 to keep the fixture small
        q_row = rng.standard_normal(3 * 768).astype(np.float16)
        kc = rng.standard_normal((n, 768)).astype(np.float16)
        vc = rng.standard_normal((n, 768)).astype(np.float16)
        out[f"q{n}"], out[f"k{n}"], out[f"v{n}"] = q_row, kc, vc
        out[f"o{n}"] = r.attention_window(q_row.astype(np.float32), kc.astype(np.float32), vc.astype(np.float32),
                                          avx2=True)
    save("attention_window.npz", **out)


def sampler_fixture(r: RefCpu):
    rng = np.random.default_rng(404)
    logits = rng.standard_normal(1024).astype(np.float32)
    prev = rng.integers(0, 1024, 40).astype(np.int32)
    prev[:10] = int(np.argmax(logits))  # the current argmax appears 10 times
    cases = [
        SampleParams.make(greedy=True),
        SampleParams.make(greedy=True, repetition_penalty=1.2),
        SampleParams.make(greedy=False, temperature=0.8, top_k=25, top_p=0.95, repetition_penalty=1.2),
        SampleParams.make(greedy=False, temperature=1.0, top_k=0, top_p=1.0),
        SampleParams.make(greedy=False, temperature=0.5, top_k=1),
    ]
    picks = []
    params = []
    for p in cases:
        for seed in (0, 1, 12345):
            for skip in (0, 3):
                picks.append(r.sample_token(logits, p, prev, seed=seed, skip=skip))
                params.append([p.greedy, p.top_k, p.end_greedy, p.min_frames, p.greedy_frames, seed, skip,
                               p.temperature, p.top_p, p.repetition_penalty])
    rng_stream = r.rng_stream(0xDEADBEEF12345678, 32)
    save("sampler.npz", logits=logits, prev=prev, picks=np.array(picks, np.int32), params=np.array(params, np.float64),
         rng_seed=np.array([0xDEADBEEF12345678], np.uint64), rng_stream=rng_stream)


def model_fixture(r: RefCpu):
    blob = mf.synth_model(MODEL_SEED, ln_random=True)
    sha = hashlib.sha256(blob).hexdigest()
    rng = np.random.default_rng(505)
    rows = mf.text_rows(rng.integers(0, mf.VOCAB, 6))
    rows[3, 1:] = rng.integers(0, 1024, 16)  # one audio row
    m = r.model(blob, threads=2)
    m.prefill(rows)
    hidden_prefill = m.hidden()
    with tempfile.TemporaryDirectory() as td:
        st = os.path.join(td, "s.state")
        m.save_state(st, rows)
        with open(st, "rb") as f:
            state_blob = f.read()
    _, n_pos, _, _, k, v, _ = mf.read_state(state_blob)
    step_row = np.array([mf.SLOT] + list(rng.integers(0, 1024, 16)), np.int32)
    gen = m.generate(4, SampleParams.make(greedy=True, min_frames=4))
    hidden_gen = m.hidden()
    pos_gen = m.position
    m.close()
    # A16 prefill (MOSS_A16=1): the mode is fixed per process, so run it in a child.
    code = (
        "import sys, numpy as np; sys.path[:0] = [%r, %r];"
        "from oracle import RefCpu; from mosship import moss_format as mf;"
        "r = RefCpu(a16_mode='1'); blob = mf.synth_model(%d, ln_random=True);"
        "rows = np.load(sys.argv[1])['rows']; m = r.model(blob, threads=2); m.prefill(rows);"
        "np.save(sys.argv[2], m.hidden())" % (os.path.join(ROOT, "oracle"), os.path.join(ROOT, "dsh-moss-tts_amd"),
                                              MODEL_SEED))
    with tempfile.TemporaryDirectory() as td:
        rp = os.path.join(td, "rows.npz")
        np.savez(rp, rows=rows)
        hp = os.path.join(td, "h.npy")
        subprocess.run([sys.executable, "-c", code, rp, hp], check=True)
        hidden_prefill_a16 = np.load(hp)
    save("model_small.npz", seed=np.array([MODEL_SEED]), sha256=np.frombuffer(bytes.fromhex(sha), np.uint8),
         rows=rows, hidden_prefill=hidden_prefill, hidden_prefill_a16=hidden_prefill_a16,
         k_prefill_l0=k[0], v_prefill_l11=v[11], step_row=step_row, gen_rows=gen["rows"], hidden_gen=hidden_gen,
         pos_gen=np.array([pos_gen]))


def main():
    r = RefCpu(a16_mode="decode")
    gemv_fixtures(r)
    quant_fixture(r)
    attention_fixture(r)
    sampler_fixture(r)
    model_fixture(r)


if __name__ == "__main__":
    main()
