"""Greedy picks with NaN logits follow the reference's scan (GPU).

sample_token's greedy branch (csrc/src/sampler.cpp:23-27) starts at index 0 and
moves only on `scratch[i] > scratch[best]`: a NaN elsewhere never wins, and a NaN
at index 0 is never left (every comparison with it is false), so the pick is 0.
Every device pick implements that: the fused local step and the per-operator pick
prologue (greedy_pick_reduce), the sample kernel's greedy branch (pick_greedy),
and the batch engine's audio-head epilogue pairs.

The logits get their NaNs from the model: a NaN fp16 scale in block 0 of a row of
a tied audio matrix makes that code's logit NaN.  Channel 2's code 517 is NaN (it
must be skipped), channel 9's code 0 is NaN (it must be picked; its embedding row
then carries the NaN into every later step, whose logits are all NaN, picking 0).
"""
import numpy as np
import pytest

from mosship import HipBatch, HipLLM, SampleParams
from mosship import moss_format as mf
from oracle import SampleParams as OSP

pytestmark = pytest.mark.gpu


def nan_model(seed=7):
    blob = bytearray(mf.synth_model(seed, ln_random=True))
    idx = mf.read_moss_index(bytes(blob))
    nan16 = np.array([np.nan], np.float16).view(np.uint16)[0]
    for ch, code in ((2, 517), (9, 0)):
        _, rows, cols, off, _ = idx[f"aemb.{ch}"]
        group = off + (code // 4) * (cols // 32) * mf.BLOCK_BYTES  # block 0 of the row's 4-row group
        blob[group + 2 * (code % 4): group + 2 * (code % 4) + 2] = int(nan16).to_bytes(2, "little")
    return bytes(blob)


@pytest.fixture(scope="module")
def setup(oracle):
    blob = nan_model()
    rng = np.random.default_rng(3)
    rows = mf.text_rows(rng.integers(0, mf.VOCAB, 24))
    m = oracle.model(blob)
    m.prefill(rows, a16=True)
    k, v = m.kv_export(len(rows))
    return blob, k, v, m.hidden()


def _reference(oracle, blob, k, v, h, frames, params):
    m = oracle.model(blob)
    m.kv_import(k, v)
    m.set_hidden(h)
    return m.generate(frames, params)["rows"]


@pytest.mark.parametrize("mode", ["fused", "per_op", "sampled_path"])
def test_single_stream_nan_picks(torch_gpu, oracle, setup, mode):
    blob, k, v, h = setup
    frames = 2
    # sampled_path: a sampling configuration whose first frames are greedy (greedy_frames), so
    # the picks run in the sample kernel's greedy branch
    kw = dict(greedy=False, temperature=0.8, top_k=25, top_p=0.95, greedy_frames=frames) \
        if mode == "sampled_path" else dict(greedy=True)
    ref = _reference(oracle, blob, k, v, h, frames, OSP.make(min_frames=frames, **kw))
    assert ref[0, 10] == 0, "channel 9 must pick its NaN code 0"
    assert ref[0, 3] != 517
    print(f"nan picks {mode}: reference frame 0 {ref[0, 1:].tolist()}", flush=True)
    g = HipLLM(blob, kv_fp32=True, per_op=mode == "per_op")
    g.kv_import(k, v, h)
    out = g.generate(frames, SampleParams.make(min_frames=frames, **kw))
    assert np.array_equal(out["rows"][:, 1:], ref[:, 1:])
    g.close()


def test_batch_nan_picks(torch_gpu, oracle, setup):
    """The batch engine's greedy frames (the head GEMM's per-16-code pairs) on 3 streams."""
    blob, k, v, h = setup
    frames = 2
    ref = _reference(oracle, blob, k, v, h, frames, OSP.make(greedy=True, min_frames=frames))
    g = HipLLM(blob)
    b = HipBatch(g, max_streams=4, capacity=64, kv_fp32=True)
    for s in range(3):
        b.set_stream(s, k, v, h)
    out = b.generate(3, frames, SampleParams.make(greedy=True, min_frames=frames))
    for s in range(3):
        assert np.array_equal(out["rows"][:, s, 1:], ref[:, 1:]), s
    b.close()
    g.close()
