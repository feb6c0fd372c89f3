"""On-device sampling (sample_token, sampler.cpp:9-79; end_reached, llm.cpp:30-35)
vs the oracle, through the C ABI (GPU).

The oracle's sampler is pinned bit-exactly to the compiled reference
(test_oracle_vs_ref, golden sampler picks).  The device draws from the same
xoshiro128** stream in the same order, so the same seed gives the same codes;
the only difference allowed is the ~1e-6 relative logit noise of the GPU's
summation order, which can move a draw that lands on a boundary (probability
~1e-6 per draw).  Teacher forcing keeps every draw on identical histories, so
one such flip costs one code, not the rest of the run.
"""
import numpy as np
import pytest

from mosship import HipBatch, HipLLM, SampleParams
from mosship import moss_format as mf
from oracle import SampleParams as OSP

pytestmark = pytest.mark.gpu

MODES = {
    "engine_default": dict(temperature=0.8, top_k=25, top_p=0.95, repetition_penalty=1.2, greedy_frames=2),
    "full_sort": dict(temperature=1.0, top_k=0, top_p=1.0),
    "narrow": dict(temperature=1.3, top_k=5, top_p=0.5, repetition_penalty=1.1),
    "no_temperature": dict(temperature=0.0, top_k=64, top_p=0.9),
}


@pytest.fixture(scope="module")
def state(oracle, golden_model):
    blob, g = golden_model
    rng = np.random.default_rng(99)
    rows = np.concatenate([g["rows"], mf.text_rows(rng.integers(0, mf.VOCAB, 30))])
    m = oracle.model(blob)
    m.prefill(rows, a16=True)
    k, v = m.kv_export(len(rows))
    return blob, k, v, m.hidden()


def _oracle(oracle, blob, k, v, h):
    m = oracle.model(blob)
    m.kv_import(k, v)
    m.set_hidden(h)
    return m


@pytest.mark.parametrize("mode", list(MODES))
def test_sampled_teacher_forced(torch_gpu, oracle, state, mode):
    blob, k, v, h = state
    frames, seed = 12, 1234 + len(mode)
    kw = MODES[mode]
    print(f"sampling mode {mode} seed {seed}", flush=True)
    ref = _oracle(oracle, blob, k, v, h).generate(frames, OSP.make(greedy=False, min_frames=frames, **kw), seed=seed)
    assert len(ref["rows"]) == frames
    g = HipLLM(blob, kv_fp32=True)
    g.kv_import(k, v, h)
    out = g.generate(frames, SampleParams.make(greedy=False, min_frames=frames, **kw), seed=seed, forced=ref["rows"])
    agree = np.mean(out["rows"][:, 1:] == ref["rows"][:, 1:])
    print(f"{mode}: agreement {agree:.4f}, distinct codes {len(np.unique(ref['rows'][:, 1:]))}")
    assert agree >= 0.99
    if mode != "no_temperature":  # sampling really happened: not the greedy codes
        gr = _oracle(oracle, blob, k, v, h).generate(frames, OSP.make(greedy=True, min_frames=frames),
                                                     forced=ref["rows"])
        assert np.mean(gr["rows"][2:, 1:] == ref["rows"][2:, 1:]) < 0.9
    g.close()


def test_sampled_free_running_and_end_gate(torch_gpu, oracle, state):
    """Free-running sampling with the sampled end gate (end_greedy = false): the
    frame where the end draw fires and every code before it follow the oracle."""
    blob, k, v, h = state
    kw = dict(temperature=0.8, top_k=25, top_p=0.95, repetition_penalty=1.2, end_greedy=False, min_frames=2)
    for seed in (5, 6, 7):
        ref = _oracle(oracle, blob, k, v, h).generate(10, OSP.make(greedy=False, **kw), seed=seed)
        g = HipLLM(blob, kv_fp32=True)
        g.kv_import(k, v, h)
        out = g.generate(10, SampleParams.make(greedy=False, **kw), seed=seed)
        print(f"seed {seed}: frames gpu {len(out['rows'])} oracle {len(ref['rows'])}", flush=True)
        assert len(out["rows"]) == len(ref["rows"])
        assert np.mean(out["rows"] == ref["rows"]) >= 0.99
        g.close()


@pytest.mark.parametrize("greedy_frames", [0, 2])
def test_batch_sampled_vs_oracle(torch_gpu, oracle, state, greedy_frames):
    """Each stream of the batched engine samples like its own LlmModel with its own seed.
    greedy_frames = 2: the first two frames run the greedy frame graph (channel picks fused
    into the next position's attention, repetition counts added a launch later), the rest
    the sampled one, on the same counts."""
    blob, k, v, h = state
    n_pos = k.shape[1]
    seeds = [11, 22, 33, 44, 55]
    kw = dict(temperature=0.8, top_k=25, top_p=0.95, repetition_penalty=1.2, min_frames=5,
              greedy_frames=greedy_frames)
    g = HipLLM(blob)
    b = HipBatch(g, max_streams=8, capacity=128, kv_fp32=True)
    hs = [h * (1.0 + 0.1 * s) for s in range(len(seeds))]  # distinct streams
    for s in range(len(seeds)):
        b.set_stream(s, k, v, hs[s])
    out = b.generate(len(seeds), 5, SampleParams.make(greedy=False, **kw), seeds=seeds)
    for s, seed in enumerate(seeds):
        ref = _oracle(oracle, blob, k, v, hs[s]).generate(5, OSP.make(greedy=False, **kw), seed=seed)
        assert out["frames"][s] == len(ref["rows"]) == 5
        agree = np.mean(out["rows"][:, s, 1:] == ref["rows"][:, 1:])
        print(f"stream {s} seed {seed}: agreement {agree:.4f}", flush=True)
        assert agree >= 0.99
        assert b.position(s) == n_pos + 4
    b.close()
    g.close()
