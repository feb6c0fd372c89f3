"""Recovery of the fused decode kernels (GPU).

The fused global step and local half need every workgroup of their launch resident at
once; each wait between workgroups is bounded, and a launch whose wait runs out is redone
on the per-operator path from the last good state (llm_model.hip: Model::generate's
recover, Model::global_step).  The condition is forced from the host: MOSS_HIP_POLL_BUDGET
gives the waits a budget of a few poll rounds, so they run out while every kernel still
exits normally.  A recovered run must give what the per-operator model gives (bit for bit
when the first launch already fails: every kernel after that is the per-operator path's),
and agree with the oracle to the usual bars whatever frame the recovery hits.
"""
import numpy as np
import pytest
from conftest import max_rel

from mosship import HipLLM, SampleParams
from mosship import moss_format as mf
from oracle import SampleParams as OSP

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture(scope="module")
def state(oracle, golden_model):
    blob, g = golden_model
    rng = np.random.default_rng(78)
    rows = np.concatenate([g["rows"], mf.text_rows(rng.integers(0, mf.VOCAB, 40))])
    m = oracle.model(blob)
    m.prefill(rows, a16=True)
    k, v = m.kv_export(len(rows))
    return blob, k, v, m.hidden()


def _model(blob, k, v, h, monkeypatch=None, budget=None, **kw):
    if budget is not None:
        monkeypatch.setenv("MOSS_HIP_POLL_BUDGET", str(budget))
    g = HipLLM(blob, kv_fp32=True, **kw)
    if budget is not None:
        monkeypatch.delenv("MOSS_HIP_POLL_BUDGET")
    g.kv_import(k, v, h)
    return g


def test_waits_that_run_out_fall_back_to_per_operator(torch_gpu, state, monkeypatch):
    """Budget of one poll round: the first fused launch of every call runs out; generate
    (greedy, repetition penalty) and global_step give the per-operator model's results."""
    blob, k, v, h = state
    frames = 6
    p = SampleParams.make(greedy=True, min_frames=frames, repetition_penalty=1.3)
    ref = _model(blob, k, v, h, per_op=True)
    g = _model(blob, k, v, h, monkeypatch, budget=1)
    print("generate with budget 1", flush=True)
    a = g.generate(frames, p)
    b = ref.generate(frames, p)
    assert g.fallbacks >= 1
    assert np.array_equal(a["rows"], b["rows"])
    assert np.array_equal(g.hidden(), ref.hidden()) and g.position == ref.position
    row = np.concatenate([[mf.SLOT], a["rows"][-1, 1:]]).astype(np.int32)
    before = g.fallbacks
    g.global_step(row)
    ref.global_step(row)
    assert g.fallbacks == before + 1
    assert np.array_equal(g.hidden(), ref.hidden()) and g.position == ref.position
    ka, va = g.kv_export(g.position)
    kb, vb = ref.kv_export(ref.position)
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    g.close()
    ref.close()


@pytest.mark.parametrize("budget", ["1@1", "1@2", "1@3", "1@6", "3", "24"])
def test_recovery_at_any_frame_matches_oracle(torch_gpu, oracle, state, monkeypatch, budget):
    """Waits that run out in a chosen launch ("1@K": one poll round from the model's K-th
    fused launch on; launch 0 is the sampled local half captured into a graph at creation,
    then generate alternates local half and global step: K = 1 hits L(0), 2 G(0) -- found
    at frame 1's readback --, 3 L(1), 6 G(2)) or wherever a few poll rounds fall short
    ("3", "24").
    Teacher-forced codes and logits against the oracle, and the final hidden state and
    position, to the usual bars."""
    blob, k, v, h = state
    frames = 8
    m = oracle.model(blob)
    m.kv_import(k, v)
    m.set_hidden(h)
    ref = m.generate(frames, OSP.make(greedy=True, min_frames=frames), logits=True)
    forced = ref["rows"].copy()
    forced[:, 0] = mf.SLOT
    g = _model(blob, k, v, h, monkeypatch, budget=budget)
    print(f"teacher-forced generate with budget {budget}", flush=True)
    out = g.generate(frames, SampleParams.make(greedy=True, min_frames=frames), forced=forced, logits=True)
    print(f"budget {budget}: {g.fallbacks} fallbacks", flush=True)
    if "@" in budget:
        assert g.fallbacks == 1
    assert np.mean(out["rows"][:, 1:] == ref["rows"][:, 1:]) >= 0.99
    assert max_rel(out["logits"], ref["logits"]) <= TOL
    assert max_rel(g.hidden(), m.hidden()) <= TOL and g.position == m.position
    g.close()
