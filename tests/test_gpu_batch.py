"""The batched multi-stream engine (moss_hip_batch_*) vs one oracle LlmModel per stream (GPU).

Every stream must behave exactly like an independent LlmModel: same KV, hidden
and greedy codes as the oracle restatement given the same state.
"""
import numpy as np
import pytest
from conftest import check_quant, d8t_rows, max_rel, q8t_rows

from mosship import HipBatch, HipLLM, SampleParams, lib
from mosship import moss_format as mf
from oracle import SampleParams as OSP

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _state(rng, n):
    k = rng.standard_normal((12, n, 768), dtype=np.float32).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((12, n, 768), dtype=np.float32).astype(np.float16).astype(np.float32)
    return k, v, rng.standard_normal(768, dtype=np.float32)


@pytest.fixture(scope="module")
def setup(golden_model):
    blob, _ = golden_model
    rng = np.random.default_rng(31)
    lens = [5, 64, 65, 130, 200]  # ragged: page boundaries on both sides
    states = [_state(rng, n) for n in lens]
    return blob, lens, states


@pytest.mark.parametrize("kv32", [True, False])
def test_batch_global_step_vs_oracle(torch_gpu, oracle, setup, kv32):
    blob, lens, states = setup
    print(f"batch global step kv32={kv32}", flush=True)
    g = HipLLM(blob)
    b = HipBatch(g, max_streams=8, capacity=256, kv_fp32=kv32)
    for s, (k, v, h) in enumerate(states):
        b.set_stream(s, k, v, h)
        assert b.position(s) == lens[s]
    rng = np.random.default_rng(5)
    rows = np.concatenate([np.full((len(lens), 1), mf.SLOT), rng.integers(0, 1024, (len(lens), 16))], 1).astype(np.int32)
    rows[1, 3] = mf.AUDIO_PAD
    b.global_step(rows)
    for s, (k, v, h) in enumerate(states):
        m = oracle.model(blob, kv_f16=not kv32)
        m.kv_import(k, v)
        m.set_hidden(h)
        m.global_step(rows[s])
        assert b.position(s) == lens[s] + 1 == m.position
        assert max_rel(b.hidden(s), m.hidden()) <= TOL
        bk, bv = b.kv_export(s, lens[s] + 1)
        ok, ov = m.kv_export(lens[s] + 1)
        assert np.array_equal(bk[:, :lens[s]], ok[:, :lens[s]])  # imported pages untouched
        assert max_rel(bk[:, lens[s]], ok[:, lens[s]]) <= TOL and max_rel(bv[:, lens[s]], ov[:, lens[s]]) <= TOL
    b.close()
    g.close()


def test_batch_generate_vs_oracle(torch_gpu, oracle, setup):
    """24 greedy frames with repetition penalty 1.2 (full frame: local transformer, heads,
    gate, global step) on 5 ragged streams, fp32 KV.  Each stream's oracle LlmModel is fed
    the batch's codes as forced rows (llm.cpp:634-733) and predicts every frame from the
    same history: >= 99 % of the predictions equal the batch's picks, positions and (for
    streams whose codes all agree) hidden states match, and codes repeat within the
    channels' histories, so the penalised picks (counts added a launch after the pick)
    are exercised."""
    blob, lens, states = setup
    g = HipLLM(blob)
    b = HipBatch(g, max_streams=8, capacity=256, kv_fp32=True)
    for s, (k, v, h) in enumerate(states):
        b.set_stream(s, k, v, h)
    frames = 24
    out = b.generate(len(lens), frames, SampleParams.make(greedy=True, min_frames=frames, repetition_penalty=1.2))
    assert (out["frames"] == frames).all()
    agree, repeats = [], 0
    for s, (k, v, h) in enumerate(states):
        m = oracle.model(blob)
        m.kv_import(k, v)
        m.set_hidden(h)
        forced = out["rows"][:, s].copy()
        forced[:, 0] = mf.SLOT
        repeats += sum(frames - len(np.unique(forced[:, 1 + ch])) for ch in range(16))
        ref = m.generate(frames, OSP.make(greedy=True, min_frames=frames, repetition_penalty=1.2), forced=forced)
        eq = out["rows"][:, s, 1:] == ref["rows"][:, 1:]
        agree.append(float(np.mean(eq)))
        assert b.position(s) == m.position
        if eq.all():
            assert max_rel(b.hidden(s), m.hidden()) <= TOL
    print("per-stream agreement", agree, "repeated codes", repeats)
    assert repeats > 0
    assert min(agree) >= 0.99


def test_batch_tiled_weights_bit_identical(torch_gpu, setup, monkeypatch):
    """The batch GEMMs (global layers, local layer, audio heads) read the matrices in the
    matrix-core order; with MOSS_HIP_GEMM_TILED=0 the Q8_0_4X4 ones: 3 sampled frames give
    bit-identical codes, hidden states and KV."""
    blob, lens, states = setup
    p = SampleParams.make(greedy=False, temperature=0.9, top_k=40, top_p=0.9, min_frames=3, repetition_penalty=1.2)
    res = []
    for tiled in ("1", "0"):
        print(f"batch tiled={tiled}", flush=True)
        monkeypatch.setenv("MOSS_HIP_GEMM_TILED", tiled)
        g = HipLLM(blob)
        monkeypatch.delenv("MOSS_HIP_GEMM_TILED")
        b = HipBatch(g, max_streams=8, capacity=256)
        for s, (k, v, h) in enumerate(states):
            b.set_stream(s, k, v, h)
        out = b.generate(len(lens), 3, p, seeds=np.arange(11, 11 + len(lens)))
        res.append((out["rows"], [b.hidden(s) for s in range(len(lens))],
                    [b.kv_export(s, b.position(s)) for s in range(len(lens))]))
        b.close()
        g.close()
    (ra, ha, ka), (rb, hb, kb) = res
    assert np.array_equal(ra, rb)
    for s in range(len(lens)):
        assert np.array_equal(ha[s], hb[s])
        assert np.array_equal(ka[s][0], kb[s][0]) and np.array_equal(ka[s][1], kb[s][1])


def test_batch_end_gate_per_stream(torch_gpu, oracle, setup):
    """min_frames = 0: each stream stops on its own end gate, like its own LlmModel."""
    blob, lens, states = setup
    g = HipLLM(blob)
    b = HipBatch(g, max_streams=8, capacity=256, kv_fp32=True)
    for s, (k, v, h) in enumerate(states):
        b.set_stream(s, k, v, h)
    out = b.generate(len(lens), 5, SampleParams.make(greedy=True, min_frames=0))
    for s, (k, v, h) in enumerate(states):
        m = oracle.model(blob)
        m.kv_import(k, v)
        m.set_hidden(h)
        ref = m.generate(5, OSP.make(greedy=True, min_frames=0))
        assert out["frames"][s] == len(ref["rows"])
        assert np.array_equal(out["rows"][:out["frames"][s], s], ref["rows"])
        assert b.position(s) == m.position


def test_batch_capacity_and_errors(torch_gpu, oracle, setup):
    blob, lens, states = setup
    g = HipLLM(blob)
    b = HipBatch(g, max_streams=2, capacity=66)
    k, v, h = states[1]  # 64 positions: 2 more fit
    b.set_stream(0, k, v, h)
    out = b.generate(1, 10, SampleParams.make(greedy=True, min_frames=10))
    m = oracle.model(blob, max_ctx=66)  # the reference's frame loop with kMaxCtx = 66 (llm.cpp:644,703)
    m.kv_import(k, v)
    m.set_hidden(h)
    ref = m.generate(10, OSP.make(greedy=True, min_frames=10))
    assert out["frames"][0] == len(ref["rows"]) == 2
    assert b.position(0) == m.position == 66
    with pytest.raises(lib.MossHipError) as e:
        b.set_stream(1, *_state(np.random.default_rng(0), 67))
    assert e.value.code == lib.EINVAL
    with pytest.raises(lib.MossHipError) as e:
        b.global_step(np.full((1, 17), 9, np.int32))  # stream 0 is at capacity
    assert e.value.code == lib.ESTATE


@pytest.mark.parametrize("model_kv32,batch_kv32", [(False, False), (True, False), (True, True), (False, True)])
def test_batch_admit_bit_exact(torch_gpu, setup, model_kv32, batch_kv32):
    """moss_hip_batch_admit hands a model's state to a stream device to device: the stream's
    K/V are the model's (kv_export), converted exactly to the batch's precision (fp32 -> fp16
    by round to nearest even, fp16 -> fp32 exact); hidden and position follow; another
    stream's pages are untouched."""
    blob, lens, states = setup
    print(f"admit model_kv32={model_kv32} batch_kv32={batch_kv32}", flush=True)
    g = HipLLM(blob, kv_fp32=model_kv32, max_ctx=256)
    k, v, h = states[3]  # 130 positions
    g.kv_import(k, v, h)
    g.global_step(np.array([mf.SLOT] + list(range(100, 116)), np.int32))  # one row the GPU computed
    b = HipBatch(g, max_streams=4, capacity=256, kv_fp32=batch_kv32)
    k1, v1, h1 = states[1]
    b.set_stream(0, k1, v1, h1)
    b.admit(2, g)
    n = g.position
    assert n == lens[3] + 1 and b.position(2) == n
    mk, mv = g.kv_export(n)
    bk, bv = b.kv_export(2, n)
    if model_kv32 and not batch_kv32:
        mk, mv = mk.astype(np.float16).astype(np.float32), mv.astype(np.float16).astype(np.float32)
    assert np.array_equal(bk, mk) and np.array_equal(bv, mv)
    assert np.array_equal(b.hidden(2), g.hidden())
    ok, ov = b.kv_export(0, lens[1])
    assert np.array_equal(ok, k1) and np.array_equal(ov, v1)
    assert np.array_equal(b.hidden(0), h1)
    b.close()
    g.close()


def test_batch_admit_then_generate(torch_gpu, oracle, golden_model):
    """The reference's per-job flow feeding the batch (engine.cpp:447-470): a voice prefix is
    prefilled once and snapshotted; per job the model restores it (restore_prefix) and
    prefills the job's text rows after it, and the batch admits the job device to device.
    Then 16 lock-step greedy frames with penalty 1.2 for the 3 jobs, each against its own
    oracle LlmModel that ran the same prefix and prefill (A16): teacher-forced predictions on
    the batch's codes >= 99 %, hidden states of the jobs whose codes all agree <= 1e-3."""
    blob, _ = golden_model
    rng = np.random.default_rng(23)
    prefix = mf.text_rows(rng.integers(0, mf.VOCAB, 40))
    prefix[10:30, 1:] = rng.integers(0, 1024, (20, 16))  # a voice prompt's audio rows
    jobs = [mf.text_rows(rng.integers(0, mf.VOCAB, n)) for n in (9, 26, 47)]
    g = HipLLM(blob, kv_fp32=True, prefill_a16=True, max_ctx=256)
    g.prefill(prefix)
    g.snapshot_prefix()
    b = HipBatch(g, max_streams=4, capacity=256, kv_fp32=True)
    for j, rows in enumerate(jobs):
        g.restore_prefix()
        assert g.position == len(prefix)
        g.prefill(rows, start=len(prefix))
        b.admit(j, g)
        assert b.position(j) == len(prefix) + len(rows)
    frames, rep = 16, 1.2
    out = b.generate(len(jobs), frames, SampleParams.make(greedy=True, min_frames=frames, repetition_penalty=rep))
    agree = []
    for j, rows in enumerate(jobs):
        m = oracle.model(blob, max_ctx=256)
        m.prefill(prefix, a16=True)
        m.prefill(rows, start=len(prefix), a16=True)
        forced = out["rows"][:, j].copy()
        forced[:, 0] = mf.SLOT
        ref = m.generate(frames, OSP.make(greedy=True, min_frames=frames, repetition_penalty=rep), forced=forced)
        eq = out["rows"][:, j, 1:] == ref["rows"][:, 1:]
        agree.append(float(np.mean(eq)))
        assert b.position(j) == m.position
        if eq.all():
            assert max_rel(b.hidden(j), m.hidden()) <= TOL
    print("admitted jobs: agreement", agree, flush=True)
    assert min(agree) >= 0.99
    b.close()
    g.close()


# The W8A8 decode (the reference with MOSS_A16 unset) end to end: every GEMM input is
# re-quantised per 32-block, so a one-ulp input difference can move one value by a full
# step (amax / 127) and the change cascades; the single-stream W8A8 decode is held to the
# same bars (test_gpu_model.py).  The arithmetic is pinned stage by stage: the quantisers
# of the LN rows, the reduces and fc_in's epilogue by tests/test_gpu_quant_capture.py (the
# same kernels), the attention quantisers of the batch below.
W8A8_E2E_TOL = 3e-2


def test_batch_w8a8_attention_quantisers(torch_gpu, oracle, setup):
    """W8A8 batch: the int8 operand of every attention of a frame -- the paged global
    attention (12 layers), the local attention (position 0, 1) and the fused pick + local
    attention (positions 2..16) -- equals the oracle's quantize_row of the fp32 output it
    recorded, bit for bit, for every stream, read in the matrix-core order."""
    blob, lens, states = setup
    g = HipLLM(blob, decode_a8=True)
    b = HipBatch(g, max_streams=8, capacity=256, kv_fp32=True)
    for s, (k, v, h) in enumerate(states):
        b.set_stream(s, k, v, h)
    b.capture(True)
    out = b.generate(len(lens), 2, SampleParams.make(greedy=True, min_frames=2, repetition_penalty=1.2))
    assert (out["frames"] == 2).all()
    caps = b.capture_attention(8)
    n = len(lens)
    for e, c in enumerate(caps):
        q = q8t_rows(c["q"], n, 768)
        d = d8t_rows(c["d"], n, 768)
        for s in range(n):
            assert np.all(np.isfinite(c["out"][s]))
            check_quant(oracle, c["out"][s], q[s], d[s], f"entry {e} stream {s}")
    print(f"29 attentions x {n} streams: int8 operands bit-exact", flush=True)
    with pytest.raises(lib.MossHipError):  # the W8A16 batch has no W8A8 operand to record
        HipBatch(HipLLM(blob), max_streams=2, capacity=64).capture(True)
    b.close()
    g.close()


def test_batch_w8a8_vs_oracle(torch_gpu, oracle, setup):
    """W8A8 batch (model created with decode_a8) against one W8A8 oracle LlmModel per stream:
    one global step (hidden within the W8A8 bar, imported pages untouched); 12 greedy frames
    with penalty 1.2 whose codes the oracles predict, fed the batch's codes, at >= 95 %; and
    the W8A8 batch differs from the W8A16 batch on the same state (the mode reaches its kernels)."""
    blob, lens, states = setup
    g = HipLLM(blob, decode_a8=True)
    b = HipBatch(g, max_streams=8, capacity=256, kv_fp32=True)
    g16 = HipLLM(blob)
    b16 = HipBatch(g16, max_streams=8, capacity=256, kv_fp32=True)
    for s, (k, v, h) in enumerate(states):
        b.set_stream(s, k, v, h)
        b16.set_stream(s, k, v, h)
    rng = np.random.default_rng(6)
    rows = np.concatenate([np.full((len(lens), 1), mf.SLOT), rng.integers(0, 1024, (len(lens), 16))], 1).astype(np.int32)
    b.global_step(rows)
    b16.global_step(rows)
    herr, sep = [], []
    for s, (k, v, h) in enumerate(states):
        m = oracle.model(blob, decode_a8=True)
        m.kv_import(k, v)
        m.set_hidden(h)
        m.global_step(rows[s])
        herr.append(max_rel(b.hidden(s), m.hidden()))
        sep.append(max_rel(b.hidden(s), b16.hidden(s)))
        bk, _ = b.kv_export(s, lens[s] + 1)
        assert np.array_equal(bk[:, :lens[s]], k)
    print(f"w8a8 batch global step: hidden vs W8A8 oracle {max(herr):.2e}, vs W8A16 batch {min(sep):.2e}", flush=True)
    assert max(herr) <= W8A8_E2E_TOL and min(sep) > 1e-4
    frames = 12
    out = b.generate(len(lens), frames, SampleParams.make(greedy=True, min_frames=frames, repetition_penalty=1.2))
    agree = []
    for s, (k, v, h) in enumerate(states):
        m = oracle.model(blob, decode_a8=True)
        m.kv_import(k, v)
        m.set_hidden(h)
        m.global_step(rows[s])
        forced = out["rows"][:, s].copy()
        forced[:, 0] = mf.SLOT
        ref = m.generate(frames, OSP.make(greedy=True, min_frames=frames, repetition_penalty=1.2), forced=forced)
        agree.append(float(np.mean(out["rows"][:, s, 1:] == ref["rows"][:, 1:])))
    print("w8a8 batch teacher-forced agreement", agree, flush=True)
    assert np.mean(agree) >= 0.95
    for x in (b, b16, g, g16):
        x.close()
