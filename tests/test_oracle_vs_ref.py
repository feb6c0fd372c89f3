"""Randomised bit-exact agreement of the C oracle with the compiled reference (CPU;
skipped where oracle/_ref was not built)."""
import os
import subprocess
import sys

import numpy as np
import pytest
from conftest import ROOT

from mosship import moss_format as mf
from oracle import REF_SO, SampleParams


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_gemv_bit_exact(oracle, ref, seed):
    rng = np.random.default_rng(seed)
    for rows, cols in [(2304, 768), (768, 3072), (1024, 768)]:
        w = mf.synth_q8x4(rng, rows, cols)
        x = (rng.standard_normal(cols) * 4).astype(np.float32)
        assert np.array_equal(oracle.gemv(w, rows, cols, x).view(np.uint32),
                              ref.gemv(w, rows, cols, x, threads=4).view(np.uint32))


def test_thread_count_does_not_change_output(ref):
    """Reference invariant (AGENTS.md:164): thread count never changes the result."""
    rng = np.random.default_rng(9)
    w = mf.synth_q8x4(rng, 3072, 768)
    x = rng.standard_normal(768).astype(np.float32)
    assert np.array_equal(ref.gemv(w, 3072, 768, x, threads=1), ref.gemv(w, 3072, 768, x, threads=7))


def test_quantize_bit_exact(oracle, ref):
    rng = np.random.default_rng(3)
    for scale in (1e-3, 1.0, 50.0):
        x = (rng.standard_normal(3072) * scale).astype(np.float32)
        qo, dho, do = oracle.quantize_row(x)
        qr, dhr, dr = ref.quantize_row(x)
        assert np.array_equal(qo, qr) and np.array_equal(dho, dhr) and np.array_equal(do, dr)


def test_sampler_bit_exact(oracle, ref):
    rng = np.random.default_rng(4)
    for trial in range(30):
        logits = (rng.standard_normal(1024) * 3).astype(np.float32)
        prev = rng.integers(0, 1024, rng.integers(0, 60)).astype(np.int32)
        p = SampleParams.make(greedy=bool(trial % 3 == 0), temperature=float(rng.choice([0.5, 0.8, 1.0, 1.3])),
                              top_k=int(rng.choice([0, 1, 5, 25])), top_p=float(rng.choice([0.5, 0.95, 1.0])),
                              repetition_penalty=float(rng.choice([1.0, 1.2])))
        seed = int(rng.integers(0, 2**32))
        assert oracle.sample_token(logits, p, prev, seed=seed) == ref.sample_token(logits, p, prev, seed=seed)


def test_greedy_nan_semantics(oracle, ref):
    """The greedy scan (sampler.cpp:23-27) with NaN logits: a NaN elsewhere never wins, a
    NaN at index 0 is never left (pick 0).  The GPU picks are tested against this."""
    rng = np.random.default_rng(8)
    p = SampleParams.make(greedy=True, repetition_penalty=1.2)
    for case in range(4):
        logits = rng.standard_normal(1024).astype(np.float32)
        logits[[517, 900]] = np.nan
        if case & 1:
            logits[0] = np.nan
        prev = rng.integers(0, 1024, 10).astype(np.int32) if case & 2 else None
        got = oracle.sample_token(logits, p, prev)
        assert got == ref.sample_token(logits, p, prev)
        assert got == 0 if case & 1 else got not in (0, 517, 900)


def test_model_steps_bit_exact(oracle, ref, golden_model):
    """Prefill (W8A8), then greedy frames with the 1.2 repetition penalty: rows and
    hidden state bit-identical between the restatement and the reference."""
    blob, g = golden_model
    rng = np.random.default_rng(11)
    rows = mf.text_rows(rng.integers(0, mf.VOCAB, 20))
    rows[5:9, 1:] = rng.integers(0, 1024, (4, 16))
    o = oracle.model(blob)
    r = ref.model(blob, threads=3)
    o.prefill(rows)
    r.prefill(rows)
    assert np.array_equal(o.hidden(), r.hidden())
    p = SampleParams.make(greedy=True, repetition_penalty=1.2, min_frames=6)
    go = o.generate(6, p)
    gr = r.generate(6, p)
    assert np.array_equal(go["rows"], gr["rows"])
    assert np.array_equal(o.hidden(), r.hidden())
    # teacher forcing with arbitrary codes
    forced = np.concatenate([np.full((4, 1), mf.SLOT), rng.integers(0, 1024, (4, 16))], axis=1).astype(np.int32)
    fo = o.generate(4, p, forced=forced)
    fr = r.generate(4, p, forced=forced)
    assert np.array_equal(fo["rows"], fr["rows"])
    assert np.array_equal(o.hidden(), r.hidden())


def test_gate_dump_mode_bit_exact(oracle, ref, golden_model, tmp_path):
    """With a gate dump the reference takes the gate from the full text head
    (llm.cpp:653-679, A16 in decode mode): the oracle's gate-dump mode matches its
    CSV (argmax id exact, the printed differences to their 4 decimals) and its codes."""
    blob, g = golden_model
    o = oracle.model(blob)
    r = ref.model(blob, threads=2)
    o.prefill(g["rows"])
    r.prefill(g["rows"])
    p = SampleParams.make(greedy=True, min_frames=0)
    path = str(tmp_path / "gate.csv")
    go = o.generate(8, p, gate=True)
    gr = r.generate(8, p, gate_path=path)
    assert np.array_equal(go["rows"], gr["rows"])
    lines = open(path).read().splitlines()
    assert lines[0] == "frame,argmax_id,argmax_minus_slot,slot_minus_end"
    rows = [ln.split(",") for ln in lines[1:]]
    assert len(rows) == len(go["gate"])
    for f, (fr, am, am_slot, slot_end) in enumerate(rows):
        l_end, l_slot, am_o, av = go["gate"][f]
        assert int(fr) == f and int(am) == int(am_o)
        assert f"{av - l_slot:.4f}" == am_slot and f"{l_slot - l_end:.4f}" == slot_end


# The reference in its default activation mode (MOSS_A16 unset: W8A8 decode and
# prefill, gemv.cpp:23-48).  The mode is read once per process, so it runs in a
# child process; it writes its outputs for the parent to compare.
_A8_CHILD = """
import sys, numpy as np
sys.path[:0] = [sys.argv[1], sys.argv[2]]
from oracle import RefCpu, SampleParams
r = RefCpu(a16_mode="off")
assert r.lib.ref_act16_enabled() == 0
blob = open(sys.argv[3], "rb").read()
rows = np.load(sys.argv[4])
forced = np.load(sys.argv[5])
m = r.model(blob, threads=3)
m.prefill(rows)
p = SampleParams.make(greedy=True, repetition_penalty=1.2, min_frames=6)
g = m.generate(6, p)["rows"]
h1 = m.hidden().copy()
f = m.generate(4, p, forced=forced)["rows"]
np.savez(sys.argv[6], gen=g, hidden_gen=h1, forced=f, hidden=m.hidden())
"""


def test_w8a8_decode_bit_exact(oracle, golden_model, tmp_path):
    """The oracle's decode_a8 mode (every decode GEMV quantises its input per 32-block
    and runs the W8A8 row dot, audio heads included) against the reference run with
    MOSS_A16 unset: prefill, 6 greedy frames with the 1.2 penalty, 4 teacher-forced
    frames -- rows and hidden states bit-identical."""
    if not os.path.exists(REF_SO):
        pytest.skip("oracle/_ref/libmossref.so not built here")
    blob, _ = golden_model
    rng = np.random.default_rng(21)
    rows = mf.text_rows(rng.integers(0, mf.VOCAB, 24))
    rows[6:12, 1:] = rng.integers(0, 1024, (6, 16))
    forced = np.concatenate([np.full((4, 1), mf.SLOT), rng.integers(0, 1024, (4, 16))], axis=1).astype(np.int32)
    paths = [str(tmp_path / n) for n in ("m.moss", "rows.npy", "forced.npy", "out.npz")]
    open(paths[0], "wb").write(blob)
    np.save(paths[1], rows)
    np.save(paths[2], forced)
    subprocess.run([sys.executable, "-c", _A8_CHILD, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "dsh-moss-tts_amd"),
                    *paths], check=True, timeout=300)
    ref = np.load(paths[3])
    o = oracle.model(blob, decode_a8=True)
    o.prefill(rows)
    p = SampleParams.make(greedy=True, repetition_penalty=1.2, min_frames=6)
    assert np.array_equal(o.generate(6, p)["rows"], ref["gen"])
    assert np.array_equal(o.hidden(), ref["hidden_gen"])
    assert np.array_equal(o.generate(4, p, forced=forced)["rows"], ref["forced"])
    assert np.array_equal(o.hidden(), ref["hidden"])
    # the W8A16 decode of the same state differs: the mode switch reaches the decode GEMVs
    o16 = oracle.model(blob)
    o16.prefill(rows)
    o16.generate(6, p)
    assert not np.array_equal(o16.hidden(), ref["hidden_gen"])
