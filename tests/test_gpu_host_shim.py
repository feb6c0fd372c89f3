"""The C++ drop-in moss::LlmModel (dsh-moss-tts_amd/host) driven through a
moss_llm-style CLI, vs the oracle and the compiled reference (GPU).  The drop-in
runs with its defaults (fp16 KV, W8A8 prefill as the reference's), so the oracle
emulates the fp16 KV rounding.

Covers the boundary a reference maintainer would link: load, prefill,
generate with timing / on_frame / teacher forcing, and the .mosskv prefix and
MOSSST1 state files (byte layout checked against the reference's loader)."""
import json
import os
import subprocess

import numpy as np
import pytest
from conftest import ROOT, max_rel

from mosship import moss_format as mf
from oracle import REF_SO
from oracle import SampleParams as OSP

pytestmark = pytest.mark.gpu
BIN = os.path.join(ROOT, "tests", "host", "moss_llm_hip")


# The file/flow tests compare decoded codes with the oracle, so the drop-in runs
# its prefill in the reference's MOSS_A16=1 mode (W8A16, smooth in its inputs);
# the default W8A8 prefill is checked on its own below.
A16_ENV = dict(os.environ, MOSS_A16="1")


def _run(*args, env=A16_ENV):
    print("moss_llm_hip", *args, flush=True)
    out = subprocess.run([BIN, *map(str, args)], capture_output=True, text=True, timeout=120, env=env)
    assert out.returncode == 0, out.stderr
    return json.loads(out.stdout)


@pytest.fixture(scope="module")
def files(tmp_path_factory, golden_model):
    blob, g = golden_model
    d = tmp_path_factory.mktemp("shim")
    w = d / "w.moss"
    w.write_bytes(blob)
    rows = g["rows"]
    prompt = d / "rows.txt"
    prompt.write_text("# golden prompt\n" + "\n".join(" ".join(map(str, r)) for r in rows) + "\n")
    return blob, rows, str(w), str(prompt), d


def test_shim_prefill_generate_state(torch_gpu, oracle, files):
    if not os.path.exists(BIN):
        pytest.fail("tests/host/moss_llm_hip not built (make -C dsh-moss-tts_amd)")
    blob, rows, w, prompt, d = files
    state = str(d / "s.state")
    res = _run("--weights", w, "--prompt", prompt, "--frames", 4, "--min-frames", 4, "--greedy", "--rep", 1.2,
               "--save-state", state)
    m = oracle.model(blob, kv_f16=True)
    m.prefill(rows, a16=True)
    _, n_pos, rows_fp, weights_fp, k, v, hidden = mf.read_state(open(state, "rb").read())
    assert n_pos == len(rows) and rows_fp == mf.fp_rows(rows) and weights_fp == mf.fp_weights(blob)
    assert max_rel(hidden, m.hidden()) <= 1e-3
    ok_, ov_ = m.kv_export(len(rows))
    assert max_rel(k, ok_) <= 1e-3 and max_rel(v, ov_) <= 1e-3
    ref = m.generate(4, OSP.make(greedy=True, min_frames=4, repetition_penalty=1.2))
    codes = np.array(res["codes"])
    assert res["frames"] == 4 == res["callbacks"] and res["position"] == m.position
    assert np.mean(codes == ref["rows"][:, 1:]) >= 0.99
    assert res["global_ms_per_frame"] > 0
    if os.path.exists(REF_SO):  # the reference's own loader accepts the file (fingerprints included)
        from oracle import RefCpu
        r = RefCpu().model(blob, threads=2)
        r.load_state(state, rows, ignore_fp=False)
        assert r.position == len(rows)
        assert np.array_equal(r.hidden(), hidden)


def test_shim_prefix_flow(torch_gpu, oracle, files):
    """Voice-prefix flow: prefill + save the first K rows, reload them from the file in a
    fresh process, prefill the rest at start = K; both runs agree exactly and follow the
    oracle; the reference's own load_prefix accepts the file."""
    blob, rows, w, prompt, d = files
    K = 4
    prefix = str(d / "p.mosskv")
    common = ["--weights", w, "--prompt", prompt, "--prefix-rows", K, "--frames", 3, "--min-frames", 3, "--greedy",
              "--rep", 1.0]
    a = _run(*common, "--save-prefix", prefix)
    b = _run(*common, "--load-prefix", prefix)
    assert a["codes"] == b["codes"] and a["hidden0"] == b["hidden0"] and a["position"] == b["position"]
    m = oracle.model(blob, kv_f16=True)
    m.prefill(rows[:K], a16=True)
    m.prefill(rows[K:], start=K, a16=True)
    ref = m.generate(3, OSP.make(greedy=True, min_frames=3))
    assert a["position"] == m.position
    assert np.mean(np.array(a["codes"]) == ref["rows"][:, 1:]) >= 0.99
    with open(prefix, "rb") as f:
        assert f.read(8) == b"MOSSPFX1"
    if os.path.exists(REF_SO):
        from oracle import RefCpu
        r = RefCpu().model(blob, threads=2)
        r.load_prefix(prefix, rows[:K])
        assert r.position == K
        with pytest.raises(RuntimeError):
            r.load_prefix(prefix, rows[:K - 1])  # rows fingerprint mismatch


def test_shim_teacher_forcing(torch_gpu, oracle, files):
    blob, rows, w, prompt, d = files
    m = oracle.model(blob, kv_f16=True)
    m.prefill(rows, a16=True)
    ref = m.generate(3, OSP.make(greedy=True, min_frames=3))
    forced = d / "forced.txt"
    forced.write_text("\n".join(" ".join(map(str, r[1:])) for r in ref["rows"]) + "\n")
    res = _run("--weights", w, "--prompt", prompt, "--frames", 3, "--min-frames", 3, "--greedy", "--rep", 1.0,
               "--force-codes", str(forced))
    assert res["codes"] == ref["rows"][:, 1:].tolist() and res["frames"] == 3
    # forcing its own greedy codes leaves the oracle where free running left it
    mf_ = oracle.model(blob, kv_f16=True)
    mf_.prefill(rows, a16=True)
    mf_.generate(3, OSP.make(greedy=True, min_frames=3), forced=ref["rows"])
    h = mf_.hidden()
    assert res["position"] == mf_.position
    assert abs(res["hidden0"] - h[0]) <= 1e-3 * np.abs(h).max()


def test_shim_sampling_and_gate_dump(torch_gpu, oracle, files):
    """moss_llm's default sampling (main.cpp:133-140) with the sampled end gate and a
    gate dump: codes, frame count and the CSV follow the oracle for the same seed."""
    blob, rows, w, prompt, d = files
    gate = str(d / "gate.csv")
    res = _run("--weights", w, "--prompt", prompt, "--frames", 8, "--min-frames", 2, "--sample", "--seed", 42,
               "--end-mode", "sample", "--dump-gate", gate)
    m = oracle.model(blob, kv_f16=True)
    m.prefill(rows, a16=True)
    ref = m.generate(8, OSP.make(greedy=False, temperature=0.8, top_k=25, top_p=0.95, repetition_penalty=1.2,
                                 end_greedy=False, min_frames=2), seed=42, gate=True)
    assert res["frames"] == len(ref["rows"])
    assert np.mean(np.array(res["codes"]).reshape(-1, 16) == ref["rows"][:, 1:]) >= 0.99
    lines = open(gate).read().splitlines()
    assert lines[0] == "frame,argmax_id,argmax_minus_slot,slot_minus_end"
    assert len(lines) - 1 == len(ref["gate"])
    for f, ln in enumerate(lines[1:]):
        fr, am, am_slot, slot_end = ln.split(",")
        l_end, l_slot, am_o, av = ref["gate"][f]
        assert int(fr) == f and int(am) == int(am_o)
        assert abs(float(am_slot) - (av - l_slot)) <= 2e-4 and abs(float(slot_end) - (l_slot - l_end)) <= 2e-4


REF_CLI = os.path.join(ROOT, "oracle", "_ref", "moss_llm_gpu")


@pytest.mark.parametrize("mode", ["greedy", "sample"])
def test_reference_cli_on_the_drop_in(torch_gpu, oracle, files, mode):
    """The reference's own moss_llm (src/main.cpp, compiled unchanged against the
    drop-in header, oracle/Makefile) runs on the GPU and follows the oracle."""
    if not os.path.exists(REF_CLI):
        pytest.skip("oracle/_ref/moss_llm_gpu not built (needs the reference sources)")
    blob, rows, w, prompt, d = files
    args = ["--weights", w, "--prompt", prompt, "--frames", 6, "--threads", 4]
    if mode == "greedy":
        args += ["--greedy", "--min-frames", 6]
        p = OSP.make(greedy=True, repetition_penalty=1.2, min_frames=6)
    else:
        args += ["--sample", "--seed", 9, "--end-mode", "sample", "--min-frames", 3]
        p = OSP.make(greedy=False, temperature=0.8, top_k=25, top_p=0.95, repetition_penalty=1.2, end_greedy=False,
                     min_frames=3)
    print("moss_llm_gpu", *args, flush=True)
    out = subprocess.run([REF_CLI, *map(str, args)], capture_output=True, text=True, timeout=120, env=A16_ENV)
    assert out.returncode == 0, out.stderr
    res = json.loads(out.stdout)
    m = oracle.model(blob, kv_f16=True)
    m.prefill(rows, a16=True)
    ref = m.generate(6, p, seed=9 if mode == "sample" else 0)
    assert res["frames"] == len(ref["rows"]) >= 3 and res["prompt_rows"] == len(rows)
    assert np.mean(np.array(res["codes"]).reshape(-1, 16) == ref["rows"][:, 1:]) >= 0.99


def test_shim_default_w8a8_prefill(torch_gpu, oracle, files):
    """Without MOSS_A16 the drop-in prefills in W8A8 like the reference: its state file
    holds KV and hidden within the W8A8 end-to-end bar of the oracle's W8A8 prefill."""
    blob, rows, w, prompt, d = files
    state = str(d / "w8.state")
    _run("--weights", w, "--prompt", prompt, "--frames", 1, "--greedy", "--save-state", state,
         env={k: v for k, v in os.environ.items() if k != "MOSS_A16"})
    m = oracle.model(blob, kv_f16=True)
    m.prefill(rows)
    _, n_pos, _, _, k, v, hidden = mf.read_state(open(state, "rb").read())
    ok_, ov_ = m.kv_export(n_pos)
    assert max_rel(hidden, m.hidden()) <= 3e-2
    assert max_rel(k, ok_) <= 3e-2 and max_rel(v, ov_) <= 3e-2


def test_shim_rejects_bad_files(torch_gpu, files):
    blob, rows, w, prompt, d = files
    bad = d / "bad.state"
    bad.write_bytes(b"MOSSST1\x00" + bytes(100))
    out = subprocess.run([BIN, "--weights", w, "--prompt", prompt, "--load-state", str(bad)], capture_output=True,
                         text=True, timeout=120)
    assert out.returncode == 2 and "bad header" in out.stderr
