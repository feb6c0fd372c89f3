"""The reference's C API (csrc/include/moss/tts.h: moss_create / moss_set_voice /
moss_text_tokens / moss_set_sampling / moss_speak / moss_destroy, implemented by
csrc/src/capi.cpp over TtsEngine, both compiled unchanged) end to end on the GPU
drop-ins (GPU).

oracle/_ref/tts_cpu, tts_gpu and tts_gpu_codec are one harness (oracle/capi_main.cpp)
linked three ways: the reference's CPU LlmModel and AudioDecoder; the GPU LlmModel
with the reference's AudioDecoder; both GPU drop-ins.  Each creates an engine,
sets a synthetic voice, and speaks the same text twice, keeping the int16 PCM its
callback receives (capi.cpp's own float -> int16 conversion).

The model is the seeded synthetic one with its end gate disabled, because
moss_speak cannot set min_frames (capi.cpp:66-78) and a random model's gate
would stop at a random frame: the end token's row of wte gets zero scales
(l_end = 0) and the slot token's row all-positive int8 values, with the local
ln_f shifted by +5 so its output is positive (l_slot > 0).
"""
import json
import os
import subprocess

import numpy as np
import pytest
from conftest import GOLDEN, ROOT

from mosship import codec_format as cf
from mosship import moss_format as mf

pytestmark = pytest.mark.gpu
REF_DIR = os.path.join(ROOT, "oracle", "_ref")
TEXT = "The quick brown fox jumps over the lazy dog, and the morning sun rises slowly above the quiet hills."


def gate_free_model(seed=1234):
    blob = bytearray(mf.synth_model(seed))
    idx = mf.read_moss_index(bytes(blob))
    _, rows, cols, off, _ = idx["wte"]
    nb = cols // 32
    for b in range(nb):
        o = off + ((mf.END // 4) * nb + b) * mf.BLOCK_BYTES + 2 * (mf.END % 4)
        blob[o:o + 2] = b"\x00\x00"  # fp16 scale 0 of the end row
        o = off + ((mf.SLOT // 4) * nb + b) * mf.BLOCK_BYTES + 8 + 32 * (mf.SLOT % 4)
        blob[o:o + 32] = bytes([127]) * 32  # int8 +127 across the slot row
    _, _, _, off, _ = idx["local.lnf.b"]
    blob[off:off + 768 * 4] = np.full(768, 5.0, np.float32).tobytes()
    return bytes(blob)


@pytest.fixture(scope="module")
def weights(tmp_path_factory):
    for exe in ("tts_cpu", "tts_gpu"):
        if not os.path.exists(os.path.join(REF_DIR, exe)):
            pytest.skip(f"oracle/_ref/{exe} not built (needs the reference sources where the build ran)")
    d = tmp_path_factory.mktemp("capi")
    llm, dec = d / "llm.moss", d / "dec.moss"
    llm.write_bytes(gate_free_model())
    dec.write_bytes(cf.synth_codec(seed=3, dtype=mf.DT_F16))
    return str(llm), str(dec), os.path.join(GOLDEN, "tokenizer.mossvocab")


def speak(exe, weights, workdir, seed, greedy, frames, env_extra, unset=()):
    llm, dec, tok = weights
    os.makedirs(workdir, exist_ok=True)
    env = dict(os.environ, **env_extra)
    for k in unset:
        env.pop(k, None)
    print(f"{exe} seed={seed} greedy={greedy} env={env_extra} unset={list(unset)}", flush=True)
    p = subprocess.run([os.path.join(REF_DIR, exe), llm, dec, tok, workdir, TEXT, str(seed), str(int(greedy)),
                        str(frames)], capture_output=True, text=True, timeout=300, env=env)
    assert p.returncode == 0, p.stderr[-2000:]
    lines = [json.loads(ln) for ln in p.stdout.splitlines() if ln.startswith("{\"")]
    head = next(x for x in lines if "version" in x)
    calls = [x for x in lines if "speak" in x]
    assert [c["speak"] for c in calls] == [1, 2]
    pcm = [np.fromfile(os.path.join(workdir, f"speak{i}.pcm"), np.int16) for i in (1, 2)]
    for c in calls:
        print(f"  speak {c['speak']}: {c['samples']} samples in {c['ms']:.1f} ms, fallbacks {c['fallbacks']}",
              flush=True)
    return head, calls, pcm


@pytest.mark.parametrize("greedy,seed", [(True, 0), (False, 42)])
def test_tts_api_gpu_llm_matches_cpu(torch_gpu, weights, tmp_path, greedy, seed):
    """MOSS_A16=1 (W8A16 prefill and decode, where the GPU path's codes are the reference's):
    every int16 sample equals the CPU build's, for both calls."""
    frames = 8
    env = {"MOSS_A16": "1", "MOSS_HIP_KV": "fp32"}
    gh, gc, gp = speak("tts_gpu", weights, str(tmp_path / "gpu"), seed, greedy, frames, env)
    ch, cc, cp = speak("tts_cpu", weights, str(tmp_path / "cpu"), seed, greedy, frames, env)
    assert gh["version"] == ch["version"] and gh["text_tokens"] == ch["text_tokens"]
    spf = cf.SAMPLES_PER_FRAME  # int16 values per frame (two interleaved channels)
    for i in range(2):
        assert gc[i]["sample_rate"] == cc[i]["sample_rate"] == 48000
        assert gp[i].size == cp[i].size == frames * spf, (gp[i].size, cp[i].size)
        assert np.array_equal(gp[i], cp[i]), f"speak {i + 1}: int16 PCM differs"
        assert gc[i]["fallbacks"] == 0
    assert np.array_equal(gp[0], gp[1])  # the same text and seed again


def test_tts_api_both_gpu_dropins(torch_gpu, weights, tmp_path):
    """Both GPU drop-ins under the C API (the fused LLM kernels and the codec graphs share the
    GPU): the codes are the CPU build's, so the int16 PCM differs only by the GPU codec's
    ~1e-6 relative float error, i.e. at most 1 LSB where a sample lands next to a rounding
    boundary; the process's fused-launch fallbacks (moss_hip_fallbacks_total) and the wall
    time of each moss_speak are reported."""
    if not os.path.exists(os.path.join(REF_DIR, "tts_gpu_codec")):
        pytest.skip("oracle/_ref/tts_gpu_codec not built")
    env = {"MOSS_A16": "1", "MOSS_HIP_KV": "fp32"}
    gh, gc, gp = speak("tts_gpu_codec", weights, str(tmp_path / "gpuc"), 0, True, 8, env)
    ch, cc, cp = speak("tts_cpu", weights, str(tmp_path / "cpu"), 0, True, 8, env)
    for i in range(2):
        assert gp[i].size == cp[i].size
        diff = np.abs(gp[i].astype(np.int32) - cp[i].astype(np.int32))
        print(f"  speak {i + 1}: {int(np.count_nonzero(diff))} of {diff.size} samples differ, max {int(diff.max())} LSB; "
              f"GPU {gc[i]['ms']:.1f} ms vs CPU {cc[i]['ms']:.1f} ms; fallbacks {gc[i]['fallbacks']}", flush=True)
        assert diff.max() <= 1
        assert gc[i]["fallbacks"] >= 0


def test_tts_api_release_default(torch_gpu, weights, tmp_path):
    """MOSS_A16 unset: moss_create puts the release setting, MOSS_A16=decode (capi.cpp:51-52,
    the _putenv_s call, here setenv), before the engine loads -- W8A16 decode after a W8A8
    prefill on the GPU drop-in, as in the CPU build; both runs complete the same frames."""
    gh, gc, gp = speak("tts_gpu", weights, str(tmp_path / "gpu"), 0, True, 6, {"MOSS_HIP_KV": "fp32"},
                       unset=("MOSS_A16",))
    ch, cc, cp = speak("tts_cpu", weights, str(tmp_path / "cpu"), 0, True, 6, {}, unset=("MOSS_A16",))
    assert gh["a16_env_before"] == ch["a16_env_before"] == "(unset)"
    assert gh["a16_env_after"] == ch["a16_env_after"] == "decode"
    for i in range(2):
        assert gp[i].size == cp[i].size == 6 * cf.SAMPLES_PER_FRAME
    same = float(np.mean(gp[0] == cp[0]))
    print(f"  release mode: {same:.4f} of int16 samples equal to the CPU build (W8A8 prefill)", flush=True)
