"""The GPU audio codec decoder (moss_hip_codec_*, reference csrc/src/decoder.cpp:26-281)
against the codec oracle (oracle/codec_oracle.py, float64; pinned to the reference
decoder compiled from its sources by tests/test_codec_oracle.py, including where the
windows bind and where the streaming caches are trimmed).

Bar: max |gpu - oracle| / max |oracle| <= 1e-3 over the samples (fp32 products and
accumulation against float64, through 12 layers).  Measured errors are printed."""
import numpy as np
import pytest
from conftest import max_rel

import codec_oracle as co
from mosship import HipCodec, MossHipError
from mosship import codec_format as cf
from mosship.moss_format import DT_F16, DT_F32, read_moss_index

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _codes(frames, seed):
    return np.random.default_rng(seed).integers(0, cf.CB_SIZE, (cf.NQ, frames)).astype(np.int32)


@pytest.fixture(scope="module")
def blob16():
    return cf.synth_codec(seed=11, dtype=DT_F16, ln_random=True)


@pytest.fixture(scope="module")
def w16(blob16):
    return co.load(blob16)


@pytest.fixture(scope="module")
def codec16(torch_gpu, blob16):
    c = HipCodec(blob16)
    yield c
    c.close()


@pytest.mark.parametrize("dtype", [DT_F16, DT_F32])
@pytest.mark.parametrize("frames", [1, 3, 9])
def test_decode_vs_oracle(torch_gpu, dtype, frames):
    """Whole-utterance decode (decoder.cpp:247-281) of fp16 (the release) and fp32 matrices."""
    blob = cf.synth_codec(seed=5, dtype=dtype, ln_random=True)
    codes = _codes(frames, 9 + frames)
    c = HipCodec(blob)
    y = c.decode(codes)
    ref = co.decode(blob, codes)
    err = max_rel(y, ref)
    print(f"decode dtype={dtype} frames={frames}: max_rel {err:.2e}", flush=True)
    assert y.shape == (frames * cf.SAMPLES_PER_FRAME,) and np.isfinite(y).all()
    assert err <= TOL
    assert c.last_ms > 0 and all(ms > 0 for ms in c.stage_ms)
    c.close()


def test_decode_window_binds(codec16, w16):
    """70 frames: the last stage runs 2240 rows against its 1600-position window (the
    case test_codec_oracle pins the oracle on against the reference)."""
    codes = _codes(70, 13)
    y = codec16.decode(codes)
    err = max_rel(y, co.decode(w16, codes))
    print(f"decode 70 frames: max_rel {err:.2e}", flush=True)
    assert err <= TOL


def test_stream_trims_every_stage(codec16, w16):
    """140 frames in 4 chunks of 35 (each run as pieces of 32 + 3 frames): every stage's
    ring passes its window (500, 800, 1200, 1600 positions); each chunk against the
    oracle's stream, and the streamed samples against the GPU's whole decode."""
    codes = _codes(140, 33)
    codec16.reset_stream()
    st = co.Stream(w16)
    parts, errs = [], []
    for a in range(0, 140, 35):
        y = codec16.decode_chunk(codes[:, a:a + 35])
        errs.append(max_rel(y, st.chunk(codes[:, a:a + 35])))
        parts.append(y)
    print("stream chunk errors", [f"{e:.2e}" for e in errs], flush=True)
    assert max(errs) <= TOL
    whole = codec16.decode(codes)
    assert max_rel(np.concatenate(parts), whole) <= 1e-4


@pytest.mark.parametrize("chunks", [(1, 1, 2, 4, 8, 3), (5, 9, 2)])
def test_stream_small_windows(torch_gpu, blob16, w16, chunks):
    """Windows of 8, 12, 16, 20 positions (every stage's ring wraps within a few frames)
    and chunk sizes from 1 frame, pieces of at most 4 frames: each chunk against the
    oracle's stream with the same windows."""
    ctx = (8, 12, 16, 20)
    c = HipCodec(blob16, max_chunk_frames=4, contexts=ctx)
    st = co.Stream(w16, contexts=ctx)
    codes = _codes(sum(chunks), 7)
    a, errs = 0, []
    for n in chunks:
        errs.append(max_rel(c.decode_chunk(codes[:, a:a + n]), st.chunk(codes[:, a:a + n])))
        a += n
    print("small-window chunk errors", [f"{e:.2e}" for e in errs], flush=True)
    assert max(errs) <= TOL
    c.close()


def test_graph_replays_equal_direct_launches(torch_gpu, blob16):
    """decode_chunk replays one hipGraph per piece size; the same chunks with direct
    launches give bit-identical samples (same kernels, same inputs), replays included."""
    codes = _codes(24, 3)
    g = HipCodec(blob16)
    e = HipCodec(blob16, eager=True)
    a = 0
    for n in (4, 4, 8, 4, 4):
        yg = g.decode_chunk(codes[:, a:a + n])
        ye = e.decode_chunk(codes[:, a:a + n])
        assert np.array_equal(yg, ye), (a, n)
        a += n
    g.close()
    e.close()


def test_piece_size_does_not_change_results(torch_gpu, blob16):
    """A chunk cut into pieces of 2 or of 32 frames gives the same samples to fp32
    rounding (the stream is causal per row)."""
    codes = _codes(11, 5)
    small = HipCodec(blob16, max_chunk_frames=2)
    big = HipCodec(blob16)
    assert max_rel(small.decode_chunk(codes), big.decode_chunk(codes)) <= 1e-5
    small.close()
    big.close()


def test_reset_and_decode_leave_stream_consistent(codec16):
    """reset_stream restarts positions at 0; decode() runs on a state of its own and
    does not disturb the stream (decoder.cpp:105-115, 247)."""
    codes = _codes(12, 17)
    codec16.reset_stream()
    first = codec16.decode_chunk(codes[:, :6])
    codec16.decode(_codes(5, 1))
    second = codec16.decode_chunk(codes[:, 6:])
    codec16.reset_stream()
    again = codec16.decode_chunk(codes[:, :6])
    assert np.array_equal(first, again)
    whole = codec16.decode(codes)
    assert max_rel(np.concatenate([first, second]), whole) <= 1e-4


def test_codec_errors(torch_gpu, blob16, codec16):
    bad = _codes(2, 0)
    bad[3, 1] = 1024
    with pytest.raises(MossHipError) as e:
        codec16.decode_chunk(bad)
    assert e.value.code == 1
    bad[3, 1] = -1
    with pytest.raises(MossHipError):
        codec16.decode(bad)
    with pytest.raises(MossHipError) as e:
        HipCodec(b"NOPE" + blob16[4:])
    assert e.value.code == 3
    idx = read_moss_index(blob16)
    # drop a tensor: rename its index entry so the loader cannot find it
    off = 16 + 80 * list(idx).index("d5.l1.f2.w")
    broken = bytearray(blob16)
    broken[off:off + 2] = b"zz"
    with pytest.raises(MossHipError) as e:
        HipCodec(bytes(broken))
    assert e.value.code == 3 and "d5.l1.f2.w" in str(e.value)
    # a Q8_0_4X4 (dtype 4) matrix is not a codec matrix
    off = 16 + 80 * list(idx).index("d1.l0.attn.w")
    broken = bytearray(blob16)
    broken[off + 48] = 4
    with pytest.raises(MossHipError) as e:
        HipCodec(bytes(broken))
    assert e.value.code == 4
