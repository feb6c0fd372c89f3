"""The audio codec decoder's oracle (oracle/codec_oracle.py, numpy float64), pinned
against the reference decoder compiled from its own sources (oracle/_ref) and
against properties the mathematics fixes.  CPU only."""
import numpy as np
import pytest

import codec_oracle as co
from conftest import max_rel
from mosship import codec_format as cf
from mosship.moss_format import DT_F16, DT_F32, read_moss_index

TOL = 1e-4  # float64 restatement vs the fp32 reference, through 12 layers


def _codes(frames, seed):
    return np.random.default_rng(seed).integers(0, cf.CB_SIZE, (cf.NQ, frames)).astype(np.int32)


@pytest.fixture(scope="module")
def blob16():
    return cf.synth_codec(seed=11, dtype=DT_F16, ln_random=True)


@pytest.fixture(scope="module")
def dec16(ref, blob16):
    from oracle import RefDecoder
    d = RefDecoder(ref, blob16, threads=4)
    yield d
    d.close()


def test_synthetic_file_layout():
    """The tensor set the reference loader asks for (decoder.cpp:26-68), with the
    export's dtype rule (export_decoder.py:86): fp16 only where cols % 32 == 0."""
    idx = read_moss_index(cf.synth_codec(seed=1, dtype=DT_F16))
    assert len(idx) == 2 + 3 * cf.NQ + sum(2 + 10 * n for n in cf.LAYERS)
    for name, (dt, rows, cols, _, nb) in idx.items():
        want = DT_F16 if rows > 1 and cols % 32 == 0 else DT_F32
        assert dt == want, name
        assert nb == rows * cols * (2 if dt == DT_F16 else 4)
    assert idx["d7.out.w"][1] == cf.FINAL_PATCH and idx["d1.in.w"][2] == cf.Q_OUT // 4


def test_patch_is_the_documented_reshape():
    """patch() in [t][c] layout equals the [C][T] formulation
    reshape(d, p, t).permute(0, 2, 1).reshape(d, t * p) of the reference's notes."""
    rng = np.random.default_rng(0)
    t, c, p = 5, 12, 4
    x = rng.standard_normal((t, c))
    ct = x.T.reshape(c // p, p, t).transpose(0, 2, 1).reshape(c // p, t * p)
    assert np.array_equal(co.patch(x, p), ct.T)


def test_rope_rotation_properties():
    """Position 0 is the identity; every position keeps each pair's norm; positions
    compose (R(a) R(b) = R(a + b)) up to the fp32 angle rounding."""
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, cf.D_MODEL))
    c0, s0 = co.rope_tables(np.zeros(3, np.int64))
    assert np.allclose(co.rope(x, c0, s0), x, atol=0, rtol=0)
    c, s = co.rope_tables(np.array([7, 100, 999]))
    y = co.rope(x, c, s)
    pair = lambda a: np.hypot(a[:, 0::2], a[:, 1::2])
    assert np.allclose(pair(y), pair(x), rtol=1e-12)
    ca, sa = co.rope_tables(np.array([3, 3, 3]))
    cb, sb = co.rope_tables(np.array([4, 4, 4]))
    c7, s7 = co.rope_tables(np.array([7, 7, 7]))
    assert np.allclose(co.rope(co.rope(x, ca, sa), cb, sb), co.rope(x, c7, s7), atol=1e-5)


def test_attention_window_one_returns_v():
    """A window of 1 keeps only the query's own key: the output is its v."""
    rng = np.random.default_rng(2)
    q, k, v = (rng.standard_normal((6, cf.D_MODEL)) for _ in range(3))
    pos = np.arange(6)
    assert np.allclose(co.attention(q, k, v, pos, pos, 1), v, rtol=0, atol=1e-15)


@pytest.mark.parametrize("dtype", [DT_F16, DT_F32])
def test_oracle_vs_reference_decode(ref, dtype):
    from oracle import RefDecoder
    blob = cf.synth_codec(seed=5, dtype=dtype, ln_random=True)
    d = RefDecoder(ref, blob, threads=4)
    try:
        codes = _codes(3, 9)
        y_ref = d.decode(codes)
    finally:
        d.close()
    assert y_ref.shape == (3 * cf.SAMPLES_PER_FRAME,) and np.isfinite(y_ref).all()
    assert max_rel(co.decode(blob, codes), y_ref) <= TOL


def test_oracle_vs_reference_window_binds(dec16, blob16):
    """70 frames: the last stage runs 2240 rows against a 1600-frame window (the
    earlier stages stay inside theirs).  The oracle matches the reference; without
    the window it gives the same samples up to stage-4 row 1600 and different
    ones after it, so the window is exercised where it binds and nowhere else."""
    codes = _codes(70, 13)
    y_ref = dec16.decode(codes)
    w = co.load(blob16)
    y = co.decode(w, codes)
    assert max_rel(y, y_ref) <= TOL
    y_open = co.decode(w, codes, windows=(0, 0, 0, 0))  # no window anywhere
    cut = 1600 * cf.FINAL_PATCH  # samples of stage-4 rows below the window
    assert np.array_equal(y_open[:cut], y[:cut])
    assert max_rel(y_open[cut:], y[cut:]) > 5 * TOL


def test_streaming_chunks_match_whole_decode(dec16, blob16):
    """Chunks decoded in order give the whole-utterance samples (causal attention,
    the same windows), in the reference and in the oracle's streaming form."""
    codes = _codes(30, 21)
    whole = dec16.decode(codes)
    dec16.reset_stream()
    parts = [dec16.decode_chunk(codes[:, a:b]) for a, b in ((0, 5), (5, 14), (14, 30))]
    assert max_rel(np.concatenate(parts), whole) <= 1e-5
    st = co.Stream(blob16)
    mine = [st.chunk(codes[:, a:b]) for a, b in ((0, 5), (5, 14), (14, 30))]
    for m, p in zip(mine, parts):
        assert max_rel(m, p) <= TOL


def test_streaming_context_trims_every_stage(dec16, blob16):
    """140 frames in 4 chunks: every stage's cache passes its context (500, 800,
    1200, 1600 frames) and is trimmed; the oracle's stream follows the reference's."""
    codes = _codes(140, 33)
    dec16.reset_stream()
    st = co.Stream(blob16)
    for a in range(0, 140, 35):
        y_ref = dec16.decode_chunk(codes[:, a:a + 35])
        assert max_rel(st.chunk(codes[:, a:a + 35]), y_ref) <= TOL, a
