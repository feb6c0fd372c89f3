"""File formats (.moss v1, 4x4 packing, MOSSST1 state) against the compiled reference (CPU)."""
import os
import tempfile

import numpy as np
import pytest

from mosship import moss_format as mf
from oracle import SampleParams


def test_tensor_list_and_size():
    specs = mf.tensor_specs()
    assert len(specs) == 177
    blob = mf.synth_model(1)
    assert len(blob) == 125047648  # llm_q8x4.moss size in scripts/model_lock.json
    idx = mf.read_moss_index(blob)
    assert set(idx) == {s.name for s in specs}
    dt, rows, cols, off, nbytes = idx["g0.attn.w"]
    assert (dt, rows, cols, nbytes) == (mf.DT_Q8X4, 2304, 768, 1880064)
    assert all(v[3] % 32 == 0 for v in idx.values())


def test_pack_roundtrip_and_layout():
    rng = np.random.default_rng(0)
    q = rng.integers(-127, 128, (8, 64), dtype=np.int8)
    d = rng.random((8, 2)).astype(np.float16)
    w = mf.pack_q8x4(q, d).reshape(2, 2, 136)
    # group 1, block 0: scales of rows 4..7, then row 5's int8 at byte 8 + 32
    assert w[1, 0, 2:4].tobytes() == d[5, 0].tobytes()
    assert w[1, 0, 40:72].view(np.int8).tolist() == q[5, :32].tolist()
    q2, d2 = mf.unpack_q8x4(w.reshape(2, -1), 8, 64)
    assert np.array_equal(q2, q) and np.array_equal(d2.view(np.uint16), d.view(np.uint16))


def test_rows_fingerprint_matches_reference_state(ref, golden_model):
    """A state file written here loads in the reference (its rows fingerprint check passes)
    and the reference's own save_state is byte-identical to our writer."""
    blob, g = golden_model
    m = ref.model(blob, threads=2)
    m.prefill(g["rows"])
    with tempfile.TemporaryDirectory() as td:
        p = os.path.join(td, "a.state")
        m.save_state(p, g["rows"])
        data = open(p, "rb").read()
        magic, n, rows_fp, weights_fp, k, v, h = mf.read_state(data)
        assert magic == mf.STATE_MAGIC and n == len(g["rows"])
        assert rows_fp == mf.fp_rows(g["rows"])
        assert weights_fp == mf.fp_weights(blob)
        ours = mf.write_state(k, v, h, g["rows"], mf.fp_weights(blob))
        assert ours == data
        m2 = ref.model(blob, threads=1)
        p2 = os.path.join(td, "b.state")
        open(p2, "wb").write(ours)
        m2.load_state(p2, g["rows"], ignore_fp=False)
        assert np.array_equal(m2.hidden(), h)
        assert m2.position == n
        with pytest.raises(RuntimeError):
            m2.load_state(p2, g["rows"][:-1])  # rows fingerprint mismatch is rejected
        open(p2, "wb").write(ours[:-100])
        with pytest.raises(RuntimeError):
            m2.load_state(p2, g["rows"])  # truncated file is rejected


def test_missing_tensor_rejected(oracle):
    blob = mf.synth_model(2, drop="g3.proj.b")
    with pytest.raises(RuntimeError, match="g3.proj.b"):
        oracle.model(blob)


def test_misaligned_tensor_rejected(golden_model):
    """Every tensor of a .moss file sits on a 32-byte boundary (the exporter pads to it,
    tools/export_weights.py:254); an index entry moved off it is rejected."""
    blob, _ = golden_model
    mf.read_moss_index(blob)
    bad = bytearray(blob)
    n = int.from_bytes(bad[8:12], "little")
    for i in range(n):
        e0 = 16 + 80 * i
        if bytes(bad[e0:e0 + 48]).rstrip(b"\0") == b"g5.fc_in.w":
            off = int.from_bytes(bad[e0 + 64:e0 + 72], "little")
            bad[e0 + 64:e0 + 72] = (off + 4).to_bytes(8, "little")
    with pytest.raises(ValueError, match="aligned"):
        mf.read_moss_index(bytes(bad))
