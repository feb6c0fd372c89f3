"""The C oracle against golden vectors written by the compiled reference (tests/golden/).

Everything here is bit-exact: the oracle restates the reference operator by
operator and both are compiled without FP contraction.
"""
import numpy as np
import pytest
from conftest import golden

from oracle import SampleParams


@pytest.mark.parametrize("name,rows,cols", [("gemv_r8_k768.npz", 8, 768), ("gemv_r8_k3072.npz", 8, 3072),
                                            ("gemv_r16_k128.npz", 16, 128)])
def test_gemv_dequant_gemm_golden(oracle, name, rows, cols):
    g = golden(name)
    y = oracle.gemv(g["w"], rows, cols, g["x"])
    assert np.array_equal(y.view(np.uint32), g["y"].view(np.uint32))
    nb = cols // 32
    groups = g["w"].reshape(rows // 4, -1)
    for r in range(rows):
        assert np.array_equal(oracle.dequant_row(groups[r // 4], nb, r % 4), g["deq"][r])
        assert np.float32(oracle.row_dot_w8a8(groups[r // 4], nb, r % 4, g["x"])) == g["w8a8"][r]
    assert np.array_equal(oracle.gemm(g["w"], rows, cols, g["xs"], a16=True), g["gemm_a16"])
    assert np.array_equal(oracle.gemm(g["w"], rows, cols, g["xs"], a16=False), g["gemm_w8a8"])
    # the W8A8 product on operands quantised beforehand (what the GPU capture tests feed it)
    qd = [oracle.quantize_row(x) for x in g["xs"]]
    y = oracle.gemm_w8a8_q(g["w"], rows, cols, np.stack([q for q, _, _ in qd]), np.stack([d for _, _, d in qd]))
    assert np.array_equal(y.view(np.uint32), g["gemm_w8a8"].view(np.uint32))


def test_quantize_and_fp16_golden(oracle):
    g = golden("quant_fp16.npz")
    q, dh, d = oracle.quantize_row(g["x"])
    assert np.array_equal(q, g["q"])
    assert np.array_equal(dh, g["dh"])
    assert np.array_equal(d.view(np.uint32), g["d"].view(np.uint32))
    h2f = np.array([oracle.half_to_float(h) for h in g["halves"]], np.float32)
    assert np.array_equal(h2f.view(np.uint32), g["h2f"].view(np.uint32))
    f2h = np.array([oracle.float_to_half(v) for v in g["fvals"]], np.uint16)
    assert np.array_equal(f2h, g["f2h"])


def test_attention_golden(oracle):
    """attention_core restated vs the reference's AVX2 attention_window (same maths,
    different summation order): agreement to fp32 rounding, not bit-exact."""
    g = golden("attention_window.npz")
    for n in (0, 32, 130):
        q_row = g[f"q{n}"].astype(np.float32)
        k = np.concatenate([g[f"k{n}"].astype(np.float32), q_row[None, 768:1536]])
        v = np.concatenate([g[f"v{n}"].astype(np.float32), q_row[None, 1536:]])
        out = oracle.attention(k, v, q_row[:768])
        ref = g[f"o{n}"]
        assert np.max(np.abs(out - ref)) <= 2e-6 * max(1.0, np.max(np.abs(ref)))


def test_sampler_golden(oracle):
    g = golden("sampler.npz")
    assert np.array_equal(oracle.rng_stream(int(g["rng_seed"][0]), 32), g["rng_stream"])
    for pick, prm in zip(g["picks"], g["params"]):
        greedy, top_k, end_greedy, min_frames, greedy_frames, seed, skip, temp, top_p, rep = prm
        p = SampleParams.make(greedy=bool(greedy), temperature=float(temp), top_k=int(top_k), top_p=float(top_p),
                              repetition_penalty=float(rep))
        assert oracle.sample_token(g["logits"], p, g["prev"], seed=int(seed), skip=int(skip)) == pick


def test_model_golden(oracle, golden_model):
    """Full restated LlmModel vs the reference on a seeded synthetic model: W8A8
    prefill (release default), KV layout, 4 greedy frames with local steps, gate,
    heads and global steps -- hidden states and codes bit-identical."""
    blob, g = golden_model
    m = oracle.model(blob)
    m.prefill(g["rows"])
    assert np.array_equal(m.hidden().view(np.uint32), g["hidden_prefill"].view(np.uint32))
    k, v = m.kv_export(len(g["rows"]))
    assert np.array_equal(k[0], g["k_prefill_l0"])
    assert np.array_equal(v[11], g["v_prefill_l11"])
    out = m.generate(4, SampleParams.make(greedy=True, min_frames=4))
    assert np.array_equal(out["rows"], g["gen_rows"])
    assert np.array_equal(m.hidden().view(np.uint32), g["hidden_gen"].view(np.uint32))
    assert m.position == int(g["pos_gen"][0])


def test_model_prefill_a16_golden(oracle, golden_model):
    blob, g = golden_model
    m = oracle.model(blob)
    m.prefill(g["rows"], a16=True)
    assert np.array_equal(m.hidden().view(np.uint32), g["hidden_prefill_a16"].view(np.uint32))
