"""Closed forms and invariants that pin the oracle independently of the reference.

Each check is chosen so that a plausible restatement mistake (a dropped term,
a wrong sign or index, a transposed operand, a wrong rounding mode) fails it.
"""
import numpy as np
import pytest
from conftest import max_rel

from mosship import moss_format as mf
from oracle import SampleParams


def test_half_to_float_exhaustive(oracle):
    halves = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = np.array([oracle.half_to_float(h) for h in halves], np.float32)
    ref = halves.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_float_to_half_rne_matches_ieee(oracle):
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(2.0) ** rng.integers(-30, 17, 20000).astype(np.float32),
        # exact ties between two halves, normal and subnormal, both parities
        (np.arange(1, 2000, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10),
        (np.arange(1, 2000, dtype=np.float32) + 0.5) * np.float32(2.0 ** -24),
        np.array([65504, 65519.996, 65520, 65536, 1e9, 6.103515625e-05, 6.1035e-05, 2.9802322e-08,
                  2.9802326e-08, 0.0, -0.0, np.inf, -np.inf], np.float32),
    ])
    got = np.array([oracle.float_to_half_rne(v) for v in vals], np.uint16)
    ref = vals.astype(np.float16).view(np.uint16)  # numpy rounds to nearest even
    assert np.array_equal(got, ref)


def test_float_to_half_reference_rounds_ties_up(oracle):
    """The reference encoder (fp16.cpp:37-66) rounds a dropped half-ulp up, not to even."""
    one_plus_half_ulp = np.float32(1.0 + 2.0 ** -11)  # tie between 1.0 and 1.0 + 2^-10
    assert oracle.float_to_half(one_plus_half_ulp) == 0x3C01
    assert oracle.float_to_half_rne(one_plus_half_ulp) == 0x3C00


def test_dequant_closed_form(oracle):
    rng = np.random.default_rng(1)
    rows, cols = 8, 256
    q = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
    d = (rng.random((rows, cols // 32)) * 0.01).astype(np.float16)
    w = mf.pack_q8x4(q, d)
    groups = w.reshape(rows // 4, -1)
    for r in range(rows):
        got = oracle.dequant_row(groups[r // 4], cols // 32, r % 4)
        exp = (q[r].astype(np.float32).reshape(-1, 32) * d[r].astype(np.float32)[:, None]).ravel()
        assert np.array_equal(got, exp)
    q2, d2 = mf.unpack_q8x4(w, rows, cols)
    assert np.array_equal(q2, q) and np.array_equal(d2.view(np.uint16), d.view(np.uint16))


def test_quantize_closed_form(oracle):
    rng = np.random.default_rng(2)
    x = rng.standard_normal(256).astype(np.float32)
    x[32:64] = 0
    q, _, d = oracle.quantize_row(x)
    blocks = x.reshape(-1, 32)
    amax = np.abs(blocks).max(axis=1)
    exp_d = (amax / np.float32(127.0)).astype(np.float32)
    assert np.array_equal(d, exp_d)
    inv = np.where(exp_d > 0, np.float32(1.0) / np.where(exp_d > 0, exp_d, 1), 0).astype(np.float32)
    exp_q = np.clip(np.rint(blocks * inv[:, None]), -127, 127).astype(np.int8).ravel()
    assert np.array_equal(q, exp_q)
    assert (q[32:64] == 0).all()


def test_gemv_vs_fp64(oracle):
    rng = np.random.default_rng(3)
    for rows, cols in [(64, 768), (16, 3072)]:
        w = mf.synth_q8x4(rng, rows, cols)
        x = rng.standard_normal(cols).astype(np.float32)
        truth = mf.dequant_q8x4(w, rows, cols).astype(np.float64) @ x.astype(np.float64)
        assert max_rel(oracle.gemv(w, rows, cols, x), truth) < 1e-5
        # scalar order agrees as well (reference gemv.cpp:51-63)
        g = w.reshape(rows // 4, -1)
        sc = np.array([oracle.lib.mo_row_dot_a16_scalar(np.ascontiguousarray(g[r // 4]), cols // 32, r % 4, x)
                       for r in range(rows)], np.float32)
        assert max_rel(sc, truth) < 1e-5


def test_w8a8_dot_is_quantised_product(oracle):
    """W8A8: per block the int32 dot is exact, so the row dot equals
    sum_b d_w d_a sum_i q_w q_a up to fp32 rounding of the block terms."""
    rng = np.random.default_rng(4)
    rows, cols = 4, 768
    w = mf.synth_q8x4(rng, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    qa, _, da = oracle.quantize_row(x)
    qw, dw = mf.unpack_q8x4(w, rows, cols)
    for r in range(rows):
        blocks = (qw[r].astype(np.int64) * qa.astype(np.int64)).reshape(-1, 32).sum(axis=1)
        exp = float(np.sum(blocks * dw[r].astype(np.float64) * da.astype(np.float64)))
        got = oracle.row_dot_w8a8(w.reshape(1, -1)[0] if rows == 4 else w, cols // 32, r, x)
        assert abs(got - exp) <= 1e-5 * max(1.0, abs(exp))


def test_layernorm_properties(oracle):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(768) * 3 + 1.5).astype(np.float32)
    y = oracle.layernorm(x, np.ones(768, np.float32), np.zeros(768, np.float32))
    assert abs(np.mean(y.astype(np.float64))) < 1e-5
    assert abs(np.var(y.astype(np.float64)) - 1.0) < 1e-4
    w = rng.standard_normal(768).astype(np.float32)
    b = rng.standard_normal(768).astype(np.float32)
    y2 = oracle.layernorm(x, w, b)
    xd = x.astype(np.float64)
    exp = (xd - xd.mean()) / np.sqrt(xd.var() + 1e-5) * w + b
    assert max_rel(y2, exp) < 1e-5


def test_rope_properties(oracle):
    cos_t, sin_t = oracle.rope_tables(768)
    rng = np.random.default_rng(6)
    v = rng.standard_normal(768).astype(np.float32)
    assert np.array_equal(oracle.rope_apply(v, 0, cos_t, sin_t), v)  # angle 0: identity
    # pair i of each head rotates by pos * 10000^(-2i/64): norms kept, angle adds
    pos = 300
    r = oracle.rope_apply(v, pos, cos_t, sin_t).astype(np.float64).reshape(12, 32, 2)
    vv = v.astype(np.float64).reshape(12, 32, 2)
    assert np.allclose(np.hypot(r[..., 0], r[..., 1]), np.hypot(vv[..., 0], vv[..., 1]), rtol=1e-6)
    inv = 1.0 / 10000.0 ** (2 * np.arange(32) / 64.0)
    ang = np.angle(r[..., 0] + 1j * r[..., 1]) - np.angle(vv[..., 0] + 1j * vv[..., 1])
    diff = np.angle(np.exp(1j * (ang - pos * inv[None, :])))
    assert np.max(np.abs(diff)) < 1e-5
    assert np.array_equal(cos_t[:, :32], cos_t[:, 32:64])  # same table for every head


def test_attention_properties(oracle):
    rng = np.random.default_rng(7)
    q = rng.standard_normal(768).astype(np.float32)
    k = rng.standard_normal((1, 768)).astype(np.float32)
    v = rng.standard_normal((1, 768)).astype(np.float32)
    assert np.array_equal(oracle.attention(k, v, q), v[0])  # one key: weight exactly 1
    n = 50
    k = rng.standard_normal((n, 768)).astype(np.float32)
    v = rng.standard_normal((n, 768)).astype(np.float32)
    out = oracle.attention(k, v, q)
    perm = rng.permutation(n)
    assert max_rel(oracle.attention(k[perm], v[perm], q), out) < 1e-6  # key order does not matter
    # explicit softmax in fp64
    qh = q.astype(np.float64).reshape(12, 64)
    kh = k.astype(np.float64).reshape(n, 12, 64)
    s = np.einsum("hd,nhd->hn", qh, kh) * 0.125
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    exp = np.einsum("hn,nhd->hd", p, v.astype(np.float64).reshape(n, 12, 64)).ravel()
    assert max_rel(out, exp) < 1e-5


def test_gelu_new_closed_form(oracle):
    for v in [-6.0, -1.0, -0.1, 0.0, 0.3, 1.0, 2.5, 8.0]:
        exp = 0.5 * v * (1 + np.tanh(np.sqrt(2 / np.pi) * (v + 0.044715 * v ** 3)))
        assert abs(oracle.lib.mo_gelu_new(v) - exp) <= 1e-6 * max(1.0, abs(exp))


def test_sampler_greedy_and_penalty(oracle):
    logits = np.array([0.5, 2.0, 2.0, -1.0, 1.9], np.float32)
    assert oracle.sample_token(logits, SampleParams.make()) == 1  # ties: lowest index
    p = SampleParams.make(repetition_penalty=2.0)
    # index 1 seen once: 2.0 / 2 = 1.0 -> index 2 wins
    assert oracle.sample_token(logits, p, prev=np.array([1])) == 2
    # both seen: 1.0, 1.0 -> index 4 (1.9) wins
    assert oracle.sample_token(logits, p, prev=np.array([1, 2])) == 4
    # compounding per occurrence: 2.0/2/2 = 0.5 (twice), 1.9/2/2 = 0.475 -> three-way tie at 0.5,
    # the lowest index (0) wins
    assert oracle.sample_token(logits, p, prev=np.array([1, 1, 2, 2, 4, 4])) == 0
    # negative logits are multiplied (-0.4 * 3 = -1.2 < -1.0), not divided (-0.133 would win)
    neg = np.array([-1.0, -3.0, -0.4], np.float32)
    assert oracle.sample_token(neg, SampleParams.make(repetition_penalty=3.0), prev=np.array([2])) == 0
    # out-of-range history entries are ignored
    assert oracle.sample_token(logits, p, prev=np.array([-5, 99])) == 1


def test_rng_xoshiro_known_answer(oracle):
    """xoshiro128** by its published recurrence (Blackman & Vigna), seeded as sampler.h:27-34."""
    def ref_stream(seed, n):
        M = 0xFFFFFFFF
        rotl = lambda x, k: ((x << k) | (x >> (32 - k))) & M
        s = [seed & M, ((seed >> 32) ^ 0x9E3779B9) & M, 0x243F6A88, 0xB7E15162]

        def nxt():
            res = (rotl((s[1] * 5) & M, 7) * 9) & M
            t = (s[1] << 9) & M
            s[2] ^= s[0]; s[3] ^= s[1]; s[1] ^= s[2]; s[0] ^= s[3]; s[2] ^= t
            s[3] = rotl(s[3], 11)
            return res
        for _ in range(8):
            nxt()
        return [nxt() for _ in range(n)]
    for seed in (0, 1, 0x123456789ABCDEF):
        assert list(oracle.rng_stream(seed, 20)) == ref_stream(seed, 20)


def test_planted_mistake_is_caught(oracle):
    """A wrong row index in the 4x4 unpack (row k read at 8 + 32*(k^1)) breaks the
    fp64 cross-check: the dequant pin is not vacuous."""
    rng = np.random.default_rng(8)
    rows, cols = 4, 128
    w = mf.synth_q8x4(rng, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    truth = mf.dequant_q8x4(w, rows, cols).astype(np.float64) @ x.astype(np.float64)
    blk = w.reshape(cols // 32, 136).copy()
    swapped = blk.copy()
    swapped[:, 8:40], swapped[:, 40:72] = blk[:, 40:72], blk[:, 8:40]
    wrong = oracle.gemv(swapped.reshape(1, -1), rows, cols, x)
    assert max_rel(wrong, truth) > 1e-2
    assert max_rel(oracle.gemv(w, rows, cols, x), truth) < 1e-5


@pytest.mark.parametrize("n_rows", [1, 5])
def test_prefill_equals_row_by_row(oracle, golden_model, n_rows):
    """Reference invariant (doc/推理加速计划.md:488): batched prefill == row by row
    in A16 mode, where both use the same row dot."""
    blob, g = golden_model
    rows = g["rows"][:n_rows]
    a = oracle.model(blob)
    a.prefill(rows, a16=True)
    b = oracle.model(blob)
    for r in rows:
        b.global_step(r)
    assert np.array_equal(a.hidden(), b.hidden())
    ka, va = a.kv_export(n_rows)
    kb, vb = b.kv_export(n_rows)
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
