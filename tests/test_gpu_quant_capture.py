"""Every in-kernel W8A8 quantiser pinned bit for bit, and every W8A8 stage checked on
its own int8 operand (GPU).

The W8A8 paths (the reference's prefill, and its decode with MOSS_A16 unset,
csrc/src/gemv.cpp:23-48, llm.cpp:319-328) re-quantise every GEMM input per
32-block (quantize_row_q8_0_scaled, csrc/src/quant.cpp:28-54).  On the GPU that
happens inside other kernels: the prefill's LayerNorm rows, its attention
epilogue and fc_in's epilogue, and the in-LDS quantiser of every GEMV stage of
the fused decode kernels.  End to end a W8A8 result cannot be held tight (a
one-ulp input difference moves a value by a full quantisation step), so with
the library's capture on, each quantiser also records the fp32 vector it
quantised and what it produced, and this module checks, stage by stage:

* the int8 values and the fp32 block scales equal the oracle's quantize_row of
  that very fp32 vector, bit for bit;
* each W8A8 stage's output is within 1e-5 of the oracle's W8A8 row dots
  (row_dot_q8_4x4, gemv_avx2.cpp:105-121) on the GPU's own int8 operand (only
  the fp32 summation order differs), and each LayerNorm / attention between
  them within 1e-5 of the oracle's on the GPU's own input;
* the captured int8 operand of the prefill is read in the matrix-core order the
  GEMMs use, by this module's own restatement of that layout.
"""
import numpy as np
import pytest
from conftest import check_quant, d8t_rows, max_rel, q8t_rows

from mosship import HipLLM, SampleParams, lib
from mosship import moss_format as mf

pytestmark = pytest.mark.gpu
TOL = 1e-5
H, FF = 768, 3072
FLIPS = []  # int8 values of LN1 a full step apart when the oracle quantises its own LN1 output


class Weights:
    """Tensors of a .moss blob by name (fp32 vectors, Q8_0_4X4 matrices as bytes)."""

    def __init__(self, blob):
        self.blob = blob
        self.idx = mf.read_moss_index(blob)

    def vec(self, name):
        _, _, _, off, nb = self.idx[name]
        return np.frombuffer(self.blob, np.float32, count=nb // 4, offset=off)

    def mat(self, name):
        _, rows, cols, off, nb = self.idx[name]
        return np.frombuffer(self.blob, np.uint8, count=nb, offset=off), rows, cols

    def row(self, oracle, name, r):
        """Row r of a Q8_0_4X4 matrix, dequantised (lookup_row, llm.cpp:114-146)."""
        w, rows, cols = self.mat(name)
        grp = w.reshape(rows // 4, -1)[r // 4]
        return oracle.dequant_row(grp, cols // 32, r % 4)


def w8a8(oracle, W, name, q, d):
    w, rows, cols = W.mat(name)
    return oracle.gemm_w8a8_q(w, rows, cols, np.asarray(q).astype(np.int8), d)


def gelu(v):  # gelu_new (llm.cpp:22-25), in float64
    v = np.asarray(v, np.float64)
    return 0.5 * v * (1.0 + np.tanh(0.7978845608028654 * (v + 0.044715 * v ** 3)))


def rope(oracle, vec, pos, tabs):
    return oracle.rope_apply(np.ascontiguousarray(vec, np.float32), pos, *tabs)


def check_block(oracle, W, pre, c, pos, keys, vals, kv32, what):
    """One block's captured stages (decode layout, lib.CAP) against the oracle: c = this
    block's capture, keys / vals [pos + 1][768] its cache rows as the GPU holds them."""
    tabs = oracle.rope_tables(pos + 1)
    ln1 = oracle.layernorm(c["xin"], W.vec(pre + "ln1.w"), W.vec(pre + "ln1.b"))
    assert max_rel(c["ln1"], ln1) <= TOL, what + " ln1"
    check_quant(oracle, c["ln1"], c["ln1_q"], c["ln1_d"], what + " ln1 quant")
    # how the end-to-end W8A8 differences arise: the oracle's own LN1 of the same input, within
    # ~1e-7, quantises to int8 values a full step away from the GPU's wherever a value sits on a
    # rounding boundary
    FLIPS.append(int(np.count_nonzero(oracle.quantize_row(ln1)[0] != c["ln1_q"].astype(np.int8))))
    qkv = w8a8(oracle, W, pre + "attn.w", c["ln1_q"], c["ln1_d"])[0] + W.vec(pre + "attn.b")
    q = rope(oracle, qkv[:H], pos, tabs)
    k = rope(oracle, qkv[H:2 * H], pos, tabs)
    v = qkv[2 * H:]
    assert max_rel(c["qkv"][:H], q) <= TOL, what + " q"
    kv_tol = TOL if kv32 else 1e-3  # the fp16 cache's rounding of the same value
    assert max_rel(c["qkv"][H:2 * H], k) <= kv_tol and max_rel(c["qkv"][2 * H:], v) <= kv_tol, what + " k/v"
    assert np.array_equal(keys[pos], c["qkv"][H:2 * H]) and np.array_equal(vals[pos], c["qkv"][2 * H:]), \
        what + ": the cache row is not the value handed on"
    att = oracle.attention(keys[:pos + 1], vals[:pos + 1], c["qkv"][:H])
    assert max_rel(c["att"], att) <= TOL, what + " attention"
    check_quant(oracle, c["att"], c["att_q"], c["att_d"], what + " attention quant")
    return check_mlp(oracle, W, pre, c, what)


def check_mlp(oracle, W, pre, c, what, resid=None):
    """proj + residual, LN2, fc_in + gelu, fc_out + residual of one captured step."""
    resid = c["xin"] if resid is None else resid
    xm = resid + (w8a8(oracle, W, pre + "proj.w", c["att_q"], c["att_d"])[0] + W.vec(pre + "proj.b"))
    assert max_rel(c["xm"], xm) <= TOL, what + " proj"
    ln2 = oracle.layernorm(c["xm"], W.vec(pre + "ln2.w"), W.vec(pre + "ln2.b"))
    assert max_rel(c["ln2"], ln2) <= TOL, what + " ln2"
    check_quant(oracle, c["ln2"], c["ln2_q"], c["ln2_d"], what + " ln2 quant")
    hh = gelu(w8a8(oracle, W, pre + "fc_in.w", c["ln2_q"], c["ln2_d"])[0] + W.vec(pre + "fc_in.b"))
    assert max_rel(c["h"], hh) <= TOL, what + " fc_in"
    clamps = check_quant(oracle, c["h"], c["h_q"], c["h_d"], what + " fc_in quant")
    xo = c["xm"] + (w8a8(oracle, W, pre + "fc_out.w", c["h_q"], c["h_d"])[0] + W.vec(pre + "fc_out.b"))
    assert max_rel(c["xout"], xo) <= TOL, what + " fc_out"
    return clamps


@pytest.fixture(scope="module")
def prefilled(oracle, golden_model):
    """A 60-position state (the oracle's A16 prefill of the golden prompt + random rows)."""
    blob, g = golden_model
    rng = np.random.default_rng(5)
    rows = np.concatenate([g["rows"], mf.text_rows(rng.integers(0, mf.VOCAB, 60 - len(g["rows"])))])
    rows[5:15, 1:] = rng.integers(0, 1024, (10, 16))
    m = oracle.model(blob)
    m.prefill(rows, a16=True)
    k, v = m.kv_export(len(rows))
    return blob, k, v, m.hidden()


@pytest.mark.parametrize("kv32", [True, False])
def test_fused_global_step_w8a8(torch_gpu, oracle, prefilled, kv32):
    """Three W8A8 fused global steps (decode_global_kernel<A8>): per block the in-LDS
    quantisers of QKV, proj, fc_in and fc_out bit-exact, every stage <= 1e-5 on the
    GPU's own operands, blocks chained exactly, hidden = ln_f of the last block."""
    blob, k, v, h = prefilled
    W = Weights(blob)
    om = oracle.model(blob)
    print(f"fused global w8a8 kv32={kv32}", flush=True)
    g = HipLLM(blob, kv_fp32=kv32, decode_a8=True)
    g.kv_import(k, v, h)
    g.capture(True)
    rng = np.random.default_rng(41)
    clamps = 0
    for step in range(3):
        pos = g.position
        row = np.array([mf.SLOT] + list(rng.integers(0, 1024, 16)), np.int32)
        row[3] = mf.AUDIO_PAD
        g.global_step(row)
        caps = g.capture_steps(lib.CAP_GLOBAL)
        keys, vals = g.kv_export(pos + 1)
        assert max_rel(caps[0]["xin"], om.embed_row(row)) <= 1e-6, "embedding"
        for l in range(12):
            if l > 0:
                assert np.array_equal(caps[l]["xin"], caps[l - 1]["xout"]), f"block {l} input"
            clamps += check_block(oracle, W, f"g{l}.", caps[l], pos, keys[l], vals[l], kv32, f"step {step} block {l}")
        hid = oracle.layernorm(caps[11]["xout"], W.vec("lnf.w"), W.vec("lnf.b"))
        assert max_rel(g.hidden(), hid) <= TOL
    print(f"  3 steps x 12 blocks pinned; {clamps} fc_in values at +-127; LN1 int8 values one step apart "
          f"from the oracle's quantisation of its own LN1: {sum(FLIPS)} of {len(FLIPS) * 768}", flush=True)
    FLIPS.clear()
    g.close()


def test_fused_local_half_w8a8(torch_gpu, oracle, prefilled):
    """A W8A8 greedy frame's local half (decode_local_kernel<A8>): at each of the 17
    local positions the quantisers of proj, fc_in, fc_out and the audio head (and of
    QKV at position 0) bit-exact, every stage <= 1e-5 on the GPU's own operands, and
    the logits the picks read equal to the oracle's W8A8 head on the captured operand."""
    blob, k, v, h = prefilled
    W = Weights(blob)
    print("fused local half w8a8", flush=True)
    g = HipLLM(blob, kv_fp32=True, decode_a8=True)
    g.kv_import(k, v, h)
    g.capture(True)
    out = g.generate(1, SampleParams.make(greedy=True, min_frames=1), logits=True)
    caps = g.capture_steps(lib.CAP_LOCAL)
    codes = out["rows"][0, 1:]
    tabs = oracle.rope_tables(17)
    keys = np.stack([c["qkv"][H:2 * H] for c in caps])
    vals = np.stack([c["qkv"][2 * H:] for c in caps])
    for lpos in range(17):
        c = caps[lpos]
        what = f"local {lpos}"
        if lpos == 0:  # the block input is the global hidden state: QKV computed in the launch
            assert np.array_equal(c["xin"], h)
            ln1 = oracle.layernorm(h, W.vec("local.ln1.w"), W.vec("local.ln1.b"))
            assert max_rel(c["ln1"], ln1) <= TOL
            check_quant(oracle, c["ln1"], c["ln1_q"], c["ln1_d"], what + " ln1 quant")
            qkv = w8a8(oracle, W, "local.attn.w", c["ln1_q"], c["ln1_d"])[0] + W.vec("local.attn.b")
            ref = np.concatenate([rope(oracle, qkv[:H], 0, tabs), rope(oracle, qkv[H:2 * H], 0, tabs), qkv[2 * H:]])
            assert max_rel(c["qkv"], ref) <= TOL, what + " qkv"
            resid = h
        else:  # an embedding row: q|k|v from the load-time table (the per-operator W8A8 GEMV)
            resid = W.row(oracle, "wte", mf.SLOT) if lpos == 1 else W.row(oracle, f"aemb.{lpos - 2}", codes[lpos - 2])
            ln1 = oracle.layernorm(resid, W.vec("local.ln1.w"), W.vec("local.ln1.b"))
            q8, _, d8 = oracle.quantize_row(ln1)
            qkv = w8a8(oracle, W, "local.attn.w", q8, d8)[0] + W.vec("local.attn.b")
            ref = np.concatenate([rope(oracle, qkv[:H], lpos, tabs), rope(oracle, qkv[H:2 * H], lpos, tabs),
                                  qkv[2 * H:]])
            assert max_rel(c["qkv"], ref) <= 1e-3, what + " qkv table row"
        att = oracle.attention(keys[:lpos + 1], vals[:lpos + 1], c["qkv"][:H])
        assert max_rel(c["att"], att) <= TOL, what + " attention"
        check_quant(oracle, c["att"], c["att_q"], c["att_d"], what + " attention quant")
        check_mlp(oracle, W, "local.", c, what, resid=resid)
        if lpos >= 1:  # local ln_f + the tied audio head of channel lpos - 1
            lnf = oracle.layernorm(c["xout"], W.vec("local.lnf.w"), W.vec("local.lnf.b"))
            assert max_rel(c["lnf"], lnf) <= TOL, what + " local ln_f"
            check_quant(oracle, c["lnf"], c["lnf_q"], c["lnf_d"], what + " head quant")
            logits = w8a8(oracle, W, f"aemb.{lpos - 1}", c["lnf_q"], c["lnf_d"])[0]
            assert max_rel(out["logits"][0, lpos - 1], logits) <= TOL, what + " head"
    print(f"  17 local positions pinned; codes {codes[:6].tolist()}...", flush=True)
    g.close()


def split_prefill_capture(raw, m):
    """Per layer, the named sections of a CAP_PREFILL capture (layout in moss_hip.h)."""
    m16 = (m + 15) // 16 * 16
    f32 = [("xin", H), ("ln1", H), ("att", H), ("xm", H), ("ln2", H), ("h", FF), ("xout", H)]
    q8 = [("ln1", H), ("att", H), ("ln2", H), ("h", FF)]
    per = 4 * m * (6 * H + FF) + m16 * (3 * H + FF) + 4 * m16 * (3 * 24 + 96)
    assert raw.size == 12 * per
    layers = []
    for l in range(12):
        base, o, d = l * per, 0, {}
        for name, K in f32:
            d[name] = raw[base + o: base + o + 4 * m * K].view(np.float32).reshape(m, K)
            o += 4 * m * K
        for name, K in q8:
            d[name + "_q"] = q8t_rows(raw[base + o: base + o + m16 * K], m, K)
            o += m16 * K
        for name, K in q8:
            d[name + "_d"] = d8t_rows(raw[base + o: base + o + 4 * m16 * K // 32], m, K)
            o += 4 * m16 * K // 32
        layers.append(d)
    return layers


@pytest.mark.parametrize("m", [256, 37])
def test_prefill_w8a8(torch_gpu, oracle, m):
    """The W8A8 prefill (config 3: 256 rows; and 37, with padded row tiles): for every row
    and layer the four quantisers (LN1 in ln_rows / the fc_out reduce, the attention
    epilogue, LN2 in the proj reduce, fc_in's epilogue) bit-exact against quantize_row of
    the fp32 row they quantised; on sampled rows every stage <= 1e-5 on the GPU's own
    int8 operands, read in the matrix-core order; layers chained exactly."""
    blob = mf.synth_model(7, ln_random=True)
    W = Weights(blob)
    rng = np.random.default_rng(m)
    rows = mf.text_rows(rng.integers(0, mf.VOCAB, m))
    rows[m // 2:, 1:] = rng.integers(0, 1024, (m - m // 2, 16))
    print(f"prefill w8a8 m={m}", flush=True)
    g = HipLLM(blob, kv_fp32=True)
    g.capture(True)
    g.prefill(rows)
    caps = split_prefill_capture(g.capture_read(lib.CAP_PREFILL), m)
    keys, vals = g.kv_export(m)
    tabs = oracle.rope_tables(m)
    sample = sorted({0, 1, 15, 16, m // 2, m - 2, m - 1} | set(rng.integers(0, m, 5).tolist()))
    clamps = 0
    for l, c in enumerate(caps):
        pre = f"g{l}."
        if l > 0:
            assert np.array_equal(c["xin"], caps[l - 1]["xout"]), f"layer {l} input"
        for r in range(m):  # every quantised row, bit for bit
            check_quant(oracle, c["ln1"][r], c["ln1_q"][r], c["ln1_d"][r], f"layer {l} row {r} ln1")
            check_quant(oracle, c["att"][r], c["att_q"][r], c["att_d"][r], f"layer {l} row {r} attention")
            check_quant(oracle, c["ln2"][r], c["ln2_q"][r], c["ln2_d"][r], f"layer {l} row {r} ln2")
            clamps += check_quant(oracle, c["h"][r], c["h_q"][r], c["h_d"][r], f"layer {l} row {r} fc_in")
        s = np.array(sample)
        ln1 = np.stack([oracle.layernorm(c["xin"][r], W.vec(pre + "ln1.w"), W.vec(pre + "ln1.b")) for r in s])
        assert max_rel(c["ln1"][s], ln1) <= TOL, f"layer {l} ln1"
        qkv = w8a8(oracle, W, pre + "attn.w", c["ln1_q"][s], c["ln1_d"][s]) + W.vec(pre + "attn.b")
        for i, r in enumerate(s):
            kr = rope(oracle, qkv[i, H:2 * H], r, tabs)
            assert max_rel(keys[l][r], kr) <= TOL and max_rel(vals[l][r], qkv[i, 2 * H:]) <= TOL, f"layer {l} k/v {r}"
            q = rope(oracle, qkv[i, :H], r, tabs)
            att = oracle.attention(keys[l][:r + 1], vals[l][:r + 1], q)
            assert max_rel(c["att"][r], att) <= TOL, f"layer {l} attention row {r}"
        xm = c["xin"][s] + (w8a8(oracle, W, pre + "proj.w", c["att_q"][s], c["att_d"][s]) + W.vec(pre + "proj.b"))
        assert max_rel(c["xm"][s], xm) <= TOL, f"layer {l} proj"
        ln2 = np.stack([oracle.layernorm(c["xm"][r], W.vec(pre + "ln2.w"), W.vec(pre + "ln2.b")) for r in s])
        assert max_rel(c["ln2"][s], ln2) <= TOL, f"layer {l} ln2"
        hh = gelu(w8a8(oracle, W, pre + "fc_in.w", c["ln2_q"][s], c["ln2_d"][s]) + W.vec(pre + "fc_in.b"))
        assert max_rel(c["h"][s], hh) <= TOL, f"layer {l} fc_in"
        xo = c["xm"][s] + (w8a8(oracle, W, pre + "fc_out.w", c["h_q"][s], c["h_d"][s]) + W.vec(pre + "fc_out.b"))
        assert max_rel(c["xout"][s], xo) <= TOL, f"layer {l} fc_out"
    hid = oracle.layernorm(caps[11]["xout"][m - 1], W.vec("lnf.w"), W.vec("lnf.b"))
    assert max_rel(g.hidden(), hid) <= TOL
    print(f"  {m} rows x 12 layers x 4 quantisers bit-exact; {len(sample)} rows staged; "
          f"{clamps} fc_in values at +-127", flush=True)
    g.close()


def test_capture_is_off_by_default_and_w8a16_records_nothing(torch_gpu, prefilled):
    """Without capture (and for the W8A16 paths) nothing is recorded."""
    blob, k, v, h = prefilled
    g = HipLLM(blob, kv_fp32=True, decode_a8=True)
    g.kv_import(k, v, h)
    g.global_step(np.array([mf.SLOT] + [1] * 16, np.int32))
    with pytest.raises(lib.MossHipError):
        g.capture_read(lib.CAP_GLOBAL)
    g.close()
    g = HipLLM(blob, kv_fp32=True, prefill_a16=True)
    g.capture(True)
    g.prefill(mf.text_rows(np.arange(20)))
    with pytest.raises(lib.MossHipError):
        g.capture_read(lib.CAP_PREFILL)
    g.close()
