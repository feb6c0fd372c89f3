"""HIP operators through the C ABI vs the CPU oracle (GPU).

Tolerance: max|y - ref| / max|ref| <= 1e-3 for every floating-point output
(the W8A16 GEMV and attention contract); dequantisation is bit-exact.
"""
import numpy as np
import pytest
from conftest import max_rel

from mosship import lib
from mosship import moss_format as mf

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


# (16384, 768), (8196, 768), (8192, 3072), (8200, 1536): the large-N LDS streaming kernel (>= 2048 groups),
# including a ragged last round of groups and the 2- and 4-slice K = 1536 / 3072 units.
@pytest.mark.parametrize("rows,cols", [(2304, 768), (768, 768), (3072, 768), (768, 3072), (1024, 768), (8, 768),
                                       (4, 128), (16384, 768), (8196, 768), (8192, 3072), (8200, 1536)])
def test_gemv_f32_vs_oracle(torch_gpu, oracle, rows, cols):
    torch = torch_gpu
    print(f"gemv f32 rows={rows} cols={cols}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols)
    w = mf.synth_q8x4(rng, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    lib.gemv_q8x4(_dev(torch, w), rows, cols, _dev(torch, x), y)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    ref = oracle.gemv(w, rows, cols, x)
    assert max_rel(got, ref) <= TOL
    # and against the exact fp64 product of the exactly dequantised matrix
    truth = mf.dequant_q8x4(w, rows, cols).astype(np.float64) @ x.astype(np.float64)
    assert max_rel(got, truth) <= 1e-5


def test_gemv_config0_f16(torch_gpu, oracle):
    """K=768, N=2304, x fp16 N(0,1), y fp16 with fp32 accumulation."""
    torch = torch_gpu
    rows, cols = 2304, 768
    rng = np.random.default_rng(2304)
    w = mf.synth_q8x4(rng, rows, cols)
    x = rng.standard_normal(cols).astype(np.float16)
    y = torch.empty(rows, dtype=torch.float16, device="cuda")
    lib.gemv_q8x4(_dev(torch, w), rows, cols, _dev(torch, x), y)
    torch.cuda.synchronize()
    ref = oracle.gemv(w, rows, cols, x.astype(np.float32))
    assert max_rel(y.cpu().numpy().astype(np.float32), ref) <= TOL


def test_gemv_large_n_sampled(torch_gpu, oracle):
    """N = 262144 (213 MB of weights): every sampled 4-row group checked against the oracle."""
    torch = torch_gpu
    rows, cols = 262144, 768
    rng = np.random.default_rng(5)
    w = mf.synth_q8x4(rng, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    lib.gemv_q8x4(_dev(torch, w), rows, cols, _dev(torch, x), y)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    groups = np.unique(np.concatenate([[0, rows // 4 - 1], rng.integers(0, rows // 4, 400)]))
    sub = w.reshape(rows // 4, -1)[groups]
    ref = oracle.gemv(sub, 4 * len(groups), cols, x)
    got_sub = got.reshape(-1, 4)[groups].ravel()
    assert max_rel(got_sub, ref) <= TOL
    assert np.isfinite(got).all()


@pytest.mark.parametrize("rows,cols", [(2304, 768), (768, 3072), (3072, 768), (1024, 768), (8, 256), (16384, 768)])
def test_gemv_w8a8_vs_oracle(torch_gpu, oracle, rows, cols):
    """The W8A8 GEMV (the reference's gemv_par with MOSS_A16 unset; the register kernel
    below 8192 rows, the LDS-streaming one from 8192, e.g. the text head): the activation
    quantisation is bit-exact and every block's integer dot exact, so only the fp32
    summation order differs from the oracle's AVX2-order W8A8 rows (<= 1e-5), while the
    W8A16 product of the same input is much farther away."""
    torch = torch_gpu
    rng = np.random.default_rng(rows + cols)
    w = mf.synth_q8x4(rng, rows, cols)
    x = (rng.standard_normal(cols) * 2).astype(np.float32)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    lib.gemv_q8x4_w8a8(_dev(torch, w.reshape(-1)), rows, cols, _dev(torch, x), y)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    ref = oracle.gemm(w, rows, cols, x[None], a16=False)[0]
    a16 = oracle.gemv(w, rows, cols, x)
    print(f"w8a8 gemv {rows}x{cols}: max rel {max_rel(got, ref):.2e} (vs w8a16 {max_rel(a16, ref):.2e})", flush=True)
    assert max_rel(got, ref) <= 1e-5
    assert max_rel(a16, ref) > 100 * max(max_rel(got, ref), 1e-7)


def test_dequant_rows_bit_exact(torch_gpu, oracle):
    torch = torch_gpu
    rng = np.random.default_rng(11)
    rows, cols = 1024, 768
    w = mf.synth_q8x4(rng, rows, cols)
    idx = np.array([0, 1, 2, 3, 4, 511, 1023, 9, 7, -1, 1024], np.int32)
    out = torch.empty((len(idx), cols), dtype=torch.float32, device="cuda")
    lib.dequant_rows_q8x4(_dev(torch, w), rows, cols, _dev(torch, idx), out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isnan(got[-2:]).all()  # out-of-range indices are flagged, never read
    groups = w.reshape(rows // 4, -1)
    for i, r in enumerate(idx[:-2]):
        assert np.array_equal(got[i].view(np.uint32), oracle.dequant_row(groups[r // 4], cols // 32, r % 4).view(np.uint32))


def _attn_case(oracle, ctx, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(768).astype(np.float32)
    k = rng.standard_normal((ctx, 768)).astype(np.float32)
    v = rng.standard_normal((ctx, 768)).astype(np.float32)
    cos_t, sin_t = oracle.rope_tables(max(ctx, 1))
    for p in range(ctx):  # K stored post-RoPE at its position, q at ctx-1
        k[p] = oracle.rope_apply(k[p], p, cos_t, sin_t)
    q = oracle.rope_apply(q, ctx - 1, cos_t, sin_t)
    return q, k, v


def _to_cache(rows_768, ctx_stride, dtype):
    n = rows_768.shape[0]
    c = np.zeros((12, ctx_stride, 64), dtype)
    c[:, :n, :] = rows_768.reshape(n, 12, 64).transpose(1, 0, 2).astype(dtype)
    return c


@pytest.mark.parametrize("ctx", [1, 17, 33, 64, 65, 128, 256, 257, 512, 767, 1024, 1025, 2048, 4096, 16641])
@pytest.mark.parametrize("kv", ["f16", "f32"])
def test_attention_decode_vs_oracle(torch_gpu, oracle, ctx, kv):
    torch = torch_gpu
    print(f"attention ctx={ctx} kv={kv}", flush=True)
    q, k, v = _attn_case(oracle, ctx, ctx)
    npdt = np.float16 if kv == "f16" else np.float32
    stride = ctx + 5
    kc, vc = _to_cache(k, stride, npdt), _to_cache(v, stride, npdt)
    out = torch.empty(768, dtype=torch.float32, device="cuda")
    lib.attn_decode(_dev(torch, q), _dev(torch, kc), _dev(torch, vc), 12, stride, ctx, out)
    out16 = torch.empty(768, dtype=torch.float16, device="cuda")
    lib.attn_decode(_dev(torch, q), _dev(torch, kc), _dev(torch, vc), 12, stride, ctx, out16)
    torch.cuda.synchronize()
    ref = oracle.attention(k.astype(npdt).astype(np.float32), v.astype(npdt).astype(np.float32), q)
    assert max_rel(out.cpu().numpy(), ref) <= TOL
    assert max_rel(out16.cpu().numpy().astype(np.float32), ref) <= TOL


def test_attention_decode_back_to_back(torch_gpu, oracle):
    """Past 256 keys the heads are cut into slices whose partials the first slice of
    each head merges: consecutive calls with different slice counts on one stream
    never take a partial of an earlier call (some of whose slots they reuse)."""
    torch = torch_gpu
    for ctx in (2048, 300, 257, 5000, 1300):
        print(f"attention back-to-back ctx={ctx}", flush=True)
        q, k, v = _attn_case(oracle, ctx, ctx + 11)
        kc, vc = _to_cache(k, ctx, np.float16), _to_cache(v, ctx, np.float16)
        out = torch.empty(768, dtype=torch.float32, device="cuda")
        lib.attn_decode(_dev(torch, q), _dev(torch, kc), _dev(torch, vc), 12, ctx, ctx, out)
        torch.cuda.synchronize()
        ref = oracle.attention(k.astype(np.float16).astype(np.float32), v.astype(np.float16).astype(np.float32), q)
        assert max_rel(out.cpu().numpy(), ref) <= TOL


def test_attention_decode_graph_replays(torch_gpu, oracle):
    """One split-KV call captured in a graph replays with the tag it was captured
    with; the merging slice clears every partial word it read, so no replay takes
    the previous replay's partials.  New q, K and V go in before each replay (with
    eager calls of other sizes on the same stream between replays), and every
    replay is checked against the oracle."""
    torch = torch_gpu
    ctx = 1500
    s = torch.cuda.Stream()
    q_d = torch.zeros(768, dtype=torch.float32, device="cuda")
    k_d = torch.zeros((12, ctx, 64), dtype=torch.float16, device="cuda")
    v_d = torch.zeros_like(k_d)
    out = torch.zeros(768, dtype=torch.float32, device="cuda")
    side = torch.empty(768, dtype=torch.float32, device="cuda")
    with torch.cuda.stream(s):  # first call on the stream: its scratch is made here
        lib.attn_decode(q_d, k_d, v_d, 12, ctx, ctx, out)
    s.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        lib.attn_decode(q_d, k_d, v_d, 12, ctx, ctx, out)
    for rep in range(4):
        print(f"attention graph replay {rep}", flush=True)
        q, k, v = _attn_case(oracle, ctx, 100 + rep)
        q_d.copy_(_dev(torch, q))
        k_d.copy_(_dev(torch, _to_cache(k, ctx, np.float16)))
        v_d.copy_(_dev(torch, _to_cache(v, ctx, np.float16)))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref = oracle.attention(k.astype(np.float16).astype(np.float32), v.astype(np.float16).astype(np.float32), q)
        assert max_rel(out.cpu().numpy(), ref) <= TOL, rep
        with torch.cuda.stream(s):  # eager calls of other slice counts between replays
            n = 300 + 400 * rep  # 300 .. 1500 keys of the ctx-1500 cache
            lib.attn_decode(q_d, k_d, v_d, 12, ctx, n, side)
        s.synchronize()


def test_attention_decode_first_call_under_capture_refused(torch_gpu):
    """The first sliced call on a stream allocates its scratch, which a graph
    capture cannot hold: it is refused with ESTATE and nothing is enqueued; an
    uncaptured call first makes the same capture work."""
    torch = torch_gpu
    ctx = 600
    s = torch.cuda.Stream()
    q = torch.zeros(768, dtype=torch.float32, device="cuda")
    k = torch.zeros((12, ctx, 64), dtype=torch.float16, device="cuda")
    out = torch.zeros(768, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        with pytest.raises(lib.MossHipError) as e:
            lib.attn_decode(q, k, k, 12, ctx, ctx, out)
    assert e.value.code == lib.ESTATE
    with torch.cuda.stream(s):
        lib.attn_decode(q, k, k, 12, ctx, ctx, out)
    s.synchronize()
    graph2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph2, stream=s):
        lib.attn_decode(q, k, k, 12, ctx, ctx, out)
    for _ in range(3):
        graph2.replay()
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()


def test_attention_single_key_returns_v(torch_gpu):
    """ctx = 1: softmax over one key is 1, so the output is that key's v exactly."""
    torch = torch_gpu
    rng = np.random.default_rng(3)
    q = rng.standard_normal(768).astype(np.float32)
    k = rng.standard_normal((1, 768)).astype(np.float32)
    v = rng.standard_normal((1, 768)).astype(np.float32)
    out = torch.empty(768, dtype=torch.float32, device="cuda")
    lib.attn_decode(_dev(torch, q), _dev(torch, _to_cache(k, 1, np.float32)), _dev(torch, _to_cache(v, 1, np.float32)),
                    12, 1, 1, out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), v[0])


def test_operator_errors(torch_gpu):
    torch = torch_gpu
    w = torch.zeros(3264, dtype=torch.uint8, device="cuda")
    x = torch.zeros(768, dtype=torch.float32, device="cuda")
    y = torch.zeros(6, dtype=torch.float32, device="cuda")
    with pytest.raises(lib.MossHipError) as e:
        lib.gemv_q8x4(w, 6, 768, x, y)  # rows % 4 != 0
    assert e.value.code == lib.EINVAL


@pytest.mark.parametrize("rows,cols,m", [(2304, 768, 64), (768, 3072, 64), (3072, 768, 256), (1024, 768, 1),
                                         (768, 768, 17), (16, 128, 100), (2304, 768, 200)])
def test_gemm_mfma_vs_oracle(torch_gpu, oracle, rows, cols, m):
    """MFMA W8A16 GEMM (fp16 hi/lo activation split) vs the oracle's A16 gemm_par."""
    torch = torch_gpu
    print(f"gemm rows={rows} cols={cols} m={m}", flush=True)
    rng = np.random.default_rng(rows + cols + m)
    w = mf.synth_q8x4(rng, rows, cols)
    x = (rng.standard_normal((m, cols)) * rng.choice([0.01, 1.0, 30.0], (m, 1))).astype(np.float32)
    y = torch.empty((m, rows), dtype=torch.float32, device="cuda")
    lib.gemm_q8x4(_dev(torch, w), rows, cols, _dev(torch, x), m, y)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    ref = oracle.gemm(w, rows, cols, x, a16=True)
    for i in range(m):  # per row: rows of very different scale
        assert max_rel(got[i], ref[i]) <= TOL
    assert max_rel(got, ref) <= 1e-5


def test_quantize_rows_bit_exact(torch_gpu, oracle):
    """W8A8 activation quantisation (quant.cpp:28-54) on the GPU == the oracle, bit for bit:
    int8 values and fp32 block scales, including an all-zero block, exact .5 ties and
    values at the clamp."""
    torch = torch_gpu
    rng = np.random.default_rng(17)
    m, cols = 9, 3072
    x = (rng.standard_normal((m, cols)) * rng.choice([1e-3, 1.0, 50.0], (m, 1))).astype(np.float32)
    x[0, :32] = 0.0                                      # d = 0 -> id = 0 -> q = 0
    x[1, :32] = np.arange(32, dtype=np.float32) - 15.5    # ties at k + 0.5 after scaling
    x[1, 31] = 127.0                                      # amax = 127: scale 1, ties stay ties
    x[2, 64:96] = rng.standard_normal(32) * 1e30          # huge values
    q = torch.empty((m, cols), dtype=torch.int8, device="cuda")
    d = torch.empty((m, cols // 32), dtype=torch.float32, device="cuda")
    lib.quantize_rows(_dev(torch, x), m, cols, q, d)
    torch.cuda.synchronize()
    for i in range(m):
        oq, _, od = oracle.quantize_row(x[i])
        assert np.array_equal(q[i].cpu().numpy(), oq), i
        assert np.array_equal(d[i].cpu().numpy(), od), i


@pytest.mark.parametrize("rows,cols,m", [(2304, 768, 64), (768, 3072, 256), (1024, 768, 1), (16, 768, 100)])
def test_gemm_w8a8_vs_oracle(torch_gpu, oracle, rows, cols, m):
    """W8A8 GEMM on the int8 matrix cores vs the oracle's W8A8 gemm_par (row_dot_q8_4x4
    order) on the same quantised activations: only the fp32 accumulation order of the
    per-block scaled integer dots differs."""
    torch = torch_gpu
    print(f"gemm w8a8 rows={rows} cols={cols} m={m}", flush=True)
    rng = np.random.default_rng(rows * 3 + cols + m)
    w = mf.synth_q8x4(rng, rows, cols)
    x = (rng.standard_normal((m, cols)) * rng.choice([0.01, 1.0, 30.0], (m, 1))).astype(np.float32)
    q = torch.empty((m, cols), dtype=torch.int8, device="cuda")
    d = torch.empty((m, cols // 32), dtype=torch.float32, device="cuda")
    y = torch.empty((m, rows), dtype=torch.float32, device="cuda")
    xd = _dev(torch, x)
    lib.quantize_rows(xd, m, cols, q, d)
    lib.gemm_q8x4_w8a8(_dev(torch, w), rows, cols, q, d, m, y)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    ref = oracle.gemm(w, rows, cols, x, a16=False)
    for i in range(m):
        assert max_rel(got[i], ref[i]) <= 1e-5, i
