"""moss_hip_attn_decode_noalloc (the single-query attention entry point that
allocates nothing: its scratch is a static device array) against
moss_hip_attn_decode on the same inputs, through the C ABI (GPU).

Both run the same kernel with the same slicing, so the outputs must be equal
bit for bit; each is also held to the oracle's attention at <= 1e-3."""
import numpy as np
import pytest
from conftest import max_rel

from mosship import lib

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _case(rng, ctx, stride, heads):
    q = rng.standard_normal(heads * 64).astype(np.float32)
    k = rng.standard_normal((ctx, heads * 64)).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((ctx, heads * 64)).astype(np.float16).astype(np.float32)
    kc = np.zeros((heads, stride, 64), np.float16)
    vc = np.zeros((heads, stride, 64), np.float16)
    kc[:, :ctx] = k.reshape(ctx, heads, 64).transpose(1, 0, 2)
    vc[:, :ctx] = v.reshape(ctx, heads, 64).transpose(1, 0, 2)
    return q, k, v, kc, vc


def _ref(q, k, v, heads):
    """Softmax attention per head in float64, scale 1/8 after the dot (llm.cpp:189-217)."""
    out = np.empty(heads * 64)
    for h in range(heads):
        sl = slice(64 * h, 64 * h + 64)
        s = k[:, sl].astype(np.float64) @ q[sl].astype(np.float64) * 0.125
        e = np.exp(s - s.max())
        out[sl] = (e / e.sum()) @ v[:, sl].astype(np.float64)
    return out


def _run(torch, q, kc, vc, heads, stride, ctx, noalloc, out_dtype=None):
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    out = torch.full((heads * 64,), float("nan"), dtype=out_dtype or torch.float32, device="cuda")
    lib.attn_decode(dev(q), dev(kc), dev(vc), heads, stride, ctx, out, noalloc=noalloc)
    torch.cuda.synchronize()
    return out.cpu().numpy().astype(np.float32)


def test_noalloc_matches_allocating_entry(torch_gpu):
    """Two calls in a row, the second on a smaller input (fewer keys, fewer heads,
    fp16 output), then one short enough for a single workgroup per head."""
    torch = torch_gpu
    rng = np.random.default_rng(11)
    for ctx, stride, heads, o16 in ((2048, 2050, 12, False), (700, 701, 8, True), (200, 256, 12, False)):
        print(f"noalloc ctx={ctx} heads={heads} out_f16={o16}", flush=True)
        q, k, v, kc, vc = _case(rng, ctx, stride, heads)
        odt = torch.float16 if o16 else torch.float32
        a = _run(torch, q, kc, vc, heads, stride, ctx, noalloc=False, out_dtype=odt)
        b = _run(torch, q, kc, vc, heads, stride, ctx, noalloc=True, out_dtype=odt)
        assert np.array_equal(a, b)
        assert max_rel(b, _ref(q, k, v, heads)) <= TOL


def test_noalloc_graph_replays(torch_gpu):
    """Captured once and replayed with new inputs, eager no-allocation calls with other
    key counts (other slice counts, so other grids on the same static scratch: its
    arrival counts and generation stepped by a different launch) between the
    replays: every replay equals the allocating entry point's result on its inputs,
    and so does every eager call in between."""
    torch = torch_gpu
    ctx, stride, heads = 1500, 1500, 12
    rng = np.random.default_rng(12)
    s = torch.cuda.Stream()
    q_d = torch.zeros(heads * 64, dtype=torch.float32, device="cuda")
    k_d = torch.zeros((heads, stride, 64), dtype=torch.float16, device="cuda")
    v_d = torch.zeros_like(k_d)
    out = torch.zeros(heads * 64, dtype=torch.float32, device="cuda")
    side = torch.zeros_like(out)
    with torch.cuda.stream(s):
        lib.attn_decode(q_d, k_d, v_d, heads, stride, ctx, out, noalloc=True)
    s.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        lib.attn_decode(q_d, k_d, v_d, heads, stride, ctx, out, noalloc=True)
    for rep in range(4):
        print(f"noalloc graph replay {rep}", flush=True)
        q, k, v, kc, vc = _case(rng, ctx, stride, heads)
        q_d.copy_(torch.from_numpy(q).cuda())
        k_d.copy_(torch.from_numpy(kc).cuda())
        v_d.copy_(torch.from_numpy(vc).cuda())
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert np.array_equal(got, _run(torch, q, kc, vc, heads, stride, ctx, noalloc=False))
        assert max_rel(got, _ref(q, k, v, heads)) <= TOL
        n = 300 + 300 * rep
        lib.attn_decode(q_d, k_d, v_d, heads, stride, n, side, noalloc=True)
        torch.cuda.synchronize()
        assert np.array_equal(side.cpu().numpy(), _run(torch, q, kc, vc, heads, stride, n, noalloc=False))


def test_noalloc_rejects_too_many_heads(torch_gpu):
    torch = torch_gpu
    heads, ctx = 17, 600
    q = torch.zeros(heads * 64, dtype=torch.float32, device="cuda")
    k = torch.zeros((heads, ctx, 64), dtype=torch.float16, device="cuda")
    out = torch.zeros_like(q)
    with pytest.raises(lib.MossHipError) as e:
        lib.attn_decode(q, k, k, heads, ctx, ctx, out, noalloc=True)
    assert e.value.code == lib.EINVAL and "16 heads" in str(e.value)
