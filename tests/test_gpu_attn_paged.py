"""moss_hip_attn_paged (the batch engine's paged global attention as an operator) against the
oracle's attention_core (llm.cpp:189-217), row by row, through the C ABI (GPU).

Rows sit on pages scattered through the pool by a shuffled block table; the key counts cover a
single key, the span edges (63, 64, 65, 127, 128, 129), ragged long rows and a row clamped by
max_keys; row_stream maps rows to streams out of order."""
import numpy as np
import pytest
from conftest import max_rel

from mosship import lib

pytestmark = pytest.mark.gpu
TOL = 1e-3
PAGE = 64


def _case(rng, keys, heads, npdt, page=PAGE):
    """Pools [page][heads][page][64] holding each stream's keys on shuffled pages, the table,
    and the rows [n][heads * 64] of K and V each stream holds (as the pool stores them)."""
    streams = len(keys)
    per = (max(keys) + page - 1) // page
    n_pages = streams * per + 3  # a few pages nobody owns
    perm = rng.permutation(n_pages)[: streams * per].reshape(streams, per).astype(np.int32)
    kp = rng.standard_normal((n_pages, heads, page, 64)).astype(npdt)
    vp = rng.standard_normal((n_pages, heads, page, 64)).astype(npdt)
    kr, vr = [], []
    for s, n in enumerate(keys):
        pos = np.arange(n)
        pg = perm[s, pos // page]
        kr.append(kp[pg, :, pos % page, :].reshape(n, heads * 64).astype(np.float32))
        vr.append(vp[pg, :, pos % page, :].reshape(n, heads * 64).astype(np.float32))
    return kp, vp, perm, per, kr, vr


def _ref(oracle, k, v, q, heads):
    if heads == 12:
        return oracle.attention(k, v, q)
    out = np.empty(heads * 64)
    for h in range(heads):  # float64, scale after the dot (llm.cpp:200)
        sl = slice(64 * h, 64 * h + 64)
        s = k[:, sl].astype(np.float64) @ q[sl].astype(np.float64) * 0.125
        e = np.exp(s - s.max())
        out[sl] = (e / e.sum()) @ v[:, sl].astype(np.float64)
    return out


@pytest.mark.parametrize("kv", ["f16", "f32"])
@pytest.mark.parametrize("heads", [12, 5])
def test_attn_paged_vs_oracle(torch_gpu, oracle, kv, heads):
    torch = torch_gpu
    rng = np.random.default_rng(heads * 7 + (kv == "f16"))
    keys = [1, 2, 63, 64, 65, 127, 128, 129, 300, 700, 1015, 1024] + list(rng.integers(64, 1025, 8))
    npdt = np.float16 if kv == "f16" else np.float32
    print(f"attn_paged kv={kv} heads={heads} keys={keys}", flush=True)
    kp, vp, table, per, kr, vr = _case(rng, keys, heads, npdt)
    rows = len(keys)
    row_stream = rng.permutation(rows).astype(np.int32)  # row r is stream row_stream[r]
    row_pos = np.array([keys[s] - 1 for s in row_stream], np.int32)
    q = rng.standard_normal((rows, heads * 64)).astype(np.float32)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    for odt in (torch.float32, torch.float16):
        out = torch.full((rows, heads * 64), float("nan"), dtype=odt, device="cuda")
        lib.attn_paged(dev(q), dev(kp), dev(vp), heads, dev(table), per, PAGE, dev(row_pos), max(keys), out,
                       row_stream=dev(row_stream))
        torch.cuda.synchronize()
        got = out.float().cpu().numpy()
        for r, s in enumerate(row_stream):
            ref = _ref(oracle, kr[s], vr[s], q[r], heads)
            assert max_rel(got[r], ref) <= TOL, (r, int(s), keys[s])


def test_attn_paged_clamps_to_max_keys(torch_gpu, oracle):
    """A row whose position lies past max_keys attends the first max_keys keys (a stream parked at
    capacity); rows without row_stream are streams 0, 1, ..."""
    torch = torch_gpu
    rng = np.random.default_rng(5)
    keys = [200, 200, 200]
    kp, vp, table, per, kr, vr = _case(rng, keys, 12, np.float16)
    row_pos = np.array([199, 150, 5000], np.int32)
    q = rng.standard_normal((3, 768)).astype(np.float32)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    out = torch.empty((3, 768), dtype=torch.float32, device="cuda")
    lib.attn_paged(dev(q), dev(kp), dev(vp), 12, dev(table), per, PAGE, dev(row_pos), 200, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for r, n in enumerate((200, 151, 200)):
        assert max_rel(got[r], oracle.attention(kr[r][:n], vr[r][:n], q[r])) <= TOL, r


def test_attn_paged_rejects_bad_arguments(torch_gpu):
    torch = torch_gpu
    z = torch.zeros(768, dtype=torch.float32, device="cuda")
    i = torch.zeros(4, dtype=torch.int32, device="cuda")
    with pytest.raises(lib.MossHipError) as e:  # 2 pages of 64 cannot hold 200 keys
        lib.attn_paged(z.view(1, 768), z, z, 12, i, 2, 64, i, 200, z.view(1, 768))
    assert e.value.code == lib.EINVAL
    with pytest.raises(lib.MossHipError) as e:  # a 64-key span would cross a page of 100
        lib.attn_paged(z.view(1, 768), z, z, 12, i, 4, 100, i, 200, z.view(1, 768))
    assert e.value.code == lib.EINVAL and "multiple of 64" in str(e.value)


def test_attn_paged_pages_of_128(torch_gpu, oracle):
    """Pages of 128 positions: each page holds two 64-key spans, at offsets 0 and 64."""
    torch = torch_gpu
    rng = np.random.default_rng(128)
    keys = [1, 64, 65, 127, 128, 129, 255, 256, 257, 600, 1000]
    kp, vp, table, per, kr, vr = _case(rng, keys, 12, np.float16, page=128)
    rows = len(keys)
    row_pos = np.array([n - 1 for n in keys], np.int32)
    q = rng.standard_normal((rows, 768)).astype(np.float32)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    out = torch.full((rows, 768), float("nan"), dtype=torch.float32, device="cuda")
    lib.attn_paged(dev(q), dev(kp), dev(vp), 12, dev(table), per, 128, dev(row_pos), max(keys), out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for r in range(rows):
        assert max_rel(got[r], oracle.attention(kr[r], vr[r], q[r])) <= TOL, (r, keys[r])
