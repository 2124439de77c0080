"""GPU parity: 8-bit-KV decode attention (kvattn.decode_sdpa) through the C
ABI against the oracle (exact arithmetic over the dequantized cache), on
the reference's own sweep (tests/engine/test_kvattn.py:78-128,196-211,
253-279) and the 4 x 32-head / 4-KV-head, head-dim-128 decode workload at
8k and 32k keys.  Bar: max |err| / max |ref| <= 1e-2, cosine >= 0.9999, and
the reference's own 8e-3 * max(1, |ref|) for bf16 outputs."""
import numpy as np
import pytest
import torch

import oracle as O
from knurlogic_amd import kvattn
from tests.util import assert_close, bf16_normal, to_numpy, to_torch, u32_to_torch

pytestmark = pytest.mark.gpu
DT = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _case(dev, B, H, Hk, L, N, D, g=None, seed=0, dtype="bfloat16"):
    g = g or (64 if D % 64 == 0 else 32)
    rng = np.random.default_rng(seed)
    k = O.round_to(rng.standard_normal((B, Hk, N, D)).astype(np.float32), dtype)
    v = O.round_to(rng.standard_normal((B, Hk, N, D)).astype(np.float32), dtype)
    q = O.round_to(rng.standard_normal((B, H, L, D)).astype(np.float32), dtype)
    K = O.quantize(k, g, 8, dtype)
    V = O.quantize(v, g, 8, dtype)
    tq = to_torch(q, dev, DT[dtype])
    tK = (u32_to_torch(K[0], dev), to_torch(K[1], dev, DT[dtype]), to_torch(K[2], dev, DT[dtype]))
    tV = (u32_to_torch(V[0], dev), to_torch(V[1], dev, DT[dtype]), to_torch(V[2], dev, DT[dtype]))
    return (q, K, V, g), (tq, tK, tV)


def _check(host, gpu, mask, tmask=None, dtype="bfloat16"):
    q, K, V, g = host
    tq, tK, tV = gpu
    D = q.shape[-1]
    scale = D ** -0.5
    assert kvattn.supports(tq, tK, tV, 8, g, tmask if tmask is not None else mask)
    got = kvattn.decode_sdpa(tq, tK, tV, scale, tmask if tmask is not None else mask, g, 8)
    assert got.shape == tq.shape and got.dtype == tq.dtype
    ref = O.kv8_decode(q, K, V, scale, mask, g, 8, "float32")
    got = to_numpy(got)
    assert np.isfinite(got).all()
    assert_close(got, ref, what="kv8")
    if dtype == "bfloat16":
        assert np.abs(got - ref).max() < 8e-3 * max(1.0, np.abs(ref).max())
    return got, ref


@pytest.mark.parametrize("D", [128, 256, 512])
@pytest.mark.parametrize("H,Hk", [(4, 4), (8, 2), (16, 2), (16, 1)])
@pytest.mark.parametrize("N", [1, 7, 256, 1000, 4099])
def test_a_decode_step_matches_the_oracle(dev, D, H, Hk, N):
    _check(*_case(dev, 1, H, Hk, 1, N, D), None)


@pytest.mark.parametrize("L,H,Hk", [(2, 8, 2), (4, 4, 2), (3, 2, 2), (4, 16, 2), (8, 8, 1)])
def test_a_short_causal_query(dev, L, H, Hk):
    _check(*_case(dev, 1, H, Hk, L, 700, 128, seed=L), "causal")


@pytest.mark.parametrize("dtype", ["float32", "float16"])
@pytest.mark.parametrize("D,H,Hk,L", [(128, 8, 2, 1), (512, 8, 2, 1), (384, 32, 1, 1)])
def test_float32_and_float16_queries(dev, dtype, D, H, Hk, L):
    """q, scales and biases in float32 / float16, on each kernel: all rows
    per wave (D = 128), one row tile per workgroup (D = 512, 4 rows), a row
    tile per wave (D = 384, 32 rows)."""
    _check(*_case(dev, 2, H, Hk, L, 900, D, dtype=dtype), None, dtype=dtype)


@pytest.mark.parametrize("g", [32, 128])
def test_other_group_sizes(dev, g):
    _check(*_case(dev, 1, 8, 2, 1, 500, 128, g=g), None)


@pytest.mark.parametrize("D,g", [(256, 32), (128, 16), (512, 32), (512, 16), (384, 128), (512, 512)])
def test_groups_narrower_than_a_lane_run_and_other_head_dims(dev, D, g):
    """The shapes kv8_partial's per-wave state does not cover, taken by the
    16-row-tile kernel: groups below D/4, head dims 384 and 512."""
    _check(*_case(dev, 1, 8, 2, 1, 1000, D, g=g, seed=D + g), None)


@pytest.mark.parametrize("D,L,H,Hk", [(256, 1, 48, 1), (256, 4, 16, 1), (512, 2, 32, 1), (384, 4, 8, 2),
                                      (128, 1, 64, 2), (256, 2, 16, 1), (256, 3, 8, 1), (512, 8, 16, 2),
                                      (384, 2, 24, 1), (512, 1, 20, 1)])
def test_many_rows_per_kv_head_at_wide_head_dims(dev, D, L, H, Hk):
    """17 to 64 query rows per KV head at head dims 256-512 (and 32 rows
    at 128), causal where L > 1: a row tile per wave over shared K/V steps
    (33-64 rows at D = 256, 17-64 at 384 / 512; 20 rows: a partial second
    tile), the 16-row-tile kernel at 16, and at D = 256 with 17-32 rows the
    all-rows-per-wave one."""
    _check(*_case(dev, 1, H, Hk, L, 900, D, seed=L * H), "causal" if L > 1 else None)


def test_many_blocks_per_head(dev):
    """One (b, hk) pair over 20k keys: the combine merges more than one
    chunk of block partials."""
    _check(*_case(dev, 1, 16, 1, 1, 20000, 128, seed=9), None)


@pytest.mark.parametrize("L,H,Hk,D", [(1, 16, 2, 256), (2, 16, 2, 256), (2, 16, 1, 512), (3, 16, 1, 384)])
def test_a_ragged_left_padded_batch(dev, L, H, Hk, D):
    """Rows of different lengths, the left padding masked out; one row fully
    padded but the last keys (tests/engine/test_kvattn.py:103-113); also
    with 32 and 48 rows per KV head at D = 512 / 384 (the row-tile kernel)."""
    B, N = 3, 1200
    host, gpu = _case(dev, B, H, Hk, L, N, D, seed=3)
    pad = np.array([0, 513, N - L - 1])
    m = np.zeros((B, 1, L, N), bool)
    for b in range(B):
        for i in range(L):
            m[b, 0, i, pad[b]:N - L + i + 1] = True
    _check(host, gpu, m, torch.from_numpy(m).to(dev))


@pytest.mark.parametrize("H,Hk,D,g", [(8, 2, 128, 64), (32, 1, 128, 16), (24, 1, 256, 32)])
def test_sparse_holes_and_a_row_that_sees_nothing(dev, H, Hk, D, g):
    B, N = 3, 65
    host, gpu = _case(dev, B, H, Hk, 1, N, D, g=g, seed=4)
    m = np.ones((B, 1, 1, N), bool)
    m[..., np.arange(N) % 5 == 2] = False
    m[2] = False
    got, _ = _check(host, gpu, m, torch.from_numpy(m).to(dev))
    assert (got[2] == 0).all()


@pytest.mark.parametrize("H,Hk,L,D", [(8, 2, 1, 128), (8, 2, 1, 512), (16, 1, 4, 256)])
def test_the_bias_is_read_with_its_own_strides(dev, H, Hk, L, D):
    """A bias that is a strided view, not laid out like its scale
    (tests/engine/test_kvattn.py:201-211); and K/V that are views of a
    larger slab, as the quantized cache hands them out -- on the all-rows,
    one-tile and row-tile kernels."""
    host, (tq, tK, tV) = _case(dev, 2, H, Hk, L, 300, D, seed=5)
    wide = torch.cat([tK[2], tK[2]], dim=-1)
    Kv = (tK[0], tK[1], wide[..., :tK[2].shape[-1]])
    assert torch.equal(Kv[2], tK[2]) and Kv[2].stride() != tK[2].stride()
    slab = tuple(torch.cat([t, t[:, :, :56]], dim=2) for t in tV)
    Vv = tuple(t[:, :, :300] for t in slab)
    _check(host, (tq, Kv, Vv), "causal" if L > 1 else None)


def test_unsupported_shapes_are_refused_and_fall_back(dev):
    (q, K, V, g), (tq, tK, tV) = _case(dev, 1, 8, 2, 1, 64, 128)
    assert not kvattn.supports(tq, tK, tV, 4, g)
    assert not kvattn.supports(tq, tK, tV, 8, g, sinks=torch.zeros(8, device=dev))
    add = torch.zeros(1, 1, 1, 64, device=dev)
    assert not kvattn.supports(tq, tK, tV, 8, g, add)
    per_head = torch.ones(1, 8, 1, 64, dtype=torch.bool, device=dev)
    assert not kvattn.supports(tq, tK, tV, 8, g, per_head)
    (_, _, _, _), (q9, K9, V9) = _case(dev, 1, 32, 1, 3, 64, 128)
    assert not kvattn.supports(q9, K9, V9, 8, 64)               # 96 rows per KV head
    # the fallback (the packed-triple attention on the GPU) computes the same attention
    got = kvattn.quantized_sdpa(tq, tK, tV, 128 ** -0.5, None, g, 8)
    ref = O.kv8_decode(q, K, V, 128 ** -0.5, None, g, 8, "float32")
    assert_close(to_numpy(got), ref, what="fallback")


def test_sdpa_dispatch_counts_hits_and_misses(dev, monkeypatch):
    from tests.toy_attention import scaled_dot_product_attention as model_attention
    monkeypatch.setattr(kvattn, "_BASE", {"fn": model_attention})    # what patch_model records
    (q, K, V, g), (tq, tK, tV) = _case(dev, 1, 8, 2, 1, 100, 128)

    class Cache:
        kv8_fetch = None

    c = Cache()
    keys = torch.zeros(1)
    kvattn.reset(True)
    c.kv8_fetch = (keys, tK, tV, g)
    out = kvattn.sdpa(tq, keys, None, c, 128 ** -0.5, None)
    assert kvattn.STATS["hits"] == 1 and c.kv8_fetch is None
    ref = O.kv8_decode(q, K, V, 128 ** -0.5, None, g, 8, "float32")
    assert_close(to_numpy(out), ref, what="dispatch")
    # keys transformed after the fetch: a counted miss, dense attention
    kd = torch.from_numpy(O.dequantize(*K, g, 8)).to(dev).to(torch.bfloat16)
    vd = torch.from_numpy(O.dequantize(*V, g, 8)).to(dev).to(torch.bfloat16)
    c.kv8_fetch = (kd, tK, tV, g)
    out2 = kvattn.sdpa(tq, kd * 2, vd, c, 128 ** -0.5, None)
    assert kvattn.STATS["misses"] == 1 and out2.shape == tq.shape
    assert torch.equal(out2, model_attention(tq, kd * 2, vd, scale=128 ** -0.5))   # dense: the model's own


@pytest.mark.parametrize("N", [8192, 32768])
@pytest.mark.parametrize("L", [1, 4])
def test_the_decode_workload(dev, N, L):
    """4 sequences, 32 query heads over 4 KV heads, head dim 128, 8-bit
    group-64 K/V; 1 query token, or 4 under a causal mask (MTP verify)."""
    _check(*_case(dev, 4, 32, 4, L, N, 128, seed=N + L), "causal" if L > 1 else None)



def test_graph_replays_match_the_eager_call(dev):
    """decode_sdpa captured in a HIP graph after a warm call on the capturing
    stream; several replays, with eager work and synchronisation between
    them, each equal to the eager result."""
    host, gpu = _case(dev, 2, 16, 2, 1, 6000, 128, seed=31)
    tq, tK, tV = gpu
    scale = 128 ** -0.5
    eager = kvattn.decode_sdpa(tq, tK, tV, scale, None, 64, 8)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        kvattn.decode_sdpa(tq, tK, tV, scale, None, 64, 8)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = kvattn.decode_sdpa(tq, tK, tV, scale, None, 64, 8)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        again = kvattn.decode_sdpa(tq, tK, tV, scale, None, 64, 8)
        torch.cuda.synchronize()
        assert torch.equal(again, eager)
    del g
