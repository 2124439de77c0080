"""GPU parity: quantized_matmul (decode GEMV M <= 16, prefill GEMM M > 16)
and gather_qmm through the C ABI, against the oracle on identical seeded
inputs.  Bar: max |y - ref| / max |ref| <= 1e-2 and cosine >= 0.9999
(fp32 accumulation, bf16 out)."""
import functools

import numpy as np
import pytest
import torch

import knurlogic_amd as K
import oracle as O
from tests.util import assert_close, bf16_normal, to_numpy, to_torch, u32_to_torch

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _weights(rng, shape, bits, group, dev):
    w = bf16_normal(rng, shape, 0.02)
    wq, s, b = O.quantize(w, group, bits)
    return (wq, s, b), (u32_to_torch(wq, dev), to_torch(s, dev, BF), to_torch(b, dev, BF))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("M", [1, 2, 3, 16, 17, 33, 48, 64, 200])
def test_qmm_small(dev, bits, group, M):
    rng = np.random.default_rng(1000 * bits + group + M)
    N, K_ = 320, 512
    (wq, s, b), (tw, ts, tb) = _weights(rng, (N, K_), bits, group, dev)
    x = bf16_normal(rng, (M, K_))
    y = K.quantized_matmul(to_torch(x, dev, BF), tw, ts, tb, True, group, bits)
    assert y.shape == (M, N) and y.dtype == BF
    ref = O.quantized_matmul(x, wq, s, b, True, group, bits, "float32")
    assert_close(to_numpy(y), ref, what=f"M={M} bits={bits} g={group}")


@functools.lru_cache(maxsize=4)
def _big_weights(bits, shape):
    w = bf16_normal(np.random.default_rng(7 + bits + shape[0]), shape, 0.02)
    return O.quantize(w, 64, bits)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [1, 16, 512])
@pytest.mark.parametrize("shape", [(14336, 4096), (4096, 14336)])
def test_qmm_decode_and_prefill_shapes(dev, bits, M, shape):
    """The dense workload: W [14336, 4096] and its reverse, M = 1, 16, 512,
    every output element against the oracle (the GEMV, the skinny kernel's
    K split and the GEMM's 128-column blocks and 4-way K split alike)."""
    N, K_ = shape
    wq, s, b = _big_weights(bits, shape)
    tw, ts, tb = u32_to_torch(wq, dev), to_torch(s, dev, BF), to_torch(b, dev, BF)
    x = bf16_normal(np.random.default_rng(7 + bits + M + N), (M, K_))
    y = to_numpy(K.quantized_matmul(to_torch(x, dev, BF), tw, ts, tb, True, 64, bits))
    assert y.shape == (M, N)
    ref = O.quantized_matmul(x, wq, s, b, True, 64, bits, "float32")
    assert_close(y, ref, what=f"{shape} M={M} bits={bits}")
    # and block by block: a wrong 128-column block must not hide in the
    # whole-matrix maximum
    for c in range(0, N, 2048):
        assert_close(y[:, c:c + 2048], ref[:, c:c + 2048], what=f"{shape} M={M} bits={bits} cols {c}+")


def test_qmm_decode_4096_square_every_column(dev):
    """The single-layer decode workload: 4-bit g64 W [4096, 4096] ~ N(0, 0.02)
    quantized on the GPU, x [1, 4096] ~ N(0, 1) bf16, every output column
    against the oracle's matmul over the oracle's own quantization (the GPU
    quantization is checked bit for bit on the way)."""
    rng = np.random.default_rng(20251)
    w = bf16_normal(rng, (4096, 4096), 0.02)
    x = bf16_normal(rng, (1, 4096))
    wq, s, b = K.quantize(to_torch(w, dev, BF), group_size=64, bits=4)
    rq, rs, rb = O.quantize(w, 64, 4)
    np.testing.assert_array_equal(wq.view(torch.int32).cpu().numpy().view(np.uint32), rq)
    np.testing.assert_array_equal(to_numpy(s), rs)
    np.testing.assert_array_equal(to_numpy(b), rb)
    y = to_numpy(K.quantized_matmul(to_torch(x, dev, BF), wq, s, b, True, 64, 4))
    ref = O.quantized_matmul(x, rq, rs, rb, True, 64, 4, "float32")
    assert y.shape == (1, 4096)
    assert_close(y, ref, what="[4096, 4096] M=1")


def test_rows_are_independent_bit_for_bit(dev):
    """Row m of a call depends only on row m (the reference's padding
    contract, tests/engine/test_per_chip_rounding.py:30-41): within each
    kernel family (as in mlx, where qmv and qmm differ) a row's bits do not
    change with the number of other rows."""
    rng = np.random.default_rng(11)
    (wq, s, b), (tw, ts, tb) = _weights(rng, (256, 512), 4, 64, dev)
    x = to_torch(bf16_normal(rng, (128, 512)), dev, BF)
    # direct-to-LDS MFMA kernel: 2..16 rows
    y16 = K.quantized_matmul(x[:16], tw, ts, tb, True, 64, 4)
    for m in (2, 5, 9, 15):
        ym = K.quantized_matmul(x[:m], tw, ts, tb, True, 64, 4)
        assert torch.equal(ym, y16[:m]), m
    # skinny MFMA kernel: 17..64 rows (32- and 64-row tiles); the padded
    # 9..31-row calls of the reference land here as 32-row calls
    y64 = K.quantized_matmul(x[:64], tw, ts, tb, True, 64, 4)
    for m in (17, 31, 32, 40):
        ym = K.quantized_matmul(x[:m], tw, ts, tb, True, 64, 4)
        assert torch.equal(ym, y64[:m]), m
    # GEMM: 65..128 rows
    y128 = K.quantized_matmul(x, tw, ts, tb, True, 64, 4)
    y96 = K.quantized_matmul(x[:96], tw, ts, tb, True, 64, 4)
    assert torch.equal(y96, y128[:96])


@pytest.mark.parametrize("M,shape", [(16, (14336, 4096)), (16, (4096, 14336)), (5, (14336, 4096))])
def test_qmm_repeats_bit_for_bit(dev, M, shape):
    """The same call four times gives the same bits (the skinny kernels'
    LDS pipelines and the split-K reduction are deterministic)."""
    g = torch.Generator(device=dev).manual_seed(M)
    w = (torch.randn(*shape, device=dev, generator=g) * 0.02).to(BF)
    wq, s, b = K.quantize(w, 64, 4)
    x = torch.randn(M, shape[1], device=dev, generator=g).to(BF)
    ys = [K.quantized_matmul(x, wq, s, b) for _ in range(4)]
    for y in ys[1:]:
        assert torch.equal(y, ys[0])


def test_linearity_at_full_size(dev):
    """qmm(2x) == 2 qmm(x) bit for bit (power-of-two scaling is exact), and
    qmm(x1 + x2) ~ qmm(x1) + qmm(x2), at the [14336, 4096] 4-bit shape."""
    g = torch.Generator(device=dev).manual_seed(1)
    w = (torch.randn(14336, 4096, device=dev, generator=g) * 0.02).to(BF)
    wq, s, b = K.quantize(w, 64, 4)
    x = torch.randn(16, 4096, device=dev, generator=g).to(BF)
    y = K.quantized_matmul(x, wq, s, b)
    assert torch.equal(K.quantized_matmul(x * 2, wq, s, b), y * 2)
    x1 = torch.randn(1, 4096, device=dev, generator=g).to(BF)
    x2 = torch.randn(1, 4096, device=dev, generator=g).to(BF)
    ysum = K.quantized_matmul((x1.float() + x2.float()).to(BF), wq, s, b).float()
    lin = K.quantized_matmul(x1, wq, s, b).float() + K.quantized_matmul(x2, wq, s, b).float()
    # x1 + x2 is rounded to bf16 before the product: allow that and bf16 outputs
    assert_close(ysum.cpu().numpy(), lin.cpu().numpy(), max_rel=2e-2, min_cos=0.999,
                 what="linearity")


def test_zero_rows_and_shape_errors(dev):
    rng = np.random.default_rng(12)
    (wq, s, b), (tw, ts, tb) = _weights(rng, (64, 128), 4, 64, dev)
    y = K.quantized_matmul(torch.zeros(0, 128, device=dev, dtype=BF), tw, ts, tb)
    assert y.shape == (0, 64)
    with pytest.raises(ValueError):
        K.quantized_matmul(torch.zeros(2, 96, device=dev, dtype=BF), tw, ts, tb)
    with pytest.raises(ValueError):
        K.quantized_matmul(torch.zeros(2, 128, device=dev, dtype=BF), tw, ts, None)
    with pytest.raises(ValueError):
        K.quantized_matmul(torch.zeros(2, 128, dtype=BF), tw, ts, tb)   # CPU tensor


# --- gather_qmm ----------------------------------------------------------------

@pytest.mark.parametrize("T,k", [(1, 8), (5, 3), (16, 8), (40, 4)])
@pytest.mark.parametrize("bits", [4, 8])
def test_gather_qmm_unsorted_and_sorted(dev, T, k, bits):
    rng = np.random.default_rng(T * 10 + k + bits)
    E, N, K_ = 12, 96, 256
    (wq, s, b), (tw, ts, tb) = _weights(rng, (E, N, K_), bits, 64, dev)
    x = bf16_normal(rng, (T, 1, 1, K_))
    inds = rng.integers(0, E, (T, k)).astype(np.int32)
    ref = O.gather_qmm(x, wq, s, b, rhs_indices=inds, bits=bits, out_dtype="float32")
    tx = to_torch(x, dev, BF)
    ti = torch.from_numpy(inds).to(dev)
    y = K.gather_qmm(tx, tw, ts, tb, rhs_indices=ti, bits=bits)
    assert y.shape == (T, k, 1, N)
    assert_close(to_numpy(y), ref, what="unsorted")
    # the sorted form SwitchGLU uses for T*k >= 64: x rows gathered by order // k
    flat = inds.reshape(-1)
    order = np.argsort(flat, kind="stable")
    xs = x.reshape(T, 1, K_)[order // k]
    ys = K.gather_qmm(to_torch(xs, dev, BF), tw, ts, tb,
                      rhs_indices=torch.from_numpy(flat[order]).to(dev), bits=bits,
                      sorted_indices=True)
    assert ys.shape == (T * k, 1, N)
    assert_close(to_numpy(ys)[np.argsort(order)].reshape(T, k, 1, N), ref, what="sorted")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("group", [32, 64])
@pytest.mark.parametrize("M,N,K_", [(2, 100, 256), (7, 64, 768), (15, 200, 1280), (16, 1000, 4096),
                                    (9, 64, 256 * 33)])
def test_qmm_direct_lds_rows(dev, bits, group, M, N, K_):
    """2..16 rows, 4/8 bits, groups of 32/64: the direct-to-LDS kernel.
    Ragged N (rows past N read zeros), one chunk, odd chunk counts, and a
    33-chunk K cut into 7 splits of 5 (the last split shorter)."""
    rng = np.random.default_rng(31 * M + N + K_ + bits + group)
    (wq, s, b), (tw, ts, tb) = _weights(rng, (N, K_), bits, group, dev)
    x = bf16_normal(rng, (M, K_))
    y = K.quantized_matmul(to_torch(x, dev, BF), tw, ts, tb, True, group, bits)
    ref = O.quantized_matmul(x, wq, s, b, True, group, bits, "float32")
    assert_close(to_numpy(y), ref, what=f"M={M} N={N} K={K_} bits={bits} g={group}")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M,N,K_", [(16, 32, 8192), (5, 48, 16384)])
def test_long_k_few_rows_splits_k(dev, bits, M, N, K_):
    """Few weight rows and a long K: the skinny kernel splits K across
    workgroups and the fp32 partials are summed in split order."""
    rng = np.random.default_rng(M + N + bits)
    (wq, s, b), (tw, ts, tb) = _weights(rng, (N, K_), bits, 64, dev)
    x = bf16_normal(rng, (M, K_))
    y = K.quantized_matmul(to_torch(x, dev, BF), tw, ts, tb, True, 64, bits)
    ref = O.quantized_matmul(x, wq, s, b, True, 64, bits, "float32")
    assert_close(to_numpy(y), ref, what=f"split K M={M} K={K_}")


@pytest.mark.parametrize("bits", [4, 8])
def test_gather_qmm_many_rows_per_expert(dev, bits):
    """~100 rows per expert: 64-row tiles, several per expert, and a ragged last tile."""
    rng = np.random.default_rng(31 + bits)
    E, N, K_, T, k = 4, 80, 384, 200, 2
    (wq, s, b), (tw, ts, tb) = _weights(rng, (E, N, K_), bits, 64, dev)
    x = bf16_normal(rng, (T, 1, 1, K_))
    inds = rng.integers(0, E, (T, k)).astype(np.int32)
    y = K.gather_qmm(to_torch(x, dev, BF), tw, ts, tb, rhs_indices=torch.from_numpy(inds).to(dev),
                     bits=bits)
    ref = O.gather_qmm(x, wq, s, b, rhs_indices=inds, bits=bits, out_dtype="float32")
    assert_close(to_numpy(y), ref, what="many rows per expert")


@pytest.mark.parametrize("bits", [4, 8])
def test_gather_qmm_long_rows(dev, bits):
    """One row per expert tile with 14336-long rows (4-bit rows in one batch
    of loads on 8-wave workgroups, 8-bit rows in two on 16-wave ones) and
    200 output rows (the last workgroup partly past N), against the
    oracle."""
    rng = np.random.default_rng(14336 + bits)
    E, N, K_, T, k = 3, 200, 14336, 3, 2
    (wq, s, b), (tw, ts, tb) = _weights(rng, (E, N, K_), bits, 64, dev)
    x = bf16_normal(rng, (T, 1, 1, K_))
    inds = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    y = K.gather_qmm(to_torch(x, dev, BF), tw, ts, tb, rhs_indices=torch.from_numpy(inds).to(dev), bits=bits)
    ref = O.gather_qmm(x, wq, s, b, rhs_indices=inds, bits=bits, out_dtype="float32")
    assert_close(to_numpy(y), ref, what=f"gather_qmm K={K_} bits={bits}")


def test_gather_qmm_with_lhs_indices_and_bad_experts(dev):
    rng = np.random.default_rng(21)
    E, N, K_ = 4, 64, 128
    (wq, s, b), (tw, ts, tb) = _weights(rng, (E, N, K_), 4, 64, dev)
    x = bf16_normal(rng, (3, 2, K_))                      # X=3 batches of M=2 rows
    lhs = np.array([2, 0, 1, 2], np.int32)
    rhs = np.array([1, 3, 0, 9], np.int32)                # expert 9 is out of range
    y = K.gather_qmm(to_torch(x, dev, BF), tw, ts, tb, torch.from_numpy(lhs).to(dev),
                     torch.from_numpy(rhs).to(dev))
    assert y.shape == (4, 2, N)
    got = to_numpy(y)
    for p in range(3):
        ref = O.quantized_matmul(x[lhs[p]], wq[rhs[p]], s[rhs[p]], b[rhs[p]], True, 64, 4, "float32")
        assert_close(got[p], ref, what=f"pair {p}")
    assert (got[3] == 0).all()


def test_gather_qmm_moe_decode_shape(dev):
    """The Qwen3.5-MoE expert shapes (128 experts, 2048 -> 768, 4-bit g64),
    top-8 of 16 tokens: gate projection through gather_qmm."""
    rng = np.random.default_rng(22)
    E, N, K_, T, k = 128, 768, 2048, 16, 8
    (wq, s, b), (tw, ts, tb) = _weights(rng, (E, N, K_), 4, 64, dev)
    x = bf16_normal(rng, (T, 1, 1, K_))
    inds = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    y = K.gather_qmm(to_torch(x, dev, BF), tw, ts, tb,
                     rhs_indices=torch.from_numpy(inds).to(dev))
    ref = O.gather_qmm(x, wq, s, b, rhs_indices=inds, out_dtype="float32")
    assert_close(to_numpy(y), ref, what="moe decode")


def test_strided_views_are_read_as_their_values(dev):
    """Non-contiguous w / scales / biases / x (column slices of wider
    tensors): the ops copy them contiguous and keep every copy alive until
    the kernel is enqueued (a freed copy can hand its memory to the next)."""
    rng = np.random.default_rng(31)
    N, K_, E = 96, 256, 5
    (wq, s, b), (tw, ts, tb) = _weights(rng, (E, N, K_), 4, 64, dev)
    wide = lambda t: torch.cat([t, t], dim=-1)[..., :t.shape[-1]]
    vw, vs, vb = wide(tw), wide(ts), wide(tb)
    assert not (vw.is_contiguous() or vs.is_contiguous() or vb.is_contiguous())
    x = bf16_normal(rng, (3, K_))
    vx = wide(to_torch(x, dev, BF))
    y = K.quantized_matmul(vx, vw[2], vs[2], vb[2], bits=4)
    assert_close(to_numpy(y), O.quantized_matmul(x, wq[2], s[2], b[2], True, 64, 4, "float32"),
                 what="qmm views")
    inds = np.array([[4, 0], [1, 1], [3, 2]], np.int32)
    g = K.gather_qmm(vx.reshape(3, 1, 1, K_), vw, vs, vb, rhs_indices=torch.from_numpy(inds).to(dev), bits=4)
    ref = O.gather_qmm(x.reshape(3, 1, 1, K_), wq, s, b, rhs_indices=inds, bits=4, out_dtype="float32")
    assert_close(to_numpy(g), ref, what="gather views")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M,N,K_", [(129, 200, 512), (300, 200, 4096), (256, 4096, 14336 // 4),
                                    (513, 130, 1024), (300, 200, 576), (257, 1030, 2880)])
def test_large_m_tiles_and_split_k(dev, bits, M, N, K_):
    """The 256 x 128 GEMM: ragged M and N edges, and K split across
    workgroups (fp32 partials summed in split order) when tiles are few; K of
    9 and 45 k-tiles, which end part-way through the 4-deep load ring."""
    rng = np.random.default_rng(M * 31 + N + K_ + bits)
    (wq, s, b), (tw, ts, tb) = _weights(rng, (N, K_), bits, 64, dev)
    x = bf16_normal(rng, (M, K_))
    y = K.quantized_matmul(to_torch(x, dev, BF), tw, ts, tb, bits=bits)
    ref = O.quantized_matmul(x, wq, s, b, True, 64, bits, "float32")
    assert_close(to_numpy(y), ref, what=f"M={M}")
