"""GPU: the batched quantized matmul (kmi_qmm_batched, both orientations)
and mlx-lm's quantized scaled-dot-product attention built on it
(kvattn.quantized_sdpa, after .../_mlx_vlm/models/base.py:260-302), against
the oracle.  The kernel dequantizes weight tiles in fp32 and feeds them to
the matrix cores as two bf16 parts (hi + lo, exact to 2^-17) where the
oracle keeps them exact, so the products meet the float bar (max rel err
<= 1e-2, cosine >= 0.9999), not bit equality.  All of mlx's affine widths
(2, 3, 4, 5, 6, 8 bits) are covered."""
import numpy as np
import pytest
import torch

import oracle as O
from knurlogic_amd import kvattn, ops
from knurlogic_amd import kvcache as KC
from tests.util import assert_close, bf16_normal, to_numpy, to_torch, u32_to_torch

pytestmark = pytest.mark.gpu


def _quantized(rng, shape, group, bits, dev, std=0.02):
    w = bf16_normal(rng, shape, std)
    wq, s, b = O.quantize(w, group, bits)
    return (wq, s, b), (u32_to_torch(wq, dev), to_torch(s, dev, torch.bfloat16), to_torch(b, dev, torch.bfloat16))


CASES = [
    # (x batch, w batch, M, K, N)
    ((), (), 1, 256, 512),
    ((3,), (3,), 5, 128, 256),
    ((2, 4), (1, 4), 16, 384, 128),        # w broadcast over the outer batch dimension
    ((2, 4, 3), (2, 4, 1), 1, 128, 640),   # w broadcast over the inner one: folded into M
    ((2,), (2,), 70, 192, 320),            # several row tiles, ragged edges
]


@pytest.mark.parametrize("transpose", [True, False])
@pytest.mark.parametrize("bits,group", [(4, 64), (8, 64), (4, 32), (8, 128), (2, 64), (3, 32), (5, 64),
                                        (6, 128)])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_batched_qmm_matches_the_oracle(dev, transpose, bits, group, case):
    xb, wb, M, K, N = CASES[case]
    if (K if transpose else N) % group:
        pytest.skip("the quantized axis is not a multiple of the group")
    rng = np.random.default_rng(100 + case)
    x = bf16_normal(rng, xb + (M, K))
    shape = wb + ((N, K) if transpose else (K, N))
    (wq, s, b), (tw, ts, tb) = _quantized(rng, shape, group, bits, dev)
    ref = O.quantized_matmul_batched(x, wq, s, b, transpose, group, bits, "float32")
    got = ops.quantized_matmul(to_torch(x, dev, torch.bfloat16), tw, ts, tb, transpose, group, bits)
    assert tuple(got.shape) == ref.shape
    assert_close(to_numpy(got), ref, what=f"case {case} transpose={transpose}")


@pytest.mark.parametrize("K", [1, 7, 1000, 8192])
def test_transpose_false_over_long_and_ragged_reductions(dev, K):
    """Attention's second product: K = keys, any length (x rows padded to
    16 bytes by the op), split across workgroups when long."""
    rng = np.random.default_rng(K)
    x = bf16_normal(rng, (3, 8, K), 0.1)
    (wq, s, b), (tw, ts, tb) = _quantized(rng, (3, K, 128), 64, 8, dev, 1.0)
    ref = O.quantized_matmul_batched(x, wq, s, b, False, 64, 8, "float32")
    got = ops.quantized_matmul(to_torch(x, dev, torch.bfloat16), tw, ts, tb, False, 64, 8)
    assert_close(to_numpy(got), ref, what=f"K={K}")


@pytest.mark.parametrize("bits", [2, 3, 5, 6])
def test_dense_projection_at_the_other_widths(dev, bits):
    """A 2-D weight at 2, 3, 5 or 6 bits (mlx's other affine widths) through
    quantized_matmul, decode and prefill row counts."""
    rng = np.random.default_rng(bits)
    (wq, s, b), (tw, ts, tb) = _quantized(rng, (320, 512), 64, bits, dev)
    for M in (1, 70):
        x = bf16_normal(rng, (M, 512))
        got = ops.quantized_matmul(to_torch(x, dev, torch.bfloat16), tw, ts, tb, True, 64, bits)
        ref = O.quantized_matmul(x, wq, s, b, True, 64, bits, "float32")
        assert_close(to_numpy(got), ref, what=f"{bits}-bit M={M}")


def test_gather_qmm_transpose_false(dev):
    """mx.gather_qmm with transpose=False (What[e] [K, N], groups along N):
    each pair's x rows times its expert's weight."""
    rng = np.random.default_rng(31)
    E, K, N, P, M = 5, 256, 192, 7, 3
    (wq, s, b), (tw, ts, tb) = _quantized(rng, (E, K, N), 64, 4, dev)
    x = bf16_normal(rng, (P, M, K))
    rhs = rng.integers(0, E, P).astype(np.int32)
    got = ops.gather_qmm(to_torch(x, dev, torch.bfloat16), tw, ts, tb, rhs_indices=torch.from_numpy(rhs).to(dev),
                         transpose=False, group_size=64, bits=4)
    ref = np.stack([O.quantized_matmul(x[p], wq[rhs[p]], s[rhs[p]], b[rhs[p]], False, 64, 4, "float32")
                    for p in range(P)])
    assert got.shape == (P, M, N)
    assert_close(to_numpy(got), ref, what="gather transpose=False")


def test_strided_slab_views_are_read_in_place(dev):
    """K/V slabs are views into a larger capacity: the batch and row strides
    are passed through, nothing is copied."""
    rng = np.random.default_rng(7)
    cap, n = 300, 211
    (wq, s, b), (tw, ts, tb) = _quantized(rng, (2, 4, cap, 128), 64, 8, dev, 1.0)
    x = bf16_normal(rng, (2, 4, 3, 128))
    view = (tw[:, :, :n], ts[:, :, :n], tb[:, :, :n])
    ref = O.quantized_matmul_batched(x, wq[:, :, :n], s[:, :, :n], b[:, :, :n], True, 64, 8, "float32")
    got = ops.quantized_matmul(to_torch(x, dev, torch.bfloat16), *view, True, 64, 8)
    assert_close(to_numpy(got), ref, what="slab view")


def test_rows_are_independent(dev):
    """An output row depends on its own input row only (the row-independence
    rule of the quantized path)."""
    rng = np.random.default_rng(9)
    (wq, s, b), (tw, ts, tb) = _quantized(rng, (2, 512, 256), 64, 4, dev)
    x = to_torch(bf16_normal(rng, (2, 40, 512)), dev, torch.bfloat16)
    full = ops.quantized_matmul(x, tw, ts, tb, False, 64, 4)
    for m in (0, 17, 39):
        one = ops.quantized_matmul(x[:, m:m + 1].contiguous(), tw, ts, tb, False, 64, 4)
        assert torch.equal(one[:, 0], full[:, m])


def _qkv(rng, B, Hq, Hk, L, N, D, bits, dev):
    q = bf16_normal(rng, (B, Hq, L, D))
    K, Kt = _quantized(rng, (B, Hk, N, D), 64, bits, dev, 1.0)
    V, Vt = _quantized(rng, (B, Hk, N, D), 64, bits, dev, 1.0)
    return q, K, V, Kt, Vt


@pytest.mark.parametrize("mask", [None, "causal", "bool", "additive", "hidden_row"])
@pytest.mark.parametrize("L,N", [(1, 1), (1, 37), (4, 600), (2, 4100)])
@pytest.mark.parametrize("bits", [8, 4])
def test_quantized_sdpa_matches_the_oracle(dev, mask, L, N, bits):
    rng = np.random.default_rng(L * 1000 + N)
    B, Hq, Hk, D = 2, 8, 2, 128
    q, K, V, Kt, Vt = _qkv(rng, B, Hq, Hk, L, N, D, bits, dev)
    m, tm = mask, mask
    if mask in ("bool", "hidden_row"):
        m = rng.random((B, 1, L, N)) > 0.3
        if mask == "hidden_row":
            m[1, 0, L - 1, :] = False
        tm = torch.from_numpy(m).to(dev)
    elif mask == "additive":
        m = O.bf16_round(rng.standard_normal((B, 1, L, N)).astype(np.float32))
        tm = to_torch(m, dev, torch.bfloat16)
    scale = D ** -0.5
    ref = O.quantized_sdpa(q, K, V, scale, m, 64, bits)
    got = kvattn.quantized_sdpa(to_torch(q, dev, torch.bfloat16), Kt, Vt, scale, tm, 64, bits)
    assert got.shape == q.shape
    assert_close(to_numpy(got), ref, what=f"mask={mask} L={L} N={N}")


def test_rep_one_and_a_mask_without_batch_axes(dev):
    """Hq == Hk (no GQA reshape) and an (L, N) mask broadcast over batch and heads."""
    rng = np.random.default_rng(21)
    B, H, L, N, D = 1, 4, 3, 50, 64
    q, K, V, Kt, Vt = _qkv(rng, B, H, H, L, N, D, 8, dev)
    m = rng.random((L, N)) > 0.5
    m[:, 0] = True
    ref = O.quantized_sdpa(q, K, V, 0.1, m, 64, 8)
    got = kvattn.quantized_sdpa(to_torch(q, dev, torch.bfloat16), Kt, Vt, 0.1, torch.from_numpy(m).to(dev), 64, 8)
    assert_close(to_numpy(got), ref, what="rep 1")


class _MlxQuantizedCache:
    """The attributes mlx-lm's base dispatch looks at on its quantized cache."""
    bits = 8
    group_size = 64


def test_sdpa_dispatch_takes_the_quantized_products_for_a_bits_cache(dev):
    rng = np.random.default_rng(22)
    B, Hq, Hk, L, N, D = 1, 8, 2, 2, 300, 128
    q, K, V, Kt, Vt = _qkv(rng, B, Hq, Hk, L, N, D, 8, dev)
    got = kvattn.sdpa(to_torch(q, dev, torch.bfloat16), Kt, Vt, _MlxQuantizedCache(), D ** -0.5, "causal")
    ref = O.quantized_sdpa(q, K, V, D ** -0.5, "causal", 64, 8)
    assert_close(to_numpy(got), ref, what="dispatch")
    with pytest.raises(ValueError):
        kvattn.sdpa(to_torch(q, dev, torch.bfloat16), Kt, Vt, _MlxQuantizedCache(), 0.1, None,
                    sinks=torch.zeros(Hq, device=dev))


def test_quantized_sdpa_over_a_quant_kv_cache_slab(dev):
    """The products read a QuantKVCache's slabs (capacity > offset) in place."""
    c = KC.QuantKVCache(8)
    g = torch.Generator(device=dev).manual_seed(3)
    for n in (100, 1, 1):
        k = torch.randn(1, 2, n, 128, device=dev, generator=g).to(torch.bfloat16)
        c.update_and_fetch(k, -k)
    K = tuple(t[:, :, :c.offset] for t in c.keys)
    V = tuple(t[:, :, :c.offset] for t in c.values)
    q = torch.randn(1, 8, 1, 128, device=dev, generator=g).to(torch.bfloat16)
    got = kvattn.quantized_sdpa(q, K, V, 0.088, None, c.group, 8)
    Kn = tuple(to_numpy(t) if t.dtype != torch.uint32 else t.view(torch.int32).cpu().numpy().view(np.uint32)
               for t in K)
    Vn = tuple(to_numpy(t) if t.dtype != torch.uint32 else t.view(torch.int32).cpu().numpy().view(np.uint32)
               for t in V)
    ref = O.quantized_sdpa(to_numpy(q), Kn, Vn, 0.088, None, c.group, 8)
    assert_close(to_numpy(got), ref, what="cache slab")


def test_bad_operands_raise(dev):
    rng = np.random.default_rng(1)
    _, (tw, ts, tb) = _quantized(rng, (2, 128, 256), 64, 4, dev)
    x = torch.zeros(2, 3, 100, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        ops.quantized_matmul(x, tw, ts, tb, False, 64, 4)          # K mismatch
    with pytest.raises(ValueError):
        ops.quantized_matmul(x.float(), tw, ts, tb, True, 64, 4)   # dtype
    with pytest.raises(ValueError):
        kvattn.masked_softmax(torch.zeros(2, 5, dtype=torch.bfloat16, device=dev),
                              torch.zeros(2, 5, device=dev))        # f32 additive mask
