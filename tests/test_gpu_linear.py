"""GPU parity: the dense layers a quantized model keeps unquantized (mlx's
nn.Linear: the MoE router and shared-expert gate) and the bias adds of the
quantized layers, through the C ABI, against the oracle.  Bar: max rel err
1e-2, cosine 0.9999 for the products (fp32 accumulation, one rounding);
the bias add is bit-exact (one bf16 addition)."""
import numpy as np
import pytest
import torch

import knurlogic_amd as K
import oracle as O
from knurlogic_amd import nn
from tests.util import assert_close, bf16_normal, to_numpy, to_torch, u32_to_torch

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


@pytest.mark.parametrize("M,K_,N", [(1, 2048, 128), (16, 2048, 128), (256, 2048, 128), (5, 2048, 1),
                                    (9, 520, 77), (3, 4096, 4096)])
def test_linear_matches_the_oracle(dev, M, K_, N):
    rng = np.random.default_rng(M + K_ + N)
    x = bf16_normal(rng, (M, K_))
    w = bf16_normal(rng, (N, K_), 0.02)
    y = K.linear(to_torch(x, dev, BF), to_torch(w, dev, BF))
    assert y.shape == (M, N) and y.dtype == BF
    assert_close(to_numpy(y), O.dense_linear(x, w, "float32"), what=f"linear {M}x{K_}x{N}")


def test_linear_with_bias_rounds_once(dev):
    """addmm(bias, x, w^T): the bias joins the fp32 sum before the one
    rounding, and a batch of leading dimensions is kept."""
    rng = np.random.default_rng(3)
    x = bf16_normal(rng, (2, 3, 256))
    w = bf16_normal(rng, (64, 256), 0.05)
    b = bf16_normal(rng, (64,))
    y = K.linear(to_torch(x, dev, BF), to_torch(w, dev, BF), to_torch(b, dev, BF))
    assert y.shape == (2, 3, 64)
    ref = O.round_to((x.astype(np.float64) @ w.astype(np.float64).T + b).astype(np.float32), "float32")
    assert_close(to_numpy(y), ref, what="linear + bias")


def test_router_gate_module_routes_like_the_oracle(dev):
    """nn.Linear as SparseMoeBlock's gate: logits, then the router."""
    rng = np.random.default_rng(4)
    x = bf16_normal(rng, (16, 2048))
    w = bf16_normal(rng, (128, 2048), 0.02)
    logits = nn.Linear(to_torch(w, dev, BF))(to_torch(x, dev, BF))
    ref = O.dense_linear(x, w)
    assert_close(to_numpy(logits), ref, what="router logits")
    # the same logits route the same way
    inds, scores = K.moe_route(logits, 8)
    ri, rs = O.route(to_numpy(logits), 8)
    np.testing.assert_array_equal(inds.cpu().numpy(), ri)
    np.testing.assert_array_equal(to_numpy(scores), rs)


def test_bias_adds_are_one_rounded_addition(dev):
    rng = np.random.default_rng(5)
    y = bf16_normal(rng, (4, 2, 1, 96))
    b = bf16_normal(rng, (6, 96))
    idx = np.array([[0, 5], [3, 3], [1, 2], [4, 0]], np.int32)
    got = K.add_bias(to_torch(y, dev, BF), to_torch(b, dev, BF), torch.from_numpy(idx).to(dev))
    ref = O.round_to(y + b[idx][:, :, None, :], "bfloat16")
    np.testing.assert_array_equal(to_numpy(got), ref)
    one = K.add_bias(to_torch(y[0, 0], dev, BF), to_torch(b[2], dev, BF))
    np.testing.assert_array_equal(to_numpy(one), O.round_to(y[0, 0] + b[2], "bfloat16"))


def test_quantized_layers_add_their_bias_in_the_library(dev):
    rng = np.random.default_rng(6)
    w = bf16_normal(rng, (3, 64, 128), 0.02)
    bias = bf16_normal(rng, (3, 64))
    wq, s, b = O.quantize(w, 64, 4)
    tq = (u32_to_torch(wq, dev), to_torch(s, dev, BF), to_torch(b, dev, BF))
    x = bf16_normal(rng, (5, 1, 1, 128))
    inds = np.array([[0], [2], [1], [1], [0]], np.int32)
    layer = nn.QuantizedSwitchLinear(*tq, to_torch(bias, dev, BF), 64, 4)
    got = layer(to_torch(x, dev, BF), torch.from_numpy(inds).to(dev))
    plain = O.gather_qmm(x, wq, s, b, rhs_indices=inds)
    ref = O.round_to(plain + bias[inds][:, :, None, :], "bfloat16")
    assert_close(to_numpy(got), ref, what="switch linear + bias")
    dense = nn.QuantizedLinear(tq[0][1], tq[1][1], tq[2][1], to_torch(bias[1], dev, BF), 64, 4)
    y = dense(to_torch(x[:, 0, 0], dev, BF))
    refd = O.round_to(O.quantized_matmul(x[:, 0, 0], wq[1], s[1], b[1], True, 64, 4) + bias[1], "bfloat16")
    assert_close(to_numpy(y), refd, what="linear + bias")
