"""GPU parity: affine quantize / dequantize through the C ABI, bit for bit
against the oracle (integer codes, scales, biases and dequantized values)."""
import numpy as np
import pytest
import torch

import knurlogic_amd as K
import oracle as O
from tests.util import bf16_normal, to_numpy, to_torch, u32_to_numpy, u32_to_torch

pytestmark = pytest.mark.gpu

DT = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _values(rng, shape, std, dtype):
    v = (rng.standard_normal(shape) * std).astype(np.float32)
    return O.round_to(v, dtype)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_quantize_is_bit_exact(dev, dtype, bits, group):
    rng = np.random.default_rng(100 + bits + group)
    w = _values(rng, (96, 384), 0.02, dtype)
    wq, s, b = K.quantize(to_torch(w, dev, DT[dtype]), group_size=group, bits=bits)
    rq, rs, rb = O.quantize(w, group, bits, dtype)
    assert wq.dtype == torch.uint32 and wq.shape == rq.shape
    assert np.array_equal(u32_to_numpy(wq), rq)
    assert np.array_equal(to_numpy(s), rs) and np.array_equal(to_numpy(b), rb)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
def test_quantize_rounds_ties_to_even(dev, dtype):
    """mlx's CPU quantizer takes std::rint of (w - bias) / scale: group
    [0, 15, 6.5, 4.5, ...] has scale -1 and bias 15, so 6.5 and 4.5 sit on
    ties (8.5, 10.5) and get codes 8 and 10 (half away from zero: 9, 11)."""
    w = np.zeros((1, 64), np.float32)
    w[0, 1], w[0, 2], w[0, 3] = 15.0, 6.5, 4.5
    w[0, 4:] = np.arange(60) % 16
    wq, s, b = K.quantize(to_torch(w, dev, DT[dtype]), group_size=64, bits=4)
    q = O.unpack_numpy(u32_to_numpy(wq), 4)[0]
    assert q[2] == 8 and q[3] == 10
    assert to_numpy(s)[0, 0] == -1.0 and to_numpy(b)[0, 0] == 15.0
    assert np.array_equal(u32_to_numpy(wq), O.quantize(w, 64, 4, dtype)[0])


def test_dequantize_takes_the_op_by_op_rounding_by_default(dev):
    """mx.dequantize on a CPU stream is a multiply then an add in the
    scales' dtype: s = 1 + 2^-7, q = 3, b = -3 gives bf16(bf16(3.0234375)
    - 3) = 0.03125, where one rounding of s*q + b would give 0.0234375."""
    words = torch.tensor([[3, 0, 0, 0, 0, 0, 0, 0]], dtype=torch.int32, device=dev).view(torch.uint32)
    sc = torch.tensor([[1.0078125]], dtype=torch.bfloat16, device=dev)
    bi = torch.tensor([[-3.0]], dtype=torch.bfloat16, device=dev)
    assert to_numpy(K.dequantize(words, sc, bi, 64, 4))[0, 0] == 0.03125
    assert to_numpy(K.dequantize(words, sc, bi, 64, 4, rounding=1))[0, 0] == 0.0234375


def test_quantize_edge_cases(dev):
    # constant groups, all-zero groups, ties and a 3-D tensor
    w = np.zeros((2, 3, 128), np.float32)
    w[0, 0, :64] = 0.5
    w[0, 1] = np.tile(np.arange(16, dtype=np.float32), 8)
    w[1, 2] = -np.tile(np.arange(16, dtype=np.float32), 8) / 8
    wq, s, b = K.quantize(to_torch(w, dev, torch.bfloat16), 64, 4)
    rq, rs, rb = O.quantize(w, 64, 4)
    assert np.array_equal(u32_to_numpy(wq), rq)
    assert np.array_equal(to_numpy(s), rs) and np.array_equal(to_numpy(b), rb)


@pytest.mark.parametrize("rounding", [K.ROUND_OP_BY_OP, K.ROUND_FUSED])
@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("out", ["bfloat16", "float16", "float32"])
def test_dequantize_is_bit_exact(dev, rounding, bits, out):
    rng = np.random.default_rng(200 + bits)
    w = bf16_normal(rng, (64, 512), 0.02)
    rq, rs, rb = O.quantize(w, 64, bits)
    got = K.dequantize(u32_to_torch(rq, dev), to_torch(rs, dev, torch.bfloat16),
                       to_torch(rb, dev, torch.bfloat16), 64, bits, dtype=DT[out],
                       rounding=rounding)
    ref = O.dequantize(rq, rs, rb, 64, bits, dtype=out, rounding=rounding)
    assert got.dtype == DT[out]
    assert np.array_equal(to_numpy(got), ref)


def test_dequantize_rounding_known_answer(dev):
    wq = np.array([[3] + [0] * 7], np.uint32)
    s = to_torch(np.array([[1.0078125]]), dev, torch.bfloat16)
    b = to_torch(np.array([[-0.0078125]]), dev, torch.bfloat16)
    two = K.dequantize(u32_to_torch(wq, dev), s, b, 64, 4, rounding=K.ROUND_OP_BY_OP)
    one = K.dequantize(u32_to_torch(wq, dev), s, b, 64, 4, rounding=K.ROUND_FUSED)
    assert to_numpy(two)[0, 0] == 3.03125 and to_numpy(one)[0, 0] == 3.015625


def test_round_trip_full_size(dev):
    """An 8-bit [14336, 4096] weight: quantize -> dequantize on the
    GPU equals the oracle's codes, and stays within one scale step."""
    g = torch.Generator(device=dev).manual_seed(0)
    w = (torch.randn(14336, 4096, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    wq, s, b = K.quantize(w, 64, 8)
    wd = K.dequantize(wq, s, b, 64, 8)
    err = (wd.float() - w.float()).abs().reshape(14336, 64, 64)
    step = s.float().abs()[..., None]
    # within |s|/2 + the bf16 rounding of s and of the output (see test_oracle)
    assert bool((err <= step * (1.0 + 2.0 ** -7 * 255) + 1e-9).all())
    # spot-check a slab bit for bit against the oracle
    rows = slice(7000, 7064)
    rq, rs, rb = O.quantize(to_numpy(w[rows]), 64, 8)
    assert np.array_equal(u32_to_numpy(wq[rows]), rq)
