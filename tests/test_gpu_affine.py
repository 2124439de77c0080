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
