"""GPU parity at prefill chunk sizes: SwitchGLU (and its weighted combine)
over the Qwen3.5-MoE expert shape -- 128 experts, top-8, 2048 -> 768 -> 2048
-- at T = 512 and 2048 tokens, for 4-bit affine experts and for VQ experts
with both codebooks (256 x 8 uint8, 4096 x 8 uint16).  The whole batch runs
on the GPU (every expert sees 32 or 128 rows); the oracle checks a sample of
tokens in full, since a token's output depends only on its own row and
experts.  Bar: max rel err 1e-2, cosine 0.9999."""
import numpy as np
import pytest
import torch

import oracle as O
from knurlogic_amd import nn
from tests.test_gpu_vq import _vq
from tests.util import assert_close, bf16_normal, to_numpy, to_torch, u32_to_torch

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
E, H, I, K_TOP = 128, 2048, 768, 8


def _affine_experts(rng, bits=4):
    """4-bit g64 expert triples drawn directly in the packed layout (uniform
    codes; scales and biases of the size N(0, 0.02) weights quantize to), so
    the 600 M weights need no host-side quantization: the matmuls are what
    is checked here, the quantizer has its own bit-exact tests."""
    mats = []
    for N, Kd in ((I, H), (I, H), (H, I)):
        wq = np.frombuffer(rng.bytes(E * N * Kd * bits // 8), np.uint32).reshape(E, N, Kd * bits // 32)
        sc = O.bf16_round(rng.uniform(0.004, 0.008, (E, N, Kd // 64)).astype(np.float32))
        bi = O.bf16_round((-7.5 * sc + rng.normal(0, 0.002, sc.shape)).astype(np.float32))
        mats.append((wq, sc, bi))
    return mats


def _routing(rng, T):
    inds = np.argsort(rng.random((T, E)), axis=1)[:, :K_TOP].astype(np.int32)   # k distinct experts per token
    _, sc = O.route(bf16_normal(rng, (T, E)), K_TOP)
    return inds, sc


def _sample(rng, T, n=40):
    """Tokens checked against the oracle: the first, the last, and random ones."""
    return np.unique(np.r_[0, T - 1, rng.choice(T, n, replace=False)])


@pytest.mark.parametrize("T", [512, 2048])
def test_affine_switch_glu_at_prefill_sizes(dev, T):
    rng = np.random.default_rng(9000 + T)
    mats = _affine_experts(rng)
    q = lambda m: nn.QuantizedSwitchLinear(u32_to_torch(m[0], dev), to_torch(m[1], dev, BF),
                                           to_torch(m[2], dev, BF), None, 64, 4)
    glu = nn.SwitchGLU(*(q(m) for m in mats))
    fns = [lambda xs, e, m=m: O.quantized_matmul(xs, m[0][e], m[1][e], m[2][e], True, 64, 4, "bfloat16")
           for m in mats]
    x = bf16_normal(rng, (T, H))
    inds, sc = _routing(rng, T)
    tx, ti = to_torch(x, dev, BF), torch.from_numpy(inds).to(dev)
    got = to_numpy(glu(tx, ti))
    comb = to_numpy(glu.combine(tx, ti, to_torch(sc, dev, BF)))
    assert got.shape == (T, K_TOP, H) and np.isfinite(got).all()
    s = _sample(rng, T)
    ref = O.switch_glu(x[s], inds[s], *fns)
    assert_close(got[s], ref, what=f"affine switch_glu T={T}")
    assert_close(comb[s], O.combine(ref, sc[s]), what=f"affine combine T={T}")


@pytest.mark.parametrize("kc", [256, 4096])
@pytest.mark.parametrize("T", [512, 2048])
def test_vq_switch_glu_at_prefill_sizes(dev, T, kc):
    rng = np.random.default_rng(9100 + T + kc)
    (hg, gg), (hu, gu), (hd, gd) = [_vq(rng, E, n, kd, kc, 0, dev) for n, kd in ((I, H), (I, H), (H, I))]
    # one codebook for the layer, as the VQ artifacts ship it
    hu, hd = (hu[0], hg[1], hu[2]), (hd[0], hg[1], hd[2])
    gu, gd = (gu[0], gg[1], gu[2]), (gd[0], gg[1], gd[2])
    glu = nn.VQSwitchGLU(*(nn.VQSwitchLinear(*g) for g in (gg, gu, gd)))
    x = bf16_normal(rng, (T, H))
    inds, sc = _routing(rng, T)
    tx, ti = to_torch(x, dev, BF), torch.from_numpy(inds).to(dev)
    got = to_numpy(glu(tx, ti))
    comb = to_numpy(glu.combine(tx, ti, to_torch(sc, dev, BF)))
    assert got.shape == (T, K_TOP, H) and np.isfinite(got).all()
    s = _sample(rng, T)
    fn = lambda h: (lambda xs, e: O.vq_matmul(xs, h[0][e], h[1], h[2][e], 0, "bfloat16"))
    ref = O.switch_glu(x[s], inds[s], fn(hg), fn(hu), fn(hd))
    assert_close(got[s], ref, what=f"vq switch_glu T={T} kc={kc}")
    assert_close(comb[s], O.combine(ref, sc[s]), what=f"vq combine T={T} kc={kc}")


@pytest.mark.parametrize("bits", [4, 8])
def test_grouped_gemm_with_k_tiles_past_a_group(dev, bits):
    """The grouped expert GEMM (from 64 routed rows per expert) on experts
    whose K runs 9 (gate/up, H = 576) and 5 (down, I = 320) k-tiles, which
    end part-way through the 4-deep load ring; 8 experts, top-2, 512 tokens
    (128 rows per expert)."""
    rng = np.random.default_rng(9200 + bits)
    e, h, i_, k, T = 8, 576, 320, 2, 512
    mats = []
    for N, Kd in ((i_, h), (i_, h), (h, i_)):
        wq = np.frombuffer(rng.bytes(e * N * Kd * bits // 8), np.uint32).reshape(e, N, Kd * bits // 32)
        sc = O.bf16_round(rng.uniform(0.004, 0.008, (e, N, Kd // 64)).astype(np.float32) / (1 << (bits - 4)))
        bi = O.bf16_round((-0.5 * ((1 << bits) - 1) * sc + rng.normal(0, 0.002, sc.shape)).astype(np.float32))
        mats.append((wq, sc, bi))
    q = lambda m: nn.QuantizedSwitchLinear(u32_to_torch(m[0], dev), to_torch(m[1], dev, BF),
                                           to_torch(m[2], dev, BF), None, 64, bits)
    glu = nn.SwitchGLU(*(q(m) for m in mats))
    fns = [lambda xs, ex, m=m: O.quantized_matmul(xs, m[0][ex], m[1][ex], m[2][ex], True, 64, bits, "bfloat16")
           for m in mats]
    x = bf16_normal(rng, (T, h))
    inds = np.argsort(rng.random((T, e)), axis=1)[:, :k].astype(np.int32)
    got = to_numpy(glu(to_torch(x, dev, BF), torch.from_numpy(inds).to(dev)))
    assert got.shape == (T, k, h) and np.isfinite(got).all()
    s = _sample(rng, T)
    assert_close(got[s], O.switch_glu(x[s], inds[s], *fns), what=f"grouped gemm {bits}-bit")
