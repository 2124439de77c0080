"""GPU parity: the scaled modes mxfp4 / mxfp8 (E2M1 / E4M3 elements, one
uint8 E8M0 scale per 32, no biases) -- dequantize, quantized_matmul (dense,
batched, either orientation) and gather_qmm / QuantizedSwitchLinear --
against the oracle's spec decoding, on the reference's own mxfp4 experts
(tests/golden/deepseek_v4_tiny_mxfp4_experts.npz) and on random codes.
Every mx value is exact in bf16, so dequantize is bit-exact; products meet
max rel err 1e-2, cosine 0.9999."""
from pathlib import Path

import numpy as np
import pytest
import torch

import knurlogic_amd as K
import oracle as O
from knurlogic_amd import checkpoint as C
from knurlogic_amd import nn
from tests.util import assert_close, bf16_normal, to_numpy, to_torch, u32_to_torch

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
GOLD = Path(__file__).resolve().parent / "golden"


def _fixture(dev):
    z = np.load(GOLD / "deepseek_v4_tiny_mxfp4_experts.npz")
    host = {p: (z[p + "__weight"], z[p + "__scales"]) for p in ("gate_proj", "up_proj", "down_proj")}
    gpu = {p: (u32_to_torch(w, dev), torch.from_numpy(s).to(dev)) for p, (w, s) in host.items()}
    return host, gpu


def _random_mx(rng, shape_rows, cols, mode, dev):
    bits = 4 if mode == "mxfp4" else 8
    wq = rng.integers(0, 2 ** 32, shape_rows + (cols * bits // 32,), dtype=np.uint64).astype(np.uint32)
    if mode == "mxfp8":
        b = wq.view(np.uint8)
        b[(b & 0x7F) == 0x7F] = 0x3F               # no NaN codes
    sc = rng.integers(118, 124, shape_rows + (cols // 32,)).astype(np.uint8)
    return (wq, sc), (u32_to_torch(wq, dev), torch.from_numpy(sc).to(dev))


@pytest.mark.parametrize("out", [torch.bfloat16, torch.float32])
def test_dequantize_the_references_mxfp4_experts_bit_exact(dev, out):
    host, gpu = _fixture(dev)
    for p in host:
        got = K.dequantize(*gpu[p], None, 32, 4, mode="mxfp4", dtype=out)
        assert np.array_equal(to_numpy(got), O.mx_dequantize(*host[p], "mxfp4").astype(np.float32))


def test_dequantize_mxfp8_bit_exact(dev):
    rng = np.random.default_rng(1)
    h, g = _random_mx(rng, (8, 16), 128, "mxfp8", dev)
    got = K.dequantize(*g, None, 32, 8, mode="mxfp8", dtype=torch.float32)
    assert np.array_equal(to_numpy(got), O.mx_dequantize(*h, "mxfp8").astype(np.float32))


def test_switch_layers_on_the_references_mxfp4_experts(dev):
    """QuantizedSwitchLinear(mode="mxfp4") over the fixture's experts: the
    gather of each token's routed experts, gate / up / down."""
    host, gpu = _fixture(dev)
    rng = np.random.default_rng(2)
    T, k = 5, 2
    inds = np.stack([rng.choice(4, k, replace=False) for _ in range(T)]).astype(np.int32)
    x = bf16_normal(rng, (T, 1, 1, 64))
    for p, K_in in (("gate_proj", 64), ("up_proj", 64)):
        lin = nn.QuantizedSwitchLinear(*gpu[p], None, None, 32, 4, "mxfp4")
        got = lin(to_torch(x, dev, BF), torch.from_numpy(inds).to(dev))         # [T, 1, k, 1, N]
        w, s = host[p]
        ref = np.stack([[O.mx_quantized_matmul(x[t, 0], w[e], s[e], "mxfp4", True, "float32")
                         for e in inds[t]] for t in range(T)])
        assert_close(to_numpy(got).reshape(ref.shape), ref, what=p)
    act = bf16_normal(rng, (T, k, 1, 32))
    down = nn.QuantizedSwitchLinear(*gpu["down_proj"], None, None, 32, 4, "mxfp4")
    got = down(to_torch(act, dev, BF), torch.from_numpy(inds).to(dev))
    w, s = host["down_proj"]
    ref = np.stack([[O.mx_quantized_matmul(act[t, j], w[inds[t, j]], s[inds[t, j]], "mxfp4", True, "float32")
                     for j in range(k)] for t in range(T)])
    assert_close(to_numpy(got).reshape(ref.shape), ref, what="down")


@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8"])
@pytest.mark.parametrize("transpose", [True, False])
@pytest.mark.parametrize("M", [1, 70])
def test_quantized_matmul_mx(dev, mode, transpose, M):
    rng = np.random.default_rng(M + (mode == "mxfp8"))
    K_, N = 256, 192
    h, g = _random_mx(rng, (N,) if transpose else (K_,), K_ if transpose else N, mode, dev)
    x = bf16_normal(rng, (M, K_))
    got = K.quantized_matmul(to_torch(x, dev, BF), *g[:1], g[1], None, transpose, 32, 4 if mode == "mxfp4" else 8,
                             mode)
    ref = O.mx_quantized_matmul(x, *h, mode, transpose, "float32")
    assert_close(to_numpy(got), ref, what=f"{mode} transpose={transpose} M={M}")


@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8"])
@pytest.mark.parametrize("M,K_,N", [(1, 4096, 200), (2, 512, 130), (5, 4096, 200), (9, 768, 64), (16, 4096, 72),
                                    (16, 320, 200), (17, 512, 130), (40, 256, 96), (64, 1024, 64), (3, 96, 40),
                                    (1, 14336, 200)])
def test_quantized_matmul_mx_decode_kernels(dev, mode, M, K_, N):
    """kmi_qmm_mx's decode kernels (M = 1: the streaming GEMV; 2..16 rows
    with K a multiple of 256: the direct-to-LDS kernel; other rows up to 64:
    the MFMA GEMV; K not a multiple of 64: the batched kernel) against the
    oracle, ragged N included."""
    rng = np.random.default_rng(M * 100 + K_ + N + (mode == "mxfp8"))
    h, g = _random_mx(rng, (N,), K_, mode, dev)
    x = bf16_normal(rng, (M, K_))
    got = K.quantized_matmul(to_torch(x, dev, BF), g[0], g[1], None, True, mode=mode)
    assert got.shape == (M, N)
    ref = O.mx_quantized_matmul(x, *h, mode, True, "float32")
    assert_close(to_numpy(got), ref, what=f"{mode} M={M} K={K_} N={N}")


def test_gather_with_a_bad_expert_gives_a_zero_row(dev):
    host, gpu = _fixture(dev)
    x = to_torch(bf16_normal(np.random.default_rng(3), (2, 1, 64)), dev, BF)
    rhs = torch.tensor([1, 7], dtype=torch.int32, device=dev)
    y = K.gather_qmm(x, *gpu["gate_proj"], None, rhs_indices=rhs, group_size=32, bits=4, mode="mxfp4")
    assert y.shape == (2, 1, 32) and not y[1].any() and y[0].abs().sum() > 0


def test_mx_checkpoint_layers_load_and_run(dev, tmp_path):
    """The fixture's experts written as an mlx-format file (no biases, no
    config): the loader reads them as mxfp4 off the tensors."""
    from safetensors.torch import save_file
    host, _ = _fixture("cpu")
    t = {}
    for p, (w, s) in host.items():
        t[f"switch_mlp.{p}.weight"] = torch.from_numpy(w.view(np.int32)).view(torch.uint32)
        t[f"switch_mlp.{p}.scales"] = torch.from_numpy(s)
    d = tmp_path / "art"
    d.mkdir()
    save_file(t, str(d / "model.safetensors"), metadata={"format": "mlx"})
    shapes = {"switch_mlp.gate_proj": (4, 32, 64), "switch_mlp.up_proj": (4, 32, 64),
              "switch_mlp.down_proj": (4, 64, 32)}
    mods = C.load_quantized(d, shapes=shapes, device=dev)
    g = mods["switch_mlp.gate_proj"]
    assert (g.mode, g.bits, g.group_size) == ("mxfp4", 4, 32)
    x = bf16_normal(np.random.default_rng(4), (1, 1, 64))
    got = g(to_torch(x, dev, BF), torch.tensor([2], dtype=torch.int32, device=dev))
    w, s = host["gate_proj"]
    assert_close(to_numpy(got).reshape(-1), O.mx_quantized_matmul(x[0], w[2], s[2], "mxfp4", True,
                                                                  "float32").reshape(-1), what="loaded mxfp4")


@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8"])
def test_quantize_mx_bit_exact(dev, mode):
    """mx.quantize on the GPU equals the oracle's OCP rule, code for code
    (signs of zeros included), bf16 and fp32 inputs."""
    rng = np.random.default_rng(7 if mode == "mxfp4" else 8)
    w = bf16_normal(rng, (48, 256), 0.05)
    w[0, :32] = 0.0
    w[1, :32] = -0.0
    w[2, 5] = 1e4                                    # a group 2^11 times larger than the rest
    for dt in (torch.bfloat16, torch.float32):
        wq, sc = K.quantize(to_torch(w, dev, dt), group_size=32, bits=4 if mode == "mxfp4" else 8, mode=mode)
        rq, rs = O.mx_quantize(w, mode)
        assert np.array_equal(sc.cpu().numpy(), rs)
        assert np.array_equal(wq.view(torch.int32).cpu().numpy().view(np.uint32), rq)


# One group of 32 per mode, scale byte 127 (X = 0), and the codes worked out
# by hand from the OCP rule: ties to the even code, saturation to the
# largest finite element, the sign kept on zero.
MX_HAND = {
    # E2M1 codes 0..7 = 0, .5, 1, 1.5, 2, 3, 4, 6; bit 3 is the sign
    "mxfp4": [(7.5, 7), (6.5, 7), (0.25, 0), (0.75, 2), (1.25, 2), (1.75, 4), (2.5, 4), (3.5, 6), (5.0, 6),
              (-0.25, 8), (-2.5, 12), (0.3, 1), (-0.0, 8), (0.0, 0)],
    # E4M3: 1.0 = 0x38, 1.125 = 0x39, 1.25 = 0x3A, 288 = 0x79, 320 = 0x7A, 448 = 0x7E, 2^-9 = 0x01
    "mxfp8": [(480.0, 0x7E), (460.0, 0x7E), (1.0625, 0x38), (1.1875, 0x3A), (2.0 ** -10, 0x00),
              (3 * 2.0 ** -10, 0x02), (-1.0625, 0xB8), (-0.0, 0x80), (0.0, 0x00), (300.0, 0x79),
              (304.0, 0x7A)],
}


def mx_hand_group(mode):
    vals, codes = zip(*MX_HAND[mode])
    w = np.zeros((1, 32), np.float32)
    w[0, :len(vals)] = vals
    c = np.zeros(32, np.uint32)
    c[:len(codes)] = codes
    return w, c


@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8"])
def test_quantize_mx_ties_saturation_and_signed_zeros(dev, mode):
    """Off-grid values, exact ties, values past the largest element and
    signed zeros: the GPU's codes equal the hand-computed ones (and the
    oracle's), scale byte 127."""
    w, want = mx_hand_group(mode)
    bits = 4 if mode == "mxfp4" else 8
    for dt in (torch.bfloat16, torch.float32):
        wq, sc = K.quantize(to_torch(w, dev, dt), mode=mode)
        assert sc.cpu().numpy().tolist() == [[127]]
        got = O.unpack_numpy(wq.view(torch.int32).cpu().numpy().view(np.uint32), bits)[0]
        assert got.tolist() == want.tolist()
        rq, rs = O.mx_quantize(w, mode)
        assert np.array_equal(wq.view(torch.int32).cpu().numpy().view(np.uint32), rq)


def test_quantize_mx_gives_the_references_checkpoint_back(dev):
    host, gpu = _fixture(dev)
    for p, (w, s) in host.items():
        d = to_torch(O.mx_dequantize(w, s, "mxfp4").astype(np.float32), dev, torch.float32)
        wq, sc = K.quantize(d, group_size=32, bits=4, mode="mxfp4")
        assert np.array_equal(sc.cpu().numpy(), s)
        assert np.array_equal(wq.view(torch.int32).cpu().numpy().view(np.uint32), w)


@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8"])
@pytest.mark.parametrize("T,k,E", [(1, 8, 16), (2, 8, 16), (3, 4, 16), (16, 8, 16), (70, 4, 16), (16, 8, 128)])
def test_switch_glu_mx_matches_the_oracle(dev, mode, T, k, E):
    """SwitchGLU over mxfp4 / mxfp8 experts in one call (gate and up
    stacked): up to 64 (token, slot) pairs token-major, more grouped by
    expert (4-row expert tiles at 128 experts); against the oracle's
    SwitchGLU over its mx matmul, and the combine against moe_combine of the
    same y, bit for bit."""
    rng = np.random.default_rng(T * 10 + k + (mode == "mxfp8") + E)
    H, I = 256, 128
    bits = 4 if mode == "mxfp4" else 8
    (hg, gg), (hu, gu), (hd, gd) = [_random_mx(rng, (E, n), kd, mode, dev) for n, kd in ((I, H), (I, H), (H, I))]
    lin = lambda g: nn.QuantizedSwitchLinear(g[0], g[1], None, None, 32, bits, mode)
    glu = nn.SwitchGLU(lin(gg), lin(gu), lin(gd))
    x = bf16_normal(rng, (T, H))
    inds = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    fn = lambda h: (lambda xs, e: O.mx_quantized_matmul(xs, h[0][e], h[1][e], mode, True, "bfloat16"))
    ref = O.switch_glu(x, inds, fn(hg), fn(hu), fn(hd))
    tx, ti = to_torch(x, dev, BF), torch.from_numpy(inds).to(dev)
    got = glu(tx, ti)
    assert got.shape == (T, k, H)
    assert_close(to_numpy(got), ref, what=f"{mode} switch_glu T={T} k={k}")
    _, sc = O.route(bf16_normal(rng, (T, E)), k)
    comb = glu.combine(tx, ti, to_torch(sc, dev, BF))
    assert_close(to_numpy(comb), O.combine(ref, sc), what="combine")
    assert torch.equal(comb, K.moe_combine(got, to_torch(sc, dev, BF)))


def test_switch_glu_mx_refuses_what_it_must(dev):
    rng = np.random.default_rng(9)
    (hg, gg), (hd, gd) = _random_mx(rng, (4, 128), 64, "mxfp4", dev), _random_mx(rng, (4, 64), 64, "mxfp4", dev)
    x = to_torch(bf16_normal(rng, (3, 64)), dev, BF)
    inds = torch.zeros(3, 8, dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        K.switch_glu_mx(x, inds, gg[0], gg[1], gd[0], gd[1], mode="nvfp4")
    with pytest.raises(ValueError):      # scales must be E8M0 bytes
        K.switch_glu_mx(x, inds, gg[0], gg[1].to(torch.bfloat16), gd[0], gd[1], mode="mxfp4")
