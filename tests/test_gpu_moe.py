"""GPU parity: the MoE row -- router, SwiGLU, combine, shared-expert gate
(bit-exact against the oracle's restatement of qwen3_5.py:35-40,108-112,
170-192), and SwitchGLU / SparseMoeBlock over 4-bit experts (the matmul bar:
max rel err 1e-2, cosine 0.9999), up to the Qwen3.5-MoE expert shapes
(128 experts, 2048 -> 768 -> 2048, top-8)."""
import numpy as np
import pytest
import torch

import knurlogic_amd as K
import oracle as O
from knurlogic_amd import nn
from tests.util import assert_close, bf16_normal, to_numpy, to_torch, u32_to_torch

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
DT = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _bits_equal(got, ref):
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    bad = np.nonzero(got.view(np.uint32) != ref.view(np.uint32))
    assert bad[0].size == 0, f"{bad[0].size} of {got.size} differ; first at {tuple(b[0] for b in bad)}: " \
                             f"{got[tuple(b[0] for b in bad)]} vs {ref[tuple(b[0] for b in bad)]}"


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("T,E,k", [(1, 128, 8), (16, 128, 8), (256, 128, 8), (7, 64, 4), (5, 1000, 16),
                                   (3, 8, 8)])
def test_route_matches_the_oracle_bit_for_bit(dev, dtype, T, E, k):
    rng = np.random.default_rng(T + E + k)
    logits = O.round_to(rng.standard_normal((T, E)).astype(np.float32), dtype)
    inds, scores = K.moe_route(to_torch(logits, dev, DT[dtype]), k)
    ri, rs = O.route(logits, k, dtype)
    assert inds.dtype == torch.int32 and inds.shape == (T, k)
    np.testing.assert_array_equal(inds.cpu().numpy(), ri)
    _bits_equal(to_numpy(scores), rs)


@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
@pytest.mark.parametrize("E,k", [(128, 8), (256, 8), (200, 8), (65, 1), (8, 8), (300, 8), (128, 9)])
def test_route_many_tokens_matches_the_oracle(dev, dtype, E, k):
    """4096 tokens, experts from 8 to 300 (a partly filled last wave of 64,
    two experts per thread past 256) and k up to 9: the router gives the
    oracle's experts and scores bit for bit."""
    rng = np.random.default_rng(E * 10 + k)
    logits = O.round_to((rng.standard_normal((4096, E)) * 2).astype(np.float32), dtype)
    inds, scores = K.moe_route(to_torch(logits, dev, DT[dtype]), k)
    ri, rs = O.route(logits, k, dtype)
    np.testing.assert_array_equal(inds.cpu().numpy(), ri)
    _bits_equal(to_numpy(scores), rs)


def test_route_ties_go_to_the_lower_expert(dev):
    """Logits on a coarse grid: many exact ties inside and at the top-k edge."""
    rng = np.random.default_rng(5)
    logits = (rng.integers(0, 4, (64, 128)) * 0.5).astype(np.float32)
    inds, scores = K.moe_route(to_torch(logits, dev, BF), 8)
    ri, rs = O.route(logits, 8, "bfloat16")
    np.testing.assert_array_equal(inds.cpu().numpy(), ri)
    _bits_equal(to_numpy(scores), rs)


def test_route_orders_a_one_ulp_near_tie_like_the_oracle(dev):
    """Probabilities one float32 ulp apart (logits 1, 0, 2^-23, -8): the
    router kernel takes expert 2 ahead of expert 1, as the oracle does."""
    lg = np.tile(np.array([[1.0, 0.0, 2.0 ** -23, -8.0]], np.float32), (3, 1))
    inds, scores = K.moe_route(to_torch(lg, dev, BF), 2)
    ri, rs = O.route(lg, 2, "bfloat16")
    assert (ri[:, :2] == [0, 2]).all()
    np.testing.assert_array_equal(inds.cpu().numpy(), ri)
    _bits_equal(to_numpy(scores), rs)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
def test_swiglu_bit_for_bit(dev, dtype):
    rng = np.random.default_rng(1)
    g = O.round_to((rng.standard_normal((37, 300)) * 4).astype(np.float32), dtype)
    u = O.round_to(rng.standard_normal((37, 300)).astype(np.float32), dtype)
    ref = O.swiglu(u, g, dtype)
    got = K.swiglu(to_torch(g, dev, DT[dtype]), to_torch(u, dev, DT[dtype]))
    _bits_equal(to_numpy(got), ref)
    # the stacked [gate | up] form
    gu = to_torch(np.concatenate([g, u], axis=-1), dev, DT[dtype])
    _bits_equal(to_numpy(K.swiglu(gu)), ref)


def test_swiglu_every_bf16_gate(dev):
    """silu on every finite bf16 gate value (65280 patterns), bit for bit
    with the oracle's float64 evaluation, with up = 1 and with random up:
    the bf16 SwiGLU runs the float32 arithmetic every expert kernel's
    epilogue shares (a float64 fallback only near bf16 rounding midpoints
    and past |gate| = 64), so this covers their activation on all inputs."""
    bits = np.arange(1 << 16, dtype=np.uint32)
    g = (bits[((bits >> 7) & 0xFF) != 0xFF] << 16).view(np.float32).reshape(1, -1)
    rng = np.random.default_rng(4)
    for u in (np.ones_like(g), O.round_to(rng.standard_normal(g.shape).astype(np.float32), "bfloat16")):
        with np.errstate(over="ignore"):
            ref = O.swiglu(u, g, "bfloat16")
        got = K.swiglu(to_torch(g, dev, BF), to_torch(u, dev, BF))
        _bits_equal(to_numpy(got), ref)


@pytest.mark.parametrize("T,H", [(19, 200), (19, 203), (70000, 16), (600, 2048)])
@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
def test_combine_bit_for_bit(dev, dtype, T, H):
    """From 2^20 outputs with H % 8 == 0 the bf16 combine takes the
    8-column kernel (with more tokens than one grid dimension holds at
    T = 70000); below that, or at H = 203, the per-element one."""
    rng = np.random.default_rng(2)
    y = O.round_to(rng.standard_normal((T, 8, H)).astype(np.float32), dtype)
    _, sc = O.route(O.round_to(rng.standard_normal((T, 32)).astype(np.float32), dtype), 8, dtype)
    got = K.moe_combine(to_torch(y, dev, DT[dtype]), to_torch(sc, dev, DT[dtype]))
    _bits_equal(to_numpy(got), O.combine(y, sc, dtype))


def test_shared_add_bit_for_bit(dev):
    rng = np.random.default_rng(3)
    y = bf16_normal(rng, (9, 160))
    sy = bf16_normal(rng, (9, 160))
    g = bf16_normal(rng, (9, 1), 2.0)
    ref = O.round_to(y + O.round_to(O.sigmoid_rounded(g) * sy, "bfloat16"), "bfloat16")
    got = K.moe_shared_add(to_torch(y, dev, BF), to_torch(g, dev, BF), to_torch(sy, dev, BF))
    _bits_equal(to_numpy(got), ref)


def _experts(rng, E, H, I, dev, bits=4):
    """Expert weights N(0, 0.02) quantized (4-bit g64): oracle triples and the
    SwitchGLU module."""
    mats = {}
    for name, shape in (("gate", (E, I, H)), ("up", (E, I, H)), ("down", (E, H, I))):
        w = bf16_normal(rng, shape, 0.02)
        mats[name] = O.quantize(w, 64, bits)
    q = lambda t: nn.QuantizedSwitchLinear(u32_to_torch(t[0], dev), to_torch(t[1], dev, BF),
                                           to_torch(t[2], dev, BF), None, 64, bits)
    glu = nn.SwitchGLU(q(mats["gate"]), q(mats["up"]), q(mats["down"]))
    fn = lambda m: (lambda xs, e: O.quantized_matmul(xs, m[0][e], m[1][e], m[2][e], True, 64, bits,
                                                     "bfloat16"))
    return glu, (fn(mats["gate"]), fn(mats["up"]), fn(mats["down"]))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("T,E,H,I,k", [(1, 16, 256, 128, 4), (5, 16, 256, 128, 4), (64, 16, 256, 128, 4),
                                       (100, 16, 256, 128, 4), (1, 128, 2048, 768, 8),
                                       (8, 128, 2048, 768, 8), (9, 128, 2048, 768, 8),
                                       (16, 128, 2048, 768, 8), (40, 128, 2048, 768, 8),
                                       (256, 128, 2048, 768, 8), (256, 4, 512, 320, 2),
                                       (600, 4, 256, 192, 2), (150, 8, 1024, 128, 4)])
def test_switch_glu_matches_the_oracle(dev, T, E, H, I, k, bits):
    """One library call (token-major up to 64 (token, slot) pairs, grouped by
    expert above: skinny expert tiles, or the grouped GEMM from 64 rows per
    expert -- 128-row tiles, 256-row tiles with an expert over two, column
    tiles past N), the separate gather_qmm path, and the fused combine."""
    rng = np.random.default_rng(T * 7 + E + bits)
    glu, fns = _experts(rng, E, H, I, dev, bits)
    assert glu.fused is not None
    x = bf16_normal(rng, (T, H))
    inds = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    tx, ti = to_torch(x, dev, BF), torch.from_numpy(inds).to(dev)
    got = glu(tx, ti)
    assert got.shape == (T, k, H)
    ref = O.switch_glu(x, inds, *fns)
    assert_close(to_numpy(got), ref, what="switch_glu")
    assert_close(to_numpy(glu.gathered(tx, ti)), ref, what="gathered")
    _, sc = O.route(bf16_normal(rng, (T, E)), k)
    comb = glu.combine(tx, ti, to_torch(sc, dev, BF))
    assert comb.shape == (T, H)
    assert_close(to_numpy(comb), O.combine(ref, sc), what="combine")


@pytest.mark.parametrize("T", [16, 40, 256])
def test_switch_glu_repeats_and_ignores_row_positions(dev, T):
    """Grouped SwitchGLU (4-, 16- and 32-row expert tiles): the same call
    gives the same bits, and permuting the tokens -- which moves rows to other
    positions inside their expert tiles -- permutes the output bit for bit
    (no row's result depends on where the sort put it)."""
    rng = np.random.default_rng(600 + T)
    E, H, I, k = 128, 2048, 768, 8
    glu, _ = _experts(rng, E, H, I, dev)
    x = bf16_normal(rng, (T, H))
    inds = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    tx, ti = to_torch(x, dev, BF), torch.from_numpy(inds).to(dev)
    ys = [glu(tx, ti) for _ in range(3)]
    for y in ys[1:]:
        assert torch.equal(y, ys[0])
    perm = torch.from_numpy(rng.permutation(T)).to(dev)
    yp = glu(tx[perm].contiguous(), ti[perm].contiguous())
    assert torch.equal(yp, ys[0][perm])


def test_switch_glu_unstacked_gate_and_up_agree(dev):
    """Without the stacked weight (gate and up that cannot be stacked):
    separate gate and up gather_qmm calls, the same SwiGLU and result."""
    rng = np.random.default_rng(11)
    E, H, I, T, k = 8, 128, 64, 6, 2
    glu, fns = _experts(rng, E, H, I, dev)
    x = bf16_normal(rng, (T, H))
    inds = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    ref = O.switch_glu(x, inds, *fns)
    tx, ti = to_torch(x, dev, BF), torch.from_numpy(inds).to(dev)
    assert_close(to_numpy(glu(tx, ti)), ref, what="stacked")
    glu.fused = None
    assert_close(to_numpy(glu(tx, ti)), ref, what="separate")


@pytest.mark.parametrize("T", [1, 16, 256])
def test_sparse_moe_block_matches_the_oracle(dev, T):
    """Router from given logits, SwitchGLU, combine and the sigmoid-gated
    quantized shared expert, at the Qwen3.5-MoE shapes."""
    rng = np.random.default_rng(40 + T)
    E, H, I, k, Is = 128, 2048, 768, 8, 512
    glu, fns = _experts(rng, E, H, I, dev)
    sw = {n: bf16_normal(rng, s, 0.02) for n, s in (("g", (Is, H)), ("u", (Is, H)), ("d", (H, Is)),
                                                    ("sg", (1, H)))}
    sq = {n: O.quantize(w, 64, 4) for n, w in sw.items()}
    ql = lambda t: nn.QuantizedLinear(u32_to_torch(t[0], dev), to_torch(t[1], dev, BF),
                                      to_torch(t[2], dev, BF), None, 64, 4)
    shared = nn.MLP(ql(sq["g"]), ql(sq["u"]), ql(sq["d"]))
    x = bf16_normal(rng, (T, H))
    logits = bf16_normal(rng, (T, E))
    tl = to_torch(logits, dev, BF)
    block = nn.SparseMoeBlock(lambda _x: tl, glu, k, shared, ql(sq["sg"]))
    got = block(to_torch(x, dev, BF))
    deq = {n: O.dequantize(*t, 64, 4, "float32") for n, t in sq.items()}
    # the oracle block with these logits: route + SwitchGLU + combine + shared
    inds, scores = O.route(logits, k)
    y = O.combine(O.switch_glu(x, inds, *fns), scores)
    a = O.swiglu(O.dense_linear(x, deq["u"]), O.dense_linear(x, deq["g"]))
    sy = O.dense_linear(a, deq["d"])
    ref = O.round_to(y + O.round_to(O.sigmoid_rounded(O.dense_linear(x, deq["sg"])) * sy, "bfloat16"),
                     "bfloat16")
    assert_close(to_numpy(got), ref, what="moe block")
    # the routed part alone, from the same logits
    assert_close(to_numpy(block.experts(to_torch(x, dev, BF), tl)), y, what="experts")


@pytest.mark.parametrize("T", [1, 2, 5, 8, 9, 16, 64, 65])
def test_moe_experts_routes_in_the_kernel_like_the_router(dev, T):
    """kmi_moe_experts (one call from the router logits): at decode sizes
    the gate/up kernel routes each token itself.  The experts and scores
    equal kmi_moe_route's bit for bit, the output equals route + SwitchGLU
    bit for bit, and both match the oracle (the matmul bar)."""
    rng = np.random.default_rng(300 + T)
    E, H, I, k = 128, 2048, 768, 8
    glu, fns = _experts(rng, E, H, I, dev)
    x = bf16_normal(rng, (T, H))
    logits = bf16_normal(rng, (T, E))
    tx, tl = to_torch(x, dev, BF), to_torch(logits, dev, BF)
    f, d = glu.fused, glu.down_proj
    out, inds, scores = K.moe_experts(tx, tl, k, f.weight, f.scales, f.biases, d.weight, d.scales, d.biases)
    ri, rs = K.moe_route(tl, k)
    assert torch.equal(inds, ri) and torch.equal(scores, rs)
    oi, os_ = O.route(logits, k)
    np.testing.assert_array_equal(inds.cpu().numpy(), oi)
    _bits_equal(to_numpy(scores), os_)
    assert torch.equal(out, glu.combine(tx, ri, rs))
    ref = O.combine(O.switch_glu(x, oi, *fns), os_)
    assert_close(to_numpy(out), ref, what=f"moe_experts T={T}")
    # and the block's routed part takes this call
    block = nn.SparseMoeBlock(None, glu, k)
    assert torch.equal(block.experts(tx, tl), out)



@pytest.mark.parametrize("T,E,H,I,pattern", [(16, 128, 2048, 768, "same"), (16, 128, 2048, 768, "half"),
                                              (32, 128, 2048, 768, "random"), (12, 256, 512, 256, "same")])
def test_moe_experts_tiles_formed_in_the_kernel(dev, T, E, H, I, pattern):
    """From the router logits, at up to 256 (token, slot) pairs over up to
    256 experts, the expert kernels form their 4-row tiles themselves (no
    sort launch).  With skewed routing -- every token, or half of them, on
    the same 8 experts, so one expert spans several tiles -- the output
    equals route + SwitchGLU (the sort's tiles) bit for bit and matches the
    oracle."""
    rng = np.random.default_rng(500 + T + E)
    k = 8
    glu, fns = _experts(rng, E, H, I, dev)
    x = bf16_normal(rng, (T, H))
    logits = bf16_normal(rng, (T, E))
    if pattern == "same":
        logits[:] = logits[0]
    elif pattern == "half":
        logits[: T // 2] = logits[0]
    tx, tl = to_torch(x, dev, BF), to_torch(logits, dev, BF)
    f, d = glu.fused, glu.down_proj
    out, inds, scores = K.moe_experts(tx, tl, k, f.weight, f.scales, f.biases, d.weight, d.scales, d.biases)
    ri, rs = K.moe_route(tl, k)
    assert torch.equal(inds, ri) and torch.equal(scores, rs)
    assert torch.equal(out, glu.combine(tx, ri, rs)), "formed tiles and the sort's tiles differ"
    oi, os_ = O.route(logits, k)
    np.testing.assert_array_equal(inds.cpu().numpy(), oi)
    if pattern == "same":
        assert len(set(oi.reshape(-1).tolist())) == k
    ref = O.combine(O.switch_glu(x, oi, *fns), os_)
    assert_close(to_numpy(out), ref, what=f"moe_experts T={T} {pattern}")
    again, _, _ = K.moe_experts(tx, tl, k, f.weight, f.scales, f.biases, d.weight, d.scales, d.biases)
    assert torch.equal(again, out)
