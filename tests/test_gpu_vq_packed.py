"""GPU parity: VQ experts in the artifacts' bit-packed on-disk layout
(kmi_vq_packed_gather_qmm / kmi_vq_packed_glu: 8-12 and 16-bit fields,
2-8-element vectors, per-group fp16 scales) against the oracle's unpack
then exact decode-then-matmul; and modules read from a written safetensors
artifact (knurlogic_amd.checkpoint) against the oracle.  Bar: max rel err
1e-2, cosine 0.9999."""
import json

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


def _packed(rng, E, N, IN, dim, kc, bits, group, dev):
    nsub = IN // dim
    codes = rng.integers(0, kc, (E, N, nsub))
    words = np.zeros((E, N, (nsub + 31) // 32 * bits), np.uint32)
    flat = C._repack(torch.from_numpy(codes), bits).view(torch.int32).numpy().view(np.uint32)
    words[...] = flat
    cb = (rng.standard_normal((kc, dim)) * 0.3).astype(np.float16)
    sc = rng.uniform(0.5, 1.5, (E, N, IN // group)).astype(np.float16)
    host = (words, cb.astype(np.float32), sc.astype(np.float32))
    gpu = (u32_to_torch(words, dev), torch.from_numpy(cb).to(dev), torch.from_numpy(sc).to(dev))
    return host, gpu


CASES = [  # (bits, kc, dim, group, IN)
    (11, 2048, 4, 64, 2048),
    (11, 2048, 2, 64, 768),
    (11, 2048, 4, 32, 96),       # a partial last block (24 fields)
    (8, 256, 4, 64, 512),
    (12, 4096, 2, 128, 1024),
    (16, 5000, 8, 64, 256),
    (9, 300, 4, 32, 128),
    (10, 1024, 8, 128, 384),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_packed_gather_matches_the_oracle(dev, case):
    bits, kc, dim, group, IN = CASES[case]
    rng = np.random.default_rng(case)
    E, N, P = 4, 96, 5
    host, gpu = _packed(rng, E, N, IN, dim, kc, bits, group, dev)
    x = bf16_normal(rng, (P, 2, IN))
    rhs = rng.integers(0, E, P).astype(np.int32)
    got = K.ops.vq_packed_gather_qmm(to_torch(x, dev, BF), *gpu, bits, group,
                                     rhs_indices=torch.from_numpy(rhs).to(dev))
    ref = np.stack([O.vq_packed_matmul(x[p], host[0][rhs[p]], host[1], host[2][rhs[p]], bits, group,
                                       "float32") for p in range(P)])
    assert got.shape == (P, 2, N)
    assert_close(to_numpy(got), ref, what=f"packed case {case}")


@pytest.mark.parametrize("T,E,H,I,k", [(1, 16, 512, 256, 4), (3, 32, 2048, 768, 8), (16, 32, 2048, 768, 8),
                                       (40, 16, 512, 256, 4)])
def test_packed_switch_glu_matches_the_oracle(dev, T, E, H, I, k):
    """One library call: up to 16 pairs per pair, more grouped by expert on
    the MFMA kernel (8- and 16-row tiles, experts over several tiles); the
    separate ops agree."""
    rng = np.random.default_rng(T + E)
    bits, kc, dim, group = 11, 2048, 4, 64
    (hg, gg), (hu, gu), (hd, gd) = [_packed(rng, E, n, kd, dim, kc, bits, group, dev)
                                    for n, kd in ((I, H), (I, H), (H, I))]
    mods = [nn.VQSwitchLinear(*g, scale_group=group, pack_bits=bits) for g in (gg, gu, gd)]
    glu = nn.VQSwitchGLU(*mods)
    x = bf16_normal(rng, (T, H))
    inds = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    fn = lambda h: (lambda xs, e: O.vq_packed_matmul(xs, h[0][e], h[1], h[2][e], bits, group, "bfloat16"))
    ref = O.switch_glu(x, inds, fn(hg), fn(hu), fn(hd))
    tx, ti = to_torch(x, dev, BF), torch.from_numpy(inds).to(dev)
    got = glu(tx, ti)
    assert got.shape == (T, k, H)
    assert_close(to_numpy(got), ref, what="packed vq switch_glu")
    assert_close(to_numpy(glu._packed_call(tx, ti)), ref, what="packed vq switch_glu (separate ops)")
    _, sc = O.route(bf16_normal(rng, (T, E)), k)
    comb = glu.combine(tx, ti, to_torch(sc, dev, BF))
    assert_close(to_numpy(comb), O.combine(ref, sc), what="packed combine")
    # one module's own call
    y = mods[2](to_torch(ref.reshape(T * k, 1, H)[:, :, :I] * 0 + bf16_normal(rng, (T * k, 1, I)), dev, BF),
                torch.from_numpy(inds.reshape(-1)).to(dev))
    assert y.shape == (T * k, 1, H)


GROUPED = [  # (bits, kc, dim, group, H, I): shapes of the expert-tile kernel
    (11, 2048, 4, 64, 512, 256),
    (11, 2048, 2, 64, 512, 192),
    (12, 4096, 2, 32, 256, 128),
    (8, 256, 4, 128, 512, 256),
    (16, 5000, 8, 64, 512, 256),
    (9, 300, 8, 32, 256, 512),
    (10, 1024, 4, 32, 384, 128),
]


@pytest.mark.parametrize("case", range(len(GROUPED)))
def test_packed_switch_glu_grouped_shapes(dev, case):
    """The expert-tile MFMA kernel across field widths, vector lengths and
    scale groups (20 tokens x top-4 over 8 experts: tiles of 16 rows, most
    experts over two tiles), SwitchGLU and combine against the oracle."""
    bits, kc, dim, group, H, I = GROUPED[case]
    rng = np.random.default_rng(100 + case)
    T, E, k = 20, 8, 4
    (hg, gg), (hu, gu), (hd, gd) = [_packed(rng, E, n, kd, dim, kc, bits, group, dev)
                                    for n, kd in ((I, H), (I, H), (H, I))]
    glu = nn.VQSwitchGLU(*(nn.VQSwitchLinear(*g, scale_group=group, pack_bits=bits) for g in (gg, gu, gd)))
    x = bf16_normal(rng, (T, H))
    inds = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    fn = lambda h: (lambda xs, e: O.vq_packed_matmul(xs, h[0][e], h[1], h[2][e], bits, group, "bfloat16"))
    ref = O.switch_glu(x, inds, fn(hg), fn(hu), fn(hd))
    tx, ti = to_torch(x, dev, BF), torch.from_numpy(inds).to(dev)
    assert_close(to_numpy(glu(tx, ti)), ref, what=f"grouped packed case {case}")
    _, sc = O.route(bf16_normal(rng, (T, E)), k)
    comb = glu.combine(tx, ti, to_torch(sc, dev, BF))
    assert_close(to_numpy(comb), O.combine(ref, sc), what=f"grouped packed combine {case}")


def test_packed_switch_glu_repeats_and_ignores_row_positions(dev):
    """Grouped packed SwitchGLU: the same call gives the same bits, and
    permuting the tokens (rows move inside their expert tiles) permutes the
    output bit for bit."""
    rng = np.random.default_rng(77)
    T, E, H, I, k, bits, kc, dim, group = 24, 32, 2048, 768, 8, 11, 2048, 4, 64
    mods = [nn.VQSwitchLinear(*_packed(rng, E, n, kd, dim, kc, bits, group, dev)[1], scale_group=group,
                              pack_bits=bits) for n, kd in ((I, H), (I, H), (H, I))]
    glu = nn.VQSwitchGLU(*mods)
    tx = to_torch(bf16_normal(rng, (T, H)), dev, BF)
    ti = torch.from_numpy(np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)).to(dev)
    ys = [glu(tx, ti) for _ in range(3)]
    for y in ys[1:]:
        assert torch.equal(y, ys[0])
    perm = torch.from_numpy(rng.permutation(T)).to(dev)
    assert torch.equal(glu(tx[perm].contiguous(), ti[perm].contiguous()), ys[0][perm])


@pytest.mark.parametrize("T", [1, 4, 16])
def test_packed_switch_glu_at_the_shipped_artifact_shape(dev, T):
    """The expert layout the reference's Gemma-4 26B VQ artifact declares
    (tests/support/artifacts/gemma-4-26b-a4b-it-VQ-6.2bpw/config.json,
    vq_modules: 128 experts, gate/up 2816 -> 704, down 704 -> 2816, a
    2048 x 2 codebook, 11-bit fields, scales per 64 inputs), top-8, full
    size: random 11-bit fields (every value is a codebook entry), SwitchGLU
    and its weighted combine against the oracle on the routed experts."""
    E, H, I, k, dim, kc, bits, group = 128, 2816, 704, 8, 2, 2048, 11, 64
    rng = np.random.default_rng(20 + T)
    g = torch.Generator(device=dev).manual_seed(20 + T)
    cb = (rng.standard_normal((kc, dim)) * 0.3).astype(np.float16)
    tcb = torch.from_numpy(cb).to(dev)

    def mat(N, IN):
        W = (IN // dim + 31) // 32 * bits
        words = torch.randint(-2 ** 31, 2 ** 31 - 1, (E, N, W), device=dev, generator=g,
                              dtype=torch.int32).view(torch.uint32)
        sc = (torch.rand(E, N, IN // group, device=dev, generator=g) + 0.5).to(torch.float16)
        return words, sc

    mats = [mat(I, H), mat(I, H), mat(H, I)]
    mods = [nn.VQSwitchLinear(w, tcb, sc, scale_group=group, pack_bits=bits, in_features=IN)
            for (w, sc), IN in zip(mats, (H, H, I))]
    glu = nn.VQSwitchGLU(*mods)
    x = bf16_normal(rng, (T, H))
    inds = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    used = sorted(set(inds.reshape(-1).tolist()))
    host = [{e: (w[e].view(torch.int32).cpu().numpy().view(np.uint32), sc[e].float().cpu().numpy())
             for e in used} for w, sc in mats]
    cbf = cb.astype(np.float32)
    fn = lambda h: (lambda xs, e: O.vq_packed_matmul(xs, h[e][0], cbf, h[e][1], bits, group, "bfloat16"))
    ref = O.switch_glu(x, inds, *(fn(h) for h in host))
    tx, ti = to_torch(x, dev, BF), torch.from_numpy(inds).to(dev)
    got = glu(tx, ti)
    assert got.shape == (T, k, H)
    assert_close(to_numpy(got), ref, what=f"artifact-shape packed vq switch_glu T={T}")
    _, scores = O.route(bf16_normal(rng, (T, E)), k)
    comb = glu.combine(tx, ti, to_torch(scores, dev, BF))
    assert_close(to_numpy(comb), O.combine(ref, scores), what="artifact-shape packed combine")


def test_packed_errors(dev):
    rng = np.random.default_rng(9)
    _, gpu = _packed(rng, 2, 8, 128, 4, 2048, 11, 64, dev)
    x = torch.zeros(1, 1, 128, dtype=BF, device=dev)
    with pytest.raises(ValueError):
        K.ops.vq_packed_gather_qmm(x, *gpu, 12, 64)                 # width is not 12-bit
    with pytest.raises(ValueError):
        K.ops.vq_packed_gather_qmm(x[..., :64].contiguous(), *gpu, 11, 64)   # K mismatch


def test_a_written_artifact_loads_and_matches_the_oracle(dev, tmp_path):
    """mlx-format affine layers and packed VQ experts written to a
    safetensors file, read back by checkpoint.load_quantized, computed on
    the GPU."""
    from safetensors.torch import save_file
    rng = np.random.default_rng(11)
    w = bf16_normal(rng, (256, 512), 0.02)
    wq, s, b = O.quantize(w, 64, 4)
    E, OUT, IN, dim, kc, bits, group = 4, 64, 256, 4, 2048, 11, 64
    host, _ = _packed(rng, E, OUT, IN, dim, kc, bits, group, "cpu")
    t = {"lin.weight": torch.from_numpy(wq.view(np.int32)).view(torch.uint32),
         "lin.scales": torch.from_numpy(s).to(BF), "lin.biases": torch.from_numpy(b).to(BF),
         "vq.codes": torch.from_numpy(host[0].view(np.int32)).view(torch.uint32),
         "vq.codebook": torch.from_numpy(host[1]).half(), "vq.vq_scales": torch.from_numpy(host[2]).half()}
    d = tmp_path / "art"
    d.mkdir()
    save_file(t, str(d / "model.safetensors"), metadata={"format": "mlx", "vq_modules": json.dumps(
        {"vq": {"experts": E, "out": OUT, "in": IN, "dim": dim, "k": kc, "group": group, "pack_bits": bits}})})
    (d / "config.json").write_text(json.dumps({"quantization": {"group_size": 64, "bits": 4}}))
    mods = C.load_quantized(d, device=dev)
    x = bf16_normal(rng, (3, 512))
    got = mods["lin"](to_torch(x, dev, BF))
    assert_close(to_numpy(got), O.quantized_matmul(x, wq, s, b, True, 64, 4, "float32"), what="loaded linear")
    xv = bf16_normal(rng, (2, 1, IN))
    rhs = np.array([3, 1], np.int32)
    gv = mods["vq"](to_torch(xv, dev, BF), torch.from_numpy(rhs).to(dev))
    ref = np.stack([O.vq_packed_matmul(xv[p], host[0][rhs[p]], host[1], host[2][rhs[p]], bits, group, "float32")
                    for p in range(2)])
    assert_close(to_numpy(gv), ref, what="loaded vq")


@pytest.mark.parametrize("T,E,H,I,dim,pattern", [(1, 128, 2048, 768, 4, "random"), (1, 128, 2816, 704, 2, "random"),
                                                 (2, 128, 2048, 768, 4, "random"), (1, 300, 512, 256, 4, "random"),
                                                 (3, 128, 2048, 768, 4, "random"), (16, 128, 2048, 768, 4, "same"),
                                                 (16, 128, 2048, 768, 4, "half")])
def test_packed_experts_from_logits(dev, T, E, H, I, dim, pattern):
    """vq_packed_experts (route, packed SwitchGLU, combine in one call; up to
    16 pairs with E <= 256 the gate/up kernel routes each pair's token;
    beyond, at up to 256 pairs over up to 256 experts, the expert-tile
    kernels form their tiles themselves, without the sort) gives moe_route's
    routing and the bits of the separate route, SwitchGLU and moe_combine
    calls, and matches the oracle's routed SwitchGLU and combine.  Random
    11-bit words (every field a codebook entry); skewed routing (every
    token, or half of them, on the same 8 experts) puts an expert's rows in
    several tiles."""
    k, kc, bits, group = 8, 2048, 11, 64
    rng = np.random.default_rng(40 + 7 * T + E + dim)
    g = torch.Generator(device=dev).manual_seed(40 + T + E)
    cb = (rng.standard_normal((kc, dim)) * 0.3).astype(np.float16)
    tcb = torch.from_numpy(cb).to(dev)

    def mat(N, IN):
        W = (IN // dim + 31) // 32 * bits
        words = torch.randint(-2 ** 31, 2 ** 31 - 1, (E, N, W), device=dev, generator=g,
                              dtype=torch.int32).view(torch.uint32)
        sc = (torch.rand(E, N, IN // group, device=dev, generator=g) + 0.5).to(torch.float16)
        return words, sc

    mats = [mat(I, H), mat(I, H), mat(H, I)]
    mods = [nn.VQSwitchLinear(w, tcb, sc, scale_group=group, pack_bits=bits, in_features=IN)
            for (w, sc), IN in zip(mats, (H, H, I))]
    glu = nn.VQSwitchGLU(*mods)
    x, lg = bf16_normal(rng, (T, H)), bf16_normal(rng, (T, E))
    if pattern == "same":
        lg[:] = lg[0]
    elif pattern == "half":
        lg[: T // 2] = lg[0]
    tx, tl = to_torch(x, dev, BF), to_torch(lg, dev, BF)
    out, inds, scores = glu.experts(tx, tl, k)
    ri, rs = K.moe_route(tl, k)
    assert torch.equal(inds, ri) and torch.equal(scores, rs), "routing differs from moe_route"
    y = glu(tx, ri)
    assert torch.equal(out, glu.combine(tx, ri, rs)), "one call and route + combine differ"
    assert torch.equal(out, K.moe_combine(y, rs)), "the down kernel's combine differs from moe_combine"
    oi, osc = O.route(lg, k)
    assert np.array_equal(to_numpy(inds), oi)
    used = sorted(set(oi.reshape(-1).tolist()))
    host = [{e: (w[e].view(torch.int32).cpu().numpy().view(np.uint32), sc[e].float().cpu().numpy())
             for e in used} for w, sc in mats]
    cbf = cb.astype(np.float32)
    fn = lambda h: (lambda xs, e: O.vq_packed_matmul(xs, h[e][0], cbf, h[e][1], bits, group, "bfloat16"))
    ref = O.switch_glu(x, oi, *(fn(h) for h in host))
    assert_close(to_numpy(y), ref, what="packed experts y")
    assert_close(to_numpy(out), O.combine(ref, osc), what="packed experts combine")
    again, _, _ = glu.experts(tx, tl, k)
    assert torch.equal(again, out)
