"""GPU parity: the VQ codebook-decode expert matmul (VQSwitchLinear's
product, 8-element vectors, uint8 / uint16 indices, fp16 codebook and
scales) and the VQ SwitchGLU, against the oracle's exact decode-then-matmul
(oracle.vq_matmul, itself pinned to the dense float64 product of the
decoded weight).  Bar: max rel err 1e-2, cosine 0.9999."""
import numpy as np
import pytest
import torch

import knurlogic_amd as K
import oracle as O
from knurlogic_amd import nn
from tests.util import assert_close, bf16_normal, to_numpy, to_torch

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _vq(rng, E, N, Kd, kc, scale_group, dev):
    """A VQ expert tensor: codes ~U[0, kc), codebook ~N(0, 0.02) fp16, scales
    ~U(0.5, 1.5) fp16 (per channel, or per group of scale_group inputs)."""
    ct = np.uint8 if kc <= 256 else np.uint16
    codes = rng.integers(0, kc, (E, N, Kd // 8)).astype(ct)
    cb = (rng.standard_normal((kc, 8)) * 0.02).astype(np.float16)
    ng = 1 if scale_group == 0 else Kd // scale_group
    sc = rng.uniform(0.5, 1.5, (E, N) if scale_group == 0 else (E, N, ng)).astype(np.float16)
    tcodes = torch.from_numpy(codes.view(np.int16) if ct == np.uint16 else codes).to(dev)
    if ct == np.uint16:
        tcodes = tcodes.view(torch.uint16)
    host = (codes, cb.astype(np.float32), sc.astype(np.float32))
    gpu = (tcodes, torch.from_numpy(cb).to(dev), torch.from_numpy(sc).to(dev))
    return host, gpu


def _ref_pairs(x, lhs, rhs, host, scale_group):
    codes, cb, sc = host
    out = []
    for p in range(len(rhs)):
        e = int(rhs[p])
        out.append(O.vq_matmul(x[lhs[p]][None], codes[e], cb, sc[e], scale_group, "float32")[0])
    return np.stack(out)


@pytest.mark.parametrize("kc", [256, 4096])
@pytest.mark.parametrize("scale_group", [0, 64])
@pytest.mark.parametrize("Kd,N", [(2048, 768), (768, 2048), (256, 100), (1024, 320)])
def test_vq_gather_matches_the_oracle(dev, kc, scale_group, Kd, N):
    rng = np.random.default_rng(kc + scale_group + Kd + N)
    E, X, P = 6, 3, 9
    host, gpu = _vq(rng, E, N, Kd, kc, scale_group, dev)
    x = bf16_normal(rng, (X, Kd))
    lhs = rng.integers(0, X, P).astype(np.int32)
    rhs = rng.integers(0, E, P).astype(np.int32)
    y = K.vq_gather_qmm(to_torch(x, dev, BF)[:, None, :], *gpu, torch.from_numpy(lhs).to(dev),
                        torch.from_numpy(rhs).to(dev), scale_group=scale_group)
    assert y.shape == (P, 1, N)
    assert_close(to_numpy(y)[:, 0], _ref_pairs(x, lhs, rhs, host, scale_group), what="vq gather")


def test_vq_linear_several_rows_and_a_bad_expert(dev):
    """x [X, M, K] with M = 3 rows per batch; an out-of-range expert gives 0."""
    rng = np.random.default_rng(7)
    E, N, Kd, kc = 4, 64, 512, 256
    host, gpu = _vq(rng, E, N, Kd, kc, 0, dev)
    lin = nn.VQSwitchLinear(*gpu)
    x = bf16_normal(rng, (2, 3, Kd))
    inds = np.array([[1], [5]], np.int32)          # batch 1 routes to expert 5: out of range
    y = lin(to_torch(x, dev, BF)[:, None], torch.from_numpy(inds).to(dev))
    assert y.shape == (2, 1, 3, N)
    got = to_numpy(y)
    ref = O.vq_matmul(x[0], host[0][1], host[1], host[2][1], 0, "float32")
    assert_close(got[0, 0], ref, what="rows")
    assert (got[1] == 0).all()


@pytest.mark.parametrize("kc,scale_group", [(256, 0), (4096, 0), (256, 64)])
@pytest.mark.parametrize("T,E,H,I,k", [(1, 16, 256, 128, 4), (5, 16, 512, 256, 4),
                                       (1, 128, 2048, 768, 8), (16, 128, 2048, 768, 8)])
def test_vq_switch_glu_matches_the_oracle(dev, kc, scale_group, T, E, H, I, k):
    rng = np.random.default_rng(T * 3 + E + kc + scale_group)
    (hg, gg), (hu, gu), (hd, gd) = [_vq(rng, E, n, kd, kc, scale_group, dev)
                                    for n, kd in ((I, H), (I, H), (H, I))]
    glu = nn.VQSwitchGLU(*(nn.VQSwitchLinear(*g, scale_group) for g in (gg, gu, gd)))
    x = bf16_normal(rng, (T, H))
    inds = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    fn = lambda h: (lambda xs, e: O.vq_matmul(xs, h[0][e], h[1], h[2][e], scale_group, "bfloat16"))
    ref = O.switch_glu(x, inds, fn(hg), fn(hu), fn(hd))
    tx, ti = to_torch(x, dev, BF), torch.from_numpy(inds).to(dev)
    got = glu(tx, ti)
    assert got.shape == (T, k, H)
    assert_close(to_numpy(got), ref, what="vq switch_glu")
    sep = glu.separate(tx, ti)
    if scale_group:
        # both run the per-pair kernels: the same sums in the same order
        assert torch.equal(sep, got), "one call and the separate ops differ"
    else:
        # the one call runs per-channel experts expert-major on MFMA (another
        # summation order than the per-pair separate ops)
        assert_close(to_numpy(sep), ref, what="vq separate ops")
    _, sc = O.route(bf16_normal(rng, (T, E)), k)
    comb = glu.combine(tx, ti, to_torch(sc, dev, BF))
    assert comb.shape == (T, H)
    assert_close(to_numpy(comb), O.combine(ref, sc), what="combine")
    # the one-call combine is the combine op applied to the same y, bit for bit
    assert torch.equal(comb, K.moe_combine(got, to_torch(sc, dev, BF)))


def test_vq_switch_glu_bad_expert_and_errors(dev):
    """An out-of-range expert contributes nothing (its y row is 0, its
    combine term 0); mismatched scores are refused."""
    rng = np.random.default_rng(41)
    E, H, I, T, k = 6, 256, 128, 3, 2
    (hg, gg), (hu, gu), (hd, gd) = [_vq(rng, E, n, kd, 256, 0, dev) for n, kd in ((I, H), (I, H), (H, I))]
    glu = nn.VQSwitchGLU(*(nn.VQSwitchLinear(*g) for g in (gg, gu, gd)))
    x = bf16_normal(rng, (T, H))
    inds = np.array([[0, 9], [2, 3], [-1, 5]], np.int32)
    tx, ti = to_torch(x, dev, BF), torch.from_numpy(inds).to(dev)
    y = to_numpy(glu(tx, ti))
    assert (y[0, 1] == 0).all() and (y[2, 0] == 0).all()
    sc = O.round_to(rng.uniform(0.1, 0.5, (T, k)).astype(np.float32), "bfloat16")
    comb = to_numpy(glu.combine(tx, ti, to_torch(sc, dev, BF)))
    assert_close(comb, O.combine(y, sc), what="combine with bad experts")
    with pytest.raises(ValueError):
        K.vq_switch_glu(tx, ti, gg, gu, gd, scores=torch.zeros(T, k + 1, dtype=BF, device=dev))


@pytest.mark.parametrize("T", [1, 3])
@pytest.mark.parametrize("kc", [256, 4096])
def test_vq_switch_glu_mfma_path_bad_experts(dev, T, kc):
    """Per-channel experts with K a multiple of 128 run expert-major on MFMA
    (one token: each pair its own tile; more: tiles from the GPU sort).  An
    out-of-range expert still gives a zero row, and the rest match the
    oracle."""
    rng = np.random.default_rng(7 * T + kc)
    E, H, I, k = 8, 768, 512, 4
    (hg, gg), (hu, gu), (hd, gd) = [_vq(rng, E, n, kd, kc, 0, dev) for n, kd in ((I, H), (I, H), (H, I))]
    glu = nn.VQSwitchGLU(*(nn.VQSwitchLinear(*g) for g in (gg, gu, gd)))
    x = bf16_normal(rng, (T, H))
    inds = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    inds[0, 1] = -1
    inds[-1, 3] = E + 2
    got = to_numpy(glu(to_torch(x, dev, BF), torch.from_numpy(inds).to(dev)))
    assert (got[0, 1] == 0).all() and (got[-1, 3] == 0).all()
    fn = lambda h: (lambda xs, e: O.vq_matmul(xs, h[0][e], h[1], h[2][e], 0, "bfloat16"))
    ok = (inds >= 0) & (inds < E)
    ref = O.switch_glu(x, np.where(ok, inds, 0), fn(hg), fn(hu), fn(hd))
    assert_close(got[ok], ref[ok], what="vq switch_glu (MFMA path)")


@pytest.mark.parametrize("T,E,H,I,k,kc", [(64, 4, 4096, 256, 2, 256), (48, 3, 1024, 512, 2, 4096)])
def test_vq_switch_glu_full_tiles_and_long_rows(dev, T, E, H, I, k, kc):
    """Many rows per expert (16-row tiles: x staged in two batches of rows),
    a 4096-long row (two passes over its pieces), and a codebook staged in
    64 blocks per projection."""
    rng = np.random.default_rng(T + E + H + kc)
    (hg, gg), (hu, gu), (hd, gd) = [_vq(rng, E, n, kd, kc, 0, dev) for n, kd in ((I, H), (I, H), (H, I))]
    glu = nn.VQSwitchGLU(*(nn.VQSwitchLinear(*g) for g in (gg, gu, gd)))
    x = bf16_normal(rng, (T, H))
    inds = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    fn = lambda h: (lambda xs, e: O.vq_matmul(xs, h[0][e], h[1], h[2][e], 0, "bfloat16"))
    ref = O.switch_glu(x, inds, fn(hg), fn(hu), fn(hd))
    got = glu(to_torch(x, dev, BF), torch.from_numpy(inds).to(dev))
    assert_close(to_numpy(got), ref, what=f"vq switch_glu T={T} H={H} kc={kc}")


@pytest.mark.parametrize("shared", [True, False])
def test_vq_switch_glu_tiles_across_16_rows(dev, shared):
    """Tens of rows per expert with 1-byte codes: experts of 17, 32, 33 and 46
    rows cut into 16-row tiles (the last one 1, 16, 1 and 14 rows deep);
    every output checked."""
    rng = np.random.default_rng(4242 + shared)
    T, E, H, I, k, kc = 64, 4, 1024, 512, 2, 256
    (hg, gg), (hu, gu), (hd, gd) = [_vq(rng, E, n, kd, kc, 0, dev) for n, kd in ((I, H), (I, H), (H, I))]
    if shared:
        hu, hd = (hu[0], hg[1], hu[2]), (hd[0], hg[1], hd[2])
        gu, gd = (gu[0], gg[1], gu[2]), (gd[0], gg[1], gd[2])
    glu = nn.VQSwitchGLU(*(nn.VQSwitchLinear(*g) for g in (gg, gu, gd)))
    x = bf16_normal(rng, (T, H))
    order = np.repeat(np.arange(E), [17, 32, 33, 46]).astype(np.int32)
    inds = np.stack([order[:T], order[T:]], axis=1)          # two distinct experts per token
    perm = rng.permutation(T)
    inds = inds[perm]
    assert (inds[:, 0] != inds[:, 1]).all()
    fn = lambda h: (lambda xs, e: O.vq_matmul(xs, h[0][e], h[1], h[2][e], 0, "bfloat16"))
    ref = O.switch_glu(x, inds, fn(hg), fn(hu), fn(hd))
    got = glu(to_torch(x, dev, BF), torch.from_numpy(inds).to(dev))
    assert_close(to_numpy(got), ref, what=f"vq switch_glu, tiles across 16 rows, shared={shared}")


@pytest.mark.parametrize("T,E,H,I,k,kc", [
    (8, 32, 1024, 512, 4, 100),      # a codebook of fewer than 256 entries
    (4, 4, 512, 256, 2, 256),        # experts over several 4-row tiles, a 256-wide down
    (8, 64, 2816, 704, 8, 256),      # the Gemma-4 26B expert widths; down on the VALU kernel (704 % 128)
    (2, 128, 2048, 768, 8, 256),     # 16 pairs: the token-major down with its combine
])
@pytest.mark.parametrize("shared", [True, False])
def test_vq_switch_glu_small_tiles_match_the_oracle(dev, T, E, H, I, k, kc, shared):
    """1-byte codes at one or two routed rows per expert: SwitchGLU and its
    combine against the oracle across tile splits, chunk counts and a short
    codebook, with one codebook for the layer (shared) or one per
    projection."""
    rng = np.random.default_rng(T + E + H + I + kc)
    (hg, gg), (hu, gu), (hd, gd) = [_vq(rng, E, n, kd, kc, 0, dev) for n, kd in ((I, H), (I, H), (H, I))]
    if shared:                      # the gate's codebook for all three projections
        hu, hd = (hu[0], hg[1], hu[2]), (hd[0], hg[1], hd[2])
        gu, gd = (gu[0], gg[1], gu[2]), (gd[0], gg[1], gd[2])
    glu = nn.VQSwitchGLU(*(nn.VQSwitchLinear(*g) for g in (gg, gu, gd)))
    x = bf16_normal(rng, (T, H))
    inds = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    fn = lambda h: (lambda xs, e: O.vq_matmul(xs, h[0][e], h[1], h[2][e], 0, "bfloat16"))
    ref = O.switch_glu(x, inds, fn(hg), fn(hu), fn(hd))
    tx, ti = to_torch(x, dev, BF), torch.from_numpy(inds).to(dev)
    got = glu(tx, ti)
    assert_close(to_numpy(got), ref, what=f"vq T={T} E={E} H={H} kc={kc}")
    _, sc = O.route(bf16_normal(rng, (T, E)), k)
    comb = glu.combine(tx, ti, to_torch(sc, dev, BF))
    assert_close(to_numpy(comb), O.combine(ref, sc), what="combine")


def test_vq_clamps_codes_past_the_codebook(dev):
    """Codes at or past a short codebook's size read its last entry (the
    clamp every VQ kernel applies, so such codes never read past the staged
    codebook): the same output as the codes clamped on the host."""
    rng = np.random.default_rng(77)
    T, E, H, I, k, kc = 8, 32, 1024, 512, 4, 100
    (hg, gg), (hu, gu), (hd, gd) = [_vq(rng, E, n, kd, kc, 0, dev) for n, kd in ((I, H), (I, H), (H, I))]
    wild = [g[0].clone() for g in (gg, gu, gd)]
    for w in wild:
        w[:, ::3, ::5] = 255                                   # past the 100 entries
    clamped = [torch.clamp(w, max=kc - 1) for w in wild]
    x = to_torch(bf16_normal(rng, (T, H)), dev, BF)
    inds = torch.from_numpy(np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)).to(dev)
    mk = lambda codes: nn.VQSwitchGLU(*(nn.VQSwitchLinear(c, g[1], g[2]) for c, g in zip(codes, (gg, gu, gd))))
    assert torch.equal(mk(wild)(x, inds), mk(clamped)(x, inds))


@pytest.mark.parametrize("T,kc", [(16, 4096), (1, 4096), (16, 256)])
def test_vq_switch_glu_repeats_bit_for_bit(dev, T, kc):
    """The same call twice gives the same bits: the sort's row order inside
    an expert tile varies between calls, and no result may depend on it."""
    rng = np.random.default_rng(5 * T + kc)
    E, H, I, k = 128, 2048, 768, 8
    (hg, gg), (hu, gu), (hd, gd) = [_vq(rng, E, n, kd, kc, 0, dev) for n, kd in ((I, H), (I, H), (H, I))]
    glu = nn.VQSwitchGLU(*(nn.VQSwitchLinear(*g) for g in (gg, gu, gd)))
    x = to_torch(bf16_normal(rng, (T, H)), dev, BF)
    inds = torch.from_numpy(np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)).to(dev)
    ys = [glu(x, inds) for _ in range(4)]
    for y in ys[1:]:
        assert torch.equal(y, ys[0])


@pytest.mark.parametrize("T,E,kc,pattern", [(1, 128, 256, "random"), (1, 128, 4096, "random"),
                                            (1, 300, 256, "random"), (3, 128, 4096, "random"),
                                            (16, 128, 256, "random"), (16, 256, 256, "random"),
                                            (16, 300, 256, "random"), (64, 128, 256, "random"),
                                            (16, 128, 256, "same"), (16, 128, 4096, "half"),
                                            (32, 128, 256, "random")])
def test_vq_experts_from_logits(dev, T, E, kc, pattern):
    """vq_experts (route, VQ SwitchGLU, combine in one call; at one token and
    E <= 256 the gate/up kernel routes the token itself; at up to 256 pairs
    over up to 256 experts the expert kernels form their tiles themselves,
    without the sort) gives the routing of moe_route and the output of the
    separate route and combine calls, bit for bit, and that output matches
    the oracle's routed SwitchGLU.  Skewed routing (every token, or half of
    them, on the same 8 experts) puts an expert's rows in several tiles."""
    rng = np.random.default_rng(11 * T + E + kc)
    H, I, k = 2048, 768, 8
    (hg, gg), (hu, gu), (hd, gd) = [_vq(rng, E, n, kd, kc, 0, dev) for n, kd in ((I, H), (I, H), (H, I))]
    glu = nn.VQSwitchGLU(*(nn.VQSwitchLinear(*g) for g in (gg, gu, gd)))
    x, lg = bf16_normal(rng, (T, H)), bf16_normal(rng, (T, E))
    if pattern == "same":
        lg[:] = lg[0]
    elif pattern == "half":
        lg[: T // 2] = lg[0]
    tx, tl = to_torch(x, dev, BF), to_torch(lg, dev, BF)
    out, inds, scores = glu.experts(tx, tl, k)
    ri, rs = K.moe_route(tl, k)
    assert torch.equal(inds, ri) and torch.equal(scores, rs), "routing differs from moe_route"
    assert torch.equal(out, glu.combine(tx, ri, rs)), "one call and route + combine differ"
    oi, osc = O.route(lg, k)
    assert np.array_equal(to_numpy(inds), oi)
    fn = lambda h: (lambda xs, e: O.vq_matmul(xs, h[0][e], h[1], h[2][e], 0, "bfloat16"))
    ref = O.combine(O.switch_glu(x, oi, fn(hg), fn(hu), fn(hd)), osc)
    assert_close(to_numpy(out), ref, what="vq experts")
    # a second call on the same inputs repeats the bits
    again, _, _ = glu.experts(tx, tl, k)
    assert torch.equal(again, out)
