"""Pins the CPU oracle (CPU only, no GPU).

Each test checks an oracle function against something that does not
restate it: the reference's own golden vectors, closed-form known answers,
invariants the mathematics fixes, or an independently written float64
numpy path -- chosen so a plausible mistake (a dropped term, a wrong sign,
index or rounding order) fails at least one of them.  Planted mistakes are
planted in the oracle, here on the CPU.
"""
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from tests.util import bf16_normal

GOLD = Path(__file__).resolve().parent / "golden"


# --- the reference's golden: Qwen3.5-MoE block, bf16, bit for bit -------------

def _golden_block():
    z = np.load(GOLD / "qwen35_moe_block.npz")
    gu, dn = z["experts__gate_up_proj"], z["experts__down_proj"]
    inter = gu.shape[1] // 2        # gate = first half of rows (qwen3_5_moe.py:41-45)
    fns = (lambda xs, e: O.dense_linear(xs, gu[e, :inter]),
           lambda xs, e: O.dense_linear(xs, gu[e, inter:]),
           lambda xs, e: O.dense_linear(xs, dn[e]))
    shared = (z["shared_expert__gate_proj__weight"], z["shared_expert__up_proj__weight"],
              z["shared_expert__down_proj__weight"], z["shared_expert_gate__weight"])
    return z, fns, shared


def test_moe_block_matches_the_reference_golden_bit_for_bit():
    z, fns, shared = _golden_block()
    y = O.moe_block(z["x"], z["gate__weight"], fns, shared, k=int(z["top_k"]))
    assert np.array_equal(y, z["expected"])


def test_the_golden_catches_rounding_order_mistakes(monkeypatch):
    z, fns, shared = _golden_block()
    k = int(z["top_k"])

    def twice_rounded_silu(g, dtype="bfloat16"):   # mlx's bf16 x*sigmoid(x)
        g32 = np.asarray(g, np.float32)
        sig = O.round_to(1.0 / (1.0 + np.exp(-g32.astype(np.float64))), dtype)
        return O.round_to(g32 * sig, dtype)

    def no_renorm(logits, kk, out_dtype="bfloat16"):
        lg = np.asarray(logits, np.float64)
        p = np.exp(lg - lg.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        order = np.argsort(-p, axis=-1, kind="stable")[..., :kk]
        return order.astype(np.int32), O.round_to(np.take_along_axis(p, order, -1), out_dtype)

    def unrounded_combine(y, s, dtype="bfloat16"):
        return O.round_to((np.asarray(y, np.float64) * np.asarray(s, np.float64)[..., None])
                          .sum(-2).astype(np.float32), dtype)

    for name, bad in (("silu_rounded", twice_rounded_silu), ("route", no_renorm),
                      ("combine", unrounded_combine)):
        with monkeypatch.context() as m:
            m.setattr(O, name, bad)
            y = O.moe_block(z["x"], z["gate__weight"], fns, shared, k=k)
        assert not np.array_equal(y, z["expected"]), name


# --- affine quantize: known answers and invariants -----------------------------

def test_quantize_known_answer_max_edge_negative_scale():
    """Group max 15 has the larger magnitude: scale -1, bias 15, q = 15 - w;
    the packed words then read 0x89ABCDEF / 0x01234567 (element j in word
    j/8 at bits 4*(j%8), kvattn.py:128-131 of the reference)."""
    w = np.tile(np.arange(16, dtype=np.float32), 4)[None]          # one group of 64
    wq, s, b = O.quantize(w, 64, 4)
    assert s[0, 0] == -1.0 and b[0, 0] == 15.0
    assert wq[0, 0] == 0x89ABCDEF and wq[0, 1] == 0x01234567
    assert np.array_equal(O.unpack_numpy(wq, 4)[0], (15 - w[0]).astype(np.uint32))


def test_quantize_known_answer_min_edge_positive_scale():
    w = -np.tile(np.arange(16, dtype=np.float32), 4)[None]
    wq, s, b = O.quantize(w, 64, 4)
    assert s[0, 0] == 1.0 and b[0, 0] == -15.0
    assert np.array_equal(O.unpack_numpy(wq, 4)[0], (w[0] + 15).astype(np.uint32))


def test_quantize_ties_round_to_even():
    """mlx's CPU quantizer (mlx/backend/cpu/quantized.cpp, ``quantize``) forms
    each code as std::rint((w - bias) / scale), which rounds a tie to the
    even integer.  Group [0, 15, 6.5, 4.5, ...]: scale -1, bias 15, so
    6.5 -> rint(8.5) = 8 and 4.5 -> rint(10.5) = 10 (half away from zero
    would give 9 and 11); dequantized 7 and 5."""
    w = np.zeros((1, 64), np.float32)
    w[0, 1], w[0, 2], w[0, 3] = 15.0, 6.5, 4.5
    w[0, 4:] = np.arange(60) % 16
    wq, s, b = O.quantize(w, 64, 4)
    assert s[0, 0] == -1.0 and b[0, 0] == 15.0
    q = O.unpack_numpy(wq, 4)[0]
    assert q[2] == 8 and q[3] == 10
    assert O.dequantize(wq, s, b, 64, 4)[0, 2] == 7.0


def test_quantize_all_zero_group():
    wq, s, b = O.quantize(np.zeros((1, 64), np.float32), 64, 8)
    assert (wq == 0).all() and b[0, 0] == 0.0 and s[0, 0] == O.bf16_round(np.float32(-1e-7))


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_quantize_invariants(bits, group):
    rng = np.random.default_rng(bits * 1000 + group)
    w = bf16_normal(rng, (64, 512), 0.02)
    wq, s, b = O.quantize(w, group, bits)
    q = O.unpack_numpy(wq, bits).astype(np.int64)
    assert q.min() >= 0 and q.max() <= 2 ** bits - 1
    wh = O.dequantize_numpy_f64(wq, s, b, group, bits)
    # round trip within |scale|/2 plus the bf16 rounding of the scale
    # (unit roundoff 2^-8: <= 2^-8 |s| per code step) -- except where snapping the scale so 0
    # is a code point shrank it and the far end of the range clipped at the
    # top code: there the error is below one (snapped) step
    sg = np.repeat(np.abs(s.astype(np.float64)), group, axis=-1)
    n_bins = 2 ** bits - 1
    err = np.abs(wh - w)
    assert (err <= sg * (1.0 + 2.0 ** -7 * n_bins) + 1e-12).all()
    over = err > sg * (0.5 + 2.0 ** -8 * (n_bins + 1)) + 1e-12
    assert (q[over] == n_bins).all()
    # the larger-magnitude edge of each group is stored as the bias: exact
    g = w.reshape(64, -1, group)
    edge = np.where(np.abs(g.min(-1)) > np.abs(g.max(-1)), g.min(-1), g.max(-1))
    assert np.array_equal(b, edge.astype(np.float32))
    # and reconstructs exactly at its own position (code 0)
    idx = np.argmax(g == edge[..., None], axis=-1)
    qe = np.take_along_axis(q.reshape(64, -1, group), idx[..., None], -1)[..., 0]
    assert (qe == 0).all()


@pytest.mark.parametrize("bits", [3, 5, 6])
def test_odd_widths_pack_as_one_bit_stream(bits):
    """3, 5 and 6-bit codes sit back to back in the row's little-endian
    bit stream (a code may straddle two words): the codes unpacked by the
    bitwise reader re-pack, bit by bit, into exactly the quantizer's words."""
    rng = np.random.default_rng(bits)
    w = bf16_normal(rng, (3, 96), 0.02)
    wq, s, b = O.quantize(w, 32, bits)
    assert wq.shape == (3, 96 * bits // 32)
    q = O.unpack_fields(wq, bits, 96)
    words = np.zeros_like(wq)
    for r in range(3):
        for j in range(96):
            for t in range(bits):
                if (int(q[r, j]) >> t) & 1:
                    p = j * bits + t
                    words[r, p // 32] |= np.uint32(1 << (p % 32))
    assert np.array_equal(words, wq)
    # and the C dequantize reads the same codes
    deq = O.dequantize(wq, s, b, 32, bits, dtype="float32", rounding=O.ROUND_FUSED)
    ref = np.repeat(s, 32, -1) * q.astype(np.float32) + np.repeat(b, 32, -1)
    assert np.abs(deq - ref).max() <= 1e-6 * np.abs(ref).max()


def test_six_bit_round_trip_is_within_the_eight_bit_bar_times_four():
    """The reference offers 6-bit KV (kvquant.py:22); its step is four times
    the 8-bit one, so a fetch of N(0,1) stays within 4 x 0.05."""
    rng = np.random.default_rng(2)
    x = bf16_normal(rng, (2, 40, 64))
    wq, s, b = O.quantize(x, 64, 6)
    assert np.abs(O.dequantize(wq, s, b, 64, 6) - x).max() < 0.2


def test_eight_bit_round_trip_is_within_the_references_bar():
    """tests/engine/test_kvquant.py:37-43: an 8-bit fetch of N(0,1) bf16 is
    within 0.05 of what went in."""
    rng = np.random.default_rng(1)
    x = bf16_normal(rng, (2, 40, 64))
    wq, s, b = O.quantize(x, 64, 8)
    assert np.abs(O.dequantize(wq, s, b, 64, 8) - x).max() < 0.05


# --- dequantize: closed form, rounding order ----------------------------------

def test_dequantize_closed_form():
    codes = np.arange(16, dtype=np.uint32)
    word0 = np.uint32(sum(int(c) << (4 * i) for i, c in enumerate(codes[:8])))
    word1 = np.uint32(sum(int(c) << (4 * i) for i, c in enumerate(codes[8:])))
    wq = np.array([[word0, word1] * 4], np.uint32)                 # 64 elements
    out = O.dequantize(wq, np.array([[0.5]], np.float32), np.array([[-1.0]], np.float32), 64, 4)
    assert np.array_equal(out[0], 0.5 * np.tile(np.arange(16), 4) - 1.0)


def test_dequantize_rounding_orders_differ_where_they_must():
    """s = 1 + 2^-7, q = 3, b = -2^-7: T(T(s*q)+b) = 3.03125 (two ties to
    even), T(fma) = 3.015625 -- the switch is real."""
    wq = np.array([[3] + [0] * 7], np.uint32)                       # element 0 -> q 3
    s = np.array([[1.0078125]], np.float32)
    b = np.array([[-0.0078125]], np.float32)
    two = O.dequantize(wq, s, b, 64, 4, rounding=O.ROUND_OP_BY_OP)
    one = O.dequantize(wq, s, b, 64, 4, rounding=O.ROUND_FUSED)
    assert two[0, 0] == 3.03125 and one[0, 0] == 3.015625


def test_dequantize_matches_numpy_within_one_rounding():
    rng = np.random.default_rng(2)
    w = bf16_normal(rng, (32, 256), 0.02)
    for bits in (4, 8):
        wq, s, b = O.quantize(w, 64, bits)
        exact = O.dequantize_numpy_f64(wq, s, b, 64, bits)
        fused = O.dequantize(wq, s, b, 64, bits, rounding=O.ROUND_FUSED)
        assert np.array_equal(fused, O.bf16_round(exact.astype(np.float32)))
        f32 = O.dequantize(wq, s, b, 64, bits, dtype="float32", rounding=O.ROUND_FUSED)
        assert np.abs(f32 - exact).max() <= np.abs(exact).max() * 2 ** -23


# --- quantized_matmul / gather_qmm ------------------------------------------------

@pytest.mark.parametrize("bits", [4, 8])
def test_qmm_equals_float64_brute_force(bits):
    rng = np.random.default_rng(3)
    w = bf16_normal(rng, (48, 256), 0.02)
    x = bf16_normal(rng, (5, 256))
    wq, s, b = O.quantize(w, 64, bits)
    ref = x.astype(np.float64) @ O.dequantize_numpy_f64(wq, s, b, 64, bits).T
    got = O.quantized_matmul(x, wq, s, b, True, 64, bits, "float32")
    assert np.abs(got - ref).max() <= np.abs(ref).max() * 1e-6
    # transpose=False: w quantized along its output axis
    wt = bf16_normal(rng, (256, 64), 0.02)
    wqt, st, bt = O.quantize(wt, 64, bits)
    reft = x.astype(np.float64) @ O.dequantize_numpy_f64(wqt, st, bt, 64, bits)
    gott = O.quantized_matmul(x, wqt, st, bt, False, 64, bits, "float32")
    assert np.abs(gott - reft).max() <= np.abs(reft).max() * 1e-6


def test_qmm_is_linear_and_row_independent():
    rng = np.random.default_rng(4)
    w = bf16_normal(rng, (64, 128), 0.02)
    wq, s, b = O.quantize(w, 64, 4)
    x = bf16_normal(rng, (7, 128))
    y = O.quantized_matmul(x, wq, s, b, True, 64, 4, "float32")
    assert np.array_equal(O.quantized_matmul(2 * x, wq, s, b, True, 64, 4, "float32"), 2 * y)
    for m in range(7):
        assert np.array_equal(O.quantized_matmul(x[m:m + 1], wq, s, b, True, 64, 4, "float32"),
                              y[m:m + 1])


def test_gather_qmm_is_per_row_expert_selection():
    rng = np.random.default_rng(5)
    E, N, K, T, k = 6, 32, 128, 5, 3
    w = bf16_normal(rng, (E, N, K), 0.02)
    wq, s, b = O.quantize(w, 64, 4)
    x = bf16_normal(rng, (T, 1, 1, K))
    inds = rng.integers(0, E, (T, k))
    got = O.gather_qmm(x, wq, s, b, rhs_indices=inds, out_dtype="float32")
    assert got.shape == (T, k, 1, N)
    for t in range(T):
        for j in range(k):
            e = inds[t, j]
            ref = x[t, 0].astype(np.float64) @ O.dequantize_numpy_f64(wq[e], s[e], b[e], 64, 4).T
            assert np.abs(got[t, j] - ref).max() <= np.abs(ref).max() * 1e-6 + 1e-30


# --- router --------------------------------------------------------------------

def test_route_known_answer_and_ties():
    inds, scores = O.route(np.array([[0.0, 1.0, 2.0, 3.0]], np.float32), 2, "float32")
    assert list(inds[0]) == [3, 2]
    e = np.exp([3.0, 2.0])
    assert np.allclose(scores[0], e / e.sum(), rtol=1e-6)
    inds, _ = O.route(np.zeros((1, 5), np.float32), 3)
    assert list(inds[0]) == [0, 1, 2]


def test_route_uniform_rows_by_hand():
    """Equal logits: e = 1, n = E, r = float32(1/E), p = r.  E = 3, k = 2:
    r = 0x3EAAAAAB, t = 2r exactly, scores = r / 2r = 0.5; experts 0, 1
    (ties to the lower index).  A hidden expert (-inf) gets e = 0 and is
    never chosen ahead of a visible one."""
    inds, scores = O.route(np.zeros((1, 3), np.float32), 2, "float32")
    assert list(inds[0]) == [0, 1] and list(scores[0]) == [0.5, 0.5]
    inds, scores = O.route(np.array([[-np.inf, 0.0, -np.inf, 0.0, 0.0]], np.float32), 3, "float32")
    assert list(inds[0]) == [1, 3, 4]
    assert scores[0, 0].view(np.uint32) == 0x3EAAAAAB          # float32(1/3): r / (3r rounded)
    assert scores.sum() == np.float32(1.0)


def test_route_one_ulp_apart_is_ordered_by_the_rounded_probabilities():
    """Two experts whose float32 probabilities differ by exactly one ulp:
    logits (bf16) 1, 0, 2^-23, -8.  exp(-1 + 2^-23) and exp(-1), each
    correctly rounded, are 0x3E590343 and 0x3E590342 after the reciprocal
    multiply, so top-2 is experts 0 and 2 -- not 0 and 1, which the
    lower-index tie rule would give were they equal.  (mlx's own SIMD exp
    is within a few ulp of this, so whether mlx picks expert 1 or 2 on such
    a row is not fixed by this rule: top-k membership at one-ulp near-ties
    is parity unpinned.)"""
    lg = np.array([[1.0, 0.0, 2.0 ** -23, -8.0]], np.float32)
    assert (O.bf16_round(lg) == lg).all()
    inds, scores = O.route(lg, 2, "float32")
    assert list(inds[0]) == [0, 2]
    # the two probabilities, as the oracle forms them, one ulp apart
    e = np.exp((lg - lg.max()).astype(np.float64)).astype(np.float32)
    n = e.astype(np.float64).sum().astype(np.float32)
    pr = e * (np.float32(1.0) / n)
    assert pr[0, 2].view(np.uint32) == 0x3E590343 and pr[0, 1].view(np.uint32) == 0x3E590342
    # a planted mistake: exp rounded through float32 arithmetic on a coarser
    # grid (x - m in bf16) makes the two equal and flips the choice to 1
    coarse = O.bf16_round((lg - lg.max()).astype(np.float32))
    assert coarse[0, 1] == coarse[0, 2]


def test_route_agrees_with_an_independent_fp32_router():
    """HF transformers' Qwen MoE router on torch's CPU kernels (softmax in
    float32, top-k, p / sum(p) in float32, cast to bf16) -- the
    implementation the reference's golden was made with -- computes the
    same float32 op sequence as mlx (softmax with one reciprocal of the
    normaliser).  Over 20000 rows of 128 bf16 logits the oracle picks the
    same top-8 set everywhere and the same bf16 scores, bit for bit, in all
    but a handful of boundary cases (one bf16 ulp apart, where torch's SIMD
    exp lands an ulp away from the correctly rounded one)."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0)
    lg = O.bf16_round(rng.standard_normal((20000, 128)).astype(np.float32))
    p = torch.softmax(torch.from_numpy(lg), -1)
    top, ind = p.topk(8, -1)
    ref = (top / top.sum(-1, keepdim=True)).to(torch.bfloat16).float().numpy()
    ind = ind.numpy()
    inds, scores = O.route(lg, 8)
    # torch picks freely among equal probabilities at the 8th place (equal
    # bf16 logits); everywhere else the sets must agree
    p9 = np.sort(p.numpy(), -1)[:, ::-1][:, 7:9]
    clear = p9[:, 0] > p9[:, 1]
    assert clear.mean() > 0.9
    assert (np.sort(inds, -1) == np.sort(ind, -1))[clear].all()
    # compare each expert's score (torch orders equal probabilities freely)
    got = np.take_along_axis(scores, np.argsort(inds, -1), -1)[clear]
    want = np.take_along_axis(ref, np.argsort(ind, -1), -1)[clear]
    diff = got != want
    assert diff.mean() < 1e-4, diff.mean()
    assert np.all(np.abs(got - want)[diff] <= np.abs(want[diff]) * 2 ** -7)


# --- KV8 decode attention ---------------------------------------------------------

def _kv_case(rng, B, H, Hk, L, N, D, g=64):
    k = bf16_normal(rng, (B, Hk, N, D))
    v = bf16_normal(rng, (B, Hk, N, D))
    q = bf16_normal(rng, (B, H, L, D))
    return q, O.quantize(k, g, 8), O.quantize(v, g, 8)


@pytest.mark.parametrize("mask", [None, "causal", "holes"])
def test_kv8_matches_float64_attention_over_the_dequantized_cache(mask):
    rng = np.random.default_rng(6)
    B, H, Hk, L, N, D = 2, 8, 2, 3, 150, 128
    q, K, V = _kv_case(rng, B, H, Hk, L, N, D)
    if mask == "holes":
        m = np.ones((B, 1, L, N), bool)
        m[..., np.arange(N) % 5 == 2] = False
        m[1, 0, 0, :] = False                      # a row that sees no key
        mask = m
    kd = O.dequantize_numpy_f64(*K, 64, 8)
    vd = O.dequantize_numpy_f64(*V, 64, 8)
    scale = D ** -0.5
    qs = (q * np.float32(scale)).astype(np.float64)  # q pre-scaled in fp32 (kvattn.py:101)
    ref = O.sdpa_numpy_f64(qs, kd, vd, 1.0, mask)
    got = O.kv8_decode(q, K, V, scale, mask, 64, 8, "float32")
    assert np.abs(got - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())
    if isinstance(mask, np.ndarray):
        assert (got[1, :, 0] == 0).all()          # every key masked -> 0 (kvattn.py:11-12)


def test_causal_rows_see_their_own_prefix():
    """kvattn._mask_rows: row i of an L-row block sees keys <= N - L + i."""
    m = O.mask_rows("causal", 1, 3, 6)
    assert m[0].tolist() == [[1, 1, 1, 1, 0, 0], [1, 1, 1, 1, 1, 0], [1, 1, 1, 1, 1, 1]]
    assert O.mask_rows("causal", 2, 1, 6) is None


# --- batched quantized_matmul and mlx-lm's quantized attention -----------------

def _on_grid(rng, lead, R, C, group, bits):
    """Packed words, scales, biases and the dense float64 weight they encode,
    built from random codes with numpy bit operations (independent of the
    oracle's packing and dequantize).  The weight is [..., R, C] quantized
    along C in groups of `group`."""
    q = rng.integers(0, 1 << bits, size=lead + (R, C), dtype=np.uint64)
    epw = 32 // bits
    words = np.zeros(lead + (R, C // epw), np.uint64)
    for i in range(epw):
        words |= q[..., i::epw] << np.uint64(bits * i)
    s = bf16_normal(rng, lead + (R, C // group), 0.01)
    b = bf16_normal(rng, lead + (R, C // group), 0.05)
    dense = np.repeat(s.astype(np.float64), group, -1) * q.astype(np.float64) + \
        np.repeat(b.astype(np.float64), group, -1)
    return words.astype(np.uint32), s, b, dense


@pytest.mark.parametrize("transpose", [True, False])
@pytest.mark.parametrize("bits,group", [(4, 64), (8, 32), (4, 128)])
def test_batched_qmm_on_grid_weights_equals_the_dense_product(transpose, bits, group):
    """A transposed operand, a group read along the wrong axis or a batch
    entry paired with the wrong weight all fail this."""
    rng = np.random.default_rng(11)
    M, K, N = 3, 256, 128
    R, C = (N, K) if transpose else (K, N)
    wq, s, b, dense = _on_grid(rng, (1, 3), R, C, group, bits)
    x = bf16_normal(rng, (2, 1, M, K))
    got = O.quantized_matmul_batched(x, wq, s, b, transpose, group, bits, "float32")
    wmat = np.swapaxes(dense, -1, -2) if transpose else dense
    ref = np.matmul(x.astype(np.float64), wmat)
    assert got.shape == (2, 3, M, N)
    assert np.abs(got - ref).max() <= 1e-6 * np.abs(ref).max()


def _qsdpa_case(rng, B, Hq, Hk, L, N, D, bits=8):
    q = bf16_normal(rng, (B, Hq, L, D))
    k = bf16_normal(rng, (B, Hk, N, D))
    v = bf16_normal(rng, (B, Hk, N, D))
    return q, O.quantize(k, 64, bits), O.quantize(v, 64, bits)


@pytest.mark.parametrize("mask", [None, "causal", "bool", "additive"])
def test_quantized_sdpa_matches_float64_attention(mask):
    """Within the bf16 roundings of q*scale, the scores and the
    probabilities (relative 2^-8 each), the result is float64 attention
    over the dequantized cache.  A transposed V product or the scale
    applied twice fails by far more."""
    rng = np.random.default_rng(12)
    B, Hq, Hk, L, N, D = 2, 8, 2, 3, 96, 128
    q, K, V = _qsdpa_case(rng, B, Hq, Hk, L, N, D)
    kd, vd = O.dequantize_numpy_f64(*K, 64, 8), O.dequantize_numpy_f64(*V, 64, 8)
    scale = D ** -0.5
    ref_mask, m = mask, mask
    if mask == "bool":
        m = rng.random((B, 1, L, N)) > 0.3
        ref_mask = m
    elif mask == "additive":
        m = O.bf16_round(rng.standard_normal((B, 1, L, N)).astype(np.float32))
        ref_mask = None
    qs = O.bf16_round(q * np.float32(scale)).astype(np.float64)
    if mask == "additive":
        s = np.einsum("bhld,bhnd->bhln", qs.reshape(B, Hk, Hq // Hk, L, D).reshape(B, Hq, L, D),
                      np.repeat(kd, Hq // Hk, axis=1)) + m
        p = np.exp(s - s.max(-1, keepdims=True))
        ref = np.einsum("bhln,bhnd->bhld", p / p.sum(-1, keepdims=True), np.repeat(vd, Hq // Hk, axis=1))
    else:
        ref = O.sdpa_numpy_f64(qs, kd, vd, 1.0, ref_mask)
    got = O.quantized_sdpa(q, K, V, scale, m, 64, 8)
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err < 2e-2, err


def test_quantized_sdpa_hidden_row_is_the_plain_mean_of_v():
    """A row whose every key is hidden scores finfo(bf16).min everywhere, so
    its softmax is uniform: with N a power of two the probabilities 1/N are
    exact in bf16 and the row is the mean of the dequantized V, rounded once
    (not 0, the 8-bit kernel's rule)."""
    rng = np.random.default_rng(13)
    B, Hq, Hk, L, N, D = 1, 4, 2, 2, 64, 64
    q, K, V = _qsdpa_case(rng, B, Hq, Hk, L, N, D, bits=4)
    m = np.ones((B, 1, L, N), bool)
    m[0, 0, 1, :] = False
    got = O.quantized_sdpa(q, K, V, 0.125, m, 64, 4)
    vd = O.dequantize_numpy_f64(*V, 64, 4)
    mean = vd.mean(axis=2)                                  # [B, Hk, D]
    want = O.bf16_round(mean.astype(np.float32))
    for h in range(Hq):
        assert np.array_equal(got[0, h, 1], want[0, h // 2])


# --- mxfp4 / mxfp8 ------------------------------------------------------------------

def test_mx_element_encodings_are_the_ocp_spec():
    """Known answers of the OCP Microscaling spec: the E2M1 values, E4M3's
    largest normal (S.1111.110 = 448), smallest normal (2^-6) and
    subnormal (2^-9), its NaN, and E8M0 = 2^(e - 127)."""
    q = np.arange(16, dtype=np.uint32)
    word = np.zeros((1, 2), np.uint32)
    for j in range(16):
        word[0, j // 8] |= np.uint32(int(q[j]) << (4 * (j % 8)))
    v = O.mx_dequantize(np.tile(word, (1, 2)), np.array([[127]], np.uint8), "mxfp4")[0, :16]
    assert v.tolist() == [0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6]
    assert O.e4m3([0x7E, 0x08, 0x01, 0xFE, 0x38])[:5].tolist() == [448.0, 2.0 ** -6, 2.0 ** -9, -448.0, 1.0]
    assert np.isnan(O.e4m3([0x7F])[0]) and np.isnan(O.e4m3([0xFF])[0])
    assert O.e8m0([127, 128, 0]).tolist() == [1.0, 2.0, 2.0 ** -127] and np.isnan(O.e8m0([255])[0])


def test_mx_matmul_equals_the_decoded_product():
    rng = np.random.default_rng(5)
    for mode, bits in (("mxfp4", 4), ("mxfp8", 8)):
        wq = rng.integers(0, 2 ** 32, (16, 64 * bits // 32), dtype=np.uint64).astype(np.uint32)
        if mode == "mxfp8":                      # no NaN codes
            b = wq.view(np.uint8)
            b[(b & 0x7F) == 0x7F] = 0
        sc = rng.integers(120, 134, (16, 2)).astype(np.uint8)
        x = bf16_normal(rng, (3, 64))
        ref = x.astype(np.float64) @ O.mx_dequantize(wq, sc, mode).T
        got = O.mx_quantized_matmul(x, wq, sc, mode, True, "float32")
        assert np.abs(got - ref).max() <= 1e-6 * np.abs(ref).max()


# --- packed VQ codes ------------------------------------------------------------------

def _pack_fields_bitwise(codes, bits):
    """Rows of integer codes -> uint32 words, one bit at a time: bit t of
    field j goes to stream position j*bits + t, stream position p to bit
    p % 32 of word p // 32, rows padded to whole 32-field blocks."""
    rows, n = codes.shape
    words = np.zeros((rows, (n + 31) // 32 * bits), np.uint32)
    for r in range(rows):
        for j in range(n):
            for t in range(bits):
                if (int(codes[r, j]) >> t) & 1:
                    p = j * bits + t
                    words[r, p // 32] |= np.uint32(1 << (p % 32))
    return words


@pytest.mark.parametrize("bits,n", [(11, 48), (8, 40), (12, 32), (9, 7)])
def test_unpack_fields_reads_the_bitwise_packing(bits, n):
    rng = np.random.default_rng(bits * 100 + n)
    codes = rng.integers(0, 1 << bits, (3, n))
    words = _pack_fields_bitwise(codes, bits)
    assert words.shape == (3, (n + 31) // 32 * bits)
    assert np.array_equal(O.unpack_fields(words, bits, n), codes)


def test_eight_bit_fields_are_the_byte_layout():
    """At 8 bits the packed stream is the uint8 code layout (little-endian
    words), whole blocks."""
    rng = np.random.default_rng(1)
    codes = rng.integers(0, 256, (2, 64)).astype(np.uint8)
    words = codes.view(np.uint32)
    assert np.array_equal(O.unpack_fields(words, 8, 64), codes)


def test_vq_packed_matmul_equals_decode_then_dense():
    rng = np.random.default_rng(2)
    OUT, IN, dim, kc, group = 24, 256, 4, 2048, 64
    codes = rng.integers(0, kc, (OUT, IN // dim))
    words = _pack_fields_bitwise(codes, 11)
    cb = O.f16_round(rng.standard_normal((kc, dim)).astype(np.float32) * 0.3)
    sc = O.f16_round((0.5 + rng.random((OUT, IN // group))).astype(np.float32))
    x = bf16_normal(rng, (3, IN))
    ref = x.astype(np.float64) @ O.vq_decode_numpy(codes, cb, sc, group).T
    got = O.vq_packed_matmul(x, words, cb, sc, 11, group, "float32")
    assert np.abs(got - ref).max() <= 1e-6 * np.abs(ref).max()


# --- VQ decode matmul ----------------------------------------------------------------

@pytest.mark.parametrize("code_dtype,kc", [(np.uint8, 256), (np.uint16, 4096)])
def test_vq_matmul_equals_decode_then_dense(code_dtype, kc):
    rng = np.random.default_rng(7)
    OUT, IN, dim = 40, 96, 8
    cb = O.f16_round(rng.standard_normal((kc, dim)) * 0.02)
    codes = rng.integers(0, kc, (OUT, IN // dim)).astype(code_dtype)
    sc = O.f16_round(rng.uniform(0.5, 1.5, OUT))
    x = bf16_normal(rng, (3, IN))
    ref = x.astype(np.float64) @ O.vq_decode_numpy(codes, cb, sc).T
    got = O.vq_matmul(x, codes, cb, sc, out_dtype="float32")
    assert np.abs(got - ref).max() <= 1e-6 * np.abs(ref).max()
    # one decoded element by hand
    o, i = 3, 17
    assert np.isclose(O.vq_decode_numpy(codes, cb, sc)[o, i],
                      sc[o] * cb[codes[o, i // dim], i % dim])


def test_the_references_mxfp4_experts_decode_as_the_spec_quantizes():
    """The reference's tiny DeepSeek-V4 checkpoint (mlx-format, mxfp4
    experts; tests/golden/make_mxfp4_fixture.py): per the OCP scheme each
    group's shared exponent is floor(log2 max|w|) - 2, so its largest
    element magnitude is 4 or 6 (codes 6, 7), and all values are finite."""
    z = np.load(GOLD / "deepseek_v4_tiny_mxfp4_experts.npz")
    for p in ("gate_proj", "up_proj", "down_proj"):
        w, s = z[p + "__weight"], z[p + "__scales"]
        v = O.mx_dequantize(w, s, "mxfp4")
        assert np.isfinite(v).all()
        elem = v / np.repeat(O.e8m0(s), 32, axis=-1)
        gmax = np.abs(elem).reshape(*elem.shape[:-1], -1, 32).max(-1)
        assert set(np.unique(gmax).tolist()) <= {4.0, 6.0}


def test_requantizing_the_references_mxfp4_experts_gives_them_back():
    """mx_quantize of the fixture's decoded values reproduces its codes and
    E8M0 scales exactly: the floor(log2 amax) - 2 exponent, RNE to E2M1 and
    the packing order all agree with the checkpoint (a ceil-based scale
    would move every group whose max element is 4 or 6 to another code)."""
    z = np.load(GOLD / "deepseek_v4_tiny_mxfp4_experts.npz")
    for p in ("gate_proj", "up_proj", "down_proj"):
        w, s = z[p + "__weight"], z[p + "__scales"]
        wq2, s2 = O.mx_quantize(O.mx_dequantize(w, s, "mxfp4"), "mxfp4")
        assert np.array_equal(s2, s) and np.array_equal(wq2, w)


def test_mx_quantize_round_trip_and_saturation():
    rng = np.random.default_rng(9)
    w = rng.standard_normal((4, 64)) * 0.05
    w[0, :32] = 0.0                                   # an all-zero group
    for mode in ("mxfp4", "mxfp8"):
        wq, s = O.mx_quantize(w, mode)
        back = O.mx_dequantize(wq, s, mode)
        assert s[0, 0] == 0 and not back[0, :32].any()
        # worst case in element units: saturation of [6, 8) to 6 (E2M1) or of
        # [448, 512) to 448 (E4M3), which bounds the rounding error as well
        worst = 2.0 if mode == "mxfp4" else 64.0
        scale = np.repeat(O.e8m0(s), 32, -1)
        assert (np.abs(back - w) <= scale * worst + 1e-12).all()


@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8"])
def test_mx_quantize_hand_computed_ties_and_saturation(mode):
    """The OCP conversion worked out by hand for one group (scale byte 127):
    ties to the even code, saturation to the largest finite element, the
    sign of zero kept (the table is shared with the GPU test)."""
    from tests.test_gpu_mx import mx_hand_group
    w, want = mx_hand_group(mode)
    wq, sc = O.mx_quantize(w, mode)
    assert sc.tolist() == [[127]]
    assert O.unpack_numpy(wq, 4 if mode == "mxfp4" else 8)[0].tolist() == want.tolist()
