"""CPU oracle for the quantized-weight path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference computes on its
quantized-weight hot path, so the HIP kernels can be checked against it.
Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import it, and only as the checker; the product (``knurlogic_amd``)
never imports it.

The reference (Knurlogic 0.1.9) is pure Python over mlx 0.32.3 / mlx-lm
0.32.0, pinned at pyproject.toml:32-33 and NOT vendored, so there is no
reference source to compile into an ``oracle/_ref`` build; the arithmetic is
restated from mlx's published algorithms and from the reference's own call
sites, and pinned as follows (each function's docstring names its pins):

* quantize/dequantize packing -- pinned by the reference's KV8 kernel, which
  reads mlx-packed words as ``(word >> (e*BITS)) & MASK``
  (src/knurlogic/engine/kvattn.py:128-131); closed-form known answers in
  tests/test_oracle.py.
* quantize's edge rule -- pinned by invariants only (codes in range, the
  larger-magnitude edge reconstructs exactly, round trip within |scale|/2,
  the reference's 8-bit round-trip bound, tests/engine/test_kvquant.py:37-43).
  The exact choice of edge/sign is mlx's published rule, not checkable
  against mlx here: parity unpinned beyond those invariants.
* dequantize's bf16 rounding order -- a switch (``rounding``); the default is
  mlx's CPU op-by-op order.  Which order mlx 0.32.3 takes is parity unpinned.
* quantized_matmul / gather_qmm -- float64 brute force through an
  independently written numpy dequantize, linearity and row independence,
  and the reference's 2e-3 bar (tests/engine/test_deepseek_v4_bf16.py:247-270).
  The batched form (both orientations, broadcast batches) -- on-grid
  weights packed independently of the oracle, against a dense float64
  product.
* mxfp4 / mxfp8 -- the OCP MX element and scale encodings, pinned by the
  spec's known answers (E2M1 table, E4M3 extremes and NaN, E8M0 powers of
  two).  How mlx orders the packed codes is its 4 / 8-bit affine order.
  mx quantize follows the OCP conversion rule (shared exponent, ties to
  even, saturation, the sign of zero kept): parity with mlx's quantizer
  is unpinned; hand-computed codes check the rule as stated.
* quantized attention (mlx-lm's base.py:260-302) -- float64 attention
  (``sdpa_numpy_f64``) within the bf16 roundings the path makes, and the
  exact uniform softmax of a fully hidden row.
* router / SwiGLU / combine / shared expert -- the reference's golden
  ``qwen_reference.npz`` key ``qwen3_5_moe/bf16/0.mlp`` (HF transformers'
  bf16 block, bit for bit), committed as tests/golden/qwen35_moe_block.npz.
* KV8 decode attention -- float64 brute force with a separately written
  numpy softmax, mask cases of tests/engine/test_kvattn.py:86-113,253-279.
* VQ decode matmul -- closed form (decode, then dense matmul in numpy);
  the bundled VQ runtime is not in the reference, so bit-level parity with
  it is unpinned.  The packed field order (LSB first in a little-endian
  word stream) is pinned against an independent bit-by-bit writer; that the
  bundled runtime reads the same order is unpinned (it is not vendored).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

_lib = None


def build() -> Path:
    """Compile oracle.c into liboracle.so (gcc + OpenMP)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.orc_quantize_affine.argtypes = [P, I64, I64, I, I, P, P, P]
        L.orc_dequantize_affine.argtypes = [P, P, P, I64, I64, I, I, I, I, P]
        L.orc_qmm.argtypes = [P, I64, I64, I64, P, P, P, I, I, I, P, I]
        L.orc_kv8_decode.argtypes = [P, I64, I64, I64, I64, P, P, P, P, P, P,
                                     I64, I64, I, I, ctypes.c_float, P, P, I]
        L.orc_vq_matmul.argtypes = [P, I64, I64, I64, P, I, P, I64, I, P,
                                    I64, P, I]
        for f in ("orc_quantize_affine", "orc_dequantize_affine", "orc_qmm",
                  "orc_kv8_decode", "orc_vq_matmul"):
            getattr(L, f).restype = None
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def threads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


# --- exact dtype rounding (float32 <-> bf16 / fp16 bit patterns) ------------

DTYPES = ("bfloat16", "float16", "float32")


def bf16_round(a) -> np.ndarray:
    """float32 -> nearest-even bfloat16, kept as float32."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).copy()
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    u = np.where(nan, u | 0x00400000,
                 u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1)))
    return (u & np.uint32(0xFFFF0000)).astype(np.uint32).view(np.float32)


def f16_round(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(a, dtype: str) -> np.ndarray:
    if dtype == "bfloat16":
        return bf16_round(a)
    if dtype == "float16":
        return f16_round(a)
    return np.asarray(a, dtype=np.float32)


def bf16_bits(a) -> np.ndarray:
    """float32 holding bf16 values -> uint16 bit patterns."""
    return (bf16_round(a).view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(u) -> np.ndarray:
    return (np.asarray(u, np.uint16).astype(np.uint32) << 16).view(np.float32)


# --- affine quantize / dequantize / quantized_matmul -------------------------

def quantize(w, group_size: int = 64, bits: int = 4, dtype: str = "bfloat16"):
    """mx.quantize(w, group_size, bits, mode="affine") on the last axis.
    ``w`` holds the values of a ``dtype`` tensor.  Returns (wq uint32,
    scales, biases) with scales/biases rounded to ``dtype``, as float32."""
    w = _f32(w)
    shp = w.shape
    cols = shp[-1]
    if cols % group_size or (cols * bits) % 32 or bits not in (2, 3, 4, 5, 6, 8):
        raise ValueError("last axis must divide by the group and pack in 32 bits")
    rows = int(np.prod(shp[:-1], dtype=np.int64))
    wq = np.zeros((rows, cols * bits // 32), np.uint32)
    s = np.zeros((rows, cols // group_size), np.float32)
    b = np.zeros((rows, cols // group_size), np.float32)
    lib().orc_quantize_affine(_p(w), rows, cols, group_size, bits, _p(wq), _p(s), _p(b))
    tail = shp[:-1]
    return (wq.reshape(*tail, -1), round_to(s, dtype).reshape(*tail, -1),
            round_to(b, dtype).reshape(*tail, -1))


ROUND_OP_BY_OP = 0
ROUND_FUSED = 1


def dequantize(wq, scales, biases, group_size: int = 64, bits: int = 4,
               dtype: str = "bfloat16", rounding: int = ROUND_OP_BY_OP):
    """mx.dequantize(...) -> values of ``dtype`` (as float32).  ``rounding``
    selects T(T(s*q)+b) (0, default) or T(fma(s, q, b)) (1)."""
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    s, b = _f32(scales), _f32(biases)
    cols = wq.shape[-1] * 32 // bits
    rows = int(np.prod(wq.shape[:-1], dtype=np.int64))
    out = np.zeros((rows, cols), np.float32)
    lib().orc_dequantize_affine(_p(wq), _p(s), _p(b), rows, cols, group_size,
                                bits, DTYPES.index(dtype), rounding, _p(out))
    return out.reshape(*wq.shape[:-1], cols)


def unpack_numpy(wq, bits: int) -> np.ndarray:
    """The integer codes of packed words, written independently of the C
    oracle (vectorised shifts) -- the cross-check of the packing order.
    Widths that do not divide 32 read the row's little-endian bit stream
    (``unpack_fields``)."""
    wq = np.asarray(wq, np.uint32)
    if 32 % bits:
        return unpack_fields(wq, bits, wq.shape[-1] * 32 // bits)
    epw = 32 / bits
    epw = int(epw)
    shifts = (np.arange(epw, dtype=np.uint32) * bits)
    q = (wq[..., :, None] >> shifts) & np.uint32((1 << bits) - 1)
    return q.reshape(*wq.shape[:-1], wq.shape[-1] * epw)


def dequantize_numpy_f64(wq, scales, biases, group_size: int, bits: int):
    """s*q+b in float64, the exact dequantized weight (numpy, independent
    of the C code)."""
    q = unpack_numpy(wq, bits).astype(np.float64)
    s = np.repeat(np.asarray(scales, np.float64), group_size, axis=-1)
    b = np.repeat(np.asarray(biases, np.float64), group_size, axis=-1)
    return s * q + b


def quantized_matmul(x, wq, scales, biases, transpose: bool = True,
                     group_size: int = 64, bits: int = 4, out_dtype: str = "bfloat16",
                     nthreads: int = 0):
    """mx.quantized_matmul for a 2-D weight: exact product, rounded once to
    ``out_dtype``.  x [..., K]."""
    x = _f32(x)
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    s, b = _f32(scales), _f32(biases)
    K = x.shape[-1]
    M = int(np.prod(x.shape[:-1], dtype=np.int64))
    if transpose:
        N = wq.shape[0]
        assert wq.shape[1] * 32 // bits == K
    else:
        N = wq.shape[1] * 32 // bits
        assert wq.shape[0] == K
    y = np.zeros((M, N), np.float32)
    lib().orc_qmm(_p(x), M, K, N, _p(wq), _p(s), _p(b), group_size, bits,
                  int(bool(transpose)), _p(y), nthreads or threads())
    return round_to(y, out_dtype).reshape(*x.shape[:-1], N)


def gather_qmm(x, wq, scales, biases, lhs_indices=None, rhs_indices=None,
               transpose: bool = True, group_size: int = 64, bits: int = 4,
               out_dtype: str = "bfloat16"):
    """mx.gather_qmm (reached through QuantizedSwitchLinear,
    .../_mlx_vlm/models/switch_layers.py:71-86): x [..., M, K], w
    [E, N, K*bits/32]; out[i] = x[lhs[i]] @ What[rhs[i]]^T with lhs/rhs
    broadcast together; lhs defaults to each batch element of x.
    Computed one expert at a time (rows grouped by expert)."""
    x = _f32(x)
    wq = np.asarray(wq, np.uint32)
    M, K = x.shape[-2], x.shape[-1]
    xb = x.reshape(-1, M, K)
    xbatch = x.shape[:-2]
    if lhs_indices is None:
        lhs_indices = np.arange(int(np.prod(xbatch, dtype=np.int64))).reshape(xbatch)
    if rhs_indices is None:
        rhs_indices = np.arange(wq.shape[0]).reshape(wq.shape[:-2])
    lhs, rhs = np.broadcast_arrays(np.asarray(lhs_indices), np.asarray(rhs_indices))
    ishape = lhs.shape
    lhs, rhs = lhs.reshape(-1), rhs.reshape(-1)
    N = wq.shape[-2] if transpose else wq.shape[-1] * 32 // bits
    out = np.zeros((lhs.size, M, N), np.float32)
    for e in np.unique(rhs):
        sel = np.nonzero(rhs == e)[0]
        xs = xb[lhs[sel]].reshape(-1, K)
        y = quantized_matmul(xs, wq[e], scales[e], biases[e], transpose,
                             group_size, bits, "float32")
        out[sel] = y.reshape(sel.size, M, N)
    return round_to(out, out_dtype).reshape(*ishape, M, N)


def quantized_matmul_batched(x, wq, scales, biases, transpose: bool = True,
                             group_size: int = 64, bits: int = 4,
                             out_dtype: str = "bfloat16"):
    """mx.quantized_matmul with batch dimensions on w, broadcast against
    x's (numpy broadcasting of x [..., M, K] and w [..., R, C]); each batch
    entry is the 2-D ``quantized_matmul`` above (exact product rounded once).
    The products of mlx-lm's quantized attention
    (.../_mlx_vlm/models/base.py:281-297) and of QuantizedMultiLinear
    (.../_mlx_vlm/models/mla.py:80-87).  Pinned by on-grid weights packed
    independently (tests/test_oracle.py)."""
    x = _f32(x)
    wq = np.asarray(wq, np.uint32)
    s, b = _f32(scales), _f32(biases)
    M, K = x.shape[-2], x.shape[-1]
    batch = np.broadcast_shapes(x.shape[:-2], wq.shape[:-2])
    xb = np.broadcast_to(x, batch + (M, K)).reshape(-1, M, K)
    wb = np.broadcast_to(wq, batch + wq.shape[-2:]).reshape(-1, *wq.shape[-2:])
    sb = np.broadcast_to(s, batch + s.shape[-2:]).reshape(-1, *s.shape[-2:])
    bb = np.broadcast_to(b, batch + b.shape[-2:]).reshape(-1, *b.shape[-2:])
    N = wq.shape[-2] if transpose else wq.shape[-1] * 32 // bits
    out = np.zeros((xb.shape[0], M, N), np.float32)
    for i in range(xb.shape[0]):
        out[i] = quantized_matmul(xb[i], wb[i], sb[i], bb[i], transpose, group_size, bits,
                                  "float32", nthreads=1)
    return round_to(out, out_dtype).reshape(*batch, M, N)


#: mx.finfo(mx.bfloat16).min, what a hidden score becomes
BF16_LOWEST = -3.3895313892515355e38


def align_mask(mask, ndim: int):
    """align_attention_mask_to_scores (.../_mlx_vlm/models/base.py:242-257):
    size-1 axes inserted before the last two until the ranks match."""
    m = np.asarray(mask)
    while m.ndim < ndim:
        m = np.expand_dims(m, max(m.ndim - 2, 0))
    return m


def quantized_sdpa(q, K, V, scale: float, mask=None, group_size: int = 64, bits: int = 8):
    """mlx-lm's quantized_scaled_dot_product_attention
    (.../_mlx_vlm/models/base.py:260-302) in bfloat16: q *= scale (rounded),
    scores = quantized_matmul(q, K, transpose=True) (rounded), a bool mask
    puts finfo(bf16).min where it is False, an additive mask is added
    (rounded), "causal" keeps key j for query l of L when j <= N - L + l;
    softmax(precise=True) in float32, probabilities rounded; out =
    quantized_matmul(p, V, transpose=False) (rounded).  q [B, Hq, L, D]; K,
    V = (packed, scales, biases) of [B, Hk, N, *].  Pinned against
    ``sdpa_numpy_f64`` and by the uniform softmax of a fully hidden row
    (tests/test_oracle.py)."""
    q = _f32(q)
    B, Hq, L, D = q.shape
    Hk = np.asarray(K[0]).shape[-3]
    rep = Hq // Hk
    # mlx casts the Python scalar to the queries' dtype before `queries *= scale`
    qs = bf16_round(q * bf16_round(np.float32(scale)))
    Ke, Ve = tuple(K), tuple(V)
    if rep > 1:
        qs = qs.reshape(B, Hk, rep, L, D)
        Ke = tuple(np.expand_dims(np.asarray(t), -3) for t in Ke)
        Ve = tuple(np.expand_dims(np.asarray(t), -3) for t in Ve)
    scores = quantized_matmul_batched(qs, *Ke, True, group_size, bits, "bfloat16")
    N = scores.shape[-1]
    if mask is not None:
        if isinstance(mask, str):
            m = np.arange(N - L, N)[:, None] >= np.arange(N)[None]
        else:
            m = align_mask(mask, scores.ndim)
        if m.dtype == bool:
            scores = np.where(m, scores, np.float32(BF16_LOWEST)).astype(np.float32)
        else:
            scores = bf16_round((scores + _f32(m)).astype(np.float32))
    mx = scores.max(axis=-1, keepdims=True)
    e = np.exp((scores - mx).astype(np.float32))
    p = bf16_round((e / e.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32))
    out = quantized_matmul_batched(p, *Ve, False, group_size, bits, "bfloat16")
    return out.reshape(B, Hq, L, -1)


# --- the scaled (microscaling) modes -------------------------------------------

#: OCP MX FP4 (E2M1) magnitudes of codes 0..7 (the spec's table); bit 3 is the sign
E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def e4m3(codes) -> np.ndarray:
    """OCP MX FP8 E4M3 (bias 7, no infinities, S.1111.111 = NaN) -> float64."""
    c = np.asarray(codes, np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 15
    m = (c & 7).astype(np.float64)
    v = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    v = np.where((e == 15) & (m == 7), np.nan, v)
    return s * v


def e8m0(scales) -> np.ndarray:
    """OCP MX E8M0 scale: 2^(e - 127); 255 is NaN."""
    e = np.asarray(scales, np.int64)
    return np.where(e == 255, np.nan, np.exp2(e - 127.0))


def mx_dequantize(wq, scales, mode: str) -> np.ndarray:
    """mx.dequantize(mode="mxfp4" | "mxfp8") in float64: codes packed as mlx
    packs 4 / 8-bit codes (``unpack_numpy``), one uint8 E8M0 scale per 32.
    The scaled modes of the reference's loader (engine/model/packed.py:20,
    load_model.py:153-173).  Pinned by the spec's known answers."""
    bits = 4 if mode == "mxfp4" else 8
    q = unpack_numpy(wq, bits).astype(np.int64)
    if mode == "mxfp4":
        v = np.where(q & 8, -1.0, 1.0) * E2M1[q & 7]
    else:
        v = e4m3(q)
    return v * np.repeat(e8m0(scales), 32, axis=-1)


def mx_quantize(w, mode: str):
    """mx.quantize(w, group_size=32, mode="mxfp4" | "mxfp8") per the OCP MX
    scheme: per group of 32, X = floor(log2 max|w|) - emax (emax 2 for E2M1,
    8 for E4M3), E8M0 byte X + 127 (clamped to 0..254; an all-zero group
    takes 0), elements w / 2^X rounded to nearest (ties to the even code)
    and saturated to the largest finite element, the input's sign kept
    (negative zeros included).  -> (wq uint32, scales uint8).

    Parity unpinned: this is the OCP MX v1.0 conversion, and mlx's own
    quantizer is not in the reference tree.  The reference's mxfp4
    checkpoint holds random codes under random scales, all on the grid, so
    re-quantizing it checks only the shared exponent of groups whose
    largest code is 4 or 6 -- not ties, saturation or the sign of zero;
    those are checked against hand-computed codes (tests/test_oracle.py)."""
    w = np.asarray(w, np.float64)
    rows = w.reshape(-1, w.shape[-1])
    G = rows.shape[1] // 32
    g = rows.reshape(rows.shape[0], G, 32)
    amax = np.abs(g).max(-1)
    emax, bits = (2, 4) if mode == "mxfp4" else (8, 8)
    with np.errstate(divide="ignore"):
        X = np.floor(np.log2(np.where(amax > 0, amax, 1.0))) - emax
    e = np.clip(np.where(amax > 0, X + 127, 0), 0, 254).astype(np.int64)
    v = g / np.exp2(e - 127.0)[..., None]
    if mode == "mxfp4":
        grid = E2M1
    else:
        grid = e4m3(np.arange(127))                 # codes 0..126: every finite magnitude
    mag = np.abs(v)
    # nearest grid value, ties to the even code; past the top: the top code
    idx = np.searchsorted(grid, mag)                 # first grid value >= mag
    idx = np.clip(idx, 1, len(grid) - 1)
    lo, hi = grid[idx - 1], grid[idx]
    pick_hi = (mag - lo > hi - mag) | ((mag - lo == hi - mag) & (idx % 2 == 0))
    code = np.where(pick_hi, idx, idx - 1)
    code = np.where(mag >= grid[-1], len(grid) - 1, code)
    # the input's sign is kept on every code, zero included (-0 is code 8 /
    # 0x80): the reference's checkpoint holds such negative zeros
    code = code | np.where(np.signbit(v), 8 if mode == "mxfp4" else 0x80, 0)
    codes = code.reshape(rows.shape[0], -1).astype(np.uint32)
    epw = 32 // bits
    q = codes.reshape(rows.shape[0], -1, epw)
    words = np.zeros(q.shape[:2], np.uint32)
    for i in range(epw):
        words |= q[..., i] << np.uint32(bits * i)
    tail = w.shape[:-1]
    return words.reshape(*tail, -1), e.astype(np.uint8).reshape(*tail, -1)


def mx_quantized_matmul(x, wq, scales, mode: str, transpose: bool = True,
                        out_dtype: str = "bfloat16"):
    """mx.quantized_matmul(mode=mxfp4 | mxfp8) for a 2-D weight: the exact
    product in float64, rounded once."""
    w = mx_dequantize(wq, scales, mode)
    y = np.asarray(x, np.float64) @ (w.T if transpose else w)
    return round_to(y.astype(np.float32), out_dtype)


# --- the Qwen3.5-MoE router, SwiGLU and SwitchGLU ----------------------------

def route(logits, k: int, out_dtype: str = "bfloat16"):
    """SparseMoeBlock's router (src/knurlogic/engine/families/qwen/
    architecture/qwen3_5.py:174-179): ``probs = mx.softmax(logits.astype(
    float32))``, top-k, ``scores / scores.sum()`` in float32, rounded to the
    logits' dtype.

    The softmax follows mlx 0.32.3's CPU kernel for a float32 row
    (mlx/backend/cpu/softmax.cpp, ``softmax<float, float>``), one float32
    rounding per step: m = max(x); e_i = exp(x_i - m); n = sum(e); r = 1/n
    (the normaliser is inverted once); p_i = e_i * r.  The renormalisation
    is two float32 array ops: t = sum of the k selected p, score = p / t.
    Two parts are fixed here where mlx's own code cannot be matched bit for
    bit without it: exp is the correctly rounded float32 exp (mlx uses its
    SIMD polynomial, within a few ulp), and both sums are the exact sum
    rounded once to float32 (mlx adds in SIMD-lane order).  Differences of
    an ulp or two in float32 reach the rounded scores at a bf16 / fp16
    rounding boundary, and they can also reorder two probabilities that lie
    within those ulps of each other and so change which expert is selected:
    top-k membership at such near-ties (and at exact ties, which mlx's
    argpartition breaks in its own order) is parity unpinned.  Here the
    top-k set follows the rounded probabilities; ties go to the lower
    expert index.
    Returns (inds [T, k] int32 in descending-probability order, scores)."""
    x = np.asarray(logits, np.float32)
    m = x.max(axis=-1, keepdims=True)
    e = np.exp((x - m).astype(np.float64)).astype(np.float32)
    n = e.astype(np.float64).sum(axis=-1, keepdims=True).astype(np.float32)
    r = np.float32(1.0) / n
    p = e * r
    # stable descending order: larger prob first, lower index on ties
    order = np.argsort(-p, axis=-1, kind="stable")[..., :k]
    top = np.take_along_axis(p, order, axis=-1)
    t = top.astype(np.float64).sum(axis=-1, keepdims=True).astype(np.float32)
    return order.astype(np.int32), round_to(top / t, out_dtype)


def silu_rounded(g, dtype: str = "bfloat16"):
    """_silu: silu in float32, rounded once to the input dtype
    (qwen3_5.py:39-40, vendored edit 8)."""
    g64 = np.asarray(g, np.float64)
    return round_to((g64 / (1.0 + np.exp(-g64))).astype(np.float32), dtype)


def sigmoid_rounded(g, dtype: str = "bfloat16"):
    """_sigmoid (qwen3_5.py:35-36)."""
    g64 = np.asarray(g, np.float64)
    return round_to((1.0 / (1.0 + np.exp(-g64))).astype(np.float32), dtype)


def swiglu(up, gate, dtype: str = "bfloat16"):
    """_SwiGLU: _silu(gate) * up, the product rounded to dtype
    (qwen3_5.py:108-112)."""
    return round_to(silu_rounded(gate, dtype) * np.asarray(up, np.float32), dtype)


def switch_glu(x, inds, gate_fn, up_fn, down_fn, dtype: str = "bfloat16"):
    """SwitchGLU.__call__ (.../_mlx_vlm/models/switch_layers.py:172-193) with
    the _SwiGLU activation: per (token, slot) the expert's gate and up
    projections (each rounded to dtype), the activation, and the down
    projection (rounded).  ``*_fn(x_rows [R, K], expert) -> [R, N]`` float32
    values already rounded to dtype.  Sorting only reorders rows, so the
    result is the same sorted or not.  Returns [T, k, H]."""
    x = np.asarray(x, np.float32)
    T, H = x.shape
    kk = inds.shape[-1]
    flat = inds.reshape(-1)
    out = None
    for e in np.unique(flat):
        sel = np.nonzero(flat == e)[0]
        xs = x[sel // kk]
        a = swiglu(up_fn(xs, e), gate_fn(xs, e), dtype)
        d = down_fn(a, e)
        if out is None:
            out = np.zeros((T * kk, d.shape[-1]), np.float32)
        out[sel] = d
    return out.reshape(T, kk, -1)


def combine(y, scores, dtype: str = "bfloat16"):
    """(y * scores[..., None]).sum(-2) (qwen3_5.py:182): each product rounded
    to dtype, the k products summed in float32 and rounded once."""
    prod = round_to(np.asarray(y, np.float32) * np.asarray(scores, np.float32)[..., None], dtype)
    return round_to(prod.astype(np.float64).sum(axis=-2).astype(np.float32), dtype)


def dense_linear(x, w, dtype: str = "bfloat16"):
    """A dtype linear layer x @ w^T, exact sum rounded once."""
    return round_to((np.asarray(x, np.float64) @ np.asarray(w, np.float64).T)
                    .astype(np.float32), dtype)


def moe_block(x, gate_w, expert_fns, shared=None, k: int = 8, dtype: str = "bfloat16"):
    """SparseMoeBlock.__call__ (qwen3_5.py:170-192): router, SwitchGLU,
    weighted combine, plus the sigmoid-gated shared expert when ``shared``
    = (gate_w, up_w, down_w, shared_gate_w) is given (dense dtype weights).
    x [T, H]."""
    logits = dense_linear(x, gate_w, dtype)
    inds, scores = route(logits, k, dtype)
    y = switch_glu(x, inds, *expert_fns, dtype=dtype)
    y = combine(y, scores, dtype)
    if shared is not None:
        sg, su, sd, sgate = shared
        a = round_to(silu_rounded(dense_linear(x, sg, dtype), dtype)
                     * dense_linear(x, su, dtype), dtype)
        sy = dense_linear(a, sd, dtype)
        sy = round_to(sigmoid_rounded(dense_linear(x, sgate, dtype), dtype) * sy, dtype)
        y = round_to(y + sy, dtype)
    return y


# --- 8-bit-KV decode attention -----------------------------------------------

def mask_rows(mask, B: int, L: int, N: int):
    """kvattn._mask_rows (src/knurlogic/engine/kvattn.py:241-253): (B, L, N)
    bool, or None when every key is visible.  ``mask`` is None, "causal" or
    a bool array broadcastable to (B, 1, L|1, N) / (B, L|1, N)."""
    if mask is None or (isinstance(mask, str) and L == 1):
        return None
    if isinstance(mask, str):
        rows = np.arange(N - L, N)[:, None]
        m = rows >= np.arange(N)[None]
        return np.broadcast_to(m[None], (B, L, N)).copy()
    m = np.asarray(mask, bool)
    if m.ndim == 4:
        m = m[:, 0]
    while m.ndim < 3:
        m = m[None]
    return np.broadcast_to(m, (B, L, N)).copy()


def kv8_decode(q, K, V, scale: float, mask=None, group: int = 64, bits: int = 8,
               out_dtype: str = "bfloat16"):
    """kvattn.decode_sdpa's result (exact arithmetic, see oracle.c).
    q [B, H, L, D] values; K, V = (packed, scales, biases) of [B, Hk, N, *]."""
    q = _f32(q)
    B, H, L, D = q.shape
    kw, ks, kb = (np.ascontiguousarray(K[0], np.uint32), _f32(K[1]), _f32(K[2]))
    vw, vs, vb = (np.ascontiguousarray(V[0], np.uint32), _f32(V[1]), _f32(V[2]))
    Hk, N = kw.shape[1], kw.shape[2]
    m = mask_rows(mask, B, L, N)
    mp = None
    if m is not None:
        m8 = np.ascontiguousarray(m, np.uint8)
        mp = _p(m8)
    out = np.zeros((B, H, L, D), np.float32)
    lib().orc_kv8_decode(_p(q), B, H, L, D, _p(kw), _p(ks), _p(kb), _p(vw), _p(vs),
                         _p(vb), Hk, N, group, bits, float(scale), mp, _p(out),
                         threads())
    return round_to(out, out_dtype)


def sdpa_numpy_f64(q, k, v, scale: float, mask=None):
    """Plain float64 attention over dense k/v (numpy, independent of the C
    code): softmax(q k^T * scale) v per head with GQA; masked rows whose
    every key is masked give 0 (the reference kernel's rule)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, H, L, D = q.shape
    Hk, N = k.shape[1], k.shape[2]
    rep = H // Hk
    m = mask_rows(mask, B, L, N)
    out = np.zeros((B, H, L, v.shape[-1]))
    for h in range(H):
        s = np.einsum("bld,bnd->bln", q[:, h], k[:, h // rep]) * scale
        if m is not None:
            s = np.where(m, s, -np.inf)
        mx = s.max(axis=-1, keepdims=True)
        ok = np.isfinite(mx)
        p = np.where(ok, np.exp(s - np.where(ok, mx, 0.0)), 0.0)
        den = p.sum(axis=-1, keepdims=True)
        o = np.einsum("bln,bnd->bld", p, v[:, h // rep])
        out[:, h] = np.where(den > 0, o / np.where(den > 0, den, 1.0), 0.0)
    return out


# --- VQ codebook-decode expert matmul ----------------------------------------

def vq_matmul(x, codes, codebook, scales, scale_group: int = 0,
              out_dtype: str = "bfloat16"):
    """One VQ expert matrix: y = x @ What^T with What[o, i] =
    scale[o, i/scale_group] * codebook[codes[o, i/dim]][i % dim].
    ``scale_group`` 0 means one scale per output channel."""
    x = _f32(x)
    codes = np.ascontiguousarray(codes)
    cb = _f32(codebook)
    kc, dim = cb.shape
    OUT = codes.shape[0]
    IN = codes.shape[1] * dim
    sg = scale_group or IN
    s = _f32(scales).reshape(OUT, IN // sg)
    M = int(np.prod(x.shape[:-1], dtype=np.int64))
    y = np.zeros((M, OUT), np.float32)
    cbytes = codes.dtype.itemsize
    assert cbytes in (1, 2)
    lib().orc_vq_matmul(_p(x), M, IN, OUT, _p(codes), cbytes, _p(cb), kc, dim,
                        _p(s), sg, _p(y), threads())
    return round_to(y, out_dtype).reshape(*x.shape[:-1], OUT)


def unpack_fields(words, pack_bits: int, nfields: int) -> np.ndarray:
    """The packed on-disk VQ code layout (.../heads/deepseek_v4.py:36-44,
    95-129): field j of a row at bits [j*b, j*b + b) of the row's uint32
    words read as one little-endian bit stream; ceil(nfields/32) * b words
    per row.  -> uint16 codes [..., nfields].  Pinned against a bit-by-bit
    Python writer (tests/test_oracle.py)."""
    w = np.ascontiguousarray(words, np.uint32)
    lead = w.shape[:-1]
    w2 = w.reshape(-1, w.shape[-1]).astype(np.uint64)
    j = np.arange(nfields, dtype=np.uint64)
    off = j * np.uint64(pack_bits)
    q = (off >> np.uint64(5)).astype(np.int64)
    sh = off & np.uint64(31)
    lo = w2[:, q] >> sh
    nxt = np.minimum(q + 1, w2.shape[1] - 1)
    hi = np.where(sh + np.uint64(pack_bits) > np.uint64(32),
                  w2[:, nxt] << (np.uint64(32) - sh), np.uint64(0))
    mask = np.uint64((1 << pack_bits) - 1)
    return ((lo | hi) & mask).astype(np.uint16).reshape(*lead, nfields)


def vq_packed_matmul(x, words, codebook, scales, pack_bits: int, group: int,
                     out_dtype: str = "bfloat16"):
    """One VQ expert matrix in the packed layout: the fields unpacked, then
    ``vq_matmul`` with per-group scales [OUT, IN / group]."""
    cb = np.asarray(codebook)
    dim = cb.shape[1]
    IN = np.asarray(scales).shape[-1] * group
    codes = unpack_fields(words, pack_bits, IN // dim)
    return vq_matmul(x, codes, cb, scales, group, out_dtype)


def vq_decode_numpy(codes, codebook, scales, scale_group: int = 0):
    """The dense weight of a VQ matrix, float64 (numpy, independent of C)."""
    cb = np.asarray(codebook, np.float64)
    kc, dim = cb.shape
    OUT, C = codes.shape
    w = cb[np.asarray(codes, np.int64)].reshape(OUT, C * dim)
    IN = C * dim
    sg = scale_group or IN
    s = np.repeat(np.asarray(scales, np.float64).reshape(OUT, IN // sg), sg, axis=-1)
    return s * w
