"""Decode attention read straight from an 8-bit KV cache, on MI355X.

Mirrors the reference's src/knurlogic/engine/kvattn.py: ``decode_sdpa``
(:256-291) computes mlx-sdpa semantics over the quantized (packed, scales,
biases) triples -- q pre-scaled, softmax over the keys a row may see -- with
one HIP kernel over the packed K/V (kmi_kv8_decode) instead of
dequantizing the cache; ``supports`` (:213-238) is the routing rule;
``sdpa`` (:301-320) is the dispatch a model's attention calls once
``patch_model`` (:323-339) has rebound it; ``STATS`` counts hits and misses
(:25-53); ``ENV`` / ``enabled`` (:69-75) switch the kernel.

Off the kernel, ``sdpa`` never computes attention in torch:
  * quantized K/V -- a cache with a ``bits`` attribute (mlx-lm's own), or
    the ``LazyDequant`` views this library's caches return (6 / 4-bit
    caches, queries longer than the kernel takes, masks it does not take)
    -- go through ``quantized_sdpa``, mlx-lm's quantized attention
    (.../_mlx_vlm/models/base.py:260-302) over the packed triples: three
    HIP launches, no dequantized copy of the cache;
  * dense K/V go to the model's own attention function, the one
    ``patch_model`` found and replaced (the reference likewise hands them
    to mlx-lm's base function).

A query row whose every key is masked returns 0 in the kernel (the
reference kernel's rule, :11-12), where a plain softmax would give NaN.
"""
from __future__ import annotations

import logging
import os
import sys

import torch

from . import _abi
from .ops import DTYPE_CODE, _on_gpu, _ptr, _stream, padded_rows, qmm_batched, row_padded

logger = logging.getLogger(__name__)

#: {on, hits, misses, last_miss}
STATS: dict = {"on": True, "hits": 0, "misses": 0, "last_miss": None}
_LOGGED: set = set()

#: query rows per KV head (GQA ratio x query length) the kernel takes
MAX_ROWS = 64

#: the kernel's on/off switch, the reference's knob (engine/kvattn.py:69):
#: unset or any other value is on
ENV = "KNURLOGIC_KV_KERNEL"
_OFF = ("0", "off", "false", "no", "disable", "disabled")

#: the model's own attention function that patch_model replaced: dense K/V
#: go back to it
_BASE: dict = {"fn": None}


def enabled() -> bool:
    """Whether the 8-bit decode kernel may be used (``ENV`` not off)."""
    return os.environ.get(ENV, "").strip().lower() not in _OFF


def reset(on: bool = True) -> None:
    STATS.update(on=bool(on), hits=0, misses=0, last_miss=None)
    _LOGGED.clear()


def count(hit: bool, why: str = "") -> None:
    """Tally one dispatch in ``STATS``: ``hit`` when the 8-bit kernel ran,
    else a miss with its reason.  The first hit and the first miss are
    logged once per ``reset``."""
    if hit:
        STATS["hits"] += 1
    else:
        STATS["misses"] += 1
        STATS["last_miss"] = why
    if hit not in _LOGGED:
        _LOGGED.add(hit)
        if hit:
            logger.info("8-bit KV decode kernel in use (kmi_kv8_decode on the packed cache)")
        else:
            logger.warning("8-bit KV decode kernel not taken for a step, fallback path "
                           "instead (%s)", why)


def _dims(q, K, V, bits):
    B, H, L, D = q.shape
    Hk = K[0].shape[1]
    Dk = K[0].shape[3] * 32 // bits
    Dv = V[0].shape[3] * 32 // bits
    return B, H, L, D, Hk, Dk, Dv


def supports(q, K, V, bits: int, group: int, mask=None, sinks=None) -> bool:
    """Whether ``decode_sdpa`` takes these shapes (else the caller falls
    back to dequantize + sdpa).  The rule of kvattn.supports
    (engine/kvattn.py:213-239): head dims 128, 256, 384 and 512, up to 64
    query rows per KV head, groups dividing D -- here multiples of 16, where
    the reference takes multiples of D/32, which adds groups of 4 and 8 that
    mlx's quantize does not make -- plus the last-axis-contiguous triples
    and matching scale/bias dtypes the C ABI reads."""
    if bits != 8 or sinks is not None or q.dim() != 4:
        return False
    B, H, L, D, Hk, Dk, Dv = _dims(q, K, V, bits)
    if Dk != D or Dv != D or D % 128 or D > 512 or H % Hk:
        return False
    # a lane's 16-d run of a key row lies in one group
    if group <= 0 or D % group or group % 16 or K[0].shape[0] != B:
        return False
    for w, sc, bi in (K, V):
        if sc.shape != bi.shape or tuple(sc.shape[:3]) != tuple(w.shape[:3]):
            return False
        if w.stride(-1) != 1 or sc.stride(-1) != 1 or bi.stride(-1) != 1:
            return False
        if sc.dtype != K[1].dtype or bi.dtype != K[1].dtype:
            return False
    R = (H // Hk) * L
    if R > MAX_ROWS:
        return False
    if q.dtype not in DTYPE_CODE or K[1].dtype not in DTYPE_CODE:
        return False
    if mask is None or isinstance(mask, str):
        return mask in (None, "causal")
    if mask.dtype != torch.bool or mask.dim() > 4:
        return False
    if mask.dim() == 4 and mask.shape[1] != 1:
        return False
    return mask.shape[-1] == K[0].shape[2] and mask.shape[-2] in (1, L)


def _mask_rows(mask, B, L, N, device):
    """kvattn._mask_rows: (B, L, N) uint8, or None when every key is visible
    or the causal rule is applied in the kernel."""
    if mask is None or isinstance(mask, str):
        return None
    m = mask
    if m.dim() == 4:
        m = m[:, 0]
    while m.dim() < 3:
        m = m[None]
    return m.expand(B, L, N).to(device=device, dtype=torch.uint8).contiguous()


def decode_sdpa(q, K, V, scale: float, mask=None, group: int = 64, bits: int = 8,
                same_layout: bool = False):
    """Attention of q (B, H, L, D) over K, V -- each the quantized triple
    (packed uint32, scales, biases) of shape (B, Hk, N, *), possibly strided
    views -- with mlx sdpa's semantics.  Returns (B, H, L, D) in q's dtype.
    ``same_layout`` is accepted for signature parity: biases are always
    read at their own strides."""
    if bits != 8:
        raise ValueError("decode_sdpa: 8-bit K/V only")
    _on_gpu(q, *K, *V)
    if not supports(q, K, V, bits, group, mask):
        raise ValueError(f"decode_sdpa: unsupported shapes q {tuple(q.shape)}, "
                         f"K {tuple(K[0].shape)}, mask {getattr(mask, 'shape', mask)}")
    B, H, L, D, Hk, _, _ = _dims(q, K, V, bits)
    N = K[0].shape[2]
    q = q.contiguous()
    out = torch.empty_like(q)
    m = _mask_rows(mask, B, L, N, q.device)
    causal = 1 if (isinstance(mask, str) and mask == "causal" and L > 1) else 0
    strides = []
    for t in (*K, *V):
        strides += [t.stride(0), t.stride(1), t.stride(2)]
    st = torch.tensor(strides, dtype=torch.int64)      # host array, read by the launcher
    L_ = _abi.load()
    nbytes = L_.kmi_kv8_workspace_bytes(B, H, Hk, L, N, D)
    ws = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=q.device)
    _abi.check(L_.kmi_kv8_decode(
        _ptr(q), DTYPE_CODE[q.dtype], B, H, L, D,
        _ptr(K[0]), _ptr(K[1]), _ptr(K[2]), _ptr(V[0]), _ptr(V[1]), _ptr(V[2]),
        st.data_ptr(), DTYPE_CODE[K[1].dtype], Hk, N, group, float(scale),
        _ptr(m), causal, _ptr(out), _ptr(ws), nbytes, _stream(q)), "kv8_decode")
    return out


#: KMI_MASK_* of include/knurlogic_amd.h
MASK_NONE, MASK_BOOL, MASK_ADD, MASK_CAUSAL = 0, 1, 2, 3


def align_mask(mask, ndim: int):
    """mlx-lm's align_attention_mask_to_scores (.../_mlx_vlm/models/
    base.py:242-257): size-1 axes inserted just before the last two until
    the mask has the scores' rank, so a (B, 1, L, N) batch mask does not
    alias B with the KV heads of (B, Hk, rep, L, N) scores."""
    if mask is None or isinstance(mask, str):
        return mask
    while mask.dim() < ndim:
        mask = mask.unsqueeze(max(mask.dim() - 2, 0))
    return mask


def masked_softmax(scores, mask=None, out=None):
    """The step between mlx-lm's two quantized attention products
    (base.py:285-295) on bf16 scores [..., L, N] (kmi_masked_softmax): a
    bool mask hides scores with finfo(bf16).min, a bf16 mask is added,
    "causal" hides key j from query row l when j > N - L + l; then
    softmax(precise=True), probabilities rounded to bf16.  The kernel reads
    and writes rows padded to 8 elements (``ops.padded_rows``); other
    layouts are copied.  ``out`` may be ``scores`` itself."""
    if scores.dtype != torch.bfloat16 or scores.dim() < 2 or scores.dim() > 5:
        raise ValueError("masked_softmax: bf16 scores [..., L, N] of 2 to 5 dimensions")
    _on_gpu(scores)
    if not row_padded(scores):
        src = padded_rows(tuple(scores.shape), scores.dtype, scores.device)
        src.copy_(scores)
        scores = src
    if out is None:
        out = padded_rows(tuple(scores.shape), scores.dtype, scores.device)
    elif not row_padded(out) or tuple(out.shape) != tuple(scores.shape) or out.dtype != scores.dtype:
        raise ValueError("masked_softmax: out must be a row-padded bf16 tensor of the scores' shape")
    lead = tuple(scores.shape[:-1])
    N = scores.shape[-1]
    dims = [1] * (4 - len(lead)) + list(lead)
    kind, mt, mstr = MASK_NONE, None, [0, 0, 0, 0]
    if isinstance(mask, str):
        if mask != "causal":
            raise ValueError(f"masked_softmax: mask {mask!r}")
        kind = MASK_CAUSAL
    elif mask is not None:
        _on_gpu(mask)
        if mask.dtype == torch.bool:
            kind = MASK_BOOL
        elif mask.dtype == torch.bfloat16:
            kind = MASK_ADD
        else:
            raise ValueError(f"masked_softmax: an additive mask must be bf16 like the scores (got {mask.dtype})")
        m = align_mask(mask, scores.dim())
        try:
            m = m.expand(*scores.shape)
        except RuntimeError as e:
            raise ValueError(f"masked_softmax: mask {tuple(mask.shape)} does not broadcast to "
                             f"scores {tuple(scores.shape)}") from e
        if m.stride(-1) != 1:
            m = m.contiguous()
        mt = m.view(torch.uint8) if kind == MASK_BOOL else m
        mstr = [0] * (4 - len(lead)) + [m.stride(d) for d in range(len(lead))]
    dt = torch.tensor(dims, dtype=torch.int64)
    ms = torch.tensor(mstr, dtype=torch.int64)
    _abi.check(_abi.load().kmi_masked_softmax(
        _ptr(scores), scores.stride(-2), DTYPE_CODE[scores.dtype], dt.data_ptr(), N, _ptr(mt), kind,
        ms.data_ptr(), _ptr(out), out.stride(-2), _stream(scores)), "masked_softmax")
    return out


def quantized_sdpa(queries, q_keys, q_values, scale: float, mask=None, group_size: int = 64,
                   bits: int = 8):
    """mlx-lm's quantized_scaled_dot_product_attention (.../_mlx_vlm/
    models/base.py:260-302) over quantized K/V triples (packed, scales,
    biases) of shape (B, Hk, N, *): q scaled by the scale rounded to q's
    dtype (mlx casts the scalar), the product rounded to bf16, scores =
    quantized_matmul(q, K, transpose=True) in bf16, masked, softmax(precise)
    in bf16, out = quantized_matmul(p, V, transpose=False).  GQA query heads
    share their KV head's triple (broadcast, never copied).  Three HIP
    launches (four when the keys are split across workgroups)."""
    B, Hq, L, D = queries.shape
    Hk = q_keys[0].shape[-3]
    if Hq % Hk:
        raise ValueError(f"quantized_sdpa: {Hq} query heads over {Hk} KV heads")
    rep = Hq // Hk
    q = queries
    Kt, Vt = tuple(q_keys), tuple(q_values)
    if rep > 1:
        q = q.reshape(B, Hk, rep, L, D)
        Kt = tuple(t.unsqueeze(-3) for t in Kt)
        Vt = tuple(t.unsqueeze(-3) for t in Vt)
    N = Kt[0].shape[-2]
    # scores, then probabilities in place, in rows padded to 8 elements
    buf = padded_rows(tuple(q.shape[:-1]) + (N,), q.dtype, q.device)
    # `queries *= scale` in mlx casts the Python scalar to the queries' dtype
    # first: q * bf16(scale), rounded to bf16 as x is staged
    qscale = float(torch.tensor(float(scale), dtype=torch.float32).to(q.dtype))
    scores = qmm_batched(q, *Kt, transpose=True, group_size=group_size, bits=bits, x_scale=qscale,
                         out=buf)
    p = masked_softmax(scores, mask, out=scores)
    out = qmm_batched(p, *Vt, transpose=False, group_size=group_size, bits=bits)
    return out.reshape(B, Hq, L, -1) if rep > 1 else out


def _packed(kv):
    """(triple, group, bits) of a quantized cache's LazyDequant view, else None."""
    from .kvcache import LazyDequant
    if isinstance(kv, LazyDequant):
        return kv.parts, kv.group, kv.bits
    return None


def sdpa(queries, keys, values, cache, scale, mask, sinks=None, base=None):
    """The dispatch a model's attention calls (kvattn.sdpa): the 8-bit
    kernel when ``cache`` just handed back exactly these keys for a short
    query (its ``kv8_fetch``); otherwise quantized K/V through
    ``quantized_sdpa`` on their packed triples, and dense K/V through
    ``base`` -- the calling module's own attention function, which the
    wrapper ``patch_model`` installed passes in -- or, for a direct call,
    the first attention function the last ``patch_model`` replaced."""
    hit = getattr(cache, "kv8_fetch", None)
    if hit is not None:
        cache.kv8_fetch = None
        kret, K, V, g = hit
        if kret is not keys:
            count(False, "the attention was handed other keys than the cache fetched")
        elif not supports(queries, K, V, 8, g, mask, sinks):
            count(False, f"shape outside the kernel (q {tuple(queries.shape)}, mask "
                         f"{getattr(mask, 'shape', mask)}, sinks given: {sinks is not None})")
        else:
            count(True)
            return decode_sdpa(queries, K, V, scale, mask, g, 8, same_layout=True)
    if hasattr(cache, "bits"):
        # mlx-lm's own quantized cache (a `bits` attribute): its fetch hands
        # back the triples, attention goes through the two quantized products
        if sinks is not None:
            raise ValueError("Quantized SDPA does not support attention sinks.")
        return quantized_sdpa(queries, keys, values, scale, mask, cache.group_size, cache.bits)
    pk, pv = _packed(keys), _packed(values)
    mask_ok = mask is None or isinstance(mask, str) or mask.dtype in (torch.bool, torch.bfloat16)
    if (pk is not None and pv is not None and sinks is None and queries.dtype == torch.bfloat16
            and pk[1:] == pv[1:] and mask_ok):
        return quantized_sdpa(queries, pk[0], pv[0], scale, mask, pk[1], pk[2])
    if base is None:
        base = _BASE["fn"]
    if base is None:
        raise ValueError("kvattn.sdpa: dense (or fp16 / fp32) attention runs in the model's own "
                         "scaled_dot_product_attention, which patch_model records; call patch_model first")
    return base(queries, keys, values, cache=cache, scale=scale, mask=mask, sinks=sinks)


class ModuleSdpa:
    """``sdpa`` as installed in one Python module by ``patch_model``: it
    carries that module's own attention function (``base``), so dense K/V
    met in that module go back to exactly the function it held."""

    __slots__ = ("base", "module")

    def __init__(self, base, module: str):
        self.base = base
        self.module = module

    def __call__(self, queries, keys, values, cache=None, scale=1.0, mask=None, sinks=None):
        return sdpa(queries, keys, values, cache, scale, mask, sinks, base=self.base)

    def __repr__(self):
        return f"kvattn.ModuleSdpa({self.module}, base={getattr(self.base, '__qualname__', self.base)!r})"


def _model_modules(model):
    if hasattr(model, "named_modules"):
        return [m for _, m in model.named_modules()]
    return [model]


def patch_model(model) -> int:
    """Rebind ``scaled_dot_product_attention`` in every Python module that
    defines one of the model's (sub)module classes to a ``ModuleSdpa``
    carrying that module's own function, so each module's dense K/V go back
    to the attention it had (modules with different functions keep theirs).
    Idempotent (a module already holding a ``ModuleSdpa`` keeps it);
    harmless for unquantized caches.  The first function replaced by this
    call also serves direct calls of ``sdpa``.  Returns how many modules
    hold the dispatch afterwards."""
    names = sorted({type(m).__module__ for m in _model_modules(model)} | {type(model).__module__})
    first, n = None, 0
    for name in names:
        mod = sys.modules.get(name)
        f = getattr(mod, "scaled_dot_product_attention", None)
        if f is None or not callable(f):
            continue
        if isinstance(f, ModuleSdpa):
            base = f.base
        elif f is sdpa:
            base = None
        else:
            base = f
            mod.scaled_dot_product_attention = ModuleSdpa(f, name)
        if first is None and base is not None:
            first = base
        n += 1
    if first is not None:
        _BASE["fn"] = first
    return n
