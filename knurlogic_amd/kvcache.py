"""Quantized KV caches on MI355X, with the interface of the reference's
engine/kvquant.py: ``QuantKVCache`` (one sequence, :117-188),
``BatchQuantKVCache`` (left-padded rows, :191-369), ``parse_bits`` /
``group_for`` (:25-42), ``mark_kernel`` (:455-460) and the ``state`` tuples
that from_state round-trips.

Storage.  A cache owns one ``_Slabs``: the keys and the values, each an
affine triple (packed uint32 [B, H, capacity, D*bits/32], scales and biases
[B, H, capacity, D/group] in the keys' dtype).  Slots [0, used) hold tokens;
capacity grows by whole 256-slot steps.  An append quantizes the new K and V
rows on the GPU straight into their slots (``kmi_kv_quantize_append_kv``,
the ``mx.quantize`` arithmetic bit for bit, one launch), after checking
that the rows fit the slabs they are written into.

Fetch.  ``update_and_fetch`` hands back K and V as ``LazyDequant`` views of
the filled slots: they dequantize (on the GPU) only when something uses
them as tensors.  For a short query with the 8-bit kernel on, the cache
also leaves ``kv8_fetch = (K returned, K triple, V triple, group)`` for
``kvattn.sdpa``, which then reads the packed slots directly.

Row bookkeeping of the batched cache follows mlx-lm's BatchKVCache: every
row ends at the shared write index ``_idx``; row b's tokens start at
``left_padding[b]``; ``offset[b]`` is its token count (negative while only
padding has been declared).  Offsets and paddings are host int64 tensors.
Neither class has a ``bits`` attribute (it is ``kv_bits``).
"""
from __future__ import annotations

import torch

from . import _abi
from .ops import DTYPE_CODE, _aligned16, _on_gpu, _ptr, _stream, dequantize

#: bits a person can ask for; None (or "bf16") is the unquantized cache.
BITS = (8, 6, 4)

#: queries of up to this many tokens per sequence hand their packed K/V to
#: the 8-bit decode kernel.  Measured on MI355X (B 4, 32 query / 4 KV heads,
#: D 128): at L = 4 (an MTP verify) the kernel takes 23.6 us at 8k keys and
#: 46.7 us at 32k, against 46.5 / 130 us for the packed-triple attention
#: that serves the other cases.
KERNEL_MAX_QUERY = 4

#: slots added at a time
STEP = 256

_OFF_WORDS = ("", "bf16", "16", "none", "off")


def parse_bits(v) -> int | None:
    """A KV precision as a person writes it: None, "" / "bf16" / "16" /
    "none" / "off" mean the unquantized cache (None); "8", "6", "4" (or the
    ints) the stored width.  Anything else is a ValueError."""
    if v is None:
        return None
    text = str(v).strip().lower()
    if text in _OFF_WORDS:
        return None
    bits = int(text)
    if bits not in BITS:
        raise ValueError(f"KV bits {v!r}: bf16, 8, 6 or 4")
    return bits


def group_for(dim: int) -> int:
    """The quantization group of a head dim: 64 if it divides, else 32."""
    if dim % 64 == 0:
        return 64
    if dim % 32 == 0:
        return 32
    raise ValueError(f"head dim {dim} is not a multiple of 32: its K/V "
                     f"cannot be quantized in groups")


def _group(dk: int, dv: int) -> int:
    """The one group K and V share: the smaller of their own groups."""
    return min(group_for(dk), group_for(dv))


def _steps(n: int) -> int:
    return -(-n // STEP) * STEP


# torch has few uint32 kernels (cat, index, pad, gather, roll): structural
# moves of the packed words go through an int32 view of the same bytes.
def _as_i32(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int32) if t.dtype == torch.uint32 else t


def _like(t: torch.Tensor, ref: torch.Tensor) -> torch.Tensor:
    return t.view(torch.uint32) if ref.dtype == torch.uint32 else t


def _triple_zeros(B, H, cap, dim, bits, group, dtype, device):
    packed = torch.zeros(B, H, cap, dim * bits // 32, dtype=torch.int32, device=device).view(torch.uint32)
    return (packed, torch.zeros(B, H, cap, dim // group, dtype=dtype, device=device),
            torch.zeros(B, H, cap, dim // group, dtype=dtype, device=device))


# the bench and the tests allocate bare triples with this
_alloc = _triple_zeros


def _slab_strides(parts, x: torch.Tensor, bits: int, group: int, what: str):
    """Check that x [B, H, S, D] can be written into the triple ``parts``
    (the kernel only sees strides and a capacity, so a slab of another
    batch, head count or width must be refused here), and return the six
    element strides the launcher takes."""
    wq, sc, bi = parts
    if bits not in (2, 3, 4, 5, 6, 8):
        raise ValueError(f"KV cache: {bits}-bit storage is not implemented (2, 3, 4, 5, 6, 8)")
    if x.dtype not in DTYPE_CODE or sc.dtype != x.dtype or bi.dtype != x.dtype:
        raise ValueError("KV cache: keys/values and the stored scales must share a float dtype")
    if x.dim() != 4 or wq.dim() != 4 or sc.dim() != 4 or bi.dim() != 4:
        raise ValueError(f"KV cache: {what} and its slab must be [B, H, slots, *]")
    B, H, _, D = x.shape
    if D % group or (D * bits) % 32:
        raise ValueError(f"KV cache: {what} head dim {D} does not pack at {bits} bits in groups of {group}")
    want_w = (B, H, wq.shape[2], D * bits // 32)
    want_s = (B, H, wq.shape[2], D // group)
    if tuple(wq.shape) != want_w or tuple(sc.shape) != want_s or tuple(bi.shape) != want_s:
        raise ValueError(f"KV cache: {what} {tuple(x.shape)} does not fit its slab (packed "
                         f"{tuple(wq.shape)}, scales {tuple(sc.shape)}, biases {tuple(bi.shape)})")
    if wq.stride(-1) != 1 or sc.stride(-1) != 1 or sc.stride() != bi.stride():
        raise ValueError("KV cache: the slab's last axis must be contiguous, scales laid out like biases")
    return [wq.stride(0), wq.stride(1), wq.stride(2), sc.stride(0), sc.stride(1), sc.stride(2)]


def append_quantized(parts, x: torch.Tensor, pos: int, group: int, bits: int) -> None:
    """Quantize x [B, H, S, D] along D into slots pos .. pos+S-1 of the
    triple ``parts`` (kmi_kv_quantize_append: one launch)."""
    strides = torch.tensor(_slab_strides(parts, x, bits, group, "x"), dtype=torch.int64)
    _on_gpu(x, *parts)
    B, H, S, D = x.shape
    wq, sc, bi = parts
    _abi.check(_abi.load().kmi_kv_quantize_append(
        _ptr(_aligned16(x)), DTYPE_CODE[x.dtype], B, H, S, D, group, bits, _ptr(wq), _ptr(sc), _ptr(bi),
        strides.data_ptr(), int(pos), wq.shape[2], _stream(x)), "kv_quantize_append")


def append_kv(kparts, vparts, keys: torch.Tensor, values: torch.Tensor, pos: int, group: int,
              bits: int) -> None:
    """Both appends of one update (keys into ``kparts``, values into
    ``vparts``, slots pos .. pos+S-1) in one launch
    (kmi_kv_quantize_append_kv)."""
    st = _slab_strides(kparts, keys, bits, group, "keys") + _slab_strides(vparts, values, bits, group, "values")
    if keys.dtype != values.dtype or keys.shape[:3] != values.shape[:3]:
        raise ValueError("KV cache: keys and values must share dtype and [B, H, S]")
    if kparts[0].shape[2] != vparts[0].shape[2]:
        raise ValueError("KV cache: the key and value slabs must hold the same number of slots")
    _on_gpu(keys, values, *kparts, *vparts)
    B, H, S, Dk = keys.shape
    strides = torch.tensor(st, dtype=torch.int64)
    kc, vc = _aligned16(keys), _aligned16(values)
    _abi.check(_abi.load().kmi_kv_quantize_append_kv(
        _ptr(kc), _ptr(vc), DTYPE_CODE[keys.dtype], B, H, S, Dk, values.shape[3], group, bits,
        _ptr(kparts[0]), _ptr(kparts[1]), _ptr(kparts[2]), strides.data_ptr(),
        _ptr(vparts[0]), _ptr(vparts[1]), _ptr(vparts[2]), strides.data_ptr() + 6 * 8,
        int(pos), kparts[0].shape[2], _stream(keys)), "kv_quantize_append")


class _Slabs:
    """The stored keys and values of one cache: two triples of shape
    [B, H, capacity, *].  Every structural operation returns new slabs."""

    __slots__ = ("k", "v")

    def __init__(self, k, v):
        self.k, self.v = tuple(k), tuple(v)

    @classmethod
    def empty(cls, B, H, cap, dims, bits, group, dtype, device) -> "_Slabs":
        return cls(_triple_zeros(B, H, cap, dims[0], bits, group, dtype, device),
                   _triple_zeros(B, H, cap, dims[1], bits, group, dtype, device))

    @property
    def tensors(self):
        return self.k + self.v

    @property
    def capacity(self) -> int:
        return self.k[0].shape[2]

    @property
    def rows(self) -> int:
        return self.k[0].shape[0]

    def _map(self, fn) -> "_Slabs":
        out = [_like(fn(_as_i32(t)), t) for t in self.tensors]
        return _Slabs(out[:3], out[3:])

    def window(self, lo: int, hi: int):
        """(K triple, V triple) views of slots lo .. hi-1."""
        return (tuple(t[:, :, lo:hi] for t in self.k), tuple(t[:, :, lo:hi] for t in self.v))

    def grown(self, keep: int, cap: int) -> "_Slabs":
        """New slabs of ``cap`` slots whose first ``keep`` are these."""
        def grow(t):
            g = t.new_zeros(*t.shape[:2], cap, t.shape[3])
            g[:, :, :keep] = t[:, :, :keep]
            return g
        return self._map(grow)

    def take_rows(self, idx: torch.Tensor) -> "_Slabs":
        return self._map(lambda t: t[idx.to(t.device)])

    def drop_front(self, m: int) -> "_Slabs":
        return self._map(lambda t: t[:, :, m:])

    def roll_rows(self, shifts: torch.Tensor) -> "_Slabs":
        """Row b rolled right by shifts[b] slots (wrapping)."""
        n = self.capacity
        src = (torch.arange(n)[None, :] - shifts[:, None]) % n          # [B, n]: slot s takes src[b, s]

        def roll(t):
            i = src.to(t.device)[:, None, :, None].expand(t.shape[0], t.shape[1], n, t.shape[3])
            return torch.gather(t, 2, i)
        return self._map(roll)

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.tensors)


def _stack_rows(parts: list, cap: int, like: _Slabs) -> _Slabs:
    """Slabs of sum(rows) rows and ``cap`` slots: each (slabs, shift, n) in
    ``parts`` contributes its rows with slots 0 .. n-1 placed at shift .. ,
    everything else zero."""
    B = sum(s.rows for s, _, _ in parts)
    out = []
    for j, ref in enumerate(like.tensors):
        dst = _as_i32(ref).new_zeros(B, ref.shape[1], cap, ref.shape[3])
        r = 0
        for s, shift, n in parts:
            src = _as_i32(s.tensors[j])
            dst[r:r + s.rows, :, shift:shift + n] = src[:, :, :n]
            r += s.rows
        out.append(_like(dst, ref))
    return _Slabs(out[:3], out[3:])


class LazyDequant:
    """K or V as ``update_and_fetch`` hands it back: the quantized slab
    view, dequantized (``mx.dequantize(...).astype(dtype)``) the first time
    it is used as a tensor -- by any torch function, operator or tensor
    attribute.  ``shape``, ``dtype``, ``device`` and ``ndim`` need no
    dequantization; ``parts`` / ``group`` / ``bits`` are the packed triple."""

    __slots__ = ("parts", "group", "bits", "_dtype", "_t")

    def __init__(self, parts, group: int, bits: int, dtype: torch.dtype):
        self.parts, self.group, self.bits, self._dtype = parts, group, bits, dtype
        self._t = None

    @property
    def shape(self):
        w = self.parts[0]
        return torch.Size((*w.shape[:-1], w.shape[-1] * 32 // self.bits))

    @property
    def dtype(self):
        return self._dtype

    @property
    def device(self):
        return self.parts[0].device

    @property
    def ndim(self):
        return self.parts[0].ndim

    def size(self, dim=None):
        return self.shape if dim is None else self.shape[dim]

    def materialize(self) -> torch.Tensor:
        if self._t is None:
            w, s, b = self.parts
            self._t = dequantize(w, s, b, self.group, self.bits).to(self._dtype)
        return self._t

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        return func(*_materialized(args), **_materialized(kwargs or {}))

    def __getattr__(self, name):
        return getattr(self.materialize(), name)

    def __repr__(self):
        state = "dequantized" if self._t is not None else "quantized"
        return f"LazyDequant({tuple(self.shape)}, {self._dtype}, {self.bits}-bit, {state})"

    def __getitem__(self, i):
        return self.materialize()[i]

    def __len__(self):
        return self.shape[0]

    def __matmul__(self, o):
        return self.materialize() @ materialize(o)

    def __rmatmul__(self, o):
        return materialize(o) @ self.materialize()

    def __mul__(self, o):
        return self.materialize() * materialize(o)

    __rmul__ = __mul__

    def __add__(self, o):
        return self.materialize() + materialize(o)

    __radd__ = __add__

    def __sub__(self, o):
        return self.materialize() - materialize(o)

    def __rsub__(self, o):
        return materialize(o) - self.materialize()

    def __truediv__(self, o):
        return self.materialize() / materialize(o)

    def __neg__(self):
        return -self.materialize()


def materialize(x):
    """x itself, or the tensor a LazyDequant stands for."""
    return x.materialize() if isinstance(x, LazyDequant) else x


def _materialized(obj):
    if isinstance(obj, LazyDequant):
        return obj.materialize()
    if isinstance(obj, (list, tuple)):
        return type(obj)(_materialized(o) for o in obj)
    if isinstance(obj, dict):
        return {k: _materialized(v) for k, v in obj.items()}
    return obj


class _QuantStore:
    """What both caches share: the slabs, their metadata and the update."""

    step = STEP
    slabs = None
    #: hand the packed K/V to the 8-bit decode kernel (kvattn.sdpa); per
    #: cache, set by kvattn.install's make_cache and carried by merge /
    #: extract / extend
    kv8_kernel = False
    kv8_fetch = None

    def _init_store(self, kv_bits) -> None:
        self.slabs = None
        self.kv_bits = int(kv_bits)
        self.group = None
        self.dims = None               # (key head dim, value head dim)

    # the triples as attributes (the reference's `keys` / `values`)
    @property
    def keys(self):
        return None if self.slabs is None else self.slabs.k

    @property
    def values(self):
        return None if self.slabs is None else self.slabs.v

    def _set_parts(self, k, v) -> None:
        self.slabs = None if k is None else _Slabs(k, v)

    def _append(self, keys: torch.Tensor, values: torch.Tensor, at: int):
        """Write S new tokens at slot ``at`` (growing the slabs first when
        they are full) and return what update_and_fetch returns."""
        B, H, S, Dk = keys.shape
        if self.group is None:
            self.dims = (Dk, values.shape[3])
            self.group = _group(*self.dims)
        if self.slabs is None:
            self.slabs = _Slabs.empty(B, H, _steps(S), self.dims, self.kv_bits, self.group, keys.dtype,
                                      keys.device)
        elif at + S > self.slabs.capacity:
            self.slabs = self.slabs.grown(at, at + _steps(S))
        append_kv(self.slabs.k, self.slabs.v, keys, values, at, self.group, self.kv_bits)
        return self._fetch(at + S, S, keys.dtype, values.dtype)

    def _fetch(self, used: int, S: int, kdt, vdt):
        K, V = self.slabs.window(0, used)
        k = LazyDequant(K, self.group, self.kv_bits, kdt)
        v = LazyDequant(V, self.group, self.kv_bits, vdt)
        if self.kv8_fetch is not None:
            # left by the previous step and never picked up: that step's
            # attention did not go through kvattn.sdpa
            from . import kvattn
            kvattn.count(False, "the attention never asked for it")
        hand = self.kv8_kernel and self.kv_bits == 8 and S <= KERNEL_MAX_QUERY
        self.kv8_fetch = (k, K, V, self.group) if hand else None
        return k, v

    def is_trimmable(self) -> bool:
        return True

    def empty(self) -> bool:
        return self.slabs is None

    def to_quantized(self, *a, **k):
        raise TypeError("already quantized")

    @property
    def nbytes(self) -> int:
        return 0 if self.slabs is None else self.slabs.nbytes()


class QuantKVCache(_QuantStore):
    """One sequence's attention cache, stored quantized.  ``keys`` /
    ``values`` are (packed, scales, biases) triples [B, H, slots, *];
    ``update_and_fetch`` returns K/V of the dtype it was given."""

    def __init__(self, kv_bits: int = 8):
        self._init_store(kv_bits)
        self.offset = 0

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        at = self.offset
        self.offset += keys.shape[2]
        return self._append(keys, values, at)

    def size(self) -> int:
        return self.offset

    def trim(self, n: int) -> int:
        n = min(self.offset, n)
        self.offset -= n
        return n

    @property
    def state(self):
        K, V = (None, None) if self.slabs is None else self.slabs.window(0, self.offset)
        return K, V, self.offset, self.kv_bits, self.group or 0, bool(self.kv8_kernel)

    @state.setter
    def state(self, v):
        k, vv, offset, bits, group, kernel = v
        self._set_parts(k, vv)
        self.offset, self.kv_bits = offset, int(bits)
        self.group, self.kv8_kernel = int(group) or None, bool(kernel)
        self.dims = None if k is None else (k[0].shape[3] * 32 // self.kv_bits,
                                            vv[0].shape[3] * 32 // self.kv_bits)

    @classmethod
    def merge(cls, caches):
        return BatchQuantKVCache.merge(caches)


class BatchQuantKVCache(_QuantStore):
    """Left-padded rows sharing one write index ``_idx`` (mlx-lm's
    BatchKVCache bookkeeping), stored quantized."""

    def __init__(self, left_padding, kv_bits: int = 8):
        self._init_store(kv_bits)
        self.left_padding = torch.tensor([int(p) for p in left_padding], dtype=torch.int64)
        self.offset = -self.left_padding
        self._idx = 0
        self._right_padding = None

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        at, S = self._idx, keys.shape[2]
        self._idx += S
        self.offset = self.offset + S
        return self._append(keys, values, at)

    def size(self) -> int:
        return self._idx

    def trim(self, n: int) -> int:
        n = min(self._idx, n)
        self._idx -= n
        self.offset = self.offset - n
        return n

    def prepare(self, *, left_padding=None, lengths=None, right_padding=None):
        """Declare more left padding (empty cache only), or right padding of
        the next update, which ``finalize`` rolls back into place."""
        if left_padding is not None:
            if self.slabs is not None:
                raise ValueError("left padding can only be added to an empty cache")
            extra = torch.tensor([int(p) for p in left_padding], dtype=torch.int64)
            self.left_padding = self.left_padding + extra
            self.offset = self.offset - extra
        if right_padding is not None and max(right_padding) > 0:
            self._right_padding = torch.tensor([int(p) for p in right_padding], dtype=torch.int64)

    def finalize(self):
        pad, self._right_padding = self._right_padding, None
        if pad is None:
            return
        self.slabs = self.slabs.roll_rows(pad)
        self.offset = self.offset - pad
        self.left_padding = self.left_padding + pad

    def make_mask(self, L: int, device=None) -> torch.Tensor:
        """bool [B, 1, L, _idx + L]: query row l of the next L tokens sees
        its own row's slots from the row's left padding up to itself."""
        n = torch.arange(self._idx + L)
        first = self.left_padding[:, None, None]                       # [B, 1, 1]
        last = (self._idx + torch.arange(L))[None, :, None]             # [1, L, 1]
        m = (n[None, None, :] >= first) & (n[None, None, :] <= last)
        return m[:, None].to(device if device is not None else "cpu")

    @property
    def state(self):
        K, V = (None, None) if self.slabs is None else self.slabs.window(0, self._idx)
        dk, dv = self.dims or (0, 0)
        return (K, V, self.offset, self.left_padding, self._idx, self.kv_bits, self.group or 0, dk, dv,
                bool(self.kv8_kernel))

    @state.setter
    def state(self, v):
        k, vv, self.offset, self.left_padding, self._idx, bits, group, dk, dv, kernel = v
        self._set_parts(k, vv)
        self.kv_bits, self.group = int(bits) or 8, int(group) or None
        self.dims = (int(dk), int(dv)) if dk else None
        self.kv8_kernel = bool(kernel)
        self._right_padding = getattr(self, "_right_padding", None)

    def filter(self, batch_indices):
        """Keep the rows ``batch_indices``, then drop the slots every kept
        row has as padding."""
        keep = torch.as_tensor(batch_indices, dtype=torch.int64)
        self.offset, self.left_padding = self.offset[keep], self.left_padding[keep]
        if self.slabs is not None:
            self.slabs = self.slabs.take_rows(keep)
        common = int(self.left_padding.min())
        if common > 0:
            if self.slabs is not None:
                self.slabs = self.slabs.drop_front(common)
            self._idx -= common
            self.left_padding = self.left_padding - common

    def extend(self, other):
        """Append ``other``'s rows: both caches' rows are shifted right so
        they end at the larger write index."""
        self.kv8_kernel = self.kv8_kernel or other.kv8_kernel
        for a, b in ((self, other), (other, self)):
            if a.group is None and b.group is not None:
                a.group, a.dims = b.group, b.dims
        idx = max(self._idx, other._idx)
        shifts = (idx - self._idx, idx - other._idx)
        held = [c for c in (self, other) if c.slabs is not None]
        if held:
            like = held[0].slabs
            cap = max([idx] + [c.slabs.capacity for c in held])
            parts = []
            for c, sh in zip((self, other), shifts):
                s = c.slabs
                if s is None:
                    s = _Slabs.empty(c.offset.shape[0], like.k[0].shape[1], 0, c.dims, c.kv_bits, c.group,
                                     like.k[1].dtype, like.k[0].device)
                parts.append((s, sh, c._idx))
            self.slabs = _stack_rows(parts, cap, like)
        self.left_padding = torch.cat([self.left_padding + shifts[0], other.left_padding + shifts[1]])
        self.offset = torch.cat([self.offset, other.offset])
        self._idx = idx

    def extract(self, idx: int) -> QuantKVCache:
        """Row ``idx`` as a single-sequence cache holding only its tokens."""
        c = QuantKVCache(self.kv_bits)
        c.kv8_kernel, c.group, c.dims = self.kv8_kernel, self.group, self.dims
        if self.slabs is not None:
            lo = int(self.left_padding[idx])
            k, v = self.slabs.window(lo, self._idx)
            c.slabs = _Slabs([t[idx:idx + 1].contiguous() for t in k], [t[idx:idx + 1].contiguous() for t in v])
            c.offset = self._idx - lo
        return c

    @classmethod
    def merge(cls, caches):
        """One batched cache of the given single-sequence caches, each row
        right-aligned at the longest one's length."""
        caches = list(caches)
        bits = caches[0].kv_bits
        lengths = [c.size() for c in caches]
        longest = max(lengths)
        out = cls([longest - n for n in lengths], bits)
        out.kv8_kernel = any(getattr(c, "kv8_kernel", False) for c in caches)
        if longest == 0:
            return out
        first = next(c for c in caches if c.slabs is not None)
        out.group, out.dims = first.group, first.dims
        parts = []
        for c, n in zip(caches, lengths):
            s = c.slabs if c.slabs is not None else _Slabs.empty(
                1, first.slabs.k[0].shape[1], 0, first.dims, bits, first.group, first.slabs.k[1].dtype,
                first.slabs.k[0].device)
            parts.append((s, longest - n, n))
        out.slabs = _stack_rows(parts, longest, first.slabs)
        out.offset = out.offset + longest
        out._idx = longest
        return out


def mark_kernel(caches) -> None:
    """Let the quantized caches in ``caches`` (and inside cache lists) hand
    their packed K/V to the 8-bit decode kernel."""
    for c in caches:
        if isinstance(c, _QuantStore):
            c.kv8_kernel = True
        else:
            inner = getattr(c, "caches", None)
            if isinstance(inner, (tuple, list)):
                mark_kernel(inner)


def _plain_empty(c) -> bool:
    """An unquantized, still-empty cache of the kind a model's make_cache
    builds: a class named KVCache (mlx-lm's, or a port's) holding no keys."""
    return type(c).__name__ == "KVCache" and getattr(c, "keys", None) is None


def quantize_cache_list(caches, bits: int, table=None):
    """(new list, how many were quantized): each empty plain ``KVCache``
    becomes a ``QuantKVCache(bits)``; a cache whose class is a key of
    ``table`` ({class: factory(bits)}, a family's own attention caches)
    becomes what its factory builds; a cache list (a ``caches`` tuple or
    list) is rebuilt from its converted members.  Everything else -- caches
    already holding tokens, recurrent state -- passes through."""
    table = table or {}
    count = 0

    def convert(c):
        nonlocal count
        make = table.get(type(c))
        if make is not None and getattr(c, "keys", None) is None:
            count += 1
            return make(bits)
        if _plain_empty(c):
            count += 1
            return QuantKVCache(bits)
        inner = getattr(c, "caches", None)
        if isinstance(inner, (tuple, list)):
            return type(c)(*(convert(m) for m in inner))
        return c

    return [convert(c) for c in caches], count


def install(model, bits, table=None) -> int:
    """Wrap ``model.make_cache`` so every new cache list stores attention
    K/V at ``bits`` (8, 6 or 4), and rebind the model's attention modules
    to ``kvattn.sdpa`` (``kvattn.patch_model``).  At 8 bits with the kernel enabled (``kvattn.ENV``)
    the new caches hand their packed K/V to the decode kernel;
    ``model.kv8_kernel`` records whether.  Returns how many caches
    of a probe list are quantized (0: none of this model's caches can be,
    and nothing is wrapped)."""
    bits = parse_bits(bits)
    if bits is None:
        return 0
    build = model.make_cache
    _, n = quantize_cache_list(build(), bits, table)
    if n == 0:
        return 0
    from . import kvattn
    # attention goes through kvattn.sdpa at every width (the packed-triple
    # path serves what the kernel does not take); the kernel needs 8 bits
    patched = kvattn.patch_model(model)
    kernel = bits == 8 and kvattn.enabled() and patched > 0
    kvattn.reset(kernel)
    model.kv8_kernel = kernel

    def make_cache():
        caches = quantize_cache_list(build(), bits, table)[0]
        if kernel:
            mark_kernel(caches)
        return caches

    model.make_cache = make_cache
    return n
