"""Quantized KV caches on MI355X: the reference's engine/kvquant.py
(``QuantKVCache`` :117-188, ``BatchQuantKVCache`` :191-398, ``parse_bits`` /
``group_for`` / ``_group`` :26-57) over torch tensors.

Each of K and V is stored as the affine-quantized triple (packed uint32,
scales, biases in the keys' dtype) in slabs grown 256 slots at a time.
``update_and_fetch`` quantizes the new keys / values on the GPU straight
into their slab slots (one ``kmi_kv_quantize_append`` launch each, the
``mx.quantize`` arithmetic bit for bit) and returns K and V as
``LazyDequant`` views: they become dequantized tensors the first time they
are used as tensors, so a decode step that takes the 8-bit kernel
(``kvattn.sdpa`` through the cache's ``kv8_fetch``) never dequantizes the
cache -- what mlx's lazy arrays give the reference.

The batched cache follows the row bookkeeping of mlx-lm's ``BatchKVCache``
(left-padded rows, one offset per row, a shared write index ``_idx``),
which the reference class extends; offsets and paddings are host int64
tensors.  Neither class has a ``bits`` attribute (it is ``kv_bits``), as
in the reference.
"""
from __future__ import annotations

import torch

from . import _abi
from .ops import DTYPE_CODE, _aligned16, _on_gpu, _ptr, _stream, dequantize

#: bits a person can ask for; None (or "bf16") is the unquantized cache.
#: The GPU quantizer and the decode kernel take 8 and 4 (6 raises).
BITS = (8, 6, 4)

#: query lengths up to this hand their packed K/V to the 8-bit decode
#: kernel (the reference's KERNEL_MAX_QUERY: decode steps only)
KERNEL_MAX_QUERY = 1


def parse_bits(v) -> int | None:
    """'bf16'/''/None/16 -> None; '8'/'6'/'4' -> int.  Anything else raises."""
    if v is None:
        return None
    s = str(v).strip().lower()
    if s in ("", "bf16", "16", "none", "off"):
        return None
    b = int(s)
    if b not in BITS:
        raise ValueError(f"KV bits {v!r}: bf16, 8, 6 or 4")
    return b


def group_for(dim: int) -> int:
    for g in (64, 32):
        if dim % g == 0:
            return g
    raise ValueError(f"head dim {dim} is not a multiple of 32: its K/V "
                     f"cannot be quantized in groups")


def _group(dk: int, dv: int) -> int:
    """One group size for K and V: 64 when both allow it, else 32."""
    group_for(dk), group_for(dv)
    return 64 if not (dk % 64 or dv % 64) else 32


# Structural ops on the packed words (cat, index, pad, gather, zeros) run
# on int32 views: torch implements few kernels for uint32.
def _i32(p: torch.Tensor) -> torch.Tensor:
    return p.view(torch.int32) if p.dtype == torch.uint32 else p


def _as(p: torch.Tensor, like_dtype) -> torch.Tensor:
    return p.view(torch.uint32) if like_dtype == torch.uint32 else p


def _map(parts, fn):
    return tuple(_as(fn(_i32(p)), p.dtype) for p in parts)


def _alloc(B, H, L, dim, bits, g, dtype, device):
    return (torch.zeros(B, H, L, dim * bits // 32, dtype=torch.int32, device=device).view(torch.uint32),
            torch.zeros(B, H, L, dim // g, dtype=dtype, device=device),
            torch.zeros(B, H, L, dim // g, dtype=dtype, device=device))


def _slice(parts, a, b):
    return tuple(p[..., a:b, :] for p in parts)


def _parts(v):
    return None if v is None else tuple(v)


def _sliced(parts, n):
    return None if parts is None else _slice(parts, 0, n)


def _cat(xs, ys, dim=2):
    return tuple(_as(torch.cat([_i32(x), _i32(y)], dim=dim), x.dtype) for x, y in zip(xs, ys))


def _nbytes(parts) -> int:
    return sum(p.numel() * p.element_size() for p in parts) if parts is not None else 0


def append_quantized(parts, x: torch.Tensor, pos: int, group: int, bits: int) -> None:
    """Quantize x [B, H, S, D] along D into slots pos .. pos+S-1 of the
    triple ``parts`` (kmi_kv_quantize_append: one launch)."""
    wq, sc, bi = parts
    _on_gpu(x, wq, sc, bi)
    if bits not in (2, 3, 4, 5, 6, 8):
        raise ValueError(f"KV cache: {bits}-bit storage is not implemented (2, 3, 4, 5, 6, 8)")
    if x.dtype not in DTYPE_CODE or sc.dtype != x.dtype or bi.dtype != x.dtype:
        raise ValueError("KV cache: keys/values and the stored scales must share a float dtype")
    if sc.stride(-1) != 1 or wq.stride(-1) != 1 or sc.stride() != bi.stride():
        raise ValueError("KV cache: the slab's last axis must be contiguous, scales laid out like biases")
    B, H, S, D = x.shape
    xc = _aligned16(x)
    strides = torch.tensor([wq.stride(0), wq.stride(1), wq.stride(2),
                            sc.stride(0), sc.stride(1), sc.stride(2)], dtype=torch.int64)
    _abi.check(_abi.load().kmi_kv_quantize_append(
        _ptr(xc), DTYPE_CODE[x.dtype], B, H, S, D, group, bits, _ptr(wq), _ptr(sc), _ptr(bi),
        strides.data_ptr(), int(pos), wq.shape[2], _stream(x)), "kv_quantize_append")


def _check_slab(parts, x, bits):
    wq, sc, bi = parts
    _on_gpu(x, wq, sc, bi)
    if bits not in (2, 3, 4, 5, 6, 8):
        raise ValueError(f"KV cache: {bits}-bit storage is not implemented (2, 3, 4, 5, 6, 8)")
    if x.dtype not in DTYPE_CODE or sc.dtype != x.dtype or bi.dtype != x.dtype:
        raise ValueError("KV cache: keys/values and the stored scales must share a float dtype")
    if sc.stride(-1) != 1 or wq.stride(-1) != 1 or sc.stride() != bi.stride():
        raise ValueError("KV cache: the slab's last axis must be contiguous, scales laid out like biases")
    return [wq.stride(0), wq.stride(1), wq.stride(2), sc.stride(0), sc.stride(1), sc.stride(2)]


def append_kv(kparts, vparts, keys: torch.Tensor, values: torch.Tensor, pos: int, group: int,
              bits: int) -> None:
    """Both appends of one update_and_fetch (keys into ``kparts``, values
    into ``vparts``, slots pos .. pos+S-1) in one launch
    (kmi_kv_quantize_append_kv)."""
    ks = _check_slab(kparts, keys, bits)
    vs = _check_slab(vparts, values, bits)
    if keys.dtype != values.dtype or keys.shape[:3] != values.shape[:3]:
        raise ValueError("KV cache: keys and values must share dtype and [B, H, S]")
    B, H, S, Dk = keys.shape
    Dv = values.shape[3]
    kc, vc = _aligned16(keys), _aligned16(values)
    st = torch.tensor(ks + vs, dtype=torch.int64)
    _abi.check(_abi.load().kmi_kv_quantize_append_kv(
        _ptr(kc), _ptr(vc), DTYPE_CODE[keys.dtype], B, H, S, Dk, Dv, group, bits,
        _ptr(kparts[0]), _ptr(kparts[1]), _ptr(kparts[2]), st.data_ptr(),
        _ptr(vparts[0]), _ptr(vparts[1]), _ptr(vparts[2]), st.data_ptr() + 6 * 8,
        int(pos), kparts[0].shape[2], _stream(keys)), "kv_quantize_append")


class LazyDequant:
    """K or V as ``update_and_fetch`` hands it back: the quantized slab
    view, dequantized (``mx.dequantize(...).astype(dtype)``) the first time
    it is used as a tensor -- by any torch function, operator or tensor
    attribute.  ``shape``, ``dtype``, ``device`` and ``ndim`` need no
    dequantization."""

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


def _fetch(c, n, S, kdt, vdt):
    """What ``update_and_fetch`` returns (K, V over slots 0 .. n-1, lazily
    dequantized) and, for a short 8-bit query with the kernel on, what
    ``kvattn.sdpa`` needs (the reference's _fetch, kvquant.py:89-104)."""
    g, bits = c.group, c.kv_bits
    K, V = _slice(c.keys, 0, n), _slice(c.values, 0, n)
    k, v = LazyDequant(K, g, bits, kdt), LazyDequant(V, g, bits, vdt)
    if getattr(c, "kv8_fetch", None) is not None:
        # handed out last step and never taken: its attention did not go
        # through kvattn.sdpa
        from . import kvattn
        kvattn.count(False, "the attention never asked for it")
    c.kv8_fetch = None
    if c.kv8_kernel and bits == 8 and S <= KERNEL_MAX_QUERY:
        c.kv8_fetch = (k, K, V, g)
    return k, v


def _grow(c, prev, B, H, S, Dk, Dv, dtype, device):
    """Room for S more slots after ``prev``: a new slab rounded up to 256
    slots, appended to the kept prefix (kvquant.py:143-151)."""
    g, bits = c.group, c.kv_bits
    if c.keys is None or prev + S > c.keys[0].shape[2]:
        n = (c.step + S - 1) // c.step * c.step
        nk = _alloc(B, H, n, Dk, bits, g, dtype, device)
        nv = _alloc(B, H, n, Dv, bits, g, dtype, device)
        if c.keys is None:
            c.keys, c.values = nk, nv
        else:
            c.keys = _cat(_slice(c.keys, 0, prev), nk)
            c.values = _cat(_slice(c.values, 0, prev), nv)


class QuantKVCache:
    """One sequence's attention cache, stored quantized.  ``keys`` /
    ``values`` are (packed, scales, biases) triples [B, H, slots, *];
    ``update_and_fetch`` returns K/V of the dtype it was given."""

    step = 256
    #: this cache hands its packed K/V to the 8-bit decode kernel
    #: (kvattn.sdpa); per cache, carried by merge / extract / extend
    kv8_kernel = False
    kv8_fetch = None

    def __init__(self, kv_bits: int = 8):
        self.keys = self.values = None
        self.offset = 0
        self.kv_bits = int(kv_bits)
        self.group = None
        self.dims = None               # (k head dim, v head dim)

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        B, H, S, Dk = keys.shape
        Dv = values.shape[3]
        if self.group is None:
            self.group = _group(Dk, Dv)
            self.dims = (Dk, Dv)
        prev = self.offset
        _grow(self, prev, B, H, S, Dk, Dv, keys.dtype, keys.device)
        self.offset += S
        append_kv(self.keys, self.values, keys, values, prev, self.group, self.kv_bits)
        return _fetch(self, self.offset, S, keys.dtype, values.dtype)

    def size(self) -> int:
        return self.offset

    def empty(self) -> bool:
        return self.keys is None

    def is_trimmable(self) -> bool:
        return True

    def trim(self, n: int) -> int:
        n = min(self.offset, n)
        self.offset -= n
        return n

    @property
    def state(self):
        return (_sliced(self.keys, self.offset), _sliced(self.values, self.offset), self.offset,
                self.kv_bits, self.group or 0, bool(self.kv8_kernel))

    @state.setter
    def state(self, v):
        k, vv, self.offset, bits, g, kernel = v
        self.keys, self.values = _parts(k), _parts(vv)
        self.kv_bits, self.group = int(bits), (int(g) or None)
        self.kv8_kernel = bool(kernel)
        if self.keys is not None and self.dims is None:
            self.dims = (self.keys[0].shape[3] * 32 // self.kv_bits,
                         self.values[0].shape[3] * 32 // self.kv_bits)

    def to_quantized(self, *a, **k):
        raise TypeError("already quantized")

    @classmethod
    def merge(cls, caches):
        return BatchQuantKVCache.merge(caches)

    @property
    def nbytes(self) -> int:
        return _nbytes(self.keys) + _nbytes(self.values)


def _carry(out, caches):
    """``out`` takes the kernel setting of the caches it was built from."""
    out.kv8_kernel = any(getattr(c, "kv8_kernel", False) for c in caches)
    return out


def _roll_rows(p: torch.Tensor, shifts: torch.Tensor) -> torch.Tensor:
    """Each batch row b of p rolled by shifts[b] along the slot axis
    (mlx-lm's dynamic_roll on axis 2)."""
    n = p.shape[2]
    idx = (torch.arange(n)[None, :] - shifts[:, None]) % n              # [B, n]
    idx = idx.to(p.device)[:, None, :, None].expand(p.shape[0], p.shape[1], n, p.shape[3])
    return _as(torch.gather(_i32(p), 2, idx), p.dtype)


class BatchQuantKVCache:
    """Left-padded rows (one offset per row, a shared write index
    ``_idx``), stored quantized: the reference's BatchQuantKVCache over
    mlx-lm's BatchKVCache row bookkeeping."""

    step = 256
    kv8_kernel = False
    kv8_fetch = None

    def __init__(self, left_padding, kv_bits: int = 8):
        self.keys = self.values = None
        self.left_padding = torch.as_tensor(list(left_padding), dtype=torch.int64)
        self.offset = -self.left_padding.clone()
        self._idx = 0
        self._right_padding = None
        self.kv_bits = int(kv_bits)
        self.group = None
        self.dims = None

    def _meta_from(self, o) -> None:
        if self.group is None and getattr(o, "group", None) is not None:
            self.group, self.dims = o.group, o.dims

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        B, H, S, Dk = keys.shape
        Dv = values.shape[3]
        if self.group is None:
            self.group = _group(Dk, Dv)
            self.dims = (Dk, Dv)
        prev = self._idx
        _grow(self, prev, B, H, S, Dk, Dv, keys.dtype, keys.device)
        self.offset = self.offset + S
        self._idx += S
        append_kv(self.keys, self.values, keys, values, prev, self.group, self.kv_bits)
        return _fetch(self, self._idx, S, keys.dtype, values.dtype)

    def size(self) -> int:
        return self._idx

    def empty(self) -> bool:
        return self.keys is None

    def is_trimmable(self) -> bool:
        return True

    def trim(self, n: int) -> int:
        n = min(self._idx, n)
        self._idx -= n
        self.offset = self.offset - n
        return n

    def prepare(self, *, left_padding=None, lengths=None, right_padding=None):
        """Rows right-padded in the next update are rolled back into place
        by ``finalize`` (mlx-lm's prepare; only right_padding is kept)."""
        if left_padding is not None:
            if self.keys is not None:
                raise ValueError("left padding can only be added to an empty cache")
            lp = torch.as_tensor(list(left_padding), dtype=torch.int64)
            self.left_padding = self.left_padding + lp
            self.offset = self.offset - lp
        if right_padding is not None and max(right_padding) > 0:
            self._right_padding = torch.as_tensor(list(right_padding), dtype=torch.int64)

    def finalize(self):
        if self._right_padding is not None:
            pad = self._right_padding
            self.keys = tuple(_roll_rows(p, pad) for p in self.keys)
            self.values = tuple(_roll_rows(p, pad) for p in self.values)
            self.offset = self.offset - pad
            self.left_padding = self.left_padding + pad
            self._right_padding = None

    def make_mask(self, L: int, device=None) -> torch.Tensor:
        """bool [B, 1, L, _idx + L]: what each of the next L query rows may
        see once they are appended -- its own row's keys from its left
        padding on, causal inside the new block."""
        N = self._idx + L
        n = torch.arange(N)[None, None, :]
        rows = self._idx + torch.arange(L)[None, :, None]
        m = (n >= self.left_padding[:, None, None]) & (n <= rows)
        return m[:, None].to(device if device is not None else "cpu")

    @property
    def state(self):
        dk, dv = self.dims or (0, 0)
        return (_sliced(self.keys, self._idx), _sliced(self.values, self._idx), self.offset,
                self.left_padding, self._idx, self.kv_bits, self.group or 0, dk, dv,
                bool(self.kv8_kernel))

    @state.setter
    def state(self, v):
        (k, vv, self.offset, self.left_padding, self._idx, bits, g, dk, dv, kernel) = v
        self.keys, self.values = _parts(k), _parts(vv)
        self.kv_bits, self.group = int(bits) or 8, (int(g) or None)
        self.dims = (int(dk), int(dv)) if dk else None
        self.kv8_kernel = bool(kernel)
        if not hasattr(self, "_right_padding"):
            self._right_padding = None

    def filter(self, batch_indices):
        bi = torch.as_tensor(batch_indices, dtype=torch.int64)
        if self.keys is not None:
            sel = bi.to(self.keys[0].device)
            self.keys = _map(self.keys, lambda p: p[sel])
            self.values = _map(self.values, lambda p: p[sel])
        self.offset = self.offset[bi]
        self.left_padding = self.left_padding[bi]
        m = int(self.left_padding.min().item())
        if m > 0:
            if self.keys is not None:
                self.keys = _slice(self.keys, m, None)
                self.values = _slice(self.values, m, None)
            self._idx -= m
            self.left_padding = self.left_padding - m

    def _empty_parts(self, B, H, dt, device):
        Dk, Dv = self.dims
        g, bits = self.group, self.kv_bits
        return (_alloc(B, H, 0, Dk, bits, g, dt, device), _alloc(B, H, 0, Dv, bits, g, dt, device))

    def extend(self, other):
        if self.keys is None and other.keys is None:
            self.left_padding = torch.cat([self.left_padding, other.left_padding])
            self.offset = torch.cat([self.offset, other.offset])
            return
        self._meta_from(other)
        self.kv8_kernel = self.kv8_kernel or other.kv8_kernel
        other._meta_from(self)
        src = self if self.keys is not None else other
        H, dt, dev = src.keys[0].shape[1], src.keys[1].dtype, src.keys[0].device
        max_idx = max(self._idx, other._idx)
        size = max(c.keys[0].shape[2] for c in (self, other) if c.keys is not None)

        def pad(c):
            if c.keys is None:
                k, v = c._empty_parts(c.offset.shape[0], H, dt, dev)
            else:
                k, v = c.keys, c.values
            left = max_idx - c._idx
            right = size - k[0].shape[2] - left
            if right < 0:
                k, v = _slice(k, 0, right), _slice(v, 0, right)
                right = 0
            if left or right:
                k = _map(k, lambda p: torch.nn.functional.pad(p, (0, 0, left, right)))
                v = _map(v, lambda p: torch.nn.functional.pad(p, (0, 0, left, right)))
            return k, v, c.offset, c.left_padding + left

        (k1, v1, o1, l1), (k2, v2, o2, l2) = pad(self), pad(other)
        self.keys = _cat(k1, k2, dim=0)
        self.values = _cat(v1, v2, dim=0)
        self.offset = torch.cat([o1, o2])
        self.left_padding = torch.cat([l1, l2])
        self._idx = max_idx

    def extract(self, idx: int) -> QuantKVCache:
        c = QuantKVCache(self.kv_bits)
        c.kv8_kernel = self.kv8_kernel
        c.group, c.dims = self.group, self.dims
        pad = int(self.left_padding[idx].item())
        if self.keys is not None:
            c.keys = _map(self.keys, lambda p: p[idx:idx + 1, :, pad:self._idx].contiguous())
            c.values = _map(self.values, lambda p: p[idx:idx + 1, :, pad:self._idx].contiguous())
            c.offset = c.keys[0].shape[2]
        return c

    @classmethod
    def merge(cls, caches):
        bits = next(c.kv_bits for c in caches)
        lengths = [c.size() for c in caches]
        L = max(lengths)
        if L == 0:
            return _carry(cls([0] * len(caches), bits), caches)
        first = next(c for c in caches if c.keys is not None)
        pad = [L - n for n in lengths]
        B = len(caches)
        H = first.keys[0].shape[1]
        dev = first.keys[0].device
        keys = _map(first.keys, lambda p: torch.zeros(B, H, L, p.shape[3], dtype=p.dtype, device=dev))
        values = _map(first.values, lambda p: torch.zeros(B, H, L, p.shape[3], dtype=p.dtype, device=dev))
        for i, (p, c) in enumerate(zip(pad, caches)):
            if c.keys is None:
                continue
            for dst, src in ((keys, c.keys), (values, c.values)):
                for d, s in zip(dst, src):
                    _i32(d)[i:i + 1, :, p:p + c.offset] = _i32(s)[..., :c.offset, :]
        out = _carry(cls(pad, bits), caches)
        out.group, out.dims = first.group, first.dims
        out.keys, out.values = keys, values
        out.offset = out.offset + L
        out._idx = L
        return out

    @property
    def nbytes(self) -> int:
        return _nbytes(self.keys) + _nbytes(self.values)


def mark_kernel(caches) -> None:
    """Let the quantized caches in ``caches`` hand their packed K/V to the
    8-bit decode kernel (the reference's mark_kernel, kvquant.py:452-460)."""
    for c in caches:
        if isinstance(c, (QuantKVCache, BatchQuantKVCache)):
            c.kv8_kernel = True
        elif isinstance(getattr(c, "caches", None), (tuple, list)):
            mark_kernel(c.caches)
