"""mlx's quantized ops, on torch tensors in MI355X memory.

Same names, argument meaning, defaults and packed layout as mlx 0.32.3's
``mx.quantize`` / ``mx.dequantize`` / ``mx.quantized_matmul`` /
``mx.gather_qmm`` (the ops the reference reaches at
src/knurlogic/engine/kvquant.py:46-51, src/knurlogic/engine/matmul_padding.py:94-105
and src/knurlogic/engine/families/glm5/architecture/glm5_next/_mlx_vlm/
models/switch_layers.py:38-48,71-86).  Shape errors raise ``ValueError`` as
mlx does.  Every op runs a HIP kernel of libknurlogic_amd.so on the
tensors' device and stream; nothing falls back to the CPU.
"""
from __future__ import annotations

import math

import torch

from . import _abi

DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}

#: dequantize rounding: T(T(s*q) + b) (mlx's op-by-op order) or T(fma(s, q, b))
ROUND_OP_BY_OP = 0
ROUND_FUSED = 1


def _lib():
    return _abi.load()


def _on_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("knurlogic_amd ops take tensors in GPU memory "
                             f"(got a tensor on {t.device})")


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t):
    return None if t is None else t.data_ptr()


#: quantization modes: affine, and the scaled (microscaling) ones the
#: reference's loader maps bias-less layers to (packed.py:20)
MODE_CODE = {"affine": 0, "mxfp4": 1, "mxfp8": 2}
_MX_BITS = {"mxfp4": 4, "mxfp8": 8}


def _check_mode(mode: str, allow_mx: bool = False):
    if mode == "affine" or (allow_mx and mode in _MX_BITS):
        return
    raise ValueError(f"mode {mode!r}: {'affine, mxfp4 and mxfp8 are' if allow_mx else 'only affine is'} "
                     "implemented here")


def _check_mx(what, scales, biases, group_size, bits, mode):
    if biases is not None:
        raise ValueError(f"{what}: {mode} has no biases")
    if scales.dtype != torch.uint8:
        raise ValueError(f"{what}: {mode} scales are uint8 E8M0 exponents (got {scales.dtype})")
    if group_size != 32 or bits != _MX_BITS[mode]:
        raise ValueError(f"{what}: {mode} takes group_size 32 and {_MX_BITS[mode]} bits")


def _check_experts(what, H, E, w_gu, s_gu, b_gu, w_down, s_down, b_down, group_size, bits):
    """Stacked SwitchGLU experts against x's width H and E experts: gate|up
    w_gu [E, 2I, H*bits/32], s_gu (/ b_gu) [E, 2I, H/group]; down w_down
    [E, H, I*bits/32], s_down (/ b_down) [E, H, I/group].  The kernels take
    only the sizes, so a tensor smaller than these would be read past its
    end.  Returns I."""
    if w_gu.dim() != 3 or w_down.dim() != 3:
        raise ValueError(f"{what}: w_gu and w_down must be [E, rows, words]")
    I2 = w_gu.shape[1]
    if I2 % 2:
        raise ValueError(f"{what}: w_gu has {I2} rows (gate and up stacked: 2I)")
    I = I2 // 2
    if H % group_size or I % group_size or (H * bits) % 32 or (I * bits) % 32:
        raise ValueError(f"{what}: H={H}, I={I} do not divide into groups of {group_size} and whole words")
    want = {
        "w_gu": (w_gu, (E, 2 * I, H * bits // 32)),
        "s_gu": (s_gu, (E, 2 * I, H // group_size)),
        "w_down": (w_down, (E, H, I * bits // 32)),
        "s_down": (s_down, (E, H, I // group_size)),
    }
    if b_gu is not None or b_down is not None:
        want["b_gu"] = (b_gu, (E, 2 * I, H // group_size))
        want["b_down"] = (b_down, (E, H, I // group_size))
    for name, (t, shape) in want.items():
        if t is None or tuple(t.shape) != shape:
            got = None if t is None else tuple(t.shape)
            raise ValueError(f"{what}: {name} is {got}, expected {shape} "
                             f"(E={E}, H={H}, I={I}, bits={bits}, group {group_size})")
    return I


def _resolve(group_size, bits, mode: str):
    """mlx's mode-dependent defaults for an omitted group_size / bits: affine
    64 and 4, mxfp4 32 and 4, mxfp8 32 and 8."""
    if mode in _MX_BITS:
        return (32 if group_size is None else int(group_size),
                _MX_BITS[mode] if bits is None else int(bits))
    return 64 if group_size is None else int(group_size), 4 if bits is None else int(bits)


def _workspace(nbytes: int, device) -> torch.Tensor | None:
    if nbytes == 0:
        return None
    return torch.empty(int(nbytes), dtype=torch.uint8, device=device)


def _aligned16(t: torch.Tensor) -> torch.Tensor:
    """t contiguous at a 16-byte aligned address (the quantize kernels read
    8 elements per lane as one 16-byte load)."""
    t = t.contiguous()
    return t.clone() if t.data_ptr() % 16 else t


def quantize(w: torch.Tensor, group_size: int | None = None, bits: int | None = None,
             mode: str = "affine"):
    """``mx.quantize``: (wq uint32 [..., K*bits/32], scales, biases
    [..., K/group_size]) in w's dtype, groups along the last axis (omitted
    group_size / bits: 64 and 4).  mxfp4 / mxfp8: (wq, scales uint8 E8M0),
    group 32 and 4 / 8 bits, which are also the only values taken (mlx
    returns no biases)."""
    _check_mode(mode, allow_mx=True)
    group_size, bits = _resolve(group_size, bits, mode)
    if mode != "affine":
        if group_size != 32 or bits != _MX_BITS[mode]:
            raise ValueError(f"quantize: {mode} takes group_size 32 and {_MX_BITS[mode]} bits "
                             f"(got {group_size} and {bits})")
        _on_gpu(w)
        if w.dtype not in DTYPE_CODE or w.ndim < 1 or w.shape[-1] % 32:
            raise ValueError(f"quantize: {mode} needs a float tensor whose last axis is a multiple of 32")
        bits_mx = _MX_BITS[mode]
        wc = w.contiguous()
        cols = wc.shape[-1]
        rows = wc.numel() // cols if cols else 0
        wq = torch.empty(*wc.shape[:-1], cols * bits_mx // 32, dtype=torch.uint32, device=w.device)
        sc = torch.empty(*wc.shape[:-1], cols // 32, dtype=torch.uint8, device=w.device)
        _abi.check(_lib().kmi_quantize_mx(_ptr(wc), DTYPE_CODE[w.dtype], rows, cols, MODE_CODE[mode], _ptr(wq),
                                          _ptr(sc), _stream(w)), "quantize")
        return wq, sc
    _on_gpu(w)
    if w.dtype not in DTYPE_CODE:
        raise ValueError(f"quantize: dtype {w.dtype} not in bf16/fp16/fp32")
    if w.ndim < 1 or w.shape[-1] % group_size or (w.shape[-1] * bits) % 32:
        raise ValueError(f"quantize: the last axis ({w.shape[-1] if w.ndim else None}) "
                         f"must be a multiple of the group size {group_size}")
    w = _aligned16(w)
    cols = w.shape[-1]
    rows = w.numel() // cols if cols else 0
    lead = tuple(w.shape[:-1])
    wq = torch.empty(*lead, cols * bits // 32, dtype=torch.uint32, device=w.device)
    scales = torch.empty(*lead, cols // group_size, dtype=w.dtype, device=w.device)
    biases = torch.empty_like(scales)
    L = _lib()
    _abi.check(L.kmi_quantize_affine(_ptr(w), DTYPE_CODE[w.dtype], rows, cols, group_size,
                                     bits, _ptr(wq), _ptr(scales), _ptr(biases), _stream(w)),
               "quantize")
    return wq, scales, biases


def dequantize(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor | None = None,
               group_size: int | None = None, bits: int | None = None, mode: str = "affine",
               dtype: torch.dtype | None = None, rounding: int = ROUND_OP_BY_OP):
    """``mx.dequantize``: scale * q + bias in ``dtype`` (default: scales'
    dtype).  ``rounding`` picks the storage rounding order.  mxfp4 / mxfp8:
    element * 2^(scale - 127), uint8 E8M0 scales, no biases (default dtype
    bfloat16).  Omitted group_size / bits take mlx's defaults for the mode."""
    _check_mode(mode, allow_mx=True)
    group_size, bits = _resolve(group_size, bits, mode)
    if mode != "affine":
        _check_mx("dequantize", scales, biases, group_size, bits, mode)
        _on_gpu(w, scales)
        out_dtype = dtype or torch.bfloat16
        cols = w.shape[-1] * 32 // bits
        if scales.shape[:-1] != w.shape[:-1] or scales.shape[-1] * 32 != cols:
            raise ValueError(f"dequantize: shapes {tuple(w.shape)}, scales {tuple(scales.shape)} ({mode})")
        wc, sc = w.contiguous(), scales.contiguous()
        rows = wc.numel() // wc.shape[-1] if wc.shape[-1] else 0
        out = torch.empty(*w.shape[:-1], cols, dtype=out_dtype, device=w.device)
        _abi.check(_lib().kmi_dequantize_mx(_ptr(wc), _ptr(sc), rows, cols, MODE_CODE[mode], _ptr(out),
                                            DTYPE_CODE[out_dtype], _stream(w)), "dequantize")
        return out
    if biases is None:
        raise ValueError("dequantize: affine mode needs biases")
    _on_gpu(w, scales, biases)
    out_dtype = dtype or scales.dtype
    if out_dtype not in DTYPE_CODE or scales.dtype not in DTYPE_CODE:
        raise ValueError(f"dequantize: dtype {out_dtype} / scales {scales.dtype}")
    if w.dtype not in (torch.uint32, torch.int32):
        raise ValueError(f"dequantize: packed weights must be uint32 (got {w.dtype})")
    cols = w.shape[-1] * 32 // bits
    if scales.shape[:-1] != w.shape[:-1] or scales.shape[-1] * group_size != cols \
            or biases.shape != scales.shape:
        raise ValueError(f"dequantize: shapes {tuple(w.shape)}, scales {tuple(scales.shape)}, "
                         f"biases {tuple(biases.shape)} do not match group {group_size}, bits {bits}")
    if biases.dtype != scales.dtype:
        raise ValueError("dequantize: scales and biases must share a dtype")
    w, scales, biases = w.contiguous(), scales.contiguous(), biases.contiguous()
    rows = w.numel() // w.shape[-1] if w.shape[-1] else 0
    out = torch.empty(*w.shape[:-1], cols, dtype=out_dtype, device=w.device)
    L = _lib()
    _abi.check(L.kmi_dequantize_affine(_ptr(w), _ptr(scales), _ptr(biases),
                                       DTYPE_CODE[scales.dtype], rows, cols, group_size, bits,
                                       _ptr(out), DTYPE_CODE[out_dtype], int(rounding),
                                       _stream(w)), "dequantize")
    return out


def _check_affine_operands_t(x, w, scales, biases, group_size, bits, what):
    """The affine operand rules for a weight stored [..., K, N*bits/32]
    (transpose=False: groups along N)."""
    if biases is None:
        raise ValueError(f"{what}: affine mode needs biases")
    _on_gpu(x, w, scales, biases)
    if x.dtype != torch.bfloat16 or scales.dtype != torch.bfloat16 or biases.dtype != torch.bfloat16:
        raise ValueError(f"{what}: only bfloat16 activations, scales and biases are implemented")
    if w.shape[-2] != x.shape[-1] or scales.shape != biases.shape or scales.shape[:-1] != w.shape[:-1] \
            or scales.shape[-1] * group_size != w.shape[-1] * 32 // bits:
        raise ValueError(f"{what}: w {tuple(w.shape)} / scales {tuple(scales.shape)} do not take x "
                         f"{tuple(x.shape)} with transpose=False at group {group_size}")


def _check_affine_operands(x, w, scales, biases, group_size, bits, what):
    if biases is None:
        raise ValueError(f"{what}: affine mode needs biases")
    _on_gpu(x, w, scales, biases)
    if x.dtype != scales.dtype or biases.dtype != scales.dtype:
        raise ValueError(f"{what}: x ({x.dtype}), scales ({scales.dtype}) and biases "
                         f"({biases.dtype}) must share a dtype")
    if x.dtype != torch.bfloat16:
        raise ValueError(f"{what}: only bfloat16 activations are implemented (got {x.dtype})")
    K = x.shape[-1]
    if w.shape[-1] * 32 // bits != K:
        raise ValueError(f"{what}: x has {K} features but w packs "
                         f"{w.shape[-1] * 32 // bits} at {bits} bits")
    if scales.shape[-1] * group_size != K or scales.shape != biases.shape \
            or scales.shape[:-1] != w.shape[:-1]:
        raise ValueError(f"{what}: scales {tuple(scales.shape)} / biases "
                         f"{tuple(biases.shape)} do not match w {tuple(w.shape)} "
                         f"at group {group_size}")


def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                     biases: torch.Tensor | None = None, transpose: bool = True,
                     group_size: int | None = None, bits: int | None = None, mode: str = "affine"):
    """``mx.quantized_matmul``: x [..., M, K] @ What^T with What [..., N, K]
    (transpose=True) or x @ What with What [..., K, N] (transpose=False,
    groups along N), fp32 accumulation, the result in x's dtype.  A 2-D
    What at 4 or 8 bits with transpose=True is the dense projection
    (kmi_qmm); a batched What (leading dimensions broadcast against x's),
    transpose=False or the 2, 3, 5 and 6-bit widths run kmi_qmm_batched.
    Omitted group_size / bits take mlx's defaults for the mode."""
    _check_mode(mode, allow_mx=True)
    group_size, bits = _resolve(group_size, bits, mode)
    if transpose and w.ndim == 2 and mode != "affine":
        return _qmm_mx(x, w, scales, biases, group_size, bits, mode)
    if not transpose or w.ndim != 2 or bits not in (4, 8) or mode != "affine":
        return qmm_batched(x, w, scales, biases, transpose, group_size, bits, mode=mode)
    _check_affine_operands(x, w, scales, biases, group_size, bits, "quantized_matmul")
    K = x.shape[-1]
    N = w.shape[0]
    x2 = x.contiguous()
    M = x2.numel() // K if K else 0
    y = torch.empty(*x.shape[:-1], N, dtype=x.dtype, device=x.device)
    L = _lib()
    nbytes = L.kmi_qmm_workspace_bytes(M, K, N, group_size, bits)
    ws = _workspace(nbytes, x.device)
    # contiguous copies held in locals until the call returns: a temporary
    # freed mid-call could hand its memory to the next copy
    wc, sc, bc = w.contiguous(), scales.contiguous(), biases.contiguous()
    _abi.check(L.kmi_qmm(_ptr(x2), M, K, N, _ptr(wc), _ptr(sc), _ptr(bc), DTYPE_CODE[x.dtype],
                         group_size, bits, _ptr(y), _ptr(ws), nbytes, _stream(x)),
               "quantized_matmul")
    return y


def _qmm_mx(x, w, scales, biases, group_size, bits, mode):
    """Microscaled dense projection (kmi_qmm_mx): x [..., K] @ What[N, K]^T
    with E2M1 / E4M3 codes and uint8 E8M0 scales [N, K/32]."""
    what = "quantized_matmul"
    _check_mx(what, scales, biases, group_size, bits, mode)
    _on_gpu(x, w, scales)
    if x.dtype != torch.bfloat16:
        raise ValueError(f"{what}: only bfloat16 activations are implemented")
    if w.dtype not in (torch.uint32, torch.int32):
        raise ValueError(f"{what}: w must be packed uint32")
    K = x.shape[-1]
    N = w.shape[0]
    if K % 32 or w.shape[1] * 32 // bits != K or tuple(scales.shape) != (N, K // 32):
        raise ValueError(f"{what}: x has {K} features; w {tuple(w.shape)} / scales "
                         f"{tuple(scales.shape)} do not match a [{N}, {K}] {mode} weight")
    x2 = x.contiguous()
    if x2.data_ptr() % 16:
        x2 = x2.clone()
    M = x2.numel() // K if K else 0
    y = torch.empty(*x.shape[:-1], N, dtype=x.dtype, device=x.device)
    L = _lib()
    code = 1 if mode == "mxfp4" else 2
    nbytes = L.kmi_qmm_mx_workspace_bytes(M, K, N, code)
    ws = _workspace(nbytes, x.device)
    wc, sc = w.contiguous(), scales.contiguous()
    _abi.check(L.kmi_qmm_mx(_ptr(x2), M, K, N, _ptr(wc), _ptr(sc), DTYPE_CODE[x.dtype], code, _ptr(y),
                            _ptr(ws), nbytes, _stream(x)), what)
    return y


def _aligned_rows(x: torch.Tensor) -> torch.Tensor:
    """x with a contiguous last axis, rows and batch strides multiples of 8
    elements from a 16-byte aligned base, and readable memory up to the
    next multiple of 8 past the last row (kmi_qmm_batched reads rows in
    16-byte units); a zero-padded copy otherwise."""
    K = x.shape[-1]
    Kp = -(-K // 8) * 8
    ok = x.stride(-1) == 1 and x.data_ptr() % 16 == 0 and \
        all(st % 8 == 0 for d, st in enumerate(x.stride()[:-1]) if x.shape[d] > 1)
    if ok and Kp != K:
        last = x.storage_offset() + sum((n - 1) * st for n, st in zip(x.shape, x.stride()))
        ok = last + (Kp - K) < x.untyped_storage().nbytes() // x.element_size()
    if ok:
        return x
    xp = torch.zeros(*x.shape[:-1], Kp, dtype=x.dtype, device=x.device)
    xp[..., :K] = x
    return xp[..., :K]


def _fold(shape, strides, M, xr):
    """Batch dimensions of (x, w, scales) strides: drop size-1 dimensions,
    fold trailing dimensions that only x walks (w broadcast, x rows
    consecutive) into M, merge dimensions contiguous in all three."""
    dims = [(n, list(st)) for n, st in zip(shape, strides) if n != 1]
    while dims and dims[-1][1][1] == 0 and dims[-1][1][2] == 0 and dims[-1][1][0] == M * xr:
        M *= dims.pop()[0]
    merged = []
    for n, st in dims:
        if merged and all(merged[-1][1][i] == n * st[i] for i in range(3)):
            merged[-1] = (merged[-1][0] * n, st)
        else:
            merged.append((n, st))
    return merged, M


def padded_rows(shape, dtype, device) -> torch.Tensor:
    """An empty [..., N] tensor whose rows start 16 bytes apart at a
    multiple of 8 elements (a view into [..., N rounded up to 8])."""
    N = shape[-1]
    Np = -(-N // 8) * 8
    return torch.empty(*shape[:-1], Np, dtype=dtype, device=device)[..., :N]


def row_padded(t: torch.Tensor) -> bool:
    """Whether t [..., N] has 16-byte aligned rows of a multiple of 8
    elements, readable up to N rounded to 8, and rows otherwise contiguous."""
    if t.dim() < 2 or t.stride(-1) != 1 or t.data_ptr() % 16:
        return False
    N = t.shape[-1]
    Np = -(-N // 8) * 8
    ld = t.stride(-2)
    if ld % 8 or ld < Np:
        return False
    if any(t.stride(d) != t.shape[d + 1] * t.stride(d + 1) for d in range(t.dim() - 2)):
        return False
    last = t.storage_offset() + sum((n - 1) * st for n, st in zip(t.shape, t.stride()))
    return last + (Np - N) < t.untyped_storage().nbytes() // t.element_size()


def qmm_batched(x, w, scales, biases, transpose: bool = True, group_size: int | None = None,
                bits: int | None = None, x_scale: float = 1.0, out=None, mode: str = "affine"):
    """mx.quantized_matmul with batch dimensions on w (broadcast against
    x's) in either orientation; ``x_scale`` != 1 multiplies x by it first,
    rounded to x's dtype (mlx-lm's ``queries *= scale``).  ``out``: a
    [batch..., M, N] bf16 tensor with rows otherwise contiguous (a row
    padding is allowed) to write into.  ``mode`` mxfp4 / mxfp8: uint8 E8M0
    scales, no biases."""
    what = "quantized_matmul"
    _check_mode(mode, allow_mx=True)
    group_size, bits = _resolve(group_size, bits, mode)
    if mode != "affine":
        _check_mx(what, scales, biases, group_size, bits, mode)
        _on_gpu(x, w, scales)
        if x.dtype != torch.bfloat16:
            raise ValueError(f"{what}: only bfloat16 activations are implemented")
    else:
        if biases is None:
            raise ValueError(f"{what}: affine mode needs biases")
        _on_gpu(x, w, scales, biases)
        if x.dtype != torch.bfloat16 or scales.dtype != torch.bfloat16 or biases.dtype != torch.bfloat16:
            raise ValueError(f"{what}: only bfloat16 activations, scales and biases are implemented")
    if w.dtype not in (torch.uint32, torch.int32) or w.ndim < 2:
        raise ValueError(f"{what}: w must be packed uint32 with at least 2 dimensions")
    if bits not in (2, 3, 4, 5, 6, 8) or group_size not in (32, 64, 128):
        raise ValueError(f"{what}: bits {bits} / group {group_size} not implemented "
                         "(2, 3, 4, 5, 6, 8 / 32, 64, 128)")
    vec = x.ndim == 1
    if vec:
        x = x[None]
    K = x.shape[-1]
    if transpose:
        N, Kw, grouped = w.shape[-2], w.shape[-1] * 32 // bits, K
    else:
        N, Kw = w.shape[-1] * 32 // bits, w.shape[-2]
        grouped = N
    if Kw != K:
        raise ValueError(f"{what}: x has {K} features but w holds {Kw} (transpose={transpose})")
    if (biases is not None and scales.shape != biases.shape) or scales.shape[:-1] != w.shape[:-1] \
            or scales.shape[-1] * group_size != grouped:
        raise ValueError(f"{what}: scales {tuple(scales.shape)} / biases "
                         f"{None if biases is None else tuple(biases.shape)} "
                         f"do not match w {tuple(w.shape)} at group {group_size}")
    M = x.shape[-2]
    try:
        batch = torch.broadcast_shapes(tuple(x.shape[:-2]), tuple(w.shape[:-2]))
    except RuntimeError as e:
        raise ValueError(f"{what}: batch shapes {tuple(x.shape[:-2])} and {tuple(w.shape[:-2])} "
                         "do not broadcast") from e
    if out is not None:
        _on_gpu(out)
        if tuple(out.shape) != tuple(batch) + (M, N) or out.dtype != x.dtype or out.stride(-1) != 1 or any(
                out.stride(d) != out.shape[d + 1] * out.stride(d + 1) for d in range(out.dim() - 2)):
            raise ValueError(f"{what}: out must be a row-padded {tuple(batch) + (M, N)} {x.dtype} tensor")
        y = out
    else:
        y = torch.empty(*batch, M, N, dtype=x.dtype, device=x.device)
    if y.numel() == 0:
        return y[0] if vec else y
    x = _aligned_rows(x)
    if w.stride(-1) != 1 or (transpose and bits in (4, 8) and (w.data_ptr() % 16 or any(
            st % 4 for d, st in enumerate(w.stride()[:-1]) if w.shape[d] > 1))):
        w = w.contiguous()
        if w.data_ptr() % 16:
            w = w.clone()
    if (biases is not None and scales.stride() != biases.stride()) or scales.stride(-1) != 1:
        scales = scales.contiguous()
        biases = biases.contiguous() if biases is not None else None
    xe = x.expand(*batch, M, K)
    we = w.expand(*batch, *w.shape[-2:])
    se = scales.expand(*batch, *scales.shape[-2:])
    be = biases.expand(*batch, *biases.shape[-2:]) if biases is not None else None
    nb = len(batch)
    dims, Mf = _fold(batch, [(xe.stride(d), we.stride(d), se.stride(d)) for d in range(nb)],
                     M, xe.stride(-2))
    if len(dims) > 4:
        raise ValueError(f"{what}: more than 4 batch dimensions after merging ({len(dims)})")
    nd = len(dims)
    shape = torch.tensor([n for n, _ in dims] or [1], dtype=torch.int64)
    xs = torch.tensor([st[0] for _, st in dims] + [xe.stride(-2)], dtype=torch.int64)
    ws_ = torch.tensor([st[1] for _, st in dims] + [we.stride(-2)], dtype=torch.int64)
    ss = torch.tensor([st[2] for _, st in dims] + [se.stride(-2)], dtype=torch.int64)
    L = _lib()
    nbytes = L.kmi_qmm_batched_workspace_bytes(nd, shape.data_ptr(), Mf, K, N)
    ws = _workspace(nbytes, x.device)
    _abi.check(L.kmi_qmm_batched(
        _ptr(xe), xs.data_ptr(), _ptr(we), ws_.data_ptr(), _ptr(se), _ptr(be), ss.data_ptr(), nd,
        shape.data_ptr(), Mf, K, N, int(bool(transpose)), DTYPE_CODE[x.dtype], group_size, bits,
        MODE_CODE[mode], None, None, 0, 0, float(x_scale), _ptr(y), y.stride(-2), _ptr(ws), nbytes, _stream(x)),
        what)
    return y[0] if vec else y


def _gather_batched(x, w, scales, lhs, rhs, ishape, transpose, group_size, bits, mode, biases=None):
    """mx.gather_qmm through kmi_qmm_batched's gather form, one batch entry
    per (lhs, rhs) pair: the scaled modes, and transpose=False."""
    what = "gather_qmm"
    M, K = x.shape[-2], x.shape[-1]
    E = math.prod(w.shape[:-2])
    wc = w.reshape(E, *w.shape[-2:]).contiguous()
    sc = scales.reshape(E, *scales.shape[-2:]).contiguous()
    bc = biases.reshape(E, *biases.shape[-2:]).contiguous() if biases is not None else None
    if transpose:
        N, Kw = wc.shape[1], wc.shape[2] * 32 // bits
    else:
        N, Kw = wc.shape[2] * 32 // bits, wc.shape[1]
    if Kw != K or sc.shape[-1] * group_size != (K if transpose else N):
        raise ValueError(f"{what}: x has {K} features; w {tuple(w.shape)}, scales {tuple(scales.shape)}")
    xb = _aligned_rows(x.reshape(-1, M, K))
    P = lhs.numel()
    y = torch.empty(P, M, N, dtype=x.dtype, device=x.device)
    if P == 0:
        return y.reshape(*ishape, M, N)
    if transpose and (wc.data_ptr() % 16 or wc.stride(1) % 4 or wc.stride(0) % 4):
        raise ValueError(f"{what}: weight rows must be 16-byte aligned")
    shape = torch.tensor([P], dtype=torch.int64)
    xs = torch.tensor([xb.stride(0), xb.stride(1)], dtype=torch.int64)
    ws_ = torch.tensor([wc.stride(0), wc.stride(1)], dtype=torch.int64)
    ss = torch.tensor([sc.stride(0), sc.stride(1)], dtype=torch.int64)
    L = _lib()
    nbytes = L.kmi_qmm_batched_workspace_bytes(1, shape.data_ptr(), M, K, N)
    ws = _workspace(nbytes, x.device)
    _abi.check(L.kmi_qmm_batched(
        _ptr(xb), xs.data_ptr(), _ptr(wc), ws_.data_ptr(), _ptr(sc), _ptr(bc), ss.data_ptr(), 1, shape.data_ptr(),
        M, K, N, int(bool(transpose)), DTYPE_CODE[x.dtype], group_size, bits, MODE_CODE[mode], _ptr(rhs),
        _ptr(lhs), E, xb.shape[0], 1.0, _ptr(y), N, _ptr(ws), nbytes, _stream(x)), what)
    return y.reshape(*ishape, M, N)


#: the default lhs of a gather (every batch element of x, broadcast against
#: rhs), kept per shape: built once instead of on every call
_DEFAULT_LHS: dict = {}


def _default_lhs(xbatch, shape, dev):
    key = (xbatch, shape, str(dev))
    t = _DEFAULT_LHS.get(key)
    if t is None:
        base = torch.arange(math.prod(xbatch), device=dev, dtype=torch.int32).reshape(xbatch)
        t = torch.broadcast_to(base, shape).reshape(-1).contiguous()
        if len(_DEFAULT_LHS) > 64:
            _DEFAULT_LHS.clear()
        _DEFAULT_LHS[key] = t
    return t


def _flat_indices(x, w, lhs_indices, rhs_indices):
    """mx.gather_qmm's index semantics: lhs defaults to every batch element
    of x, rhs to every batch element of w; the two broadcast together."""
    dev = x.device
    xbatch = tuple(x.shape[:-2])
    wbatch = tuple(w.shape[:-2])
    if lhs_indices is None and rhs_indices is not None:
        rhs = torch.as_tensor(rhs_indices, device=dev)
        if rhs.dtype.is_floating_point:
            raise ValueError("gather_qmm: indices must be integers")
        try:
            shape = tuple(torch.broadcast_shapes(xbatch, tuple(rhs.shape)))
        except RuntimeError as e:
            raise ValueError(f"gather_qmm: x batch {xbatch} and indices {tuple(rhs.shape)} do not broadcast") from e
        rhs = torch.broadcast_to(rhs, shape).reshape(-1)
        rhs = (rhs if rhs.dtype == torch.int32 else rhs.to(torch.int32)).contiguous()
        return _default_lhs(xbatch, shape, dev), rhs, shape
    if lhs_indices is None:
        lhs_indices = torch.arange(math.prod(xbatch), device=dev, dtype=torch.int32).reshape(xbatch)
    if rhs_indices is None:
        rhs_indices = torch.arange(math.prod(wbatch), device=dev, dtype=torch.int32).reshape(wbatch)
    lhs = torch.as_tensor(lhs_indices, device=dev)
    rhs = torch.as_tensor(rhs_indices, device=dev)
    if lhs.dtype.is_floating_point or rhs.dtype.is_floating_point:
        raise ValueError("gather_qmm: indices must be integers")
    lhs, rhs = torch.broadcast_tensors(lhs, rhs)
    shape = tuple(lhs.shape)
    return (lhs.reshape(-1).to(torch.int32).contiguous(),
            rhs.reshape(-1).to(torch.int32).contiguous(), shape)


def gather_qmm(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
               biases: torch.Tensor | None = None, lhs_indices=None, rhs_indices=None,
               transpose: bool = True, group_size: int | None = None, bits: int | None = None,
               mode: str = "affine", sorted_indices: bool = False):
    """``mx.gather_qmm``: out[i] = x[lhs[i]] @ What[rhs[i]]^T for x
    [..., M, K] and w [..., N, K*bits/32]; out [*broadcast(lhs, rhs), M, N].
    Rows are grouped by expert on the GPU whatever ``sorted_indices`` says,
    so each routed expert's weights are read once.  The mxfp4 / mxfp8
    modes (uint8 E8M0 scales, no biases) run the batched kernel's gather
    form, either orientation."""
    _check_mode(mode, allow_mx=True)
    group_size, bits = _resolve(group_size, bits, mode)
    if x.ndim < 2 or w.ndim < 3:
        raise ValueError("gather_qmm: x needs [..., M, K] and w [..., N, K*bits/32]")
    if mode != "affine":
        _check_mx("gather_qmm", scales, biases, group_size, bits, mode)
        _on_gpu(x, w, scales)
        if x.dtype != torch.bfloat16:
            raise ValueError("gather_qmm: only bfloat16 activations are implemented")
        lhs, rhs, ishape = _flat_indices(x, w, lhs_indices, rhs_indices)
        return _gather_batched(x, w, scales, lhs, rhs, ishape, transpose, group_size, bits, mode)
    if not transpose:
        _check_affine_operands_t(x, w, scales, biases, group_size, bits, "gather_qmm")
        lhs, rhs, ishape = _flat_indices(x, w, lhs_indices, rhs_indices)
        return _gather_batched(x, w, scales, lhs, rhs, ishape, False, group_size, bits, mode, biases)
    _check_affine_operands(x, w, scales, biases, group_size, bits, "gather_qmm")
    M, K = x.shape[-2], x.shape[-1]
    N = w.shape[-2]
    E = math.prod(w.shape[:-2])
    Xb = math.prod(x.shape[:-2])
    lhs, rhs, ishape = _flat_indices(x, w, lhs_indices, rhs_indices)
    P = lhs.numel()
    y = torch.empty(*ishape, M, N, dtype=x.dtype, device=x.device)
    if P == 0:
        return y
    L = _lib()
    nbytes = L.kmi_gather_qmm_workspace_bytes(P, M, E, K, N, group_size, bits)
    ws = _workspace(nbytes, x.device)
    xc, wc, sc, bc = x.contiguous(), w.contiguous(), scales.contiguous(), biases.contiguous()
    _abi.check(L.kmi_gather_qmm(_ptr(xc), Xb, M, K, _ptr(wc), _ptr(sc), _ptr(bc), E, N,
                                _ptr(lhs), _ptr(rhs), P, DTYPE_CODE[x.dtype], group_size, bits,
                                int(bool(sorted_indices)), _ptr(y), _ptr(ws), nbytes,
                                _stream(x)), "gather_qmm")
    return y


# --- MoE glue --------------------------------------------------------------------

def moe_route(logits: torch.Tensor, k: int):
    """SparseMoeBlock's router (qwen3_5.py:174-179): softmax over the last
    axis in float32, the top ``k`` (descending; equal probabilities lower
    expert first), renormalized in float32 and rounded to the logits' dtype.
    Returns (inds int32 [..., k], scores [..., k])."""
    _on_gpu(logits)
    if logits.dtype not in DTYPE_CODE:
        raise ValueError(f"moe_route: dtype {logits.dtype}")
    E = logits.shape[-1]
    lg = logits.contiguous()
    T = lg.numel() // E if E else 0
    inds = torch.empty(*logits.shape[:-1], k, dtype=torch.int32, device=logits.device)
    scores = torch.empty(*logits.shape[:-1], k, dtype=logits.dtype, device=logits.device)
    _abi.check(_lib().kmi_moe_route(_ptr(lg), DTYPE_CODE[lg.dtype], T, E, k, _ptr(inds),
                                    _ptr(scores), _stream(lg)), "moe_route")
    return inds, scores


def swiglu(gate: torch.Tensor, up: torch.Tensor | None = None):
    """_SwiGLU: round(round(silu_f32(gate)) * up).  With ``up`` None,
    ``gate`` is one stacked [..., 2I] projection: gate = [..., :I],
    up = [..., I:]."""
    if up is None:
        I = gate.shape[-1] // 2
        src = gate.contiguous()
        g_, u_, ld = src, src[..., I:], 2 * I
        shape = (*gate.shape[:-1], I)
    else:
        if gate.shape != up.shape or gate.dtype != up.dtype:
            raise ValueError("swiglu: gate and up differ in shape or dtype")
        g_, u_ = gate.contiguous(), up.contiguous()
        I, ld, shape = gate.shape[-1], gate.shape[-1], tuple(gate.shape)
    _on_gpu(g_, u_)
    rows = math.prod(shape[:-1])
    out = torch.empty(shape, dtype=gate.dtype, device=gate.device)
    _abi.check(_lib().kmi_swiglu(_ptr(g_), _ptr(u_), ld, DTYPE_CODE[gate.dtype], rows, I,
                                 _ptr(out), _stream(gate)), "swiglu")
    return out


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None):
    """mlx's nn.Linear: x [..., K] @ weight[N, K]^T, or addmm(bias, x,
    weight^T) with one rounding of the fp32 sum plus the bias
    (kmi_linear).  bfloat16 or float16, shared by x, weight and bias."""
    _on_gpu(x, weight)
    if x.dtype not in (torch.bfloat16, torch.float16) or weight.dtype != x.dtype:
        raise ValueError(f"linear: x and weight must share bfloat16 or float16 (got {x.dtype}, {weight.dtype})")
    if weight.dim() != 2 or x.shape[-1] != weight.shape[1]:
        raise ValueError(f"linear: x {tuple(x.shape)} and weight {tuple(weight.shape)} do not match")
    N, K = weight.shape
    if K % 8:
        raise ValueError(f"linear: K={K} must be a multiple of 8")
    if bias is not None:
        _on_gpu(bias)
        if bias.shape != (N,) or bias.dtype != x.dtype:
            raise ValueError(f"linear: bias must be [{N}] of {x.dtype}")
        bias = bias.contiguous()
    xc, wc = _aligned16(x), _aligned16(weight)
    M = xc.numel() // K if K else 0
    y = torch.empty(*x.shape[:-1], N, dtype=x.dtype, device=x.device)
    _abi.check(_lib().kmi_linear(_ptr(xc), M, K, _ptr(wc), N, _ptr(bias), DTYPE_CODE[x.dtype], _ptr(y),
                                 _stream(x)), "linear")
    return y


def add_bias(y: torch.Tensor, bias: torch.Tensor, indices: torch.Tensor | None = None) -> torch.Tensor:
    """y + bias as its own rounded op (nn.QuantizedLinear's bias), or, with
    ``indices`` [...] of experts, y[..., M, N] + bias[indices][..., None, :]
    (QuantizedSwitchLinear's, switch_layers.py:82-85).  Returns a new
    tensor (kmi_add_bias on a copy of y)."""
    _on_gpu(y, bias)
    if y.dtype not in (torch.bfloat16, torch.float16) or bias.dtype != y.dtype:
        raise ValueError("add_bias: y and bias must share bfloat16 or float16")
    N = y.shape[-1]
    out = y.contiguous().clone()
    if indices is None:
        if bias.shape != (N,):
            raise ValueError(f"add_bias: bias must be [{N}]")
        idx, per, E = None, 1, 1
    else:
        _on_gpu(indices)
        if bias.dim() != 2 or bias.shape[1] != N or tuple(y.shape[:-2]) != tuple(indices.shape):
            raise ValueError("add_bias: y [..., M, N], indices [...] and bias [E, N] must agree")
        idx, per, E = indices.reshape(-1).to(torch.int32).contiguous(), y.shape[-2], bias.shape[0]
    rows = out.numel() // N
    bc = bias.contiguous()
    _abi.check(_lib().kmi_add_bias(_ptr(out), rows, N, _ptr(bc), _ptr(idx), per, E, DTYPE_CODE[y.dtype],
                                   _stream(y)), "add_bias")
    return out


def moe_combine(y: torch.Tensor, scores: torch.Tensor):
    """(y * scores[..., None]).sum(-2) with the reference's rounding: each
    product rounded to the dtype, the k products summed once.
    y [..., k, H], scores [..., k] -> [..., H]."""
    _on_gpu(y, scores)
    if y.dtype != scores.dtype or y.shape[:-1] != scores.shape:
        raise ValueError("moe_combine: y [..., k, H] and scores [..., k] must agree")
    k, H = y.shape[-2], y.shape[-1]
    T = math.prod(y.shape[:-2])
    out = torch.empty(*y.shape[:-2], H, dtype=y.dtype, device=y.device)
    yc, sc = y.contiguous(), scores.contiguous()
    _abi.check(_lib().kmi_moe_combine(_ptr(yc), _ptr(sc), DTYPE_CODE[y.dtype], T, k, H,
                                      _ptr(out), _stream(y)),
               "moe_combine")
    return out


def moe_shared_add(y: torch.Tensor, gate: torch.Tensor, shared_y: torch.Tensor):
    """y + _sigmoid(gate) * shared_y with the reference's roundings
    (qwen3_5.py:184-187); gate [..., 1] is the shared_expert_gate logit."""
    _on_gpu(y, gate, shared_y)
    if y.shape != shared_y.shape or gate.shape[:-1] != y.shape[:-1] or gate.shape[-1] != 1:
        raise ValueError("moe_shared_add: y, shared_y [..., H] and gate [..., 1] must agree")
    H = y.shape[-1]
    T = math.prod(y.shape[:-1])
    out = torch.empty_like(y)
    yc, gc, sc = y.contiguous(), gate.contiguous(), shared_y.contiguous()
    _abi.check(_lib().kmi_moe_shared_add(_ptr(yc), _ptr(gc), _ptr(sc), DTYPE_CODE[y.dtype], T, H,
                                         _ptr(out), _stream(y)), "moe_shared_add")
    return out


def switch_glu(x: torch.Tensor, indices: torch.Tensor, w_gu, s_gu, b_gu, w_down, s_down, b_down,
               scores: torch.Tensor | None = None, group_size: int = 64, bits: int = 4):
    """SwitchGLU with the _SwiGLU activation, and the weighted combine when
    ``scores`` is given, in one library call (kmi_switch_glu).

    x [..., H] bf16; indices [..., k]; the gate and up projections stacked
    per expert (w_gu [E, 2I, H*bits/32], s_gu/b_gu [E, 2I, H/group]); down
    [E, H, I*bits/32].  Returns [..., k, H], or [..., H] with scores."""
    _on_gpu(x, indices, w_gu, s_gu, b_gu, w_down, s_down, b_down, scores)
    if x.dtype != torch.bfloat16:
        raise ValueError("switch_glu: only bfloat16 activations are implemented")
    lead, H = tuple(x.shape[:-1]), x.shape[-1]
    k = indices.shape[-1]
    if tuple(indices.shape[:-1]) != lead:
        raise ValueError("switch_glu: indices [..., k] must match x [..., H]")
    E = w_gu.shape[0]
    I = _check_experts("switch_glu", H, E, w_gu, s_gu, b_gu, w_down, s_down, b_down, group_size, bits)
    T = math.prod(lead)
    xc = x.contiguous()
    ic = indices.reshape(T, k).to(torch.int32).contiguous()
    ts = [t.contiguous() for t in (w_gu, s_gu, b_gu, w_down, s_down, b_down)]
    sc = None
    if scores is not None:
        if scores.shape != indices.shape or scores.dtype != x.dtype:
            raise ValueError("switch_glu: scores must match indices in shape and x in dtype")
        sc = scores.contiguous()
        out = torch.empty(*lead, H, dtype=x.dtype, device=x.device)
    else:
        out = torch.empty(*lead, k, H, dtype=x.dtype, device=x.device)
    if T == 0:
        return out
    L = _lib()
    nbytes = L.kmi_switch_glu_workspace_bytes(T, H, I, k, E, group_size, bits)
    ws = _workspace(nbytes, x.device)
    _abi.check(L.kmi_switch_glu(_ptr(xc), T, H, I, k, _ptr(ic), _ptr(sc), *[_ptr(t) for t in ts[:3]],
                                *[_ptr(t) for t in ts[3:]], E, DTYPE_CODE[x.dtype], group_size, bits,
                                _ptr(out), _ptr(ws), nbytes, _stream(x)), "switch_glu")
    return out


def switch_glu_mx(x: torch.Tensor, indices: torch.Tensor, w_gu, s_gu, w_down, s_down,
                  scores: torch.Tensor | None = None, mode: str = "mxfp4"):
    """``switch_glu`` for experts in an OCP microscaled mode (kmi_switch_glu_mx):
    mxfp4 (E2M1) or mxfp8 (E4M3) codes, uint8 E8M0 scales per 32 inputs, no
    biases; gate and up stacked per expert (w_gu [E, 2I, H*bits/32], s_gu
    [E, 2I, H/32])."""
    _on_gpu(x, indices, w_gu, s_gu, w_down, s_down, scores)
    if mode not in _MX_BITS:
        raise ValueError(f"switch_glu_mx: mode {mode!r} (mxfp4 or mxfp8)")
    if x.dtype != torch.bfloat16:
        raise ValueError("switch_glu_mx: only bfloat16 activations are implemented")
    if s_gu.dtype != torch.uint8 or s_down.dtype != torch.uint8:
        raise ValueError("switch_glu_mx: scales must be uint8 E8M0")
    lead, H = tuple(x.shape[:-1]), x.shape[-1]
    k = indices.shape[-1]
    if tuple(indices.shape[:-1]) != lead:
        raise ValueError("switch_glu_mx: indices [..., k] must match x [..., H]")
    E = w_gu.shape[0]
    I = _check_experts("switch_glu_mx", H, E, w_gu, s_gu, None, w_down, s_down, None, 32, _MX_BITS[mode])
    T = math.prod(lead)
    xc = x.contiguous()
    ic = indices.reshape(T, k).to(torch.int32).contiguous()
    ts = [t.contiguous() for t in (w_gu, s_gu, w_down, s_down)]
    sc = None
    if scores is not None:
        if scores.shape != indices.shape or scores.dtype != x.dtype:
            raise ValueError("switch_glu_mx: scores must match indices in shape and x in dtype")
        sc = scores.contiguous()
        out = torch.empty(*lead, H, dtype=x.dtype, device=x.device)
    else:
        out = torch.empty(*lead, k, H, dtype=x.dtype, device=x.device)
    if T == 0:
        return out
    L = _lib()
    nbytes = L.kmi_switch_glu_workspace_bytes(T, H, I, k, E, 32, _MX_BITS[mode])
    ws = _workspace(nbytes, x.device)
    _abi.check(L.kmi_switch_glu_mx(_ptr(xc), T, H, I, k, _ptr(ic), _ptr(sc), *[_ptr(t) for t in ts], E,
                                   DTYPE_CODE[x.dtype], 1 if mode == "mxfp4" else 2, _ptr(out), _ptr(ws),
                                   nbytes, _stream(x)), "switch_glu_mx")
    return out


def moe_experts(x: torch.Tensor, logits: torch.Tensor, k: int, w_gu, s_gu, b_gu, w_down, s_down, b_down,
                group_size: int = 64, bits: int = 4):
    """SparseMoeBlock's routed part from its router logits in one library
    call (kmi_moe_experts): route (as ``moe_route``), SwitchGLU, weighted
    combine.  x [..., H] and logits [..., E] bf16.  Returns (out [..., H],
    inds [..., k] int32, scores [..., k])."""
    _on_gpu(x, logits, w_gu, s_gu, b_gu, w_down, s_down, b_down)
    if x.dtype != torch.bfloat16 or logits.dtype != torch.bfloat16:
        raise ValueError("moe_experts: bfloat16 activations and logits only")
    lead, H = tuple(x.shape[:-1]), x.shape[-1]
    if tuple(logits.shape[:-1]) != lead:
        raise ValueError("moe_experts: logits [..., E] must match x [..., H]")
    E = logits.shape[-1]
    if w_gu.shape[0] != E or w_down.shape[0] != E:
        raise ValueError(f"moe_experts: {E} logits per token for {w_gu.shape[0]} gate/up and "
                         f"{w_down.shape[0]} down experts")
    I = _check_experts("moe_experts", H, E, w_gu, s_gu, b_gu, w_down, s_down, b_down, group_size, bits)
    T = math.prod(lead)
    out = torch.empty(*lead, H, dtype=x.dtype, device=x.device)
    inds = torch.empty(*lead, k, dtype=torch.int32, device=x.device)
    scores = torch.empty(*lead, k, dtype=x.dtype, device=x.device)
    if T == 0:
        return out, inds, scores
    xc, lc = x.contiguous(), logits.contiguous()
    ts = [t.contiguous() for t in (w_gu, s_gu, b_gu, w_down, s_down, b_down)]
    L = _lib()
    nbytes = L.kmi_switch_glu_workspace_bytes(T, H, I, k, E, group_size, bits)
    ws = _workspace(nbytes, x.device)
    _abi.check(L.kmi_moe_experts(_ptr(xc), _ptr(lc), T, H, I, k, E, *[_ptr(t) for t in ts], DTYPE_CODE[x.dtype],
                                 group_size, bits, _ptr(out), _ptr(inds), _ptr(scores), _ptr(ws), nbytes,
                                 _stream(x)), "moe_experts")
    return out, inds, scores


# --- VQ codebook-decode experts ---------------------------------------------------

_CODE_BYTES = {torch.uint8: 1, torch.uint16: 2, torch.int16: 2}


def _vq_operands(codes, codebook, scales):
    if codes.dtype not in _CODE_BYTES:
        raise ValueError(f"vq: codes must be uint8 or uint16 (got {codes.dtype})")
    if codebook.dtype != torch.float16 or scales.dtype != torch.float16:
        raise ValueError("vq: codebook and scales must be float16")
    if codebook.ndim != 2:
        raise ValueError("vq: codebook [k, dim]")
    return _CODE_BYTES[codes.dtype], codebook.shape[0], codebook.shape[1]


def vq_gather_qmm(x: torch.Tensor, codes: torch.Tensor, codebook: torch.Tensor, scales: torch.Tensor,
                  lhs_indices=None, rhs_indices=None, scale_group: int = 0):
    """VQSwitchLinear's product: out[i] = x[lhs[i]] @ What[rhs[i]]^T with
    What[e, o, j] = scales[e, o, j / scale_group] * codebook[codes[e, o, j/dim]][j % dim]
    (scale_group 0: scales [E, N], one per output channel).  x [..., M, K];
    codes [E, N, K/dim]; out [*broadcast(lhs, rhs), M, N]."""
    cbytes, kc, dim = _vq_operands(codes, codebook, scales)
    _on_gpu(x, codes, codebook, scales)
    if x.dtype != torch.bfloat16:
        raise ValueError("vq_gather_qmm: only bfloat16 activations are implemented")
    E, N = codes.shape[0], codes.shape[1]
    M, K = x.shape[-2], x.shape[-1]
    if codes.shape[2] * dim != K:
        raise ValueError(f"vq_gather_qmm: codes {tuple(codes.shape)} do not cover K={K}")
    lhs, rhs, ishape = _vq_indices(x, E, lhs_indices, rhs_indices)
    P = lhs.numel()
    y = torch.empty(*ishape, M, N, dtype=x.dtype, device=x.device)
    if P == 0:
        return y
    # one (pair, row) per kernel row: x rows lhs*M + m, experts repeated
    m = torch.arange(M, device=x.device, dtype=torch.int32)
    rows = (lhs.view(-1, 1) * M + m).reshape(-1).contiguous()
    experts = rhs.view(-1, 1).expand(P, M).reshape(-1).contiguous()
    xc = x.reshape(-1, K).contiguous()
    cc, cbc, sc = codes.contiguous(), codebook.contiguous(), scales.contiguous()
    _abi.check(_lib().kmi_vq_gather_qmm(_ptr(xc), xc.shape[0], K, _ptr(cc), cbytes, _ptr(cbc), kc, dim,
                                        _ptr(sc), scale_group, E, N, _ptr(rows), _ptr(experts), P * M,
                                        DTYPE_CODE[x.dtype], _ptr(y), _stream(x)), "vq_gather_qmm")
    return y


def _vq_packed_operands(codes, codebook, scales, pack_bits, group, K, what):
    if codes.dtype not in (torch.uint32, torch.int32) or codes.ndim != 3:
        raise ValueError(f"{what}: packed codes must be uint32 [E, N, W]")
    if codebook.dtype != torch.float16 or scales.dtype != torch.float16 or codebook.ndim != 2:
        raise ValueError(f"{what}: codebook [k, dim] and scales must be float16")
    kc, dim = codebook.shape
    if K % dim or K % group:
        raise ValueError(f"{what}: K={K} is not a multiple of dim {dim} and group {group}")
    W = (K // dim + 31) // 32 * pack_bits
    if codes.shape[2] != W:
        raise ValueError(f"{what}: codes rows are {codes.shape[2]} wide; K={K} at dim {dim} is {W} "
                         f"packed {pack_bits}-bit words")
    if tuple(scales.shape) != (codes.shape[0], codes.shape[1], K // group):
        raise ValueError(f"{what}: scales {tuple(scales.shape)} do not match codes {tuple(codes.shape)} "
                         f"at group {group}")
    return kc, dim


def vq_packed_gather_qmm(x: torch.Tensor, codes: torch.Tensor, codebook: torch.Tensor, scales: torch.Tensor,
                         pack_bits: int, group: int, lhs_indices=None, rhs_indices=None,
                         rows_are_pairs: bool = False):
    """VQSwitchLinear's product over the bit-packed code layout of the VQ
    artifacts (kmi_vq_packed_gather_qmm): What[e, o, i] =
    scales[e, o, i / group] * codebook[field(e, o, i / dim)][i % dim],
    fields of ``pack_bits`` bits; out[i] = x[lhs[i]] @ What[rhs[i]]^T.
    ``rows_are_pairs``: the caller guarantees lhs[i] == i (x holds one row
    per pair), so no row list is built."""
    _on_gpu(x, codes, codebook, scales)
    if x.dtype != torch.bfloat16:
        raise ValueError("vq_packed_gather_qmm: only bfloat16 activations are implemented")
    M, K = x.shape[-2], x.shape[-1]
    kc, dim = _vq_packed_operands(codes, codebook, scales, pack_bits, group, K, "vq_packed_gather_qmm")
    E, N = codes.shape[0], codes.shape[1]
    xc = x.reshape(-1, K).contiguous()
    if rows_are_pairs:
        # one x row per pair (x row p): the expert list is all the kernel needs
        rhs = torch.as_tensor(rhs_indices, device=x.device).reshape(-1)
        rhs = (rhs if rhs.dtype == torch.int32 else rhs.to(torch.int32)).contiguous()
        P, ishape = rhs.numel(), (rhs.numel(),)
        if M != 1 or xc.shape[0] != P:
            raise ValueError("vq_packed_gather_qmm: rows_are_pairs takes x [P, 1, K] with P = len(rhs)")
    else:
        lhs, rhs, ishape = _vq_indices(x, E, lhs_indices, rhs_indices)
        P = lhs.numel()
    y = torch.empty(*ishape, M, N, dtype=x.dtype, device=x.device)
    if P == 0:
        return y
    cc, cbc, sc = codes.contiguous(), codebook.contiguous(), scales.contiguous()
    if rows_are_pairs:
        rows, div, experts = None, 1, rhs
    else:
        m = torch.arange(M, device=x.device, dtype=torch.int32)
        rows = (lhs.view(-1, 1) * M + m).reshape(-1).contiguous()
        div = 1
        experts = rhs.view(-1, 1).expand(P, M).reshape(-1).contiguous()
    _abi.check(_lib().kmi_vq_packed_gather_qmm(
        _ptr(xc), xc.shape[0], K, _ptr(cc), pack_bits, _ptr(cbc), kc, dim, _ptr(sc), group, E, N,
        _ptr(rows), div, _ptr(experts), P * M, DTYPE_CODE[x.dtype], _ptr(y), _stream(x)), "vq_packed_gather_qmm")
    return y


def vq_packed_glu(x: torch.Tensor, indices: torch.Tensor, gate, up, pack_bits: int, group: int):
    """SwitchGLU's gate and up products over packed VQ experts with
    _SwiGLU, one launch (kmi_vq_packed_glu): x [..., H], indices [..., k]
    -> act [..., k, I]; gate / up = (codes, codebook, scales)."""
    _on_gpu(x, indices, *gate, *up)
    if x.dtype != torch.bfloat16:
        raise ValueError("vq_packed_glu: only bfloat16 activations are implemented")
    H = x.shape[-1]
    kc, dim = _vq_packed_operands(gate[0], gate[1], gate[2], pack_bits, group, H, "vq_packed_glu")
    _vq_packed_operands(up[0], up[1], up[2], pack_bits, group, H, "vq_packed_glu")
    if up[0].shape != gate[0].shape or up[1].shape != gate[1].shape:
        raise ValueError("vq_packed_glu: gate and up differ in shape")
    E, I = gate[0].shape[0], gate[0].shape[1]
    lead, k = tuple(indices.shape[:-1]), indices.shape[-1]
    T = math.prod(lead)
    if tuple(x.shape[:-1]) != lead:
        raise ValueError("vq_packed_glu: x [..., H] and indices [..., k] must share leading dimensions")
    act = torch.empty(*lead, k, I, dtype=x.dtype, device=x.device)
    if T * k == 0:
        return act
    experts = indices.reshape(-1).to(torch.int32).contiguous()
    xc = x.reshape(T, H).contiguous()
    g = tuple(t.contiguous() for t in gate)
    u = tuple(t.contiguous() for t in up)
    _abi.check(_lib().kmi_vq_packed_glu(
        _ptr(xc), T, H, I, _ptr(g[0]), _ptr(g[2]), _ptr(g[1]), _ptr(u[0]), _ptr(u[2]), _ptr(u[1]), pack_bits,
        kc, dim, group, E, None, k, _ptr(experts), T * k, DTYPE_CODE[x.dtype], _ptr(act), _stream(x)),
        "vq_packed_glu")
    return act


def vq_packed_switch_glu(x: torch.Tensor, indices: torch.Tensor, gate, up, down, pack_bits: int, group: int,
                         scores: torch.Tensor | None = None):
    """SwitchGLU over packed VQ experts in one library call
    (kmi_vq_packed_switch_glu): gate/up with the _SwiGLU epilogue, down, and
    with scores [..., k] the weighted combine.  gate / up / down = (codes,
    codebook, scales).  x [..., H], indices [..., k] -> [..., k, H], or
    [..., H] with scores."""
    _on_gpu(x, indices, *gate, *up, *down, scores)
    if x.dtype != torch.bfloat16:
        raise ValueError("vq_packed_switch_glu: only bfloat16 activations are implemented")
    H = x.shape[-1]
    kc, dim = _vq_packed_operands(gate[0], gate[1], gate[2], pack_bits, group, H, "vq_packed_switch_glu")
    _vq_packed_operands(up[0], up[1], up[2], pack_bits, group, H, "vq_packed_switch_glu")
    if up[0].shape != gate[0].shape or up[1].shape != gate[1].shape:
        raise ValueError("vq_packed_switch_glu: gate and up differ in shape")
    E, I = gate[0].shape[0], gate[0].shape[1]
    kd, dd = _vq_packed_operands(down[0], down[1], down[2], pack_bits, group, I, "vq_packed_switch_glu")
    if down[0].shape[0] != E or down[0].shape[1] != H or kd != kc or dd != dim:
        raise ValueError("vq_packed_switch_glu: down must be [E, H, *] over I inputs with gate's codebook shape")
    lead, k = tuple(indices.shape[:-1]), indices.shape[-1]
    if tuple(x.shape[:-1]) != lead:
        raise ValueError("vq_packed_switch_glu: x [..., H] and indices [..., k] must share leading dimensions")
    T = math.prod(lead)
    sc = None
    if scores is not None:
        if scores.shape != indices.shape or scores.dtype != x.dtype:
            raise ValueError("vq_packed_switch_glu: scores must match indices in shape and x in dtype")
        sc = scores.contiguous()
        out = torch.empty(*lead, H, dtype=x.dtype, device=x.device)
    else:
        out = torch.empty(*lead, k, H, dtype=x.dtype, device=x.device)
    if T == 0:
        return out
    xc = x.reshape(T, H).contiguous()
    ic = indices.reshape(T, k).to(torch.int32).contiguous()
    g, u, d = (tuple(t.contiguous() for t in m) for m in (gate, up, down))
    L = _lib()
    nbytes = L.kmi_vq_packed_switch_glu_workspace_bytes(T, H, I, k)
    ws = _workspace(nbytes, x.device)
    _abi.check(L.kmi_vq_packed_switch_glu(
        _ptr(xc), T, H, I, k, _ptr(ic), _ptr(sc), _ptr(g[0]), _ptr(g[2]), _ptr(g[1]), _ptr(u[0]), _ptr(u[2]),
        _ptr(u[1]), _ptr(d[0]), _ptr(d[2]), _ptr(d[1]), pack_bits, kc, dim, group, E, DTYPE_CODE[x.dtype],
        _ptr(out), _ptr(ws), nbytes, _stream(x)), "vq_packed_switch_glu")
    return out


def vq_packed_experts(x: torch.Tensor, logits: torch.Tensor, k: int, gate, up, down, pack_bits: int, group: int):
    """The packed VQ experts of a SparseMoeBlock from its router logits in one
    library call (kmi_vq_packed_experts): route (as ``moe_route``), packed
    VQ SwitchGLU, weighted combine.  x [..., H] and logits [..., E] bf16;
    gate / up / down = (codes, codebook, scales).  Returns (out [..., H],
    inds [..., k] int32, scores [..., k])."""
    _on_gpu(x, logits, *gate, *up, *down)
    if x.dtype != torch.bfloat16 or logits.dtype != torch.bfloat16:
        raise ValueError("vq_packed_experts: bfloat16 activations and logits only")
    H = x.shape[-1]
    kc, dim = _vq_packed_operands(gate[0], gate[1], gate[2], pack_bits, group, H, "vq_packed_experts")
    _vq_packed_operands(up[0], up[1], up[2], pack_bits, group, H, "vq_packed_experts")
    if up[0].shape != gate[0].shape or up[1].shape != gate[1].shape:
        raise ValueError("vq_packed_experts: gate and up differ in shape")
    E, I = gate[0].shape[0], gate[0].shape[1]
    kd, dd = _vq_packed_operands(down[0], down[1], down[2], pack_bits, group, I, "vq_packed_experts")
    if down[0].shape[0] != E or down[0].shape[1] != H or kd != kc or dd != dim:
        raise ValueError("vq_packed_experts: down must be [E, H, *] over I inputs with gate's codebook shape")
    lead = tuple(x.shape[:-1])
    if tuple(logits.shape) != lead + (E,):
        raise ValueError(f"vq_packed_experts: logits must be [..., {E}] over x's leading dimensions")
    T = math.prod(lead)
    out = torch.empty(*lead, H, dtype=x.dtype, device=x.device)
    inds = torch.empty(*lead, k, dtype=torch.int32, device=x.device)
    scores = torch.empty(*lead, k, dtype=x.dtype, device=x.device)
    if T == 0:
        return out, inds, scores
    xc, lc = x.reshape(T, H).contiguous(), logits.reshape(T, E).contiguous()
    g, u, d = (tuple(t.contiguous() for t in m) for m in (gate, up, down))
    L = _lib()
    nbytes = L.kmi_vq_packed_switch_glu_workspace_bytes(T, H, I, k)
    ws = _workspace(nbytes, x.device)
    _abi.check(L.kmi_vq_packed_experts(
        _ptr(xc), _ptr(lc), T, H, I, k, _ptr(g[0]), _ptr(g[2]), _ptr(g[1]), _ptr(u[0]), _ptr(u[2]), _ptr(u[1]),
        _ptr(d[0]), _ptr(d[2]), _ptr(d[1]), pack_bits, kc, dim, group, E, DTYPE_CODE[x.dtype], _ptr(out),
        _ptr(inds), _ptr(scores), _ptr(ws), nbytes, _stream(x)), "vq_packed_experts")
    return out, inds, scores


def _vq_indices(x, E, lhs_indices, rhs_indices):
    dev = x.device
    xbatch = tuple(x.shape[:-2])
    if lhs_indices is None:
        lhs_indices = torch.arange(math.prod(xbatch), device=dev, dtype=torch.int32).reshape(xbatch)
    if rhs_indices is None:
        rhs_indices = torch.arange(E, device=dev, dtype=torch.int32)
    lhs = torch.as_tensor(lhs_indices, device=dev)
    rhs = torch.as_tensor(rhs_indices, device=dev)
    lhs, rhs = torch.broadcast_tensors(lhs, rhs)
    shape = tuple(lhs.shape)
    return (lhs.reshape(-1).to(torch.int32).contiguous(), rhs.reshape(-1).to(torch.int32).contiguous(),
            shape)


def vq_glu(x: torch.Tensor, indices: torch.Tensor, gate, up, scale_group: int = 0):
    """The VQ gate and up projections of SwitchGLU with the _SwiGLU epilogue,
    one kernel: gate / up = (codes, codebook, scales).  x [..., H],
    indices [..., k] -> act [..., k, I]."""
    (cg, bg, sg_), (cu, bu, su) = gate, up
    cbytes, kc, dim = _vq_operands(cg, bg, sg_)
    if _vq_operands(cu, bu, su) != (cbytes, kc, dim) or cu.shape != cg.shape:
        raise ValueError("vq_glu: gate and up differ in layout")
    _on_gpu(x, indices, cg, bg, sg_, cu, bu, su)
    lead, H = tuple(x.shape[:-1]), x.shape[-1]
    k = indices.shape[-1]
    E, I = cg.shape[0], cg.shape[1]
    T = math.prod(lead)
    act = torch.empty(*lead, k, I, dtype=x.dtype, device=x.device)
    if T == 0:
        return act
    xc = x.reshape(T, H).contiguous()
    ic = indices.reshape(T, k).to(torch.int32).contiguous()
    ops = [t.contiguous() for t in (cg, sg_, bg, cu, su, bu)]
    _abi.check(_lib().kmi_vq_glu(_ptr(xc), T, H, I, k, _ptr(ic), *[_ptr(t) for t in ops], cbytes, kc, dim,
                                 scale_group, E, DTYPE_CODE[x.dtype], _ptr(act), _stream(x)), "vq_glu")
    return act



def vq_switch_glu(x: torch.Tensor, indices: torch.Tensor, gate, up, down, scale_group: int = 0,
                  scores: torch.Tensor | None = None):
    """SwitchGLU over VQ experts in one library call: gate/up with the
    _SwiGLU epilogue, down, and (with scores [..., k]) the weighted combine.
    gate / up / down = (codes, codebook, scales).  x [..., H], indices
    [..., k] -> [..., k, H], or [..., H] with scores."""
    (cg, bg, sg_), (cu, bu, su), (cd, bd, sd) = gate, up, down
    cbytes, kc, dim = _vq_operands(cg, bg, sg_)
    if (_vq_operands(cu, bu, su) != (cbytes, kc, dim) or _vq_operands(cd, bd, sd) != (cbytes, kc, dim)
            or cu.shape != cg.shape):
        raise ValueError("vq_switch_glu: gate, up and down differ in layout")
    _on_gpu(x, indices, cg, bg, sg_, cu, bu, su, cd, bd, sd)
    if x.dtype != torch.bfloat16:
        raise ValueError("vq_switch_glu: only bfloat16 activations are implemented")
    lead, H = tuple(x.shape[:-1]), x.shape[-1]
    k = indices.shape[-1]
    E, I = cg.shape[0], cg.shape[1]
    if cd.shape[0] != E or cd.shape[1] != H or cd.shape[2] * dim != I:
        raise ValueError(f"vq_switch_glu: down codes {tuple(cd.shape)} do not match [E, H, I/dim]")
    T = math.prod(lead)
    if scores is not None:
        if scores.dtype != x.dtype or tuple(scores.shape) != tuple(indices.shape):
            raise ValueError("vq_switch_glu: scores must match indices and the dtype of x")
        out = torch.empty(*lead, H, dtype=x.dtype, device=x.device)
    else:
        out = torch.empty(*lead, k, H, dtype=x.dtype, device=x.device)
    if T == 0:
        return out
    xc = x.reshape(T, H).contiguous()
    ic = indices.reshape(T, k).to(torch.int32).contiguous()
    scc = scores.reshape(T, k).contiguous() if scores is not None else None
    ops = [t.contiguous() for t in (cg, sg_, bg, cu, su, bu, cd, sd, bd)]
    nbytes = _lib().kmi_vq_switch_glu_workspace_bytes(T, H, I, k)
    ws = _workspace(nbytes, x.device)
    _abi.check(_lib().kmi_vq_switch_glu(_ptr(xc), T, H, I, k, _ptr(ic), _ptr(scc) if scc is not None else None,
                                        *[_ptr(t) for t in ops], cbytes, kc, dim, scale_group, E,
                                        DTYPE_CODE[x.dtype], _ptr(out), _ptr(ws), nbytes, _stream(x)),
               "vq_switch_glu")
    return out


def vq_experts(x: torch.Tensor, logits: torch.Tensor, k: int, gate, up, down, scale_group: int = 0):
    """The VQ experts of a SparseMoeBlock from its router logits in one
    library call (kmi_vq_experts): route (as ``moe_route``), VQ SwitchGLU,
    weighted combine.  x [..., H] and logits [..., E] bf16; gate / up / down
    = (codes, codebook, scales).  Returns (out [..., H], inds [..., k]
    int32, scores [..., k])."""
    (cg, bg, sg_), (cu, bu, su), (cd, bd, sd) = gate, up, down
    cbytes, kc, dim = _vq_operands(cg, bg, sg_)
    if (_vq_operands(cu, bu, su) != (cbytes, kc, dim) or _vq_operands(cd, bd, sd) != (cbytes, kc, dim)
            or cu.shape != cg.shape):
        raise ValueError("vq_experts: gate, up and down differ in layout")
    _on_gpu(x, logits, cg, bg, sg_, cu, bu, su, cd, bd, sd)
    if x.dtype != torch.bfloat16 or logits.dtype != torch.bfloat16:
        raise ValueError("vq_experts: bfloat16 activations and logits only")
    lead, H = tuple(x.shape[:-1]), x.shape[-1]
    if tuple(logits.shape[:-1]) != lead:
        raise ValueError("vq_experts: logits [..., E] must match x [..., H]")
    E, I = cg.shape[0], cg.shape[1]
    if logits.shape[-1] != E:
        raise ValueError(f"vq_experts: {logits.shape[-1]} logits for {E} experts")
    if cd.shape[0] != E or cd.shape[1] != H or cd.shape[2] * dim != I:
        raise ValueError(f"vq_experts: down codes {tuple(cd.shape)} do not match [E, H, I/dim]")
    T = math.prod(lead)
    out = torch.empty(*lead, H, dtype=x.dtype, device=x.device)
    inds = torch.empty(*lead, k, dtype=torch.int32, device=x.device)
    scores = torch.empty(*lead, k, dtype=x.dtype, device=x.device)
    if T == 0:
        return out, inds, scores
    xc, lc = x.reshape(T, H).contiguous(), logits.reshape(T, E).contiguous()
    ops = [t.contiguous() for t in (cg, sg_, bg, cu, su, bu, cd, sd, bd)]
    L = _lib()
    nbytes = L.kmi_vq_switch_glu_workspace_bytes(T, H, I, k)
    ws = _workspace(nbytes, x.device)
    _abi.check(L.kmi_vq_experts(_ptr(xc), _ptr(lc), T, H, I, k, *[_ptr(t) for t in ops], cbytes, kc, dim,
                                scale_group, E, DTYPE_CODE[x.dtype], _ptr(out), _ptr(inds), _ptr(scores), _ptr(ws),
                                nbytes, _stream(x)), "vq_experts")
    return out, inds, scores
