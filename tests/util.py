"""Shared helpers for the parity tests (tolerances, conversions)."""
from __future__ import annotations

import numpy as np

#: the bar for floating-point outputs: max |got - ref| / max |ref| and cosine
MAX_REL = 1e-2
MIN_COS = 0.9999


def rel_err(got, ref) -> float:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = max(np.abs(ref).max(), 1e-30)
    return float(np.abs(got - ref).max() / den)


def cosine(got, ref) -> float:
    a = np.asarray(got, np.float64).ravel()
    b = np.asarray(ref, np.float64).ravel()
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    if na == 0 and nb == 0:
        return 1.0
    return float(a @ b / (na * nb))


def assert_close(got, ref, max_rel=MAX_REL, min_cos=MIN_COS, what=""):
    r, c = rel_err(got, ref), cosine(got, ref)
    assert r <= max_rel and c >= min_cos, f"{what}: max rel err {r:.3e} (bar {max_rel}), cosine {c:.6f} (bar {min_cos})"
    return r, c


def bf16_normal(rng, shape, std=1.0):
    """N(0, std) rounded to bf16, as float32 numpy."""
    import oracle
    return oracle.bf16_round((rng.standard_normal(shape) * std).astype(np.float32))


def to_torch(a, dev, dtype):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev).to(dtype)


def to_numpy(t):
    """A bf16/fp16/fp32 tensor -> float32 numpy (exact)."""
    import torch
    return t.detach().to(torch.float32).cpu().numpy()


def u32_to_torch(a, dev):
    import torch
    a = np.ascontiguousarray(a, np.uint32)
    if not a.flags.writeable:
        a = a.copy()
    return torch.from_numpy(a.view(np.int32)).to(dev).view(torch.uint32)


def u32_to_numpy(t):
    import torch
    return t.detach().view(torch.int32).cpu().numpy().view(np.uint32)
