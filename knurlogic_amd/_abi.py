"""ctypes binding of libknurlogic_amd.so (the C ABI in include/knurlogic_amd.h).

The library is the only compute path: there is no CPU fallback.  If it is
missing or no GPU is visible, every op raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libknurlogic_amd.so"

P, I64, I, SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t

#: every exported entry point: name -> (restype, argtypes)
SIGNATURES = {
    "kmi_last_error": (ctypes.c_char_p, []),
    "kmi_abi_version": (I, []),
    "kmi_quantize_affine": (I, [P, I, I64, I64, I, I, P, P, P, P]),
    "kmi_kv_quantize_append": (I, [P, I, I64, I64, I64, I64, I, I, P, P, P, P, I64, I64, P]),
    "kmi_kv_quantize_append_kv": (I, [P, P, I, I64, I64, I64, I64, I64, I, I, P, P, P, P, P, P, P, P, I64, I64, P]),
    "kmi_dequantize_affine": (I, [P, P, P, I, I64, I64, I, I, P, I, I, P]),
    "kmi_qmm": (I, [P, I64, I64, I64, P, P, P, I, I, I, P, P, SZ, P]),
    "kmi_qmm_workspace_bytes": (SZ, [I64, I64, I64, I, I]),
    "kmi_qmm_mx": (I, [P, I64, I64, I64, P, P, I, I, P, P, SZ, P]),
    "kmi_qmm_mx_workspace_bytes": (SZ, [I64, I64, I64, I]),
    "kmi_qmm_noalloc_scratch_bytes": (SZ, []),
    "kmi_qmm_noalloc": (I, [P, I64, I64, I64, P, P, P, I, I, I, P, P]),
    "kmi_gather_qmm": (I, [P, I64, I64, I64, P, P, P, I64, I64, P, P, I64, I, I, I, I,
                           P, P, SZ, P]),
    "kmi_gather_qmm_workspace_bytes": (SZ, [I64, I64, I64, I64, I64, I, I]),
    "kmi_kv8_decode": (I, [P, I, I, I, I, I, P, P, P, P, P, P, P, I, I, I, I,
                           ctypes.c_float, P, I, P, P, SZ, P]),
    "kmi_kv8_workspace_bytes": (SZ, [I, I, I, I, I, I]),
    "kmi_dequantize_mx": (I, [P, P, I64, I64, I, P, I, P]),
    "kmi_quantize_mx": (I, [P, I, I64, I64, I, P, P, P]),
    "kmi_qmm_batched": (I, [P, P, P, P, P, P, P, I, P, I64, I64, I64, I, I, I, I, I, P, P, I64, I64,
                            ctypes.c_float, P, I64, P, SZ, P]),
    "kmi_qmm_batched_workspace_bytes": (SZ, [I, P, I64, I64, I64]),
    "kmi_masked_softmax": (I, [P, I64, I, P, I64, P, I, P, P, I64, P]),
    "kmi_vq_packed_gather_qmm": (I, [P, I64, I64, P, I, P, I, I, P, I, I64, I64, P, I64, P, I64, I, P, P]),
    "kmi_vq_packed_glu": (I, [P, I64, I64, I64, P, P, P, P, P, P, I, I, I, I, I64, P, I64, P, I64, I, P, P]),
    "kmi_linear": (I, [P, I64, I64, P, I64, P, I, P, P]),
    "kmi_add_bias": (I, [P, I64, I64, P, P, I64, I64, I, P]),
    "kmi_moe_route": (I, [P, I, I64, I, I, P, P, P]),
    "kmi_swiglu": (I, [P, P, I64, I, I64, I64, P, P]),
    "kmi_moe_combine": (I, [P, P, I, I64, I, I64, P, P]),
    "kmi_moe_shared_add": (I, [P, P, P, I, I64, I64, P, P]),
    "kmi_switch_glu": (I, [P, I64, I64, I64, I, P, P, P, P, P, P, P, P, I64, I, I, I, P, P, SZ, P]),
    "kmi_switch_glu_workspace_bytes": (SZ, [I64, I64, I64, I, I64, I, I]),
    "kmi_switch_glu_mx": (I, [P, I64, I64, I64, I, P, P, P, P, P, P, I64, I, I, P, P, SZ, P]),
    "kmi_moe_experts": (I, [P, P, I64, I64, I64, I, I64, P, P, P, P, P, P, I, I, I, P, P, P, P, SZ, P]),
    "kmi_vq_gather_qmm": (I, [P, I64, I64, P, I, P, I, I, P, I, I64, I64, P, P, I64, I, P, P]),
    "kmi_vq_glu": (I, [P, I64, I64, I64, I, P, P, P, P, P, P, P, I, I, I, I, I64, I, P, P]),
    "kmi_vq_switch_glu_workspace_bytes": (SZ, [I64, I64, I64, I]),
    "kmi_vq_switch_glu": (I, [P, I64, I64, I64, I, P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I64, I,
                              P, P, SZ, P]),
    "kmi_vq_experts": (I, [P, P, I64, I64, I64, I, P, P, P, P, P, P, P, P, P, I, I, I, I, I64, I, P, P, P,
                           P, SZ, P]),
    "kmi_vq_packed_switch_glu_workspace_bytes": (SZ, [I64, I64, I64, I]),
    "kmi_vq_packed_experts": (I, [P, P, I64, I64, I64, I, P, P, P, P, P, P, P, P, P, I, I, I, I, I64, I, P, P,
                                  P, P, SZ, P]),
    "kmi_vq_packed_switch_glu": (I, [P, I64, I64, I64, I, P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I64, I,
                                     P, P, SZ, P]),
    "kmi_read_probe": (I, [P, I64, I, P, P]),
    "kmi_mfma_probe": (I, [P, I, I, P, P, P]),
}

ABI_VERSION = 1

_lib = None


class KmiError(RuntimeError):
    """A HIP-side failure (launch error, missing workspace)."""


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Load the library and bind every entry point (no GPU needed)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"knurlogic_amd: {p} is not built; run __graft_entry__.build() "
            "(hipcc --offload-arch=gfx950). There is no CPU fallback.")
    L = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    if L.kmi_abi_version() != ABI_VERSION:
        raise RuntimeError(f"knurlogic_amd: ABI {L.kmi_abi_version()} != {ABI_VERSION}")
    if path is None:
        _lib = L
    return L


def check(rc: int, what: str) -> None:
    if rc == 0:
        return
    msg = (_lib.kmi_last_error() or b"").decode(errors="replace")
    if rc == -1:
        raise ValueError(f"[{what}] {msg}")
    raise KmiError(f"[{what}] error {rc}: {msg}")
