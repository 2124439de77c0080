"""The C ABI library loads and exports every symbol include/*.h declares,
and the Python mirror refuses what it must -- no GPU needed, no compute."""
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(kmi_\w+)\s*\(", text))
    return names


def test_header_declares_the_boundary():
    names = declared()
    for must in ("kmi_quantize_affine", "kmi_dequantize_affine", "kmi_qmm", "kmi_gather_qmm",
                 "kmi_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    import ctypes
    from knurlogic_amd import _abi
    lib = ctypes.CDLL(str(_abi.LIB_PATH))
    missing = [n for n in sorted(declared()) if not hasattr(lib, n)]
    assert not missing, missing
    # and the ctypes table binds exactly the declared set
    assert set(_abi.SIGNATURES) == declared()


def test_abi_version_and_error_channel():
    from knurlogic_amd import _abi
    L = _abi.load()
    assert L.kmi_abi_version() == _abi.ABI_VERSION
    # a bad argument is refused on the host, before any GPU work
    rc = L.kmi_quantize_affine(None, 0, 1, 64, 64, 4, None, None, None, None)
    assert rc == -1 and b"null" in L.kmi_last_error()
    rc = L.kmi_qmm(1, 1, 100, 64, 1, 1, 1, 0, 64, 4, 1, None, 0, None)
    assert rc == -1 and b"multiple of the group" in L.kmi_last_error()


def test_workspace_queries_are_host_only():
    from knurlogic_amd import _abi
    L = _abi.load()
    assert L.kmi_qmm_workspace_bytes(512, 4096, 14336, 64, 4) == 0      # GEMM path
    assert L.kmi_qmm_workspace_bytes(1, 4096, 14336, 64, 4) >= 0
    assert L.kmi_gather_qmm_workspace_bytes(16, 1, 128, 2048, 768, 64, 4) > 0


def test_ops_refuse_cpu_tensors():
    torch = pytest.importorskip("torch")
    import knurlogic_amd as K
    with pytest.raises(ValueError, match="GPU memory"):
        K.quantize(torch.zeros(4, 64, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="affine"):
        K.quantize(torch.zeros(4, 64, dtype=torch.bfloat16), mode="mxfp4")
