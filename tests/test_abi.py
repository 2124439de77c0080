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
    with pytest.raises(ValueError, match="affine, mxfp4 and mxfp8"):
        K.quantize(torch.zeros(4, 64, dtype=torch.bfloat16), mode="nvfp4")
    # the mx modes take group 32 and their own width, as mlx requires
    with pytest.raises(ValueError, match="mxfp8 takes group_size 32 and 8 bits"):
        K.quantize(torch.zeros(4, 64, dtype=torch.bfloat16), bits=4, mode="mxfp8")
    with pytest.raises(ValueError, match="mxfp4 takes group_size 32"):
        K.quantize(torch.zeros(4, 64, dtype=torch.bfloat16), group_size=64, mode="mxfp4")


def test_new_entries_refuse_bad_arguments_on_the_host():
    """The batched matmul, masked softmax, packed VQ, mx dequantize and KV
    append entries check their arguments before touching the GPU (fake
    non-null pointers are never dereferenced)."""
    import ctypes
    from knurlogic_amd import _abi
    L = _abi.load()
    i64 = lambda *v: (ctypes.c_int64 * len(v))(*v)
    st = i64(0, 64)
    # mxfp4 requires 4 bits and groups of 32
    rc = L.kmi_qmm_batched(16, st, 16, st, 16, None, st, 0, None, 1, 64, 64, 1, 0, 64, 4, 1, None, None, 0, 0,
                           1.0, 16, 64, None, 0, None)
    assert rc == -1 and b"mxfp4" in L.kmi_last_error()
    # 7-bit codes do not exist in mlx
    rc = L.kmi_qmm_batched(16, st, 16, st, 16, 16, st, 0, None, 1, 64, 64, 1, 0, 64, 7, 0, None, None, 0, 0,
                           1.0, 16, 64, None, 0, None)
    assert rc == -1 and b"bits 7" in L.kmi_last_error()
    # rows of the softmax must be padded to 8 elements
    dims = i64(1, 1, 1, 2)
    rc = L.kmi_masked_softmax(16, 5, 0, dims, 5, None, 0, None, 16, 5, None)
    assert rc == -1 and b"padded" in L.kmi_last_error()
    # packed VQ: 13-bit fields are not built
    rc = L.kmi_vq_packed_gather_qmm(16, 1, 128, 16, 13, 16, 4096, 4, 16, 64, 2, 8, None, 1, 16, 1, 0, 16, None)
    assert rc == -1 and b"13-bit" in L.kmi_last_error()
    # mx dequantize: mode 3 does not exist
    rc = L.kmi_dequantize_mx(16, 16, 1, 64, 3, 16, 0, None)
    assert rc == -1 and b"mode 3" in L.kmi_last_error()
    # KV append past the slab's capacity
    rc = L.kmi_kv_quantize_append(16, 0, 1, 1, 4, 64, 64, 8, 16, 16, 16, i64(0, 0, 0, 0, 0, 0), 254, 256, None)
    assert rc == -1 and b"capacity" in L.kmi_last_error()


def test_noalloc_scratch_covers_every_planned_qmm():
    """kmi_qmm_noalloc's scratch array (KMI_QMM_SCRATCH_BYTES) holds the
    split-K partials of every shape kmi_qmm plans: the GEMM keeps
    splits x tiles <= 256 (tiles of 256 x 128 outputs) and the skinny kernel
    fewer than 1024 split workgroups of 64 x 64 outputs, so the partials never
    pass 32 MiB.  Swept here on the host (workspace queries only)."""
    import re
    from knurlogic_amd import _abi
    L = _abi.load()
    cap = L.kmi_qmm_noalloc_scratch_bytes()
    hdr = (ROOT / "include" / "knurlogic_amd.h").read_text()
    assert cap == eval(re.search(r"#define KMI_QMM_SCRATCH_BYTES \((\d+)u << (\d+)\)", hdr).expand(r"\1 << \2"))
    worst = 0
    for M in (1, 2, 5, 16, 17, 33, 64, 65, 128, 129, 200, 256, 300, 384, 512, 640, 1000, 1024, 2048, 4096):
        for K in (64, 512, 1024, 2048, 4096, 8192, 14336, 28672):
            for N in (64, 100, 768, 2048, 4096, 6144, 8192, 14336, 28672):
                for bits in (4, 8):
                    worst = max(worst, L.kmi_qmm_workspace_bytes(M, K, N, 64, bits))
    assert worst == cap      # reached (M = 512, K = 14336, N = 4096) and never passed


def test_build_refuses_a_spilling_kernel_with_counted_lds_waits():
    """The build's scratch rule: a kernel compiled from a direct-to-LDS
    source must report no scratch (a spill's scratch traffic would sit among
    the loads its counted vmcnt waits count)."""
    from knurlogic_amd import build as B
    remarks = ("x.hip:1:1: remark: Function Name: _Z4kernv [-Rpass-analysis=kernel-resource-usage]\n"
               "x.hip:1:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]\n"
               "x.hip:9:1: remark: Function Name: _Z5otherv [-Rpass-analysis=kernel-resource-usage]\n"
               "x.hip:9:1: remark:     ScratchSize [bytes/lane]: 68 [-Rpass-analysis=kernel-resource-usage]\n")
    assert B.kernel_scratch(remarks) == {"_Z4kernv": 0, "_Z5otherv": 68}
    dl = B.SRC / "qgemv_dl.hip"
    assert B.uses_lds_dma(dl) and B.uses_lds_dma(B.SRC / "qgemv_xs.hip") and B.uses_lds_dma(B.SRC / "vq_packed.hip")
    assert not B.uses_lds_dma(B.SRC / "kv8.hip")
    with pytest.raises(RuntimeError, match="scratch"):
        B.check_scratch(dl, remarks)
    # a source without direct-to-LDS loads may spill (reported, not refused)
    assert B.check_scratch(B.SRC / "kv8.hip", remarks)["_Z5otherv"] == 68
