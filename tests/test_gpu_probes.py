"""The calibration kernels behind bench.py's measured ceilings: the plain
read (kmi_read_probe) and the bf16 MFMA loop (kmi_mfma_probe) run through
the C ABI, and the MFMA probe's counters give a plausible shader clock."""
import ctypes

import pytest
import torch

from knurlogic_amd import _abi

pytestmark = pytest.mark.gpu


def test_read_probe_runs_and_refuses_bad_sizes(dev):
    L = _abi.load()
    buf = torch.ones(1 << 20, dtype=torch.uint8, device=dev)
    out = torch.zeros(1, dtype=torch.int32, device=dev)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _abi.check(L.kmi_read_probe(ctypes.c_void_p(buf.data_ptr()), buf.numel(), 64, ctypes.c_void_p(out.data_ptr()),
                                st), "read_probe")
    torch.cuda.synchronize()
    assert int(out.item()) == 0          # all-ones data never XORs to the guard value
    assert L.kmi_read_probe(ctypes.c_void_p(buf.data_ptr()), 100, 64, ctypes.c_void_p(out.data_ptr()), st) == -1


def test_mfma_probe_counts_cycles_and_ticks(dev):
    import bench
    r = bench.mfma_rate(dev, rounds=256)
    assert r["TFLOPs"] > 0 and r["clock_MHz"] is not None
    assert 300 <= r["clock_MHz"] <= 4000, r
    assert r["TFLOPs"] <= r["peak_at_clock_TFLOPs"] * 1.05, r
    L = _abi.load()
    z = ctypes.c_void_p(0)
    assert L.kmi_mfma_probe(z, 1, 1, z, z, z) == -1 and b"null" in L.kmi_last_error()
