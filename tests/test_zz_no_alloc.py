"""kmi_qmm_noalloc (the entry point that allocates nothing) against kmi_qmm
with a caller workspace, through the C ABI: bit for bit, on two calls in a
row, the second smaller than the first, so the second runs over what the
first left in the shared scratch array; and recorded into a HIP graph,
replayed with new inputs."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from knurlogic_amd import _abi
from tests.util import bf16_normal, to_torch, u32_to_torch

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _operands(dev, M, K, N, bits, seed):
    rng = np.random.default_rng(seed)
    wq, s, b = O.quantize(bf16_normal(rng, (N, K), 0.02), 64, bits)
    x = to_torch(bf16_normal(rng, (M, K)), dev, BF)
    return x, u32_to_torch(wq, dev), to_torch(s, dev, BF), to_torch(b, dev, BF)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _both(dev, M, K, N, bits, seed):
    """(kmi_qmm with a torch workspace, kmi_qmm_noalloc) on the same operands."""
    L = _abi.load()
    x, w, s, b = _operands(dev, M, K, N, bits, seed)
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    need = L.kmi_qmm_workspace_bytes(M, K, N, 64, bits)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    y_ws = torch.empty(M, N, dtype=BF, device=dev)
    y_na = torch.full((M, N), float("nan"), dtype=BF, device=dev)
    _abi.check(L.kmi_qmm(_ptr(x), M, K, N, _ptr(w), _ptr(s), _ptr(b), 0, 64, bits, _ptr(y_ws), _ptr(ws), need, st),
               "qmm")
    _abi.check(L.kmi_qmm_noalloc(_ptr(x), M, K, N, _ptr(w), _ptr(s), _ptr(b), 0, 64, bits, _ptr(y_na), st),
               "qmm_noalloc")
    torch.cuda.synchronize()
    return need, y_ws, y_na


def test_noalloc_captured_in_a_graph_replays_like_qmm(dev):
    """kmi_qmm_noalloc recorded into a HIP graph (torch.cuda.CUDAGraph) and
    replayed with new x contents written eagerly between replays: every
    replay equals kmi_qmm with a workspace, bit for bit.  This test runs
    first in its file and no other test calls the no-alloc entry, so the
    capture also covers the first call's per-device scratch lookup."""
    torch.cuda.set_device(dev)
    L = _abi.load()
    M, K, N, bits = 16, 4096, 4096, 8          # a K-split shape: the partials sit in the scratch array
    x, w, s, b = _operands(dev, M, K, N, bits, 7)
    need = L.kmi_qmm_workspace_bytes(M, K, N, 64, bits)
    assert need > 0
    y = torch.full((M, N), float("nan"), dtype=BF, device=dev)
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        rc = L.kmi_qmm_noalloc(_ptr(x), M, K, N, _ptr(w), _ptr(s), _ptr(b), 0, 64, bits, _ptr(y),
                               ctypes.c_void_p(side.cuda_stream))
    _abi.check(rc, "qmm_noalloc (captured)")
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    ref = torch.empty(M, N, dtype=BF, device=dev)
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    rng = np.random.default_rng(8)
    for i in range(4):
        x.copy_(to_torch(bf16_normal(rng, (M, K)), dev, BF))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _abi.check(L.kmi_qmm(_ptr(x), M, K, N, _ptr(w), _ptr(s), _ptr(b), 0, 64, bits, _ptr(ref), _ptr(ws),
                             need, st), "qmm")
        torch.cuda.synchronize()
        assert torch.equal(y, ref), f"replay {i}"
    del graph


def test_noalloc_matches_qmm_on_two_calls_in_a_row(dev):
    torch.cuda.set_device(dev)
    L = _abi.load()
    # 1) the prefill GEMM with a 4-way K split: its partials fill the whole array
    need1, y1, z1 = _both(dev, 512, 14336, 4096, 4, 1)
    assert need1 == L.kmi_qmm_noalloc_scratch_bytes(), need1
    assert torch.equal(y1, z1)
    # 2) a smaller call (decode rows, skinny kernel, K split): the array still
    #    holds call 1's partials, which must not leak into this result
    need2, y2, z2 = _both(dev, 16, 4096, 4096, 8, 2)
    assert 0 < need2 < need1
    assert torch.equal(y2, z2)
    # 3) and one that needs no partials at all (single-row GEMV)
    need3, y3, z3 = _both(dev, 1, 4096, 4096, 4, 3)
    assert need3 == 0 and torch.equal(y3, z3)
