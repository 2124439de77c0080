"""GPU: quantized KV caches installed into a model and attention dispatched
through kvattn.sdpa -- the reference's tests/engine/test_kvattn.py:143-191
(install, then the decode steps take the kernel and match the path
without it) and the cases the 8-bit kernel refuses (6 / 4-bit caches),
which run mlx-lm's quantized attention over the packed triples, checked
against the oracle's restatement of it.  Bars: max rel err 1e-2, cosine
0.9999."""
import importlib
import sys

import numpy as np
import pytest
import torch

import oracle as O
from knurlogic_amd import kvattn
from knurlogic_amd import kvcache as KC
from tests.util import assert_close, to_numpy

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


@pytest.fixture
def toy(monkeypatch):
    sys.modules.pop("tests.toy_attention", None)
    mod = importlib.import_module("tests.toy_attention")
    monkeypatch.setattr(kvattn, "_BASE", {"fn": None})
    monkeypatch.delenv(kvattn.ENV, raising=False)
    yield mod
    sys.modules.pop("tests.toy_attention", None)


def _kv(shape, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn(*shape, device=dev, generator=g).to(BF)


def _np_triple(parts):
    return tuple(t.cpu().view(torch.int32).numpy().view(np.uint32) if t.dtype == torch.uint32
                 else t.float().cpu().numpy() for t in parts)


def test_install_takes_the_kernel_and_matches_the_path_without_it(dev, toy, monkeypatch):
    calls = []
    real = kvattn.decode_sdpa
    monkeypatch.setattr(kvattn, "decode_sdpa", lambda *a, **k: calls.append(a[0].shape) or real(*a, **k))
    x = _kv((2, 22, 256), 1, dev)                                # a 16-token prompt, 6 forced decode steps
    dense = toy.run(toy.Model().to(dev).to(BF), x, 16)          # bf16 caches, the model's own attention

    off_model = toy.Model().to(dev).to(BF)
    monkeypatch.setenv(kvattn.ENV, "off")
    assert KC.install(off_model, 8) == 2 and off_model.kv8_kernel is False
    off = toy.run(off_model, x, 16)
    assert not calls

    on_model = toy.Model().to(dev).to(BF)
    monkeypatch.delenv(kvattn.ENV)
    assert KC.install(on_model, 8) == 2 and on_model.kv8_kernel is True
    on = toy.run(on_model, x, 16)
    assert len(calls) == 12 and all(s == (2, 8, 1, 128) for s in calls)   # every decode step, both layers
    assert kvattn.STATS["hits"] == 12 and kvattn.STATS["misses"] == 0
    assert_close(to_numpy(on), to_numpy(off), what="kernel on vs off")
    assert_close(to_numpy(on), to_numpy(dense), max_rel=3e-2, min_cos=0.999, what="8-bit vs bf16 cache")


@pytest.mark.parametrize("L", [2, 4])
def test_a_verify_step_through_the_cache_takes_the_kernel(dev, L):
    """MTP verify: L query tokens per sequence, causal inside the block,
    through an 8-bit cache with the kernel on (KERNEL_MAX_QUERY)."""
    B, H, Hk, D = 2, 32, 4, 128
    c = KC.BatchQuantKVCache([0, 0], 8)
    c.kv8_kernel = True
    prompt = _kv((B, Hk, 600, D), 1, dev)
    c.update_and_fetch(prompt, prompt * 0.5)
    c.kv8_fetch = None
    kvattn.reset(True)
    step = _kv((B, Hk, L, D), 2, dev)
    k, v = c.update_and_fetch(step, step * 0.5)
    assert c.kv8_fetch is not None
    q = _kv((B, H, L, D), 3, dev)
    out = kvattn.sdpa(q, k, v, c, D ** -0.5, "causal")
    assert kvattn.STATS["hits"] == 1 and k._t is None
    allk = torch.cat([prompt, step], 2).float().cpu().numpy()
    K = O.quantize(allk, 64, 8, "bfloat16")
    V = O.quantize(allk * 0.5, 64, 8, "bfloat16")
    ref = O.kv8_decode(q.float().cpu().numpy(), K, V, D ** -0.5, "causal", 64, 8, "float32")
    assert_close(to_numpy(out), ref, what=f"verify L={L}")


@pytest.mark.parametrize("bits", [6, 4])
@pytest.mark.parametrize("L,mask", [(1, None), (4, "causal")])
def test_narrow_caches_attend_over_the_packed_triples(dev, bits, L, mask):
    """6 and 4-bit caches (the reference's other widths): decode and verify
    go through the packed-triple attention, never a dequantized copy, and
    equal the oracle's quantized attention over the cache's own triples."""
    B, H, Hk, D = 2, 16, 4, 128
    c = KC.BatchQuantKVCache([0, 0], bits)
    c.kv8_kernel = True                                          # on, but not for this width
    prompt = _kv((B, Hk, 300, D), 4, dev)
    c.update_and_fetch(prompt, -prompt)
    step = _kv((B, Hk, L, D), 5, dev)
    k, v = c.update_and_fetch(step, -step)
    assert c.kv8_fetch is None
    q = _kv((B, H, L, D), 6, dev)
    kvattn.reset(True)
    out = kvattn.sdpa(q, k, v, c, D ** -0.5, mask)
    assert k._t is None and v._t is None                         # never dequantized
    assert kvattn.STATS["hits"] == 0
    n = c._idx
    K = _np_triple(t[:, :, :n] for t in c.keys)
    V = _np_triple(t[:, :, :n] for t in c.values)
    ref = O.quantized_sdpa(q.float().cpu().numpy(), K, V, D ** -0.5, mask, 64, bits)
    assert_close(to_numpy(out), ref, what=f"{bits}-bit L={L}")
    # and within the bar of float64 attention over the dequantized cache
    Kd = O.dequantize_numpy_f64(*K, 64, bits)
    Vd = O.dequantize_numpy_f64(*V, 64, bits)
    m = None if mask is None else (np.arange(n - L, n)[:, None] >= np.arange(n)[None])
    exact = O.sdpa_numpy_f64(q.float().cpu().numpy() * D ** -0.5, Kd, Vd, 1.0, m)
    assert_close(to_numpy(out), exact, what=f"{bits}-bit L={L} vs float64")
