"""kvattn.patch_model / enabled and kvcache.install on the CPU (no kernel
calls): which modules get rebound, which caches get quantized, and that
dense K/V go back to the model's own attention function -- the reference's
engine/kvattn.py:323-339 and engine/kvquant.py:390-452."""
import importlib
import sys

import pytest
import torch

from knurlogic_amd import kvattn
from knurlogic_amd import kvcache as KC


@pytest.fixture
def toy(monkeypatch):
    """A fresh toy model module (its attention function unpatched)."""
    sys.modules.pop("tests.toy_attention", None)
    mod = importlib.import_module("tests.toy_attention")
    monkeypatch.setattr(kvattn, "_BASE", {"fn": None})
    monkeypatch.delenv(kvattn.ENV, raising=False)
    yield mod
    sys.modules.pop("tests.toy_attention", None)


def test_patch_model_rebinds_the_models_attention_and_keeps_it_as_the_base(toy):
    orig = toy.scaled_dot_product_attention
    model = toy.Model()
    assert kvattn.patch_model(model) == 1
    bound = toy.scaled_dot_product_attention
    assert isinstance(bound, kvattn.ModuleSdpa) and bound.base is orig
    assert kvattn._BASE["fn"] is orig
    assert kvattn.patch_model(model) == 1                    # idempotent
    assert toy.scaled_dot_product_attention is bound and bound.base is orig
    assert kvattn._BASE["fn"] is orig


def _other_module(monkeypatch, name, factor):
    """A second model module whose own attention function differs from the
    toy's (it scales the toy's output), with one module class in it."""
    import types
    mod = types.ModuleType(name)
    calls = []

    def attention(queries, keys, values, cache=None, scale=1.0, mask=None, sinks=None):
        calls.append(name)
        from tests.toy_attention import scaled_dot_product_attention as plain
        return plain(queries, keys, values, cache=cache, scale=scale, mask=mask) * factor

    class Block(torch.nn.Module):
        pass

    Block.__module__ = name
    mod.scaled_dot_product_attention = attention
    mod.Block = Block
    mod.calls = calls
    monkeypatch.setitem(sys.modules, name, mod)
    return mod


def test_modules_with_different_attention_keep_their_own_base(toy, monkeypatch):
    other = _other_module(monkeypatch, "tests._toy_other_attention", 2.0)
    third = _other_module(monkeypatch, "tests._toy_third_attention", 3.0)
    own = {m.__name__: m.scaled_dot_product_attention for m in (toy, other, third)}
    model = toy.Model(layers=1)
    model.extra = other.Block()
    model.more = third.Block()
    assert kvattn.patch_model(model) == 3
    for m in (toy, other, third):
        f = m.scaled_dot_product_attention
        assert isinstance(f, kvattn.ModuleSdpa) and f.base is own[m.__name__]
    # dense K/V dispatched from each module reach that module's own function
    q, k = torch.randn(1, 2, 1, 16), torch.randn(1, 2, 5, 16)
    want = own[toy.__name__](q, k, k, scale=0.25)
    assert torch.equal(toy.scaled_dot_product_attention(q, k, k, cache=None, scale=0.25), want)
    assert torch.equal(other.scaled_dot_product_attention(q, k, k, cache=None, scale=0.25), want * 2)
    assert torch.equal(third.scaled_dot_product_attention(q, k, k, cache=None, scale=0.25), want * 3)
    assert other.calls == ["tests._toy_other_attention"] and third.calls == ["tests._toy_third_attention"]


def test_a_second_model_patched_later_serves_direct_calls(toy, monkeypatch):
    toy_orig = toy.scaled_dot_product_attention
    kvattn.patch_model(toy.Model(layers=1))
    assert kvattn._BASE["fn"] is toy_orig
    other = _other_module(monkeypatch, "tests._toy_other_attention", 2.0)
    other_orig = other.scaled_dot_product_attention

    class Second(torch.nn.Module):
        pass

    Second.__module__ = other.__name__
    assert kvattn.patch_model(Second()) == 1
    assert kvattn._BASE["fn"] is other_orig
    # the first model's module still holds its own base
    assert toy.scaled_dot_product_attention.base is toy_orig


def test_dense_kv_go_back_to_the_models_own_attention(toy):
    model = toy.Model(layers=1)
    x = torch.randn(1, 7, 256)
    want = toy.run(model, x, 5)
    kvattn.patch_model(model)
    got = toy.run(model, x, 5)                                # plain caches: every call is dense
    assert torch.equal(got, want)


def test_dense_kv_without_patch_model_is_an_error(toy):
    q = torch.zeros(1, 2, 1, 128)
    with pytest.raises(ValueError, match="patch_model"):
        kvattn.sdpa(q, q, q, None, 1.0, None)


def test_enabled_follows_the_switch(monkeypatch):
    monkeypatch.delenv(kvattn.ENV, raising=False)
    assert kvattn.enabled()
    for off in ("off", "0", "False"):
        monkeypatch.setenv(kvattn.ENV, off)
        assert not kvattn.enabled()
    monkeypatch.setenv(kvattn.ENV, "on")
    assert kvattn.enabled()


def test_install_quantizes_plain_caches_and_marks_the_kernel(toy, monkeypatch):
    model = toy.Model()
    assert KC.install(model, 8) == 2
    assert model.kv8_kernel is True and isinstance(toy.scaled_dot_product_attention, kvattn.ModuleSdpa)
    caches = model.make_cache()
    assert all(type(c) is KC.QuantKVCache and c.kv_bits == 8 and c.kv8_kernel for c in caches)
    # the switch off: quantized caches, no kernel
    other = toy.Model()
    monkeypatch.setenv(kvattn.ENV, "off")
    assert KC.install(other, 8) == 2 and other.kv8_kernel is False
    assert not any(c.kv8_kernel for c in other.make_cache())
    # 4 bits: quantized, never the 8-bit kernel
    four = toy.Model()
    monkeypatch.delenv(kvattn.ENV)
    assert KC.install(four, "4") == 2 and four.kv8_kernel is False
    assert all(c.kv_bits == 4 and not c.kv8_kernel for c in four.make_cache())
    # bf16: nothing to do
    plain = toy.Model()
    assert KC.install(plain, "bf16") == 0 and not hasattr(plain, "kv8_kernel")


def test_quantize_cache_list_recurses_and_leaves_the_rest():
    class KVCache:
        keys = None

    class Recurrent:
        keys = None

    class CacheList:
        def __init__(self, *caches):
            self.caches = caches

    class Family:
        keys = None

    filled = KVCache()
    filled.keys = torch.zeros(1)
    made = []
    out, n = KC.quantize_cache_list(
        [KVCache(), Recurrent(), CacheList(KVCache(), Recurrent()), filled, Family()], 6,
        {Family: lambda bits: made.append(bits) or KC.BatchQuantKVCache([0], bits)})
    assert n == 3 and made == [6]
    assert type(out[0]) is KC.QuantKVCache and out[0].kv_bits == 6
    assert type(out[1]) is Recurrent
    assert type(out[2]) is CacheList and type(out[2].caches[0]) is KC.QuantKVCache
    assert type(out[2].caches[1]) is Recurrent
    assert out[3] is filled
    assert type(out[4]) is KC.BatchQuantKVCache


def _triples(B, H, Hk, L, N, D, g, dtype=torch.bfloat16):
    q = torch.zeros(B, H, L, D, dtype=dtype)
    w = torch.zeros(B, Hk, N, D // 4, dtype=torch.int32)
    sc = torch.zeros(B, Hk, N, D // g, dtype=dtype)
    return q, (w, sc, sc), (w, sc.clone(), sc.clone())


@pytest.mark.parametrize("D,g,H,Hk,L,ok", [
    (128, 64, 8, 2, 1, True), (256, 32, 8, 2, 1, True), (128, 16, 8, 2, 1, True),
    (384, 128, 8, 2, 1, True), (512, 16, 8, 2, 1, True), (512, 512, 8, 2, 1, True),
    (256, 64, 64, 1, 1, True), (512, 64, 16, 1, 4, True),      # 64 rows per KV head
    (128, 8, 8, 2, 1, False), (256, 8, 8, 2, 1, False),        # groups mlx does not make
    (512, 48, 8, 2, 1, False),                                  # does not divide D
    (64, 32, 8, 2, 1, False), (640, 64, 8, 2, 1, False),       # head dims outside 128..512
    (128, 64, 32, 1, 3, False),                                 # 96 rows per KV head
])
def test_the_shape_rule(D, g, H, Hk, L, ok):
    """kvattn.supports: the reference's rule (engine/kvattn.py:213-239) on
    head dims, rows per KV head and groups, with groups narrowed to
    multiples of 16."""
    q, K, V = _triples(1, H, Hk, L, 64, D, g)
    assert kvattn.supports(q, K, V, 8, g) is ok
