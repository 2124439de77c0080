"""GPU: the quantized KV caches (knurlogic_amd/kvcache.py, after the
reference's engine/kvquant.py).  Quantize-on-append (kmi_kv_quantize_append)
writes exactly the oracle's mx.quantize of the appended rows into the slab
slots, for single and batched caches and every float dtype; a fetch is close
to what went in (the reference's 0.05 at 8 bits); a one-token decode step
takes the 8-bit kernel straight from the cache and matches the oracle."""
import numpy as np
import pytest
import torch

import oracle as O
from knurlogic_amd import kvattn
from knurlogic_amd import kvcache as KC
from tests.util import assert_close, to_numpy

pytestmark = pytest.mark.gpu
DT = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _kv(shape, seed, dev, dtype=torch.bfloat16):
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn(*shape, device=dev, generator=g).to(dtype)


def _bits(t):
    t = t.cpu()
    return t.view(torch.int32) if t.dtype == torch.uint32 else t.view(torch.int16) if t.element_size() == 2 \
        else t.view(torch.int32)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("bits", [8, 6, 4])
def test_append_writes_the_oracle_quantization_into_the_slots(dev, dtype, bits):
    c = KC.QuantKVCache(bits)
    chunks = [_kv((2, 4, n, 128), n, dev, DT[dtype]) for n in (3, 1, 300, 1)]
    for x in chunks:
        k, v = c.update_and_fetch(x, -x)
    assert c.offset == 305 and c.keys[0].shape[2] == 516 and c.group == 64
    allx = torch.cat(chunks, 2).float().cpu().numpy()
    for parts, src in ((c.keys, allx), (c.values, -allx)):
        wq, s, b = O.quantize(src, 64, bits, dtype)
        assert np.array_equal(parts[0][:, :, :305].cpu().view(torch.int32).numpy(), wq.view(np.int32))
        assert np.array_equal(parts[1][:, :, :305].float().cpu().numpy(), s)
        assert np.array_equal(parts[2][:, :, :305].float().cpu().numpy(), b)
        assert not parts[0][:, :, 305:].cpu().view(torch.int32).any()


def test_a_fetch_is_close_to_what_went_in_at_8_bits(dev):
    """The reference's bound (tests/engine/test_kvquant.py:37-43)."""
    k, v = _kv((1, 2, 40, 64), 0, dev), _kv((1, 2, 40, 64), 1, dev)
    kk, vv = KC.QuantKVCache(8).update_and_fetch(k, v)
    assert isinstance(kk, KC.LazyDequant) and kk.dtype == k.dtype and kk.shape == k.shape
    kt = KC.materialize(kk)
    assert torch.is_tensor(kt) and kt.dtype == k.dtype
    assert (kt.float() - k.float()).abs().max().item() < 0.05
    assert (vv.float() - v.float()).abs().max().item() < 0.05       # a torch op dequantizes it


def test_a_decode_step_takes_the_kernel_from_the_cache(dev):
    """kv8_kernel on: a one-token query through kvattn.sdpa reads the packed
    K/V the cache just returned (a counted hit, the cache never
    dequantized) and matches the oracle over the same quantized triples."""
    B, H, Hk, D = 2, 16, 2, 128
    c = KC.BatchQuantKVCache([0, 0], 8)
    c.kv8_kernel = True
    prompt = _kv((B, Hk, 700, D), 1, dev)
    c.update_and_fetch(prompt, prompt * 0.5)
    c.kv8_fetch = None                                  # the prefill's fetch, not a decode step
    kvattn.reset(True)
    step = _kv((B, Hk, 1, D), 2, dev)
    k, v = c.update_and_fetch(step, step * 0.5)
    assert c.kv8_fetch is not None
    q = _kv((B, H, 1, D), 3, dev)
    out = kvattn.sdpa(q, k, v, c, D ** -0.5, None)
    assert kvattn.STATS["hits"] == 1 and kvattn.STATS["misses"] == 0
    assert k._t is None and v._t is None                # never dequantized
    allk = torch.cat([prompt, step], 2).float().cpu().numpy()
    K = O.quantize(allk, 64, 8, "bfloat16")
    V = O.quantize(allk * 0.5, 64, 8, "bfloat16")
    ref = O.kv8_decode(q.float().cpu().numpy(), K, V, D ** -0.5, None, 64, 8, "float32")
    assert_close(to_numpy(out), ref, what="kv8 through the cache")
    # the same step without the kernel: attention over the cache's packed triples
    c2 = KC.QuantKVCache(8)
    k2, v2 = c2.update_and_fetch(torch.cat([prompt, step], 2)[:1], (torch.cat([prompt, step], 2) * 0.5)[:1])
    out2 = kvattn.sdpa(q[:1], k2, v2, c2, D ** -0.5, None)
    assert_close(to_numpy(out2), ref[:1], what="fallback through the cache")


def test_batched_rows_hold_the_oracle_quantization(dev):
    """merge (left padding), extend, a decode step, filter, extract: every
    row's filled slots are the oracle's quantization of that row's tokens."""
    rows = [_kv((1, 2, n, 64), n, dev) for n in (5, 12, 3)]
    caches = []
    for x in rows:
        c = KC.QuantKVCache(8)
        c.update_and_fetch(x, x)
        caches.append(c)
    b = KC.BatchQuantKVCache.merge(caches[:2])
    b.extend(KC.BatchQuantKVCache.merge(caches[2:]))
    step = _kv((3, 2, 1, 64), 9, dev)
    b.update_and_fetch(step, step)
    assert b.left_padding.tolist() == [7, 0, 9] and b.offset.tolist() == [6, 13, 4] and b._idx == 13
    for i, x in enumerate(rows):
        toks = torch.cat([x, step[i:i + 1]], 2).float().cpu().numpy()
        wq, s, _ = O.quantize(toks, 64, 8, "bfloat16")
        pad = b.left_padding[i].item()
        assert np.array_equal(b.keys[0][i:i + 1, :, pad:13].cpu().view(torch.int32).numpy(), wq.view(np.int32))
        assert np.array_equal(b.keys[1][i:i + 1, :, pad:13].float().cpu().numpy(), s)
    b.filter([0, 2])
    one = b.extract(1)
    assert one.offset == 4
    wq, _, _ = O.quantize(torch.cat([rows[2], step[2:3]], 2).float().cpu().numpy(), 64, 8, "bfloat16")
    assert np.array_equal(one.keys[0].cpu().view(torch.int32).numpy(), wq.view(np.int32))


def test_append_refuses_what_it_cannot_store(dev):
    c = KC.QuantKVCache(7)
    x = _kv((1, 1, 2, 64), 0, dev)
    with pytest.raises(ValueError):
        c.update_and_fetch(x, x)


def test_a_six_bit_cache_stores_fetches_and_attends_through_the_fallback(dev):
    """6-bit K/V (the reference's kvquant.BITS): codes straddle words in
    the row's bit stream; a fetch is within four 8-bit steps of what went
    in, and attention takes the packed-triple path (the decode kernel is
    8-bit only), within the bar of float64 attention over the dequantized
    cache."""
    c = KC.QuantKVCache(6)
    c.kv8_kernel = True
    k, v = _kv((1, 2, 50, 128), 1, dev), _kv((1, 2, 50, 128), 2, dev)
    kk, vv = c.update_and_fetch(k, v)
    wq, s, b = O.quantize(k.float().cpu().numpy(), 64, 6, "bfloat16")
    assert np.array_equal(c.keys[0][:, :, :50].cpu().view(torch.int32).numpy(), wq.view(np.int32))
    assert (KC.materialize(kk).float() - k.float()).abs().max().item() < 0.2
    assert c.kv8_fetch is None
    q = _kv((1, 8, 1, 128), 3, dev)
    kvattn.reset()
    out = kvattn.sdpa(q, kk, vv, c, 128 ** -0.5, None)
    Kd = O.dequantize_numpy_f64(*(t.cpu().view(torch.int32).numpy().view(np.uint32) if t.dtype == torch.uint32
                                  else t.float().cpu().numpy() for t in (c.keys[0][:, :, :50], c.keys[1][:, :, :50],
                                                                        c.keys[2][:, :, :50])), 64, 6)
    Vd = O.dequantize_numpy_f64(*(t.cpu().view(torch.int32).numpy().view(np.uint32) if t.dtype == torch.uint32
                                  else t.float().cpu().numpy() for t in (c.values[0][:, :, :50],
                                                                        c.values[1][:, :, :50],
                                                                        c.values[2][:, :, :50])), 64, 6)
    ref = O.sdpa_numpy_f64(q.float().cpu().numpy() * 128 ** -0.5, Kd, Vd, 1.0)
    assert_close(to_numpy(out), ref, what="6-bit fallback attention")
