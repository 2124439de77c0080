"""Host logic of the quantized KV caches (knurlogic_amd/kvcache.py, after
the reference's engine/kvquant.py): slab growth, row bookkeeping of the
batched cache (merge / extend / filter / extract / trim / right-padding
roll / masks), stored bytes, on the CPU.  The GPU quantize-append is
replaced here by the oracle's mx.quantize restatement writing into CPU
slabs, so the bookkeeping is checked on its own; tests/test_gpu_kvcache.py
runs the real path."""
import numpy as np
import pytest
import torch

import oracle as O
from knurlogic_amd import kvcache as KC

BF = torch.bfloat16


def _cpu_append(parts, x, pos, group, bits):
    wq, sc, bi = parts
    q, s, b = O.quantize(x.float().numpy(), group, bits, "bfloat16")
    S = x.shape[2]
    wq.view(torch.int32)[:, :, pos:pos + S] = torch.from_numpy(q.view(np.int32))
    sc[:, :, pos:pos + S] = torch.from_numpy(s).to(sc.dtype)
    bi[:, :, pos:pos + S] = torch.from_numpy(b).to(bi.dtype)


def _cpu_append_kv(kparts, vparts, keys, values, pos, group, bits):
    _cpu_append(kparts, keys, pos, group, bits)
    _cpu_append(vparts, values, pos, group, bits)


REAL_APPEND_KV = KC.append_kv


@pytest.fixture(autouse=True)
def cpu_append(monkeypatch):
    monkeypatch.setattr(KC, "append_quantized", _cpu_append)
    monkeypatch.setattr(KC, "append_kv", _cpu_append_kv)


def _kv(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(BF)


def _rows(c):
    """Per batch row: the packed words of the filled slots, in order."""
    return c.keys[0].view(torch.int32)


def test_bits_are_bf16_8_6_or_4():
    assert KC.parse_bits("bf16") is None and KC.parse_bits(None) is None
    assert KC.parse_bits("6") == 6 and KC.parse_bits(" 8 ") == 8
    with pytest.raises(ValueError):
        KC.parse_bits("5")


def test_group_is_64_when_both_heads_allow_it_else_32():
    assert KC._group(128, 128) == 64 and KC._group(128, 96) == 32 and KC._group(96, 96) == 32
    with pytest.raises(ValueError):
        KC.group_for(100)


def test_slabs_grow_in_256_slots_and_keep_the_prefix():
    c = KC.QuantKVCache(8)
    chunks = [_kv((1, 2, n, 64), n) for n in (3, 1, 300, 1)]
    for x in chunks:
        k, v = c.update_and_fetch(x, x)
        assert isinstance(k, KC.LazyDequant) and k.shape == (1, 2, c.offset, 64) and k.dtype == BF
    assert c.offset == 305 and c.keys[0].shape[2] == 4 + 512      # 256, then +512 at the 300-slot chunk
    ref = O.quantize(torch.cat(chunks, 2).float().numpy(), 64, 8, "bfloat16")
    assert np.array_equal(c.keys[0][:, :, :305].view(torch.int32).numpy(), ref[0].view(np.int32))
    assert np.array_equal(c.keys[1][:, :, :305].float().numpy(), ref[1])
    assert not c.keys[0].view(torch.int32)[:, :, 305:].any()
    assert not hasattr(c, "bits") and not hasattr(KC.BatchQuantKVCache([0], 8), "bits")


@pytest.mark.parametrize("bits,ratio", [(8, 1.0625 / 2), (4, 0.5625 / 2)])
def test_stored_bytes_shrink_by_the_bits(bits, ratio):
    """The reference's byte ratios (tests/engine/test_kvquant.py:22-34): a
    512-token bf16 K/V against the quantized triples."""
    c = KC.QuantKVCache(bits)
    k = _kv((1, 4, 512, 128), 0)
    c.update_and_fetch(k, k)
    assert c.nbytes / (2 * k.numel() * 2) == pytest.approx(ratio, rel=1e-6)


def _fill(n, seed):
    c = KC.QuantKVCache(8)
    x = _kv((1, 2, n, 32), seed)
    c.update_and_fetch(x, x)
    return c, x


def test_merge_left_pads_each_row_to_the_longest():
    caches, xs = zip(*[_fill(n, n) for n in (5, 12, 3)])
    b = KC.BatchQuantKVCache.merge(list(caches))
    assert b.left_padding.tolist() == [7, 0, 9] and b.offset.tolist() == [5, 12, 3] and b._idx == 12
    for i, (c, x) in enumerate(zip(caches, xs)):
        pad = b.left_padding[i].item()
        assert torch.equal(_rows(b)[i, :, pad:12], c.keys[0].view(torch.int32)[0, :, :x.shape[2]])
        assert not _rows(b)[i, :, :pad].any()


def test_extend_filter_extract_keep_each_row():
    caches, xs = zip(*[_fill(n, n) for n in (5, 12, 3)])
    b = KC.BatchQuantKVCache.merge(list(caches[:2]))
    b.extend(KC.BatchQuantKVCache.merge(list(caches[2:])))
    assert b.left_padding.tolist() == [7, 0, 9] and b.offset.tolist() == [5, 12, 3]
    step = _kv((3, 2, 1, 32), 99)
    k, _ = b.update_and_fetch(step, step)
    assert k.shape == (3, 2, 13, 32) and b.offset.tolist() == [6, 13, 4]
    b.filter([0, 2])
    assert b.left_padding.tolist() == [0, 2] and b._idx == 6 and b.size() == 6
    one = b.extract(1)
    assert type(one) is KC.QuantKVCache and one.offset == 4
    ref = torch.cat([caches[2].keys[0].view(torch.int32)[:, :, :3],
                     b.keys[0].view(torch.int32)[1:2, :, 5:6]], 2)
    assert torch.equal(one.keys[0].view(torch.int32), ref)


def test_a_trimmed_batch_rewrites_like_a_fresh_one():
    """The reference's rollback test (test_kvquant.py:51-70): trim(2) then
    replay leaves exactly what a cache fed only the committed tokens holds."""
    a, b = KC.BatchQuantKVCache([0, 0], 8), KC.BatchQuantKVCache([0, 0], 8)
    base = _kv((2, 2, 9, 32), 1)
    for c in (a, b):
        c.update_and_fetch(base, base)
    wrong = _kv((2, 2, 2, 32), 5)
    a.update_and_fetch(wrong, wrong)
    assert a.trim(2) == 2 and a.size() == 9
    right = _kv((2, 2, 2, 32), 6)
    a.update_and_fetch(right, right)
    b.update_and_fetch(right, right)
    for pa, pb in zip(a.keys + a.values, b.keys + b.values):
        assert torch.equal(pa[:, :, :11].view(torch.int16 if pa.dtype == BF else torch.int32),
                           pb[:, :, :11].view(torch.int16 if pb.dtype == BF else torch.int32))


def test_right_padding_rolls_rows_back_into_place():
    """prepare(right_padding) then finalize: each right-padded row's slots
    roll right by its padding, which joins its left padding."""
    c = KC.BatchQuantKVCache([0, 0], 8)
    c.prepare(right_padding=[2, 0])
    x = _kv((2, 2, 5, 32), 3)
    c.update_and_fetch(x, x)
    before = _rows(c).clone()
    c.finalize()
    assert c.left_padding.tolist() == [2, 0] and c.offset.tolist() == [3, 5]
    n = c.keys[0].shape[2]
    assert torch.equal(_rows(c)[0], torch.roll(before[0], 2, dims=1))
    assert torch.equal(_rows(c)[1], before[1]) and n == 256


def test_mask_sees_the_row_from_its_left_padding_causally():
    c = KC.BatchQuantKVCache([2, 0], 8)
    x = _kv((2, 2, 4, 32), 4)
    m = c.make_mask(4)
    assert m.shape == (2, 1, 4, 4) and m.dtype == torch.bool
    assert m[0, 0].tolist() == [[False, False, False, False], [False, False, False, False],
                                [False, False, True, False], [False, False, True, True]]
    assert m[1, 0].tolist() == [[True, False, False, False], [True, True, False, False],
                                [True, True, True, False], [True, True, True, True]]
    c.update_and_fetch(x, x)
    assert c.make_mask(1)[:, 0, 0].tolist() == [[False, False, True, True, True],
                                                [True, True, True, True, True]]


def test_state_round_trips():
    c, _ = _fill(7, 2)
    c.kv8_kernel = True
    d = KC.QuantKVCache.__new__(KC.QuantKVCache)
    d.dims = None
    d.state = c.state
    assert d.offset == 7 and d.group == 32 and d.kv8_kernel and d.dims == (32, 32)
    assert torch.equal(d.keys[0].view(torch.int32), c.keys[0][:, :, :7].view(torch.int32))


@pytest.mark.parametrize("what", ["batch", "heads", "width", "scales", "capacity"])
def test_an_append_that_does_not_fit_its_slab_is_refused(what):
    """The append kernel sees only strides and a capacity, so rows of
    another batch, head count or head dim (a cache reused at another batch,
    a state restored from another model) must be refused on the host rather
    than written past the slab."""
    k = _kv((2, 4, 3, 64), 0)
    kp = KC._alloc(2, 4, 256, 64, 8, 64, BF, "cpu")
    vp = KC._alloc(2, 4, 256, 64, 8, 64, BF, "cpu")
    bad = {"batch": lambda: KC._alloc(3, 4, 256, 64, 8, 64, BF, "cpu"),
           "heads": lambda: KC._alloc(2, 2, 256, 64, 8, 64, BF, "cpu"),
           "width": lambda: KC._alloc(2, 4, 256, 128, 8, 64, BF, "cpu"),
           "scales": lambda: (kp[0], kp[1][..., :0], kp[2][..., :0]),
           "capacity": lambda: KC._alloc(2, 4, 512, 64, 8, 64, BF, "cpu")}[what]()
    match = "same number of slots" if what == "capacity" else "does not fit its slab"
    with pytest.raises(ValueError, match=match):
        REAL_APPEND_KV(kp, bad, k, k, 0, 64, 8)         # the real append, not the CPU stand-in
    with pytest.raises(ValueError, match="GPU memory"):
        REAL_APPEND_KV(kp, vp, k, k, 0, 64, 8)          # a fitting slab only fails for being on the CPU
