"""The on-disk formats (knurlogic_amd/checkpoint.py), on the CPU: the
packed-layer recipe read off tensor shapes (the reference's
engine/model/packed.py:33-64), the VQ layout rules and their errors (the
cases of tests/engine/test_deepseek_v4_mtp.py:262-287), and a written
safetensors file read back into modules (tensors left on the CPU)."""
import json
import types

import numpy as np
import pytest
import torch

from knurlogic_amd import checkpoint as C
from knurlogic_amd import nn


def _shape(*s):
    return types.SimpleNamespace(shape=tuple(s))


def test_recipe_reads_bits_group_and_mode_off_the_shapes():
    w = {"a.weight": _shape(64, 512 * 4 // 32), "a.scales": _shape(64, 8), "a.biases": _shape(64, 8)}
    assert C.recipe(w, "a", 512) == {"group_size": 64, "bits": 4, "mode": "affine"}
    w8 = {"b.weight": _shape(64, 256 * 8 // 32), "b.scales": _shape(64, 8)}
    assert C.recipe(w8, "b", 256) == {"group_size": 32, "bits": 8, "mode": "mxfp8"}
    assert C.recipe(w8, "b", 256, {"mode": "nvfp4"})["mode"] == "nvfp4"
    assert C.recipe(w8, "b", 256, {"mode": "mxfp4", "x.b": {"mode": "nvfp4"}}, prefix="x.")["mode"] == "nvfp4"
    assert C.recipe({"c.weight": _shape(4, 4)}, "c", 32) is None
    with pytest.raises(ValueError, match="neither affine"):
        C.recipe({"d.weight": _shape(64, 96 * 3 // 32 * 1), "d.scales": _shape(64, 3)}, "d", 96)


def _vq_shapes(E=4, OUT=64, IN=256, dim=4, k=2048, group=64):
    bits = (k - 1).bit_length()
    width = (IN // dim + 31) // 32 * bits
    return {"m.codes": _shape(E, OUT, width), "m.codebook": _shape(k, dim),
            "m.vq_scales": _shape(E, OUT, IN // group)}


def test_vq_recipe_packed_and_unpacked_layouts():
    r = C.vq_recipe(_vq_shapes(), "m", in_dims=256)
    assert (r["pack_bits"], r["dim"], r["k"], r["group"], r["in"]) == (11, 4, 2048, 64, 256)
    un = {"m.codes": _shape(2, 8, 32), "m.codebook": _shape(256, 8), "m.vq_scales": _shape(2, 8, 4)}
    r = C.vq_recipe(un, "m")
    assert (r["pack_bits"], r["in"], r["group"], r["code_dtype"]) == (0, 256, 64, torch.uint8)


def test_vq_recipe_rejects_what_the_reference_rejects():
    good = _vq_shapes()
    E, OUT, W = good["m.codes"].shape

    def bind(**edit):
        w = dict(good)
        for t, shape in edit.items():
            if shape is None:
                w.pop(f"m.{t}")
            else:
                w[f"m.{t}"] = _shape(*shape)
        return C.vq_recipe(w, "m", E, OUT, 256)

    bind()
    with pytest.raises(ValueError, match="codebook"):
        bind(codebook=None)
    with pytest.raises(ValueError, match="codes rows"):
        bind(codes=(E, OUT, W + 1))
    with pytest.raises(ValueError, match="shape mismatch"):
        bind(codes=(E, OUT + 1, W))
    with pytest.raises(ValueError, match="shape mismatch"):
        bind(vq_scales=(E + 1, OUT, 4))
    with pytest.raises(ValueError, match="input size"):
        C.vq_recipe(_vq_shapes(IN=200, dim=4, group=40), "m")


def _write(tmp_path, tensors, meta=None, config=None):
    from safetensors.torch import save_file
    d = tmp_path / "art"
    d.mkdir()
    save_file(tensors, str(d / "model.safetensors"), metadata=meta)
    if config is not None:
        (d / "config.json").write_text(json.dumps(config))
    return d


def test_load_quantized_builds_each_layer_from_its_tensors(tmp_path):
    g = torch.Generator().manual_seed(0)
    u32 = lambda *s: torch.randint(0, 2 ** 31, s, generator=g, dtype=torch.int32).view(torch.uint32)
    bf = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16)
    E, OUT, IN, dim, k = 4, 64, 256, 4, 2048
    t = {
        "lin.weight": u32(128, 512 * 4 // 32), "lin.scales": bf(128, 8), "lin.biases": bf(128, 8),
        "sw.weight": u32(3, 32, 256 * 8 // 32), "sw.scales": bf(3, 32, 8), "sw.biases": bf(3, 32, 8),
        "dense.weight": bf(16, 16),
        "vq.codes": u32(E, OUT, (IN // dim + 31) // 32 * 11),
        "vq.codebook": torch.randn(k, dim, generator=g).half(),
        "vq.vq_scales": torch.rand(E, OUT, IN // 64, generator=g).half(),
        "vqu.codes": torch.randint(0, 256, (2, 8, 32), generator=g, dtype=torch.uint8),
        "vqu.codebook": torch.randn(256, 8, generator=g).half(),
        "vqu.vq_scales": torch.rand(2, 8, 4, generator=g).half(),
    }
    meta = {"format": "mlx", "vq_modules": json.dumps(
        {"vq": {"experts": E, "out": OUT, "in": IN, "dim": dim, "k": k, "group": 64, "pack_bits": 11}})}
    d = _write(tmp_path, t, meta, {"quantization": {"group_size": 64, "bits": 4, "sw": {"bits": 8,
                                                                                       "group_size": 32}}})
    mods = C.load_quantized(d, device="cpu")
    assert set(mods) == {"lin", "sw", "vq", "vqu"}
    assert isinstance(mods["lin"], nn.QuantizedLinear) and (mods["lin"].bits, mods["lin"].group_size) == (4, 64)
    assert isinstance(mods["sw"], nn.QuantizedSwitchLinear)
    assert (mods["sw"].bits, mods["sw"].group_size) == (8, 32)
    v = mods["vq"]
    assert isinstance(v, nn.VQSwitchLinear) and (v.pack_bits, v.scale_group, v.input_dims) == (11, 64, IN)
    assert torch.equal(v.codes.view(torch.int32), t["vq.codes"].view(torch.int32))
    vu = mods["vqu"]
    assert vu.pack_bits == 0 and vu.codes.dtype == torch.uint8 and vu.scale_group == 64
    # a module shape overrides the config
    mods = C.load_quantized(d, shapes={"lin": (128, 512)}, device="cpu")
    assert mods["lin"].bits == 4


def test_a_declared_vq_entry_must_match_and_modes_are_read_off_the_tensors(tmp_path):
    g = torch.Generator().manual_seed(1)
    t = {"vq.codes": torch.zeros(2, 8, 22, dtype=torch.int32).view(torch.uint32),
         "vq.codebook": torch.randn(2048, 4, generator=g).half(),
         "vq.vq_scales": torch.rand(2, 8, 4, generator=g).half()}
    meta = {"vq_modules": json.dumps({"vq": {"experts": 2, "out": 8, "in": 256, "dim": 4, "k": 2048,
                                              "group": 64, "pack_bits": 12}})}
    d = _write(tmp_path, t, meta)
    with pytest.raises(ValueError, match="vq_modules"):
        C.load_quantized(d, device="cpu")
    t2 = {"l.weight": torch.zeros(8, 16, dtype=torch.int32).view(torch.uint32),
          "l.scales": torch.zeros(8, 4, dtype=torch.uint8)}
    d2 = tmp_path / "b"
    d2.mkdir()
    from safetensors.torch import save_file
    save_file(t2, str(d2 / "model.safetensors"))
    (d2 / "config.json").write_text(json.dumps({"quantization": {"group_size": 32, "bits": 4,
                                                                 "mode": "nvfp4"}}))
    with pytest.raises(ValueError, match="nvfp4"):
        C.load_quantized(d2, device="cpu")
    (d2 / "config.json").write_text(json.dumps({"quantization": {"group_size": 32, "bits": 4}}))
    m = C.load_quantized(d2, device="cpu")["l"]
    assert (m.mode, m.bits, m.group_size, m.biases) == ("mxfp4", 4, 32, None)


def test_unpacked_short_vectors_are_repacked_exactly():
    """dim-4 uint16 indices (one per vector) become the 16-bit packed layout
    the packed kernel reads; the fields come back unchanged."""
    import oracle as O
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 4096, (2, 3, 40))
    t = {"m.codes": torch.from_numpy(codes.astype(np.int16)).view(torch.uint16),
         "m.codebook": torch.zeros(4096, 4, dtype=torch.float16),
         "m.vq_scales": torch.ones(2, 3, 5, dtype=torch.float16)}
    m = C.build(t, "m", device="cpu")
    assert m.pack_bits == 16 and m.input_dims == 160 and m.scale_group == 32
    back = O.unpack_fields(m.codes.view(torch.int32).numpy().view(np.uint32), 16, 40)
    assert np.array_equal(back, codes)
