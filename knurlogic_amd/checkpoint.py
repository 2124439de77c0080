"""On-disk formats of the quantized path: mlx-format safetensors checkpoints
and the VQ artifacts' expert tensors, read into this package's modules.

* A layer is stored quantized as ``<m>.weight`` (packed uint32) beside
  ``<m>.scales``, plus ``<m>.biases`` when affine.  Its recipe is read off
  the tensors (src/knurlogic/engine/model/packed.py:33-64): bits from the
  packed width over the layer's input size, group size from the scales'
  width, affine when biases are present, else the mode the artifact's
  config names for the layer or at top level, else mxfp4 (4-bit) / mxfp8
  (8-bit).  mlx-lm's loader takes per-layer entries of the config's
  ``quantization`` block first (src/knurlogic/engine/model/load_model.py:
  124-144).
* VQ experts are ``<m>.codes`` / ``<m>.codebook`` / ``<m>.vq_scales``
  (src/knurlogic/engine/families/deepseek/heads/deepseek_v4.py:36-44,
  95-129): codebook [K, dim] fp16, group = in / vq_scales' width, codes
  either ceil(in/dim/32) * ceil(log2 K) packed words per row or one uint8
  (K <= 256) / uint16 index per vector; a file may describe them in its
  ``vq_modules`` metadata (``experts/out/in/dim/k/group/pack_bits``,
  tests/engine/test_deepseek_v4_mtp.py:206-233).

The affine, mxfp4 and mxfp8 modes are built; another mode (nvfp4, ...)
raises ``ValueError`` naming it.  Files are read with safetensors (no code
executes from a file); tensors are moved to the requested device.
"""
from __future__ import annotations

import json
from pathlib import Path
from typing import Any

import torch

from .nn import QuantizedLinear, QuantizedSwitchLinear, VQSwitchLinear

#: the mode of a packed layer without biases, by bit width (packed.py:20)
SCALED_MODES = {4: "mxfp4", 8: "mxfp8"}


def artifact_quantization(model_path) -> dict[str, Any]:
    """The artifact's quantization settings: config.json's ``quantization``
    block, else its ``quantization_config`` block, else {} (also when there
    is no config.json) -- packed.py:23-30."""
    cfg_file = Path(str(model_path)) / "config.json"
    if not cfg_file.is_file():
        return {}
    cfg = json.loads(cfg_file.read_text())
    for key in ("quantization", "quantization_config"):
        if cfg.get(key):
            return cfg[key]
    return {}


def _declared_mode(quant: dict, key: str):
    """The mode the settings give layer ``key``: its own entry's, else the
    top-level one (either may be absent)."""
    entry = quant.get(key)
    if isinstance(entry, dict) and entry.get("mode"):
        return entry["mode"]
    return quant.get("mode")


def recipe(weights: dict, path: str, in_dims: int, quant: dict | None = None,
           prefix: str = "") -> dict | None:
    """How the packed layer ``path`` was quantized -- {group_size, bits,
    mode} -- read off its tensors' shapes, or None when ``weights`` holds it
    unpacked (no ``.scales``); packed.recipe, packed.py:33-64.  A layer with
    biases is affine; one without takes the mode the settings declare for
    it (``prefix + path``, then the top level) unless that is affine or
    absent, in which case its width decides (4 -> mxfp4, 8 -> mxfp8).
    ``weights`` may hold anything with a ``.shape``."""
    scales = weights.get(f"{path}.scales")
    if scales is None:
        return None
    in_dims = int(in_dims)
    words = int(weights[f"{path}.weight"].shape[-1])
    out = {"group_size": in_dims // int(scales.shape[-1]), "bits": words * 32 // in_dims}
    if f"{path}.biases" in weights:
        out["mode"] = "affine"
        return out
    mode = _declared_mode(quant or {}, prefix + path)
    if mode in (None, "affine"):
        mode = SCALED_MODES.get(out["bits"])
    if mode is None:
        raise ValueError(f"{path}: packed at {out['bits']} bits without biases, which is neither affine "
                         f"nor mxfp4/mxfp8")
    out["mode"] = mode
    return out


def in_dims_from_config(weights: dict, path: str, quant: dict) -> int | None:
    """A packed layer's input size from the config's quantization block
    (a per-layer entry first, as mlx-lm's class predicate takes it), when
    no module skeleton gives it."""
    w = weights.get(f"{path}.weight")
    if w is None:
        return None
    layer = quant.get(path)
    if layer is False:
        return None
    bits = (layer.get("bits") if isinstance(layer, dict) else None) or quant.get("bits")
    if not bits:
        return None
    return int(w.shape[-1]) * 32 // int(bits)


def vq_recipe(weights: dict, path: str, experts: int | None = None, out: int | None = None,
              in_dims: int | None = None) -> dict | None:
    """The VQ layout of ``path``, or None when it is not VQ
    (deepseek_v4._vq_module, :95-129): {experts, out, in, k, dim, group,
    pack_bits (0: one index per vector), code_dtype}.  The expert / out /
    in sizes come from the module skeleton (or a vq_modules entry) when
    given, else from the tensors: the scales' leading axes, and in = codes
    width * dim, which only the one-index-per-vector layout fixes."""
    codes, vs = weights.get(f"{path}.codes"), weights.get(f"{path}.vq_scales")
    if codes is None and vs is None:
        return None
    cb = weights.get(f"{path}.codebook")
    if codes is None or vs is None or cb is None:
        raise ValueError(f"{path}: VQ needs .codes, .codebook and .vq_scales together")
    K, dim = (int(n) for n in cb.shape)
    E = int(experts if experts is not None else vs.shape[0])
    OUT = int(out if out is not None else vs.shape[1])
    ngrp = int(vs.shape[-1])
    width = int(codes.shape[-1])
    bits = (K - 1).bit_length()
    if in_dims is None:
        # without the skeleton's size only the one-index-per-vector layout
        # is unambiguous (a packed row fixes in only to within a block)
        if width % bits == 0 and (width * dim) % ngrp:
            raise ValueError(f"{path}: packed VQ codes need the layer's input size (module shape or "
                             "the file's vq_modules entry)")
        in_dims = width * dim
    IN = int(in_dims)
    if ngrp <= 0 or IN % ngrp or IN % dim:
        raise ValueError(f"{path}: in={IN} does not divide into {ngrp} scale groups of dim-{dim} codes")
    if tuple(int(n) for n in vs.shape) != (E, OUT, ngrp) or tuple(int(n) for n in codes.shape[:2]) != (E, OUT):
        raise ValueError(f"{path}: shape mismatch: codes {tuple(codes.shape)}, vq_scales {tuple(vs.shape)} "
                         f"for {E} experts x {OUT} rows")
    nsub = IN // dim
    if width == (nsub + 31) // 32 * bits:
        pb, cdt = bits, torch.uint32
    elif width == nsub:
        pb, cdt = 0, (torch.uint8 if K <= 256 else torch.uint16)
    else:
        raise ValueError(f"{path}: codes rows are {width} wide; in={IN} at dim {dim} is "
                         f"{(nsub + 31) // 32 * bits} packed {bits}-bit words or {nsub} codes")
    return {"experts": E, "out": OUT, "in": IN, "k": K, "dim": dim, "group": IN // ngrp,
            "pack_bits": pb, "code_dtype": cdt}


def read_safetensors(paths) -> tuple[dict[str, torch.Tensor], dict[str, str]]:
    """Tensors (CPU) and merged string metadata of one or more .safetensors
    files."""
    from safetensors import safe_open
    if isinstance(paths, (str, Path)):
        paths = [paths]
    tensors: dict[str, torch.Tensor] = {}
    meta: dict[str, str] = {}
    for p in paths:
        with safe_open(str(p), framework="pt") as f:
            meta.update(f.metadata() or {})
            for k in f.keys():
                tensors[k] = f.get_tensor(k)
    return tensors, meta


def _u32(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.uint32) if t.dtype == torch.int32 else t


def _repack(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """Unpacked indices [E, N, nsub] -> the packed layout at ``bits``-bit
    fields (rows padded to whole 32-field blocks), on the CPU."""
    E, N, nsub = codes.shape
    nblk = (nsub + 31) // 32
    c = torch.zeros(E, N, nblk * 32, dtype=torch.int64)
    c[..., :nsub] = codes.to(torch.int64)
    words = torch.zeros(E, N, nblk * bits, dtype=torch.int64)
    for j in range(32):
        for_block = c[..., j::32]                                  # [E, N, nblk], field j of each block
        off = j * bits
        q, sh = off // 32, off % 32
        words[..., q::bits] |= (for_block << sh) & 0xFFFFFFFF
        if sh + bits > 32:
            words[..., q + 1::bits] |= for_block >> (32 - sh)
    return words.to(torch.int32).view(torch.uint32)


def build(weights: dict, path: str, in_dims: int | None = None, quant: dict | None = None,
          device="cuda", prefix: str = ""):
    """This package's module for the packed (or VQ) layer ``path``: a
    QuantizedLinear (2-D weight), QuantizedSwitchLinear (3-D) or
    VQSwitchLinear; None when ``path`` is stored unpacked."""
    vq = vq_recipe(weights, path, in_dims=in_dims)
    if vq is not None:
        codes = weights[f"{path}.codes"]
        cb = weights[f"{path}.codebook"].to(device=device, dtype=torch.float16)
        vs = weights[f"{path}.vq_scales"].to(device=device, dtype=torch.float16)
        pb, dim, group = vq["pack_bits"], vq["dim"], vq["group"]
        if pb:
            return VQSwitchLinear(_u32(codes).to(device), cb, vs, scale_group=group, pack_bits=pb,
                                  in_features=vq["in"])
        if dim == 8 and (group == vq["in"] or group % 64 == 0):
            per_channel = group == vq["in"]
            return VQSwitchLinear(codes.to(device=device, dtype=vq["code_dtype"]), cb,
                                  vs[..., 0].contiguous() if per_channel else vs,
                                  scale_group=0 if per_channel else group)
        bits = 8 if vq["k"] <= 256 else 16
        return VQSwitchLinear(_repack(codes, bits).to(device), cb, vs, scale_group=group, pack_bits=bits,
                              in_features=vq["in"])
    if f"{path}.scales" not in weights:
        return None
    quant = quant or {}
    if in_dims is None:
        in_dims = in_dims_from_config(weights, path, quant)
        if in_dims is None:
            raise ValueError(f"{path}: packed, but neither a module shape nor the config's quantization "
                             "block gives its input size")
    r = recipe(weights, path, in_dims, quant, prefix)
    if r["mode"] not in ("affine", "mxfp4", "mxfp8"):
        raise ValueError(f"{path}: mode {r['mode']!r} is not implemented (affine, mxfp4, mxfp8)")
    w = _u32(weights[f"{path}.weight"]).to(device)
    s = weights[f"{path}.scales"].to(device)
    if r["mode"] == "affine":
        b = weights[f"{path}.biases"].to(device=device, dtype=s.dtype)
        act = s.dtype
    else:
        b, act = None, torch.bfloat16                      # uint8 E8M0 scales, no biases
    bias = weights.get(f"{path}.bias")
    bias = bias.to(device=device, dtype=act) if bias is not None else None
    cls = QuantizedLinear if w.dim() == 2 else QuantizedSwitchLinear
    return cls(w, s, b, bias, group_size=r["group_size"], bits=r["bits"], mode=r["mode"])


def load_quantized(model_path=None, files=None, shapes: dict | None = None, device="cuda") -> dict:
    """Every packed or VQ layer of an mlx-format artifact (``model*.safetensors``
    and config.json under ``model_path``, or explicit ``files``) as this
    package's modules, {path: module}.  ``shapes`` maps a layer path to its
    dense weight shape (the module skeleton's), else input sizes come from
    the config's quantization block.  VQ layers described in a file's
    ``vq_modules`` metadata are checked against it."""
    if files is None:
        files = sorted(Path(str(model_path)).glob("model*.safetensors"))
        if not files:
            raise FileNotFoundError(f"No safetensors found in {model_path}")
    weights, meta = read_safetensors(files)
    quant = artifact_quantization(model_path) if model_path is not None else {}
    declared = json.loads(meta["vq_modules"]) if "vq_modules" in meta else {}
    paths = sorted({k.rsplit(".", 1)[0] for k in weights
                    if k.endswith(".scales") or k.endswith(".codes") or k.endswith(".vq_scales")})
    out = {}
    for p in paths:
        in_dims = None
        if shapes and p in shapes:
            in_dims = int(shapes[p][-1])
        if p in declared:
            m = declared[p]
            if in_dims is None and m.get("in") is not None:
                in_dims = int(m["in"])
            r = vq_recipe(weights, p, m.get("experts"), m.get("out"), m.get("in"))
            if r is None or r["pack_bits"] != int(m.get("pack_bits", r["pack_bits"])) or \
                    r["dim"] != int(m.get("dim", r["dim"])) or r["k"] != int(m.get("k", r["k"])) or \
                    r["group"] != int(m.get("group", r["group"])):
                raise ValueError(f"{p}: tensors do not match the file's vq_modules entry {m}")
        mod = build(weights, p, in_dims, quant, device)
        if mod is not None:
            out[p] = mod
    return out
