"""Writes tests/golden/qwen35_moe_block.npz from the reference's golden.

Source: the reference's tests/support/goldens/qwen_reference.npz, key
``qwen3_5_moe/bf16/0.mlp`` -- HF transformers 5.16.1's bf16
Qwen3_5MoeSparseMoeBlock (layer 0 of a tiny config: hidden 32, 4 experts,
top-2, expert and shared-expert intermediate 16) on a (1, 21, 32) bf16
input, which the reference holds knurlogic's MLX MoE block to bit for bit
(tests/engine/test_qwen_reference.py:215-239).  The reference stores no
weights: it re-makes them from numpy by parameter name
(tests/support/goldens/build_qwen_reference.py:174-196 ``init_weights``,
:328-339 ``component_input`` / ``component_weights``).  This script makes
the same numbers the same way and stores them beside the expected output,
so the test needs neither the reference nor its builder.

Run in the build container (the reference is only there):
    python tests/golden/make_qwen_moe_golden.py
"""
import json
import sys
import zlib
from pathlib import Path

import numpy as np

REF = Path("/root/reference/tests/support/goldens/qwen_reference.npz")
OUT = Path(__file__).resolve().parent / "qwen35_moe_block.npz"
PREFIX = "model.layers.0.mlp."
PROMPT_LEN = 21      # len(PROMPT) of the builder
WIDTH = 32           # the MoE block's input width (hidden size)


def bf16(a):
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def weight(name, shape):
    """A matrix of the builder's init: standard normal / sqrt(fan_in) from
    the stream seeded [7, crc32(name)], then rounded to bf16."""
    rng = np.random.default_rng([7, zlib.crc32(name.encode())])
    a = rng.standard_normal(shape) / np.sqrt(np.prod(shape[1:]))
    return bf16(a.astype(np.float32))


def main():
    z = np.load(REF)                      # allow_pickle stays False
    meta = json.loads(bytes(z["meta"]).decode())
    shapes = meta["qwen3_5_moe/shapes"]
    cfg = meta["qwen3_5_moe/config"]
    w = {k[len(PREFIX):]: weight(k, tuple(v)) for k, v in shapes.items()
         if k.startswith(PREFIX)}
    rng = np.random.default_rng([5, WIDTH])
    x = bf16(rng.standard_normal((1, PROMPT_LEN, WIDTH)).astype(np.float32))
    np.savez_compressed(
        OUT, x=x[0], expected=z["qwen3_5_moe/bf16/0.mlp"][0],
        top_k=np.int32(cfg["num_experts_per_tok"]),
        **{k.replace(".", "__"): v for k, v in w.items()})
    print("wrote", OUT, sorted(w), x.shape)


if __name__ == "__main__":
    sys.exit(main())
