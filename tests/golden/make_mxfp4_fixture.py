"""Writes deepseek_v4_tiny_mxfp4_experts.npz: the routed-expert tensors of
layer 0 of the reference's tiny DeepSeek-V4 golden model
(tests/support/goldens/deepseek_v4_tiny/model.safetensors, an mlx-format
checkpoint whose experts are mxfp4: packed 4-bit E2M1 codes, uint8 E8M0
scales per 32 inputs, no biases).  Data only; read with safetensors' safe
loader.  Run from the repository root where /root/reference is present:

    python tests/golden/make_mxfp4_fixture.py
"""
from pathlib import Path

import numpy as np
from safetensors import safe_open

SRC = Path("/root/reference/tests/support/goldens/deepseek_v4_tiny/model.safetensors")
OUT = Path(__file__).resolve().parent / "deepseek_v4_tiny_mxfp4_experts.npz"
PREFIX = "model.layers.0.ffn.switch_mlp."


def main():
    arrays = {}
    with safe_open(str(SRC), framework="numpy") as f:
        for k in f.keys():
            if k.startswith(PREFIX):
                arrays[k[len(PREFIX):].replace(".", "__")] = f.get_tensor(k)
    np.savez_compressed(OUT, **arrays)
    for k, v in sorted(arrays.items()):
        print(k, v.dtype, v.shape)


if __name__ == "__main__":
    main()
