"""Host-side argument checks of the MoE wrappers (no kernel calls): the
stacked expert tensors must match x's width, the expert count and each
other, since the kernels take only the sizes and would otherwise read past a
smaller tensor."""
import pytest
import torch

from knurlogic_amd import ops


def _affine(E=4, H=256, I=128, bits=4, g=64):
    u32 = torch.int32
    return dict(
        w_gu=torch.zeros(E, 2 * I, H * bits // 32, dtype=u32),
        s_gu=torch.zeros(E, 2 * I, H // g, dtype=torch.bfloat16),
        b_gu=torch.zeros(E, 2 * I, H // g, dtype=torch.bfloat16),
        w_down=torch.zeros(E, H, I * bits // 32, dtype=u32),
        s_down=torch.zeros(E, H, I // g, dtype=torch.bfloat16),
        b_down=torch.zeros(E, H, I // g, dtype=torch.bfloat16),
    )


def _check(t, H=256, E=4, g=64, bits=4):
    return ops._check_experts("moe", H, E, t["w_gu"], t["s_gu"], t["b_gu"], t["w_down"], t["s_down"],
                              t["b_down"], g, bits)


def test_matching_experts_pass_and_give_I():
    assert _check(_affine()) == 128
    assert _check(_affine(bits=8), bits=8) == 128
    mx = _affine(g=32)
    assert ops._check_experts("mx", 256, 4, mx["w_gu"], mx["s_gu"], None, mx["w_down"], mx["s_down"], None,
                              32, 4) == 128


@pytest.mark.parametrize("name,shape", [
    ("w_gu", (4, 256, 16)),        # H of 128, not 256
    ("w_gu", (3, 256, 32)),        # one expert fewer
    ("s_gu", (4, 256, 2)),         # scales for a narrower x
    ("b_gu", (4, 128, 4)),         # biases for half the rows
    ("w_down", (2, 256, 16)),      # down with fewer experts
    ("w_down", (4, 256, 8)),       # down over a smaller I
    ("s_down", (4, 128, 2)),
    ("b_down", (4, 256, 1)),
])
def test_each_mismatch_is_refused(name, shape):
    t = _affine()
    t[name] = torch.zeros(shape, dtype=t[name].dtype)
    with pytest.raises(ValueError, match=name):
        _check(t)


def test_wrong_width_or_count_is_refused():
    t = _affine()
    with pytest.raises(ValueError, match="w_gu"):
        _check(t, H=512)               # x wider than the experts
    with pytest.raises(ValueError, match="w_gu"):
        _check(t, E=8)                 # more experts routed than stored
    with pytest.raises(ValueError, match="w_gu"):
        _check(t, bits=8)              # 8-bit reading of a 4-bit tensor


def test_odd_stacked_rows_and_missing_bias_are_refused():
    t = _affine()
    t["w_gu"] = torch.zeros(4, 255, 32, dtype=torch.int32)
    with pytest.raises(ValueError, match="2I"):
        _check(t)
    t = _affine()
    t["b_down"] = None
    with pytest.raises(ValueError, match="b_down"):
        _check(t)


def test_moe_experts_refuses_cpu_tensors_before_any_kernel():
    t = _affine()
    x = torch.zeros(1, 256, dtype=torch.bfloat16)
    logits = torch.zeros(1, 4, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU memory"):
        ops.moe_experts(x, logits, 2, *t.values())
