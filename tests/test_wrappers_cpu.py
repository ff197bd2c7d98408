"""The tensor wrappers refuse host tensors before anything reaches the
library: the kernels treat every data pointer as a device address, so a CPU
tensor (or a mix of devices) must fail as a ValueError on the host, never as
a launch."""
from __future__ import annotations

import pytest
import torch

from holonomyawareattention_amd import kernels

B, T, H, d = 1, 8, 2, 6
nb, Dp, Tp = d // 3, 32, 64


def _t(*shape, dtype=torch.float32):
    return torch.zeros(shape, dtype=dtype)


CALLS = {
    "qkvg_projection": lambda: kernels.qkvg_projection(_t(B, T, 64, dtype=torch.bfloat16),
                                                       _t(3 * 64, 64, dtype=torch.bfloat16), None, None),
    "geom_scan": lambda: kernels.geom_scan(_t(B, T, H, d), _t(B, T, H, d), _t(B, T, H, d), _t(B, T, H, d),
                                           None, 0.1),
    "attention": lambda: kernels.attention(_t(B, H, Tp, Dp), _t(B, H, Tp, Dp), _t(B, H, 1, Dp, 64),
                                           _t(B, H, T, nb, 4), d, 0.5),
    "attention_masked": lambda: kernels.attention_masked(_t(B, H, Tp, Dp), _t(B, H, Tp, Dp), _t(B, H, 1, Dp, 64),
                                                         _t(B, H, T, nb, 4), _t(B, H, nb, 4), d, 0.5),
    "attention_backward": lambda: kernels.attention_backward(
        _t(B, T, H, d), None, 0.1, _t(B, H, Tp, Dp), _t(B, H, Tp, Dp), _t(B, H, 1, Dp, 64), _t(B, H, T, nb, 4),
        _t(B, H, Tp), _t(B, T, H, d), _t(B, T, H, d), d, 0.5, _t(B, T, H, d), _t(B, T, H, d), _t(B, T, H, d),
        _t(B, T, H, d), None),
    "quat_to_dense": lambda: kernels.quat_to_dense(_t(3, nb, 4), d),
    "decode_geom": lambda: kernels.decode_geom(_t(B, H, d), _t(B, H, d), _t(B, H, d), None, None, 0.1, 0,
                                               _t(B, H, nb, 4), _t(B, H, Dp), _t(B, H, 64, Dp),
                                               _t(B, H, 1, Dp, 64)),
    "decode_attention": lambda: kernels.decode_attention(_t(B, H, Dp), _t(B, H, 64, Dp), _t(B, H, 1, Dp, 64),
                                                         _t(B, H, nb, 4), 0, d, 0.5),
    "add_layernorm": lambda: kernels.add_layernorm(_t(4, 8), _t(4, 8), _t(8), _t(8)),
    "workspace_status": lambda: kernels.workspace_status(_t(64, dtype=torch.uint8), _t(1, dtype=torch.int32)),
    "attention_masked_train": lambda: kernels.attention_masked_train(
        _t(B, H, Tp, Dp), _t(B, H, Tp, Dp), _t(B, H, 1, Dp, 64), _t(B, H, T, nb, 4), _t(B, H, nb, 4), d, 0.5,
        dropout_p=0.1, seed=3),
    "attention_masked_backward": lambda: kernels.attention_masked_backward(
        _t(B, T, H, d), None, 0.1, _t(B, H, Tp, Dp), _t(B, H, Tp, Dp), _t(B, H, 1, Dp, 64), _t(B, H, T, nb, 4),
        _t(B, H, nb, 4), _t(B, H, Tp), _t(B, T, H, d), _t(B, T, H, d), d, 0.5, _t(B, T, H, d), _t(B, T, H, d),
        _t(B, T, H, d), _t(B, T, H, d), None, dropout_p=0.1, seed=3),
    "dropout_keep_mask": lambda: kernels.dropout_keep_mask(B, T, H, 0.1, 3, device="cpu"),
}


@pytest.mark.parametrize("name", sorted(CALLS))
def test_host_tensors_are_refused(name):
    with pytest.raises(ValueError, match="GPU"):
        CALLS[name]()


def test_one_gpu_reports_the_offending_tensor():
    with pytest.raises(ValueError, match="cpu"):
        kernels._one_gpu("probe", None, torch.zeros(1))
    with pytest.raises(ValueError, match="no tensor"):
        kernels._one_gpu("probe", None)


def test_dropout_arguments_are_checked_on_the_host():
    """dropout_p outside [0, 1), a seed beyond 64 bits or an offset beyond 32
    bits fail as ValueError before the library is called."""
    for p, seed, off in ((1.0, 0, 0), (-0.5, 0, 0), (float("nan"), 0, 0), (0.1, -1, 0), (0.1, 2 ** 64, 0),
                         (0.1, 0, 2 ** 32)):
        with pytest.raises(ValueError, match="dropout_p|seed"):
            kernels._dropout_args("probe", p, seed, off)
    assert kernels._dropout_args("probe", 0.25, 2 ** 64 - 1, 2 ** 32 - 1) == (0.25, 2 ** 64 - 1, 2 ** 32 - 1)
