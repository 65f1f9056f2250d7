"""CPU pins of the H3 GPU tests' bar factor (tests/test_gpu_h3.py _amplification): the bf16
attention bar carried through the value-side and output-side camera maps."""

import torch

from .test_gpu_h3 import _amplification, _bf16_step


def test_unit_values_and_identity_blocks_keep_the_plain_bar():
    vt = torch.zeros(2, 10, 3, 128)
    vt[..., 96:] = 1.0  # RMS 1 on the camera channels
    amp = _amplification(vt, torch.eye(4).expand(1, 5, 4, 4))
    assert amp.shape == (2, 5, 3, 128) and bool((amp == 1).all())


def test_value_scale_and_block_rows_multiply():
    vt = torch.zeros(1, 4, 1, 128)
    vt[..., 96:] = 3.0  # camera channels of RMS 3
    vt[..., 0:96] = 10.0  # rotary channels: not mapped, the plain bar stays
    m = torch.eye(4)
    m[1] = torch.tensor([0.5, 0.0, -1.0, 0.0])  # row 1: absolute sum 1.5
    amp = _amplification(vt, m[None, None].expand(1, 2, 4, 4))
    assert bool((amp[..., :96] == 1).all())
    assert bool((amp[..., 96::4] == 3).all()) and bool((amp[..., 97::4] == 4.5).all())
    assert bool((amp[..., 98::4] == 3).all()) and bool((amp[..., 99::4] == 3).all())


def test_bf16_step():
    x = torch.tensor([1.0, 1.99, 2.0, -6.47, 0.3])
    assert _bf16_step(x).tolist() == [2.0 ** -7, 2.0 ** -7, 2.0 ** -6, 2.0 ** -5, 2.0 ** -9]
    # it is the gap between neighbouring bf16 values: 3 + step is one, 3 + step / 4 rounds to 3
    st = float(_bf16_step(torch.tensor([3.0]))[0])
    assert float(torch.tensor([3.0 + st]).bfloat16()) == 3.0 + st
    assert float(torch.tensor([3.0 + st / 4]).bfloat16()) == 3.0
