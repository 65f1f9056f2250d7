"""The H3 parity bar for outputs mapped by per-row camera blocks (tests/test_gpu_h3.py), on the
CPU: identity blocks give the plain attention bar, a block of gain g admits g times it."""

import pytest
import torch

from .helpers import MAX_ABS
from .test_gpu_h3 import _assert_projected_close


def _case(block):
    want = torch.zeros(1, 3, 2, 128)
    m = block.expand(1, 3, 4, 4).clone()
    return want, m


def test_identity_blocks_keep_the_attention_bar():
    want, m = _case(torch.eye(4))
    _assert_projected_close(want + 0.9 * MAX_ABS * (torch.arange(128) == 5), want, m)
    with pytest.raises(AssertionError):
        _assert_projected_close(want + 1.1 * MAX_ABS * (torch.arange(128) == 5), want, m)


def test_bar_scales_with_the_block_gain_of_each_channel():
    block = torch.eye(4)
    block[2, :] = torch.tensor([1.0, -1.0, 0.5, 0.5])  # channel 2 of each group: gain 3
    want, m = _case(block)
    _assert_projected_close(want + 2.9 * MAX_ABS * (torch.arange(128) == 6), want, m)  # 6 % 4 == 2
    with pytest.raises(AssertionError):
        _assert_projected_close(want + 2.9 * MAX_ABS * (torch.arange(128) == 5), want, m)
    with pytest.raises(AssertionError):
        _assert_projected_close(want + 3.1 * MAX_ABS * (torch.arange(128) == 6), want, m)
