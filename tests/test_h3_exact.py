"""CPU pins of the unrounded camera projection that the H3 GPU tests compare against
(tests/test_gpu_h3.py _exact_projected)."""

import torch

from oracle import h3_ref as ref

from .test_gpu_h3 import _exact_projected


def test_identity_blocks_leave_the_output():
    o = torch.randn(2, 5, 3, 128, dtype=torch.float64)
    eye = torch.eye(4).expand(2, 5, 4, 4)
    assert torch.equal(_exact_projected(o, eye), o)


def test_rows_of_the_block_map_each_group():
    o = torch.zeros(1, 1, 1, 128, dtype=torch.float64)
    o[..., 96:100] = torch.tensor([1.0, 2.0, 3.0, 4.0], dtype=torch.float64)
    o[..., 5] = 7.0
    m = torch.tensor([[1.0, 0, 0, 0], [0, 0, 1.0, 0], [0.5, 0.5, 0, 0], [0, 0, 0, -1.0]])[None, None]
    y = _exact_projected(o, m)
    assert y[0, 0, 0, 96:100].tolist() == [1.0, 3.0, 1.5, -4.0]
    assert float(y[0, 0, 0, 5]) == 7.0 and float(y[..., 100:].abs().sum()) == 0.0


def test_agrees_with_the_oracle_projection_to_a_bf16_step():
    g = torch.Generator().manual_seed(9)
    x = (torch.randn(2, 7, 3, 128, generator=g) * 2).to(torch.bfloat16)
    m = torch.randn(2, 7, 4, 4, generator=g) * 0.6
    ours = _exact_projected(x.double(), m)
    theirs = ref.prope_project(x, m).double()
    assert torch.equal(ours[..., :96], theirs[..., :96])
    step = torch.ldexp(torch.ones_like(theirs), torch.frexp(theirs.abs().clamp_min(1e-30)).exponent - 8)
    assert bool(((ours - theirs).abs() <= step).all())
