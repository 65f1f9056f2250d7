"""Host side of RoPE on load: the position allocation and the cos/sin tables the kernels read
agree with the oracle's restatement of the reference (no GPU needed)."""

import itertools

import pytest
import torch

from oracle import wan_cache_ref as ref
from solarwm_amd import rope


@pytest.mark.parametrize("use_echorope,rtf", [(True, None), (False, None), (False, 12)])
def test_positions_match_oracle(use_echorope, rtf):
    cfg = rope.RopeConfig(grid_hw=(3, 4), use_echorope=use_echorope, rope_train_frames=rtf)
    T = 12
    for ns, nl, nb, cap, csf, sink_branch in itertools.product(
            (0, 1, 2), (0, 1, 3, 9, 20), (1, 3), (5, 21, 40), (0, 7, 40), (True, False)):
        kw = dict(num_sink_frames=ns, num_local_frames=nl, num_new_frames=nb,
                  max_attention_size=cap * T, frame_seqlen=T, current_start_frame=csf,
                  sink_branch=sink_branch)
        try:
            want = ref.rope_positions(use_echorope=use_echorope, rope_train_frames=rtf, **kw)
        except ValueError:
            with pytest.raises(ValueError):
                rope.positions(cfg, num_sink_frames=ns, num_local_frames=nl, num_new_frames=nb,
                               max_attention_size=cap * T, frame_tokens=T, current_start_frame=csf,
                               sink_branch=sink_branch)
            continue
        qpos, kpos = rope.positions(cfg, num_sink_frames=ns, num_local_frames=nl,
                                    num_new_frames=nb, max_attention_size=cap * T,
                                    frame_tokens=T, current_start_frame=csf,
                                    sink_branch=sink_branch)
        assert qpos == list(range(want["q_start"], want["q_start"] + nb))
        assert kpos == list(range(want["num_sink"])) + list(
            range(want["local_start"], want["local_start"] + nl))


def test_underflow_messages_name_the_reference_check():
    """A window that does not fit the positions raises the reference's ValueError of that path:
    sink/local positions (causal_model.py:859) or window-relative positions (:766)."""
    cfg = rope.RopeConfig(grid_hw=(3, 4), use_echorope=False, rope_train_frames=4)
    kw = dict(num_local_frames=5, num_new_frames=2, max_attention_size=9 * 12, frame_tokens=12,
              current_start_frame=20)
    with pytest.raises(ValueError, match=r"^EchoRoPE underflow while assigning sink/local "
                                         r"positions: B=2, R=5, sink=1, q_start=2, local_start=-1"):
        rope.positions(cfg, num_sink_frames=1, sink_branch=True, **kw)
    with pytest.raises(ValueError, match=r"^EchoRoPE underflow while assigning window-relative "
                                         r"positions: B=3, R=2, q_start=-1, local_start=0"):
        rope.positions(cfg, num_sink_frames=0, sink_branch=False,
                       **dict(kw, num_local_frames=2, num_new_frames=3))


def test_tables_match_oracle_freqs():
    f = ref.wan_rope_freqs()
    cfg = rope.RopeConfig(grid_hw=(5, 7))
    hw = rope.spatial_table(cfg, "cpu").view(-1, 21, 2).double()
    want_h = torch.stack([f[:5, 22:43].real, f[:5, 22:43].imag], -1)
    want_w = torch.stack([f[:7, 43:].real, f[:7, 43:].imag], -1)
    assert torch.allclose(hw[:5], want_h, atol=1e-7) and torch.allclose(hw[5:], want_w, atol=1e-7)
    qpos, kpos = [18, 19, 20], [0, 1, 2, 9, 20]
    t = rope.temporal_table(qpos, kpos, cfg, "cpu").double()
    for i, pq in enumerate(qpos):
        for j, pk in enumerate(kpos):
            # the pair angle of (pq - pk) is the table's pq angle minus its pk angle
            z = f[pq, :22] * f[pk, :22].conj()
            assert torch.allclose(t[i, j, :, 0], z.real, atol=1e-6)
            assert torch.allclose(t[i, j, :, 1], z.imag, atol=1e-6)
