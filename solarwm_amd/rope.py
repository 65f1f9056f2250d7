"""Wan RoPE for the cached path, applied on load by the kernels.

The reference keeps pre-RoPE K in its cache and re-ropes the visible window in float64 on every
forward (causal_model.py:791-876 -> echorope_apply :88-197): sink frames at temporal positions
0.., the local frames and the query chunk at window-relative positions.  Per head the 64 complex
channel pairs (2i, 2i+1) split into 22 temporal, 21 height and 21 width pairs
(causal_model.py:1855-1866) with angle ``position * theta^(-2j/d_part)`` (model.py:28-35).

Here a second K pool holds each frame with its height/width pairs already rotated (written once
by the append kernel; spatial positions never change), and the attention kernel turns the
query's temporal pairs by ``(p_query - p_key) * w_j`` per key frame.  Because a rotation pair
contributes ``Re(q conj(k) exp(i (p_q - p_k) w))`` to a score, this equals roping queries and
keys at their own positions.  This module builds the two cos/sin tables the kernels read and
allocates the positions exactly as the reference does.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import torch

TEMPORAL_PAIRS, SPATIAL_PAIRS = 22, 21  # head_dim 128: c - 2*(c//3), c//3 with c = 64


@dataclass(frozen=True)
class RopeConfig:
    """RoPE settings of a Wan model's self-attention (causal_model.py:549-567, :1855-1866).

    ``grid_hw``: the latent patch grid (H, W) of one frame, H * W = frame tokens (tokens are
    ordered row-major inside a frame).  ``use_echorope`` selects EchoRoPE's window-relative
    positions (the default) or block-relative RoPE, optionally frozen at ``rope_train_frames``.
    """

    grid_hw: tuple[int, int]
    use_echorope: bool = True
    rope_train_frames: int | None = None
    theta: float = 10000.0
    table_len: int = 1024  # rope_params(1024, ...)
    # every angle 0: the kernels' RoPE paths then apply no rotation (the PRoPE self-attention
    # branch, which has no RoPE, runs on them this way)
    identity: bool = False

    def __post_init__(self):
        gh, gw = self.grid_hw
        if gh <= 0 or gw <= 0:
            raise ValueError(f"grid_hw must be positive, got {self.grid_hw}")
        if self.rope_train_frames is not None and self.rope_train_frames <= 0:
            raise ValueError(f"rope_train_frames must be positive, got {self.rope_train_frames}")


def _inv_freq(dim: int, theta: float) -> torch.Tensor:
    """float64 theta^(-2j/dim), j < dim/2."""
    return 1.0 / torch.pow(torch.tensor(theta, dtype=torch.float64),
                           torch.arange(0, dim, 2, dtype=torch.float64) / dim)


def spatial_table(cfg: RopeConfig, device) -> torch.Tensor:
    """float32 [(H + W) * 21 * 2]: cos, sin of h * w_j for h < H, then of w * w_j for w < W
    (the height and width parts use the same 42-dim frequencies)."""
    gh, gw = cfg.grid_hw
    inv = _inv_freq(2 * SPATIAL_PAIRS, cfg.theta) * (0.0 if cfg.identity else 1.0)
    ang = torch.cat([torch.outer(torch.arange(gh, dtype=torch.float64), inv),
                     torch.outer(torch.arange(gw, dtype=torch.float64), inv)])
    tab = torch.stack([torch.cos(ang), torch.sin(ang)], dim=-1)
    return tab.to(torch.float32).reshape(-1).contiguous().to(device)


def temporal_table(q_positions: Sequence[int], k_positions: Sequence[int], cfg: RopeConfig,
                   device) -> torch.Tensor:
    """float32 [n_q, n_k, 22, 2]: cos, sin of (q_positions[f] - k_positions[j]) * w_i (the
    44-dim temporal frequencies), computed in float64."""
    inv = _inv_freq(2 * TEMPORAL_PAIRS, cfg.theta) * (0.0 if cfg.identity else 1.0)
    d = (torch.tensor(list(q_positions), dtype=torch.float64)[:, None]
         - torch.tensor(list(k_positions), dtype=torch.float64)[None, :])
    ang = d[..., None] * inv
    tab = torch.stack([torch.cos(ang), torch.sin(ang)], dim=-1)
    return tab.to(torch.float32).contiguous().to(device)


def positions(cfg: RopeConfig, *, num_sink_frames: int, num_local_frames: int,
              num_new_frames: int, max_attention_size: int, frame_tokens: int,
              current_start_frame: int, sink_branch: bool) -> tuple[list[int], list[int]]:
    """(query frame positions, key frame positions in window order) of one cached forward.

    Follows _rope_sink_local_and_query (causal_model.py:791-876; a sink is configured) or
    _rope_q_and_window_k (:718-789; no sink) with _window_relative_positions (:656-701) and
    _echorope_pmax_frames (:703-716).
    """
    nb, nl = num_new_frames, num_local_frames
    ns = num_sink_frames if sink_branch else 0
    if cfg.identity:  # no rotation: every position is 0
        return [0] * nb, [0] * (num_sink_frames + nl)
    pmax = min(max(1, nb, max_attention_size // max(1, frame_tokens)), cfg.table_len)
    if cfg.use_echorope:
        q_last = min(max(0, ns + nl - nb) + nb - 1, pmax - 1)
        q_start = q_last - nb + 1
        local_start = q_last - nl + 1 if nl > 0 else q_last
    elif sink_branch:
        if cfg.rope_train_frames is None:
            q_last = ns + nl - 1
        else:
            q_last = min(current_start_frame + nb - 1, cfg.rope_train_frames - 1)
        q_start = q_last - nb + 1
        local_start = q_last - nl + 1 if nl > 0 else max(ns, q_start)
    else:
        q_start, local_start = nl - nb, 0
    if q_start < 0 or local_start < 0:
        if sink_branch:  # the reference's two checks word for word (causal_model.py:859, :766)
            raise ValueError(
                f"EchoRoPE underflow while assigning sink/local positions: B={nb}, R={nl}, "
                f"sink={ns}, q_start={q_start}, local_start={local_start}, pmax={pmax}")
        raise ValueError(
            f"EchoRoPE underflow while assigning window-relative positions: B={nb}, R={nl}, "
            f"q_start={q_start}, local_start={local_start}, pmax={pmax}")
    keys = list(range(ns)) + list(range(local_start, local_start + nl))
    if keys and max(keys + [q_start + nb - 1]) >= cfg.table_len:
        raise ValueError(f"temporal positions exceed the {cfg.table_len}-entry RoPE table")
    return list(range(q_start, q_start + nb)), keys


class RopeTables:
    """Device tables shared by every layer of a model: the spatial table (fixed) and the
    temporal table per distinct (query positions, key positions) pair, which every layer of a
    pass reuses."""

    def __init__(self, cfg: RopeConfig, device):
        self.cfg = cfg
        self.device = torch.device(device)
        self.hw = spatial_table(cfg, self.device)
        self._t: dict[tuple[tuple[int, ...], tuple[int, ...]], torch.Tensor] = {}

    def temporal(self, q_positions: Sequence[int], k_positions: Sequence[int]) -> torch.Tensor:
        key = (tuple(q_positions), tuple(k_positions))
        t = self._t.get(key)
        if t is None:
            if len(self._t) > 64:
                self._t.clear()
            t = self._t[key] = temporal_table(q_positions, k_positions, self.cfg, self.device)
        return t

