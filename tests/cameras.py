"""Synthetic camera trajectories for the PRoPE tests: per latent frame a rigid world-to-camera
transform (rotation about a random axis plus a translation) and the data path's intrinsics
(fx = 969.7 / 1920, fy = 969.7 / 1080, principal point (0.5, 0.5))."""

import math

import torch

FX, FY = 969.6969696969696 / 1920.0, 969.6969696969696 / 1080.0


def trajectory(batch: int, frames: int, seed: int, t_scale: float = 0.5,
               angle: float = math.pi / 6) -> tuple[torch.Tensor, torch.Tensor]:
    """(viewmats [B, F, 4, 4], K [B, F, 3, 3]) float32; frame 0 of each stream is a random pose
    too, so no camera is the identity."""
    g = torch.Generator().manual_seed(seed)
    n = batch * frames
    axis = torch.randn(n, 3, generator=g, dtype=torch.float64)
    axis = axis / axis.norm(dim=-1, keepdim=True)
    th = (torch.rand(n, generator=g, dtype=torch.float64) * 2 - 1) * angle
    kx = torch.zeros(n, 3, 3, dtype=torch.float64)
    kx[:, 0, 1], kx[:, 0, 2], kx[:, 1, 2] = -axis[:, 2], axis[:, 1], -axis[:, 0]
    kx = kx - kx.transpose(1, 2)
    rot = (torch.eye(3, dtype=torch.float64) + th.sin()[:, None, None] * kx
           + (1 - th.cos())[:, None, None] * kx @ kx)
    v = torch.zeros(n, 4, 4, dtype=torch.float64)
    v[:, :3, :3] = rot
    v[:, :3, 3] = torch.randn(n, 3, generator=g, dtype=torch.float64) * t_scale
    v[:, 3, 3] = 1.0
    k = torch.zeros(n, 3, 3, dtype=torch.float64)
    k[:, 0, 0], k[:, 1, 1], k[:, 0, 2], k[:, 1, 2], k[:, 2, 2] = FX, FY, 0.5, 0.5, 1.0
    return (v.to(torch.float32).reshape(batch, frames, 4, 4),
            k.to(torch.float32).reshape(batch, frames, 3, 3))


def per_token(x: torch.Tensor, frame_tokens: int) -> torch.Tensor:
    """Expand per-frame tensors [B, F, ...] to per-token [B, F*T, ...] (the data path's layout)."""
    return x.repeat_interleave(frame_tokens, dim=1).contiguous()
