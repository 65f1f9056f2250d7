"""Fused PRoPE (camera projective positional encoding) on the cached path, applied by the kernels.

The reference's fused mode (solar/backends/wan22/runtime/modeling/causal_model.py:585-651,
:1170-1199; camera_prope.py:93-261) keeps raw K/V plus a camera cache with the same token layout
(causal_model.py:1948-2075).  Every forward it ropes the visible window and then maps, per group
of 4 head channels, q -> P_qᵀ q, k -> P_k⁻¹ k, v -> P_k⁻¹ v (P = lift(K_norm) · viewmat of the
token's camera), attends, and maps the output back with P_q.

Here cameras are per latent frame (the data path expands one camera per frame to all its tokens,
solar/backends/wan22/runtime/data.py:516-530), stored per frame slot next to the K/V slots:

* at append, each written frame's P⁻¹ is applied once: to V (a transformed V copy) and to the
  spatial channel groups of the height/width-roped K copy (spatial RoPE never changes);
* the temporal groups (channels 0..43, 11 groups) see a RoPE rotation that moves with the
  window, so the query takes, per (query frame, key frame), the 4x4
  W = R_k(p_k)ᵀ (P_q P_k⁻¹)ᵀ R_q(p_q) per group — built here once per pass for all layers;
* the query's spatial groups take P_qᵀ after their RoPE, and the output takes P_q.

``q·k`` summed over a group is then ``(P_qᵀ R_q q)·(P_k⁻¹ R_k k)``, the reference's score.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Sequence

import torch

from .rope import TEMPORAL_PAIRS, _inv_freq

GROUPS_T = TEMPORAL_PAIRS // 2  # 11 channel groups of 4 hold temporal RoPE pairs only
TRANSLATION_TRANSFORMS = ("linear", "logd4")


@dataclass(frozen=True)
class PropeConfig:
    """Camera settings of the fused-PRoPE self-attention (causal_model.py:549-568).

    ``camera_translation_transform``: ``"linear"`` (as stored) or ``"logd4"`` (translations
    compressed to t · log1p(|t|) / (4|t|), camera.py:31-62)."""

    camera_translation_transform: str = "linear"

    def __post_init__(self):
        if self.camera_translation_transform not in TRANSLATION_TRANSFORMS:
            raise ValueError(
                f"camera_translation_transform must be one of {TRANSLATION_TRANSFORMS}, got "
                f"{self.camera_translation_transform!r}")


# ---------------------------------------------------------------------------------------------
# camera algebra (device tensors; camera_prope.py:206-231, :307-338; camera.py:31-62)
# ---------------------------------------------------------------------------------------------
def transform_relative_viewmats(viewmats: torch.Tensor, transform: str) -> torch.Tensor:
    if transform == "linear":
        return viewmats
    work = torch.float64 if viewmats.dtype == torch.float64 else torch.float32
    t = viewmats[..., :3, 3].to(work)
    norm = torch.linalg.vector_norm(t, dim=-1, keepdim=True)
    scale = torch.where(norm > 0, torch.log1p(norm) / (4.0 * norm.clamp_min(torch.finfo(work).tiny)),
                        torch.zeros_like(norm))
    out = viewmats.clone()
    out[..., :3, 3] = (t * scale).to(viewmats.dtype)
    return out


def projection(viewmats: torch.Tensor, ks: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(P, P⁻¹) in float64: P = diag(fx, fy, 1, 1) V (the principal point is dropped) and
    P⁻¹ = V⁻¹ diag(1/fx, 1/fy, 1, 1) with V⁻¹ = [Rᵀ -Rᵀt; 0 1]."""
    v = viewmats.to(torch.float64)
    k = ks.to(torch.float64)
    one = torch.ones_like(k[..., 0, 0])
    d = torch.stack([k[..., 0, 0], k[..., 1, 1], one, one], dim=-1)
    p = d[..., :, None] * v
    rt = v[..., :3, :3].transpose(-1, -2)
    vinv = torch.zeros_like(v)
    vinv[..., :3, :3] = rt
    vinv[..., :3, 3] = -(rt @ v[..., :3, 3:4])[..., 0]
    vinv[..., 3, 3] = 1.0
    return p, vinv / d[..., None, :]


def _temporal_rotations(positions: Sequence[int], theta: float, device) -> torch.Tensor:
    """float64 [n, 11, 4, 4]: per group g, blockdiag(rot(p w_2g), rot(p w_2g+1)) with
    rot(a) = [[cos a, -sin a], [sin a, cos a]] acting on (x[2i], x[2i+1])."""
    inv = _inv_freq(2 * TEMPORAL_PAIRS, theta).to(device)
    ang = torch.tensor(list(positions), dtype=torch.float64, device=device)[:, None] * inv
    c, s = torch.cos(ang), torch.sin(ang)
    n = len(positions)
    r = torch.zeros(n, GROUPS_T, 4, 4, dtype=torch.float64, device=device)
    for half in range(2):
        cc, ss = c[:, half::2], s[:, half::2]
        i = 2 * half
        r[:, :, i, i], r[:, :, i, i + 1] = cc, -ss
        r[:, :, i + 1, i], r[:, :, i + 1, i + 1] = ss, cc
    return r


def frame_cameras(cam: torch.Tensor, *, current_start: int, num_new_tokens: int,
                  frame_tokens: int, per_frame: bool, check: bool) -> torch.Tensor:
    """The current chunk's cameras, one per latent frame ``[B, nb, ...]``.

    Per-token tensors follow the reference's slicing (current-chunk or full-trajectory length,
    causal_model.py:1927-1945) and must repeat one camera over each frame's tokens (``check``
    verifies it, at the cost of one device synchronisation).  ``per_frame`` tensors are indexed
    by latent frame (current chunk, or the full trajectory from frame 0)."""
    nb = num_new_tokens // frame_tokens
    if per_frame:
        f0 = current_start // frame_tokens
        if cam.shape[1] == nb:
            return cam
        if cam.shape[1] >= f0 + nb:
            return cam[:, f0 : f0 + nb]
        raise ValueError(f"per-frame camera tensor of {cam.shape[1]} frames does not cover frames "
                         f"[{f0}, {f0 + nb})")
    if cam.shape[1] != num_new_tokens:
        end = current_start + num_new_tokens
        if current_start < 0 or cam.shape[1] < end:
            raise ValueError(f"fused_prope camera tensor of {cam.shape[1]} tokens does not cover "
                             f"the current chunk [{current_start}, {end})")
        cam = cam[:, current_start:end]
    by_frame = cam.reshape(cam.shape[0], nb, frame_tokens, *cam.shape[2:])
    first = by_frame[:, :, :1]
    if check and not bool((by_frame == first).all()):
        raise ValueError("fused PRoPE on the slot cache needs one camera per latent frame "
                         "(every token of a frame must carry the same viewmat and K)")
    return first[:, :, 0]


# ---------------------------------------------------------------------------------------------
# the camera cache (one per model, indexed by frame slot like every layer's K/V pools)
# ---------------------------------------------------------------------------------------------
class CameraCache:
    """Per-slot cameras of the fused mode: raw view matrices and intrinsics (for the reference's
    ``_fused_prope_camera_metadata`` view) and each frame's P⁻¹ (float32 [n_slots, B, 4, 4])."""

    def __init__(self, n_slots: int, batch: int, device, cfg: PropeConfig):
        self.cfg = cfg
        self.device = torch.device(device)
        self.viewmats = torch.zeros(n_slots, batch, 4, 4, dtype=torch.float32, device=self.device)
        self.ks = torch.zeros(n_slots, batch, 3, 3, dtype=torch.float32, device=self.device)
        self.p_inv = torch.zeros(n_slots, batch, 4, 4, dtype=torch.float32, device=self.device)
        self.active = False  # no camera-conditioned frame has been written yet

    def reset(self) -> None:
        self.viewmats.zero_()
        self.ks.zero_()
        self.p_inv.zero_()
        self.active = False


@dataclass
class CameraPass:
    """Everything the layers of one forward need, computed once (``stage_camera_cache``)."""

    current_start: int
    num_new_tokens: int
    staging: tuple[int, ...]
    window: tuple[int, ...]
    kv_xform: torch.Tensor  # [n_written, B, 4, 4] P⁻¹ of the frames written this pass
    q_xform_t: torch.Tensor  # [B, n_keys_frames, nb, 11, 4, 4]
    q_xform_s: torch.Tensor  # [B, nb, 4, 4] P_qᵀ
    out_xform: torch.Tensor  # [B, nb, 4, 4] P_q
    camera: CameraCache = field(repr=False)


def stage_camera_cache(kv_cache: Sequence[Any], cam_viewmats: torch.Tensor, cam_K: torch.Tensor,
                       current_start: int, num_new_tokens: int, *,
                       sink_recache_after_switch: bool = False, per_frame: bool = False,
                       check_frame_constant: bool = True) -> CameraPass:
    """The fused camera staging of one forward (causal_model.py:1948-2066), for the slot cache.

    The frames this forward writes get their cameras in the staging slots the K/V append uses
    (so committing the K/V slot table commits the cameras too); a recompute pass that
    rewrites sink frames (``sink_recache_after_switch``) keeps the old sink cameras, as the
    reference's camera staging does.  Returns the per-pass tables for ``attend_cached``.
    """
    if cam_viewmats is None or cam_K is None:
        raise ValueError("fused_prope camera-conditioned KV-cache requires both viewmats and K")
    if not kv_cache:
        raise ValueError("fused_prope KV-cache requires a non-empty block cache")
    c0 = kv_cache[0]
    cam = c0.camera
    if cam is None or c0.rope is None:
        raise ValueError("the cache was allocated without prope= (fused PRoPE needs a pre-RoPE, "
                         "camera-aware cache)")
    g = c0.geom
    T = g.frame_tokens
    if cam_viewmats.shape[0] != g.batch or cam_K.shape[0] != g.batch:
        raise ValueError(f"fused_prope camera/cache batch mismatch: camera="
                         f"{cam_viewmats.shape[0]}, cache={g.batch}")
    if not cam.active and c0.local_end > 0:
        raise RuntimeError("fused_prope found populated raw K/V history without shared "
                           "camera metadata; reset/rebuild the cache before enabling camera")
    plan, temp, staging, window = c0.plan(int(current_start), int(num_new_tokens),
                                          sink_recache_after_switch)
    dev = cam.device
    vq = frame_cameras(cam_viewmats, current_start=current_start, num_new_tokens=num_new_tokens,
                       frame_tokens=T, per_frame=per_frame, check=check_frame_constant)
    kq = frame_cameras(cam_K, current_start=current_start, num_new_tokens=num_new_tokens,
                       frame_tokens=T, per_frame=per_frame, check=check_frame_constant)
    vq = vq.to(device=dev, dtype=torch.float32)
    kq = kq.to(device=dev, dtype=torch.float32)
    cam.active = True  # camera-conditioned frames from here on (causal_model.py:2005-2019)
    c0.metadata_present = True  # a dropped camera state is recreated (causal_model.py:2008-2011)
    tr = cam.cfg.camera_translation_transform
    p_q, p_q_inv = projection(transform_relative_viewmats(vq, tr), kq)  # [B, nb, 4, 4]

    # written frames: position ws_f + i takes chunk frame roped_offset/T + i, except positions
    # below the camera write start, which keep the camera already there
    ws_f = plan.write_start_index // T
    off_f = plan.roped_offset // T
    cam_ws = (max(plan.local_start_index, plan.sink_tokens) if plan.is_recompute
              else plan.local_start_index)
    pre = list(c0.table)
    if plan.action == "roll_and_insert" and plan.num_rolled_tokens > 0:
        sf, ef, rf = plan.sink_tokens // T, plan.num_evicted_tokens // T, plan.num_rolled_tokens // T
        pre[sf : sf + rf] = pre[sf + ef : sf + ef + rf]
    if staging:
        new_view = vq.transpose(0, 1)[off_f : off_f + len(staging)].clone()  # [n, B, 4, 4]
        new_k = kq.transpose(0, 1)[off_f : off_f + len(staging)].clone()
        new_inv = p_q_inv.transpose(0, 1)[off_f : off_f + len(staging)].to(torch.float32)
        for i, s in enumerate(staging):
            pos = ws_f + i
            if pos * T < cam_ws:  # keep the previous camera of this position
                old = pre[pos]
                new_view[i], new_k[i], new_inv[i] = cam.viewmats[old], cam.ks[old], cam.p_inv[old]
        idx = torch.tensor(list(staging), dtype=torch.long, device=dev)
        cam.viewmats.index_copy_(0, idx, new_view)
        cam.ks.index_copy_(0, idx, new_k)
        cam.p_inv.index_copy_(0, idx, new_inv.contiguous())
        kv_xform = new_inv.contiguous()
    else:
        kv_xform = torch.zeros(0, g.batch, 4, 4, dtype=torch.float32, device=dev)

    from .attention import window_positions  # the RoPE positions attend_cached uses

    nb = num_new_tokens // T
    qpos, kpos = window_positions(c0, plan, window, nb, int(current_start))
    widx = torch.tensor(list(window), dtype=torch.long, device=dev)
    pk_inv = cam.p_inv.index_select(0, widx).to(torch.float64)  # [nk, B, 4, 4]
    a = torch.einsum("bfik,jbkl->bfjil", p_q, pk_inv)  # P_q P_k⁻¹: [B, nb, nk, 4, 4]
    theta = c0.rope.cfg.theta
    rq = _temporal_rotations(qpos, theta, dev)  # [nb, 11, 4, 4]
    rk = _temporal_rotations(kpos, theta, dev)  # [nk, 11, 4, 4]
    # W = R_kᵀ Aᵀ R_q:  W_im = sum_{k,l} Rk_ki A_lk Rq_lm
    w = torch.einsum("jgki,bfjlk,fglm->bjfgim", rk, a, rq)
    return CameraPass(
        current_start=int(current_start), num_new_tokens=int(num_new_tokens),
        staging=tuple(staging), window=tuple(window), kv_xform=kv_xform,
        q_xform_t=w.to(torch.float32).contiguous(),
        q_xform_s=p_q.transpose(-1, -2).to(torch.float32).contiguous(),
        out_xform=p_q.to(torch.float32).contiguous(), camera=cam)


def commit_camera_cache(update: CameraPass | None) -> None:
    """The reference commits staged camera rows after every block succeeded
    (causal_model.py:2068-2075).  Here the cameras already sit in the staging slots, and the
    K/V commit (``apply_cache_updates``) moves them into the cache with the slot table; this
    call only checks that the pass still owns its staging slots."""
    if update is None:
        return
    if not update.camera.active:
        raise RuntimeError("camera cache was dropped after this pass was staged")


def drop_camera_cache(kv_cache: Sequence[Any]) -> None:
    """A commit made without cameras drops the camera metadata (causal_model.py:2838-2842);
    the same as ``kv_cache[0].pop("_fused_prope_camera_metadata", None)``."""
    if kv_cache:
        kv_cache[0].pop("_fused_prope_camera_metadata", None)
