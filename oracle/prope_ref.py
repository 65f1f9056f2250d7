"""CPU restatement of SolarWM's fused PRoPE on the KV-cache path — TEST INFRASTRUCTURE ONLY.

PRoPE (projective positional encoding) gives every token a camera.  With P = lift(K) · V (an
``image <- world`` map built from the camera's view matrix V and intrinsics K), attention runs on
q' = Pᵀ q, k' = P⁻¹ k, v' = P⁻¹ v, applied to each group of 4 head channels, and the output is
mapped back with P (solar/backends/wan22/runtime/modeling/camera_prope.py:93-180, :183-261).
The fused mode of the cached self-attention keeps raw K/V and a camera cache with the same token
layout (causal_model.py:1948-2075), applies ordinary RoPE first and PRoPE after it
(causal_model.py:585-651, :1170-1199).

Written from reading the reference (not imported, not copied).  Arithmetic is float64 unless
``emulate_bf16`` asks for the reference's own roundings (matrices and features in bf16,
camera_prope.py:242-245).

Pinning (tests/test_oracle_prope.py):
* ``invert_se3`` / ``invert_k`` / ``projection_matrices`` — M · M⁻¹ = I on random poses and
  intrinsics; P · P⁻¹ = I; the GTA branch (no intrinsics) is P = V; the principal point is
  dropped from K.
* ``transform_relative_viewmats`` — linear is the identity; logd4 on hand cases (|t| = 5 ->
  t · log1p(5) / 20; t = 0 stays 0; rotation untouched).
* ``apply_tiled`` — explicit per-token, per-group loops.
* ``prope_qkv_separate`` — identity cameras change nothing; one camera for every token turns
  PRoPE attention (with the output map) back into plain attention; scores depend only on the
  relative pose (a common world change leaves them unchanged, linear translation mode); a query
  and key with different cameras do change.
* ``stage_fused_camera_cache`` / ``commit_fused_camera_cache`` — token-labelled cameras follow
  exactly the rows the K/V cache moves (rolling, direct insert, recompute), and the staged
  buffer leaves the committed state untouched until commit.
* ``prope_branch_forward`` — identity cameras reduce it to the main branch's cached attention
  with an immediate commit (token-labelled cache contents equal, C1 known answer through it);
  one camera for every token gives plain cached attention's output; a common world change of
  all cameras leaves the output unchanged; a ``none`` forward leaves the cache untouched.
"""

from __future__ import annotations

from typing import Any, Callable

import torch

GROUP = 4  # PRoPE acts on consecutive groups of 4 head channels (camera_prope.py:216-226)


# ---------------------------------------------------------------------------------------------
# camera algebra (camera.py:31-62; camera_prope.py:206-231, :307-338)
# ---------------------------------------------------------------------------------------------
def transform_relative_viewmats(viewmats: torch.Tensor, transform: str = "linear") -> torch.Tensor:
    """``linear`` returns the view matrices; ``logd4`` scales each translation t to
    t · log1p(|t|) / (4 |t|) (0 stays 0), in float32 (float64 for float64 input)."""
    if transform == "linear":
        return viewmats
    if transform != "logd4":
        raise ValueError(f"unknown camera translation transform {transform!r}")
    work = torch.float64 if viewmats.dtype == torch.float64 else torch.float32
    t = viewmats[..., :3, 3].to(work)
    norm = torch.linalg.vector_norm(t, dim=-1, keepdim=True)
    scale = torch.where(norm > 0, torch.log1p(norm) / (4.0 * norm.clamp_min(torch.finfo(work).tiny)),
                        torch.zeros_like(norm))
    out = viewmats.clone()
    out[..., :3, 3] = (t * scale).to(viewmats.dtype)
    return out


def invert_se3(m: torch.Tensor) -> torch.Tensor:
    """[R t; 0 1]⁻¹ = [Rᵀ -Rᵀt; 0 1]."""
    rt = m[..., :3, :3].transpose(-1, -2)
    out = torch.zeros_like(m)
    out[..., :3, :3] = rt
    out[..., :3, 3] = -(rt @ m[..., :3, 3:4])[..., 0]
    out[..., 3, 3] = 1.0
    return out


def lift_k(ks: torch.Tensor) -> torch.Tensor:
    """3x3 -> 4x4 with a 1 in the homogeneous corner."""
    out = torch.zeros(ks.shape[:-2] + (4, 4), dtype=ks.dtype)
    out[..., :3, :3] = ks
    out[..., 3, 3] = 1.0
    return out


def invert_k(ks: torch.Tensor) -> torch.Tensor:
    """Inverse of skew-free intrinsics [[fx 0 cx] [0 fy cy] [0 0 1]]."""
    out = torch.zeros_like(ks)
    out[..., 0, 0] = 1.0 / ks[..., 0, 0]
    out[..., 1, 1] = 1.0 / ks[..., 1, 1]
    out[..., 0, 2] = -ks[..., 0, 2] / ks[..., 0, 0]
    out[..., 1, 2] = -ks[..., 1, 2] / ks[..., 1, 1]
    out[..., 2, 2] = 1.0
    return out


def normalised_intrinsics(ks: torch.Tensor) -> torch.Tensor:
    """Keep the focal lengths, drop the principal point (camera_prope.py:208-216)."""
    out = torch.zeros_like(ks)
    out[..., 0, 0] = ks[..., 0, 0]
    out[..., 1, 1] = ks[..., 1, 1]
    out[..., 2, 2] = 1.0
    return out


def projection_matrices(viewmats: torch.Tensor, ks: torch.Tensor | None,
                        dtype: torch.dtype = torch.float64):
    """(P, Pᵀ, P⁻¹) per camera, evaluated in ``dtype``: P = lift(Kn) V and
    P⁻¹ = V⁻¹ lift(Kn⁻¹) with Kn the normalised intrinsics, or P = V without intrinsics."""
    v = viewmats.to(dtype)
    if ks is None:
        p = v
        p_inv = invert_se3(v)
    else:
        kn = normalised_intrinsics(ks.to(dtype))
        p = lift_k(kn) @ v
        p_inv = invert_se3(v) @ lift_k(invert_k(kn))
    return p, p.transpose(-1, -2), p_inv


def apply_tiled(feats: torch.Tensor, matrix: torch.Tensor) -> torch.Tensor:
    """feats [B, L, H, D], matrix [B, L, 4, 4] (one per token): every group of 4 channels of
    token l becomes matrix[b, l] @ group (camera_prope.py:234-256, the per-ray branch)."""
    b, l, h, d = feats.shape
    x = feats.reshape(b, l, h, d // GROUP, GROUP)
    out = torch.einsum("blij,blhgj->blhgi", matrix.to(feats.dtype), x)
    return out.reshape(b, l, h, d)


SPATIAL0 = 44  # first channel of the height/width RoPE pairs (22 temporal pairs before them)


def fp8_prope_copies_effective(k: torch.Tensor, v: torch.Tensor, p_inv: torch.Tensor,
                               grid_hw: tuple[int, int], freqs: torch.Tensor,
                               frame_seqlen: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Raw (K, V) [B, n*T, H, D] -> the raw K and V a camera-aware fp8 cache effectively attends
    with (float64), for the per-token P⁻¹ ``p_inv`` [B, n*T, 4, 4] of ``projection_matrices``.

    The cache keeps K's copy as [temporal groups raw | P⁻¹ on the spatial groups of its
    height/width-roped values] and V's copy as P⁻¹ v, each the value a bf16 copy holds,
    quantised per (frame, stream, head) with its own absmax/448.  Undoing the copies' transforms
    on the decoded values (the exact inverse of ``p_inv`` on K's spatial groups and the conjugate
    height/width table; the same inverse on V) gives the inputs whose RoPE-then-PRoPE in
    ``cached_self_attention(prope=...)`` reproduce the decoded copies.  (``p_inv`` inverts the
    rotation by its transpose, so it is P's inverse only to float32 accuracy; its own inverse is
    used.)  Not a reference function (the reference has no fp8 cache).
    """
    p = torch.linalg.inv(p_inv.double())
    from .wan_cache_ref import fp8_fake_quant_frames, rope_frames

    nf = k.shape[1] // frame_seqlen
    zero = [0] * nf
    kr = rope_frames(k.double(), grid_hw, zero, freqs)
    kx = kr.clone()
    kx[..., SPATIAL0:] = apply_tiled(kr[..., SPATIAL0:], p_inv.double())
    kq = fp8_fake_quant_frames(kx.to(torch.bfloat16).float(), frame_seqlen).double()
    kr_eff = kq.clone()
    kr_eff[..., SPATIAL0:] = apply_tiled(kq[..., SPATIAL0:], p.double())
    k_eff = rope_frames(kr_eff, grid_hw, zero, freqs.conj())
    vx = apply_tiled(v.double(), p_inv.double()).to(torch.bfloat16)
    v_eff = apply_tiled(fp8_fake_quant_frames(vx.float(), frame_seqlen).double(), p.double())
    return k_eff, v_eff


def prope_qkv_separate(q, k, v, *, q_viewmats, q_ks, kv_viewmats, kv_ks,
                       transform: str = "linear", emulate_bf16: bool = False):
    """PRoPE with separate query and key/value cameras (camera_prope.py:93-180), in the
    ``[B, L, H, D]`` layout: returns (Pqᵀ q, Pkv⁻¹ k, Pkv⁻¹ v, out_fn) with out_fn(x) = Pq x.
    Cameras are per token: ``*_viewmats`` [B, L, 4, 4], ``*_ks`` [B, L, 3, 3] or None.

    float64 by default; ``emulate_bf16`` evaluates the matrices in float32 and applies them in
    bf16 to bf16 features, as the reference does for a bf16 model."""
    mdt = torch.float32 if emulate_bf16 else torch.float64
    fdt = torch.bfloat16 if emulate_bf16 else torch.float64
    qv = transform_relative_viewmats(q_viewmats, transform)
    kvv = transform_relative_viewmats(kv_viewmats, transform)
    pq, pq_t, _ = projection_matrices(qv, q_ks, mdt)
    _, _, pkv_inv = projection_matrices(kvv, kv_ks, mdt)
    qo = apply_tiled(q.to(fdt), pq_t.to(fdt))
    ko = apply_tiled(k.to(fdt), pkv_inv.to(fdt))
    vo = apply_tiled(v.to(fdt), pkv_inv.to(fdt))

    def out_fn(x: torch.Tensor) -> torch.Tensor:
        return apply_tiled(x.to(fdt), pq.to(fdt))

    return qo, ko, vo, out_fn


# ---------------------------------------------------------------------------------------------
# the shared camera cache of the fused mode (causal_model.py:1927-2075)
# ---------------------------------------------------------------------------------------------
STATE_KEY = "_fused_prope_camera_metadata"


def slice_current_camera_tokens(tensor: torch.Tensor, *, current_start: int,
                                num_new_tokens: int) -> torch.Tensor:
    """Accept current-chunk or full-trajectory camera tensors (causal_model.py:1927-1945)."""
    if tensor.shape[1] == num_new_tokens:
        return tensor
    end = current_start + num_new_tokens
    if current_start >= 0 and tensor.shape[1] >= end:
        return tensor[:, current_start:end]
    raise ValueError(
        f"fused_prope camera tensor of {tensor.shape[1]} tokens does not cover the current chunk "
        f"[{current_start}, {end})")


def stage_fused_camera_cache(kv_cache: list[dict[str, Any]], *, cam_viewmats: torch.Tensor,
                             cam_ks: torch.Tensor, current_start: int, num_new_tokens: int,
                             frame_seqlen: int, sink_size: int, local_attn_size: int):
    """Stage the camera rows of one forward in layer 0's cache (causal_model.py:1948-2066).

    Returns (current viewmats, current K, staged viewmats, staged K, update): the staged buffers
    are the committed camera cache after this forward's eviction and chunk write; the committed
    state changes only in ``commit_fused_camera_cache``.  Note the write window: it follows the
    K/V cache except that ``sink_recache_after_switch`` is not applied here.
    """
    cam_viewmats = slice_current_camera_tokens(cam_viewmats, current_start=current_start,
                                               num_new_tokens=num_new_tokens)
    cam_ks = slice_current_camera_tokens(cam_ks, current_start=current_start,
                                         num_new_tokens=num_new_tokens)
    cache = kv_cache[0]
    cache_size = cache["k"].shape[1]
    batch = cache["k"].shape[0]
    global_end = int(cache["global_end_index"].item())
    prev_local_end = int(cache["local_end_index"].item())
    current_end = current_start + num_new_tokens
    sink_tokens = sink_size * frame_seqlen
    is_recompute = current_end <= global_end and current_start > 0
    state = cache.get(STATE_KEY)
    if state is None:
        if prev_local_end > 0:
            raise RuntimeError("fused_prope found populated K/V history without camera metadata")
        state = {"viewmats": cam_viewmats.new_zeros(batch, cache_size, 4, 4),
                 "K": cam_ks.new_zeros(batch, cache_size, 3, 3)}
        cache[STATE_KEY] = state
    temp_v = state["viewmats"].clone()
    temp_k = state["K"].clone()
    rolling = (local_attn_size != -1 and current_end > global_end
               and num_new_tokens + prev_local_end > cache_size)
    if rolling:
        evicted = num_new_tokens + prev_local_end - cache_size
        rolled = prev_local_end - evicted - sink_tokens
        local_end_index = prev_local_end + current_end - global_end - evicted
        src = slice(sink_tokens + evicted, sink_tokens + evicted + rolled)
        dst = slice(sink_tokens, sink_tokens + rolled)
        temp_v[:, dst] = temp_v[:, src].clone()
        temp_k[:, dst] = temp_k[:, src].clone()
    else:
        local_end_index = prev_local_end + current_end - global_end
    local_start_index = local_end_index - num_new_tokens
    write_start = max(local_start_index, sink_tokens) if is_recompute else local_start_index
    off = max(0, write_start - local_start_index)
    write_len = max(0, local_end_index - write_start)
    if write_len > 0:
        temp_v[:, write_start:local_end_index] = cam_viewmats[:, off : off + write_len]
        temp_k[:, write_start:local_end_index] = cam_ks[:, off : off + write_len]
    update = {"state": state, "temp_viewmats": temp_v, "temp_K": temp_k}
    return cam_viewmats, cam_ks, temp_v, temp_k, update


def commit_fused_camera_cache(update: dict[str, Any] | None) -> None:
    """Copy the staged camera rows into the shared state (causal_model.py:2068-2075)."""
    if update is None:
        return
    update["state"]["viewmats"].copy_(update["temp_viewmats"])
    update["state"]["K"].copy_(update["temp_K"])


def visible_cameras(temp: torch.Tensor, window: list[tuple[int, int]]) -> torch.Tensor:
    """The camera rows of the attention window: ``cat`` of the same token ranges the K/V window
    takes (causal_model.py:1170-1184, :1212-1214)."""
    return torch.cat([temp[:, a:b] for a, b in window], dim=1)


def fused_prope_attention(q, k, v, *, q_viewmats, q_ks, kv_viewmats, kv_ks, attn_fn: Callable,
                          transform: str = "linear", emulate_bf16: bool = False) -> torch.Tensor:
    """attention(Pqᵀ q, Pkv⁻¹ k, Pkv⁻¹ v) mapped back by Pq (causal_model.py:1185-1196)."""
    qo, ko, vo, out_fn = prope_qkv_separate(
        q, k, v, q_viewmats=q_viewmats, q_ks=q_ks, kv_viewmats=kv_viewmats, kv_ks=kv_ks,
        transform=transform, emulate_bf16=emulate_bf16)
    return out_fn(attn_fn(qo, ko, vo))


# ---------------------------------------------------------------------------------------------
# the PRoPE self-attention branch with its own cache (CausalPropeSelfAttention.forward,
# causal_model.py:1296-1525; camera_attention_mode "parallel")
# ---------------------------------------------------------------------------------------------
def prope_branch_forward(q, k, v, cache: dict[str, Any], *, viewmats, ks, current_start: int,
                         frame_seqlen: int, sink_size: int, local_attn_size: int,
                         cache_update_policy: str = "commit_detached", transform: str = "linear",
                         attn_fn: Callable | None = None, emulate_bf16: bool = False,
                         sink_recache_after_switch: bool = False) -> torch.Tensor:
    """One forward of the branch after its projections and norms, over a dense cache dict
    (``k``, ``v``, ``global_end_index``, ``local_end_index``: the layer's ``prope_*`` entries).

    PRoPE with the chunk's own cameras (``viewmats`` [B, L, 4, 4], ``ks`` [B, L, 3, 3] per token
    of the chunk; camera_prope.py:34-90) maps q, k, v to Pᵀq, P⁻¹k, P⁻¹v; the transformed K/V go
    through the cache exactly as the main branch's (the index arithmetic of :1368-1502 is the
    same as :1028-1133, restated in ``wan_cache_ref.cached_self_attention``); the attention over
    sink | window (:1480-1505) is mapped back with P.  A non-``none`` policy writes the cache and
    advances the indices in the same forward (:1428-1451, :1512-1514), i.e. the deferred update
    of the main branch applied at once."""
    from oracle import wan_cache_ref as ref

    qo, ko, vo, out_fn = prope_qkv_separate(
        q, k, v, q_viewmats=viewmats, q_ks=ks, kv_viewmats=viewmats, kv_ks=ks,
        transform=transform, emulate_bf16=emulate_bf16)
    dt = cache["k"].dtype
    x, upd = ref.cached_self_attention(
        qo.to(dt), ko.to(dt), vo.to(dt), cache, current_start=current_start,
        frame_seqlen=frame_seqlen, sink_size=sink_size, local_attn_size=local_attn_size,
        sink_recache_after_switch=sink_recache_after_switch,
        attn_fn=attn_fn if attn_fn is not None else ref.attention)
    if cache_update_policy != "none":
        ref.apply_cache_updates([cache], [(0, upd)])
    return out_fn(x)
