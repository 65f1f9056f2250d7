"""Attention entry points with the reference's call signatures.

* :func:`attention` — drop-in for ``attention(q, k, v, ...)`` of
  solar/backends/wan22/runtime/modeling/attention.py:141-188 (dense ``[B, L, H, D]`` inputs).
* :func:`chunk_causal_attention` — the chunk-causal FlexAttention of the cache-free
  inference-window path (causal_model.py:474-534, :984-989).
* :func:`attend_cached` — the KV-cache branch of ``CausalWanSelfAttention.forward``
  (causal_model.py:1028-1235) after projection and RoPE: appends the chunk, resolves eviction and
  the sink|local window through the slot table and attends, returning the reference's
  ``(x, (current_end, local_end_index, cache_update_info))`` pair.
* :func:`apply_cache_updates` — the deferred commit ``CausalWanModel._apply_cache_updates``
  (causal_model.py:2856-2921).

Every call runs the HIP kernels of libsolarkv.so; there is no other code path.
"""

from __future__ import annotations

import math
from typing import Iterable, Sequence

import torch

from . import _lib, kernels
from .cache import CacheUpdate, SlotKVCache
from .prope import CameraPass, commit_camera_cache, stage_camera_cache
from .rope import positions as rope_positions


def _pack_dense(k: torch.Tensor, v: torch.Tensor, pool_dtype: torch.dtype):
    """Stage dense K/V [B, L, H, D] as a one-frame pool (V transposed) for the kernel, in this
    stream's reused staging buffer (no allocation or zero-fill per call)."""
    b, lk, h, _ = k.shape
    kpool, vpool = kernels.staging_pools(1, b, h, lk, pool_dtype, k.device)
    kernels.append_frames(k, v, kpool, vpool, [0], frame_tokens=lk)
    return kpool, vpool


def _dense_attention(q, k, v, softmax_scale, mask_mode=_lib.SKV_MASK_NONE, q_pos0=0, chunk=0):
    kpool, vpool = _pack_dense(k, v, k.dtype)
    return kernels.attention_frames(
        q, kpool, vpool, [0], frame_tokens=k.shape[1], softmax_scale=softmax_scale,
        mask_mode=mask_mode, q_pos0=q_pos0, chunk_tokens=chunk,
    )


def attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    q_lens: torch.Tensor | None = None,
    k_lens: torch.Tensor | None = None,
    dropout_p: float = 0.0,
    softmax_scale: float | None = None,
    q_scale: float | None = None,
    causal: bool = False,
    window_size: tuple[int, int] = (-1, -1),
    deterministic: bool = False,
    dtype: torch.dtype = torch.bfloat16,
    fa_version: int | None = None,
) -> torch.Tensor:
    """softmax(q kᵀ · scale) v for ``[B, L, H, D]`` tensors; returns ``q.dtype`` like the
    reference's flash path (attention.py:66-138).  ``q_lens``/``k_lens`` select per-sample
    prefixes (varlen); rows past ``q_lens[b]`` are returned as zeros.  Dropout, causal and
    sliding-window options are not used by the cached path and raise ``NotImplementedError``.
    """
    if dropout_p:
        raise NotImplementedError("dropout is not supported by the inference kernels")
    if causal or tuple(window_size) != (-1, -1):
        raise NotImplementedError("causal / sliding-window attention is not on this path")
    if dtype not in (torch.float16, torch.bfloat16):
        raise AssertionError("dtype must be float16 or bfloat16")  # attention.py:63-64
    out_dtype = q.dtype
    if q.shape[-1] != kernels.HEAD_DIM:
        raise ValueError(f"head_dim must be {kernels.HEAD_DIM}")
    if k.shape != v.shape or q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise ValueError("q, k, v must be [B, L, H, D] with matching B, H and k.shape == v.shape")
    # attention.py:69-87: inputs that are not half precision are cast to `dtype`, then q and k
    # to v's dtype, and the kernel computes in that dtype.  bf16 runs the bf16 MFMA kernel (fp32
    # inputs with dtype=bfloat16 are passed as fp32 and rounded to bf16 on load, the same
    # rounding); fp16 runs the same kernel on fp16 pools with fp16 MFMAs.
    half = (torch.float16, torch.bfloat16)

    def to_half(x):
        return x if x.dtype in half else x.to(dtype)

    if v.dtype in half or dtype == torch.float16:
        vh = to_half(v)
        kv_dtype = vh.dtype
        qh, kh = to_half(q).to(kv_dtype), to_half(k).to(kv_dtype)
    else:  # fp32 inputs, dtype=bfloat16: the kernels round them to bf16 on load
        kv_dtype = v.dtype
        qh, kh, vh = q.to(kv_dtype), k.to(kv_dtype), v
    if q_scale is not None:
        qh = (qh.float() * q_scale).to(kv_dtype)
    if q_lens is None and k_lens is None:
        out = _dense_attention(qh.contiguous(), kh.contiguous(), vh.contiguous(), softmax_scale)
        return out.to(out_dtype)
    b, lq = q.shape[:2]
    lk = k.shape[1]
    ql = [lq] * b if q_lens is None else [int(x) for x in q_lens.tolist()]
    kl = [lk] * b if k_lens is None else [int(x) for x in k_lens.tolist()]
    out = torch.zeros(q.shape, dtype=kv_dtype, device=q.device)
    for i in range(b):
        if ql[i] == 0:
            continue
        if kl[i] == 0:
            raise RuntimeError("attention over an empty key window")
        o = _dense_attention(
            qh[i : i + 1, : ql[i]].contiguous(),
            kh[i : i + 1, : kl[i]].contiguous(),
            vh[i : i + 1, : kl[i]].contiguous(),
            softmax_scale,
        )
        out[i : i + 1, : ql[i]] = o
    return out.to(out_dtype)


def chunk_causal_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    chunk_tokens: int,
    q_pos0: int = 0,
    softmax_scale: float | None = None,
) -> torch.Tensor:
    """Chunk-causal attention of ``build_inference_window_block_mask`` (causal_model.py:474-534):
    query ``i`` (sequence position ``q_pos0 + i``) sees keys ``< min((pos // chunk + 1) * chunk,
    Lk)``.  Inputs ``[B, L, H, D]`` (bf16 or fp32); returns ``q.dtype``.  Rows beyond the valid
    length that FlexAttention pads (the mask's "eye" rows) do not exist here: nothing is padded.
    """
    if chunk_tokens <= 0:
        raise ValueError("chunk_tokens must be positive")
    out_dtype = q.dtype
    kv_dtype = torch.bfloat16 if k.dtype not in (torch.float32, torch.bfloat16) else k.dtype
    return _dense_attention(
        q.to(kv_dtype), k.to(kv_dtype), v.to(kv_dtype), softmax_scale,
        mask_mode=_lib.SKV_MASK_CHUNK_CAUSAL, q_pos0=q_pos0, chunk=chunk_tokens,
    ).to(out_dtype)


def norm_spec(norm, heads: int, device) -> tuple[torch.Tensor, float]:
    """(float32 weight [H*D] on ``device``, eps) of a WanRMSNorm-like object (``.weight``,
    ``.eps``) or a ``(weight, eps)`` pair."""
    if isinstance(norm, tuple):
        weight, eps = norm
    else:
        weight, eps = norm.weight, norm.eps
    w = weight.detach().to(device=device, dtype=torch.float32).reshape(-1).contiguous()
    if w.numel() != heads * kernels.HEAD_DIM:
        raise ValueError(f"norm weight has {w.numel()} entries, expected {heads * kernels.HEAD_DIM}")
    return w, float(eps)


def _row_norm(x: torch.Tensor, norm, heads: int):
    """(inv_rms [B, L], weight) of ``x`` for the kernels' fused RMSNorm."""
    w, eps = norm_spec(norm, heads, x.device)
    return kernels.rms_rows(x, eps), w


def window_positions(kv_cache: SlotKVCache, plan, window: Sequence[int], nb: int,
                     current_start: int) -> tuple[list[int], list[int]]:
    """RoPE temporal positions (query frames, key frames in window order) of one cached forward:
    sink frames lead the window when a sink is configured (causal_model.py:1135-1156) and the
    query chunk is whole frames (causal_model.py:737-744, :806-810)."""
    g = kv_cache.geom
    T = g.frame_tokens
    sink_branch = g.sink_tokens > 0
    ns = (plan.window[0][1] - plan.window[0][0]) // T if sink_branch and plan.window else 0
    return rope_positions(
        kv_cache.rope.cfg, num_sink_frames=ns, num_local_frames=len(window) - ns,
        num_new_frames=nb, max_attention_size=g.max_attention_size, frame_tokens=T,
        current_start_frame=int(current_start) // T, sink_branch=sink_branch)


def attend_cached(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    kv_cache: SlotKVCache,
    current_start: int = 0,
    *,
    sink_recache_after_switch: bool = False,
    memory_frames: Sequence[int] | None = None,
    memory_positions: Sequence[int] | None = None,
    softmax_scale: float | None = None,
    out: torch.Tensor | None = None,
    camera: CameraPass | None = None,
    norm_q=None,
    norm_k=None,
) -> tuple[torch.Tensor, tuple[int, int, CacheUpdate]]:
    """One layer's cached self-attention (causal_model.py:1028-1235, post-projection/RoPE).

    ``q``, ``k``, ``v`` are the chunk's ``[B, Lq, H, D]`` query/key/value: post-RoPE for a cache
    without RoPE configuration, pre-RoPE (as the reference's cache branch receives them) for a
    cache allocated with ``rope`` (RoPE applied on load at the reference's window positions).
    The chunk is appended into staging slots, the visible window is the reference's
    ``cat[sink, local]`` (including the chunk), optionally preceded by memory-bank frames
    ``memory_frames`` (bank indices, in order), and nothing in the committed cache changes until
    :func:`apply_cache_updates`.  In a pre-RoPE cache the bank frames take the temporal RoPE
    positions ``memory_positions`` (one per bank frame; memory_kv_attention.py:97-137 rotates
    bank rows at their own positions ahead of the window's), the window its own.  ``camera`` (from ``prope.stage_camera_cache``, once per forward
    for all layers) applies fused PRoPE after RoPE (causal_model.py:1170-1199) and returns the
    output mapped back by the query cameras.  ``norm_q`` / ``norm_k`` (the layer's WanRMSNorm
    modules, or ``(weight, eps)``) take the raw projections: K is normalised inside the append
    and Q at the attention kernel's load, the reference's ``norm_q(q(x))`` / ``norm_k(k(x))``
    (causal_model.py:908-910) without a round trip through HBM.  Returns ``(out [B, Lq, H, D],
    (current_end, local_end_index, update))``.
    """
    g = kv_cache.geom
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q, k, v must all be [B, Lq, H, D] of the same shape")
    if q.shape[0] != g.batch or q.shape[2] != g.heads or q.shape[3] != g.head_dim:
        raise ValueError(
            f"chunk shape {tuple(q.shape)} does not match the cache (B={g.batch}, H={g.heads}, "
            f"D={g.head_dim})"
        )
    if kv_cache.dtype != torch.float8_e4m3fn and k.dtype != kv_cache.dtype:
        raise ValueError(f"k/v dtype {k.dtype} differs from the cache dtype {kv_cache.dtype}")
    plan, temp, staging, window = kv_cache.plan(
        int(current_start), q.shape[1], sink_recache_after_switch
    )
    T = g.frame_tokens
    rope = kv_cache.rope
    n_mem = len(memory_frames) if memory_frames else 0
    if rope is not None and n_mem:
        if memory_positions is None or len(memory_positions) != n_mem:
            raise ValueError("memory-bank frames in a pre-RoPE cache need memory_positions "
                             "(one temporal position per bank frame)")
        if camera is not None:
            raise NotImplementedError("memory-bank frames with fused PRoPE are not supported")
    elif memory_positions is not None and (rope is None or not n_mem):
        raise ValueError("memory_positions apply to bank frames of a pre-RoPE cache")
    if camera is not None:
        if kv_cache.camera is None or camera.camera is not kv_cache.camera:
            raise ValueError("camera pass was staged for a different cache (allocate with prope=)")
        if (camera.current_start != int(current_start) or camera.num_new_tokens != q.shape[1]
                or camera.staging != tuple(staging) or camera.window != tuple(window)):
            raise RuntimeError("camera pass does not match this layer's forward (stage it once per "
                               "forward, before the layers, with the same current_start and chunk)")
    elif kv_cache.camera is not None and kv_cache.camera.active:
        raise ValueError("this cache holds camera-conditioned history: pass camera= "
                         "(prope.stage_camera_cache) for every forward")
    if plan.write_len > 0:
        kernels.append_frames(
            k, v, kv_cache.kpool, kv_cache.vpool, staging, frame_tokens=T,
            src_frame0=plan.roped_offset // T, kscale=kv_cache.kscale, vscale=kv_cache.vscale,
            kr_pool=kv_cache.krpool, rope_hw=rope.hw if rope is not None else None,
            grid_hw=rope.cfg.grid_hw if rope is not None else None,
            vr_pool=kv_cache.vrpool if camera is not None else None,
            kv_xform=camera.kv_xform if camera is not None else None,
            k_norm=_row_norm(k, norm_k, g.heads) if norm_k is not None else None,
            kr_scale=kv_cache.krscale,
            vr_scale=kv_cache.vrscale if camera is not None else None,
        )
    frames = list(kv_cache.bank_slots(memory_frames)) if memory_frames else []
    frames.extend(window)
    if not frames:
        raise RuntimeError("KV-cache attention window is empty")  # causal_model.py:785-787
    rope_args = prope_args = None
    kpool, vpool = kv_cache.kpool, kv_cache.vpool
    kscale, vscale = kv_cache.kscale, kv_cache.vscale
    q_in, out_in = q, out
    if rope is not None:
        nb = q.shape[1] // T
        if nb * T != q.shape[1]:
            raise ValueError("EchoRoPE expects the query chunk to contain whole frames")
        kpool, kscale = kv_cache.krpool, kv_cache.krscale
        if camera is not None:
            prope_args = (rope.hw, rope.cfg.grid_hw, camera.q_xform_t, camera.q_xform_s,
                          camera.out_xform)
            vpool, vscale = kv_cache.vrpool, kv_cache.vrscale
        else:
            qpos, kpos = window_positions(kv_cache, plan, window, nb, int(current_start))
            if n_mem:
                kpos = [int(p) for p in memory_positions] + list(kpos)
            rope_args = (rope.hw, rope.cfg.grid_hw, rope.temporal(qpos, kpos))
        if kv_cache.dtype == torch.float8_e4m3fn and q.dtype != torch.bfloat16:
            # the fp8 RoPE kernels take bf16 queries (the bf16-pool kernels round to bf16 on load)
            q_in = q.to(torch.bfloat16)
            out_in = None
    x = kernels.attention_frames(
        q_in, kpool, vpool, frames, frame_tokens=T, softmax_scale=softmax_scale,
        kscale=kscale, vscale=vscale, out=out_in, rope=rope_args, prope=prope_args,
        q_norm=_row_norm(q, norm_q, g.heads) if norm_q is not None else None,
    )
    if x.dtype != q.dtype:
        x = x.to(q.dtype) if out is None else out.copy_(x)
    update = kv_cache.stage(plan, temp)
    return x, (plan.current_end, plan.local_end_index, update)


def prope_branch_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    kv_cache: SlotKVCache,
    current_start: int,
    cam_viewmats: torch.Tensor,
    cam_K: torch.Tensor,
    *,
    cache_update_policy: str = "commit_detached",
    sink_recache_after_switch: bool = False,
    per_frame: bool = False,
    softmax_scale: float | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """The cache branch of the PRoPE self-attention branch (``CausalPropeSelfAttention.forward``
    with a ``kv_cache``, causal_model.py:1296-1525), after its projections and q/k RMSNorm.

    ``q``, ``k``, ``v`` [B, Lq, H, D] and the chunk's cameras (per token ``[B, L, 4, 4]`` /
    ``[B, L, 3, 3]``, current chunk or full trajectory, one camera per latent frame; or per frame
    with ``per_frame``).  The reference applies PRoPE to the chunk (q -> P_qᵀ q, k, v -> P⁻¹ k,
    P⁻¹ v with the chunk's own cameras, camera_prope.py:34-90), caches the transformed K/V in the
    layer's ``prope_k`` / ``prope_v`` with the same index arithmetic as the main cache, attends
    over sink | window and maps the output back with P_q; a non-``none`` policy commits at once
    (the branch writes its cache inside its forward, causal_model.py:1428-1451, :1512-1514).
    Here the layer's branch cache (``prope_branch=`` of the allocator) keeps each frame's camera
    per slot; the kernels apply P⁻¹ at append and the query-side matrices and P_q inside the
    attention, with no RoPE.  Returns the output before the branch's ``out_proj``."""
    br = kv_cache.branch
    if br is None:
        raise ValueError("this cache has no PRoPE branch cache (allocate with prope_branch=)")
    cam = stage_camera_cache([br], cam_viewmats, cam_K, int(current_start), q.shape[1],
                             sink_recache_after_switch=sink_recache_after_switch,
                             per_frame=per_frame)
    x, (current_end, local_end, update) = attend_cached(
        q, k, v, br, current_start, sink_recache_after_switch=sink_recache_after_switch,
        softmax_scale=softmax_scale, out=out, camera=cam)
    if cache_update_policy != "none":
        br.commit(update, current_end, local_end)
        commit_camera_cache(cam)
    return x


def apply_cache_updates(
    kv_cache: Sequence[SlotKVCache],
    cache_update_infos: Iterable[tuple[int, tuple[int, int, CacheUpdate | None]]],
) -> None:
    """Deferred commit of every block's update (causal_model.py:2856-2921): the table takes the
    staged frames; indices advance unless the forward was a recompute."""
    for block_index, (current_end, local_end_index, update) in cache_update_infos:
        kv_cache[block_index].commit(update, current_end, local_end_index)


def default_softmax_scale(head_dim: int = kernels.HEAD_DIM) -> float:
    return 1.0 / math.sqrt(head_dim)
