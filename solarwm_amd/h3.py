"""MiniMax-H3's per-segment transforms on the HIP kernels: rotate-half MM-RoPE on head channels
[0, 96) and the camera PRoPE of channels [96, 128) (``skv_h3_rope_prope``), the camera matrices
they take, and ``prope_qkv_separate`` built on them.

Drop-in counterparts of the reference's fused transforms: ``rope_prope`` for
fused_prope.py:426-438 (BSHD in, BSHD out, same bf16 roundings), ``prope_project`` for
fused_prope.py:162-167 (BHSD view in, BHSD view of BSHD memory out), ``prope_qkv_separate`` for
torch_prope.py:218-241.  The camera matrices (``suffix_matrices``) are a few 4x4 products per
row, computed with the reference's own tensor operations (torch_prope.py:22-48, :187-215) in
the features' dtype on the features' device; the per-row work on q / k / v / outputs is the
HIP kernel.
"""

from __future__ import annotations

import ctypes
from functools import partial

import torch

from . import _lib, kernels

WAN_FIXED_FX = 969.6969696969696 / (960.0 * 2.0)  # camera.py:22
WAN_FIXED_FY = 969.6969696969696 / (540.0 * 2.0)  # camera.py:23
ROTARY_CHANNELS = 96  # rotate-half MM-RoPE on [0, 96); the camera projection on [96, 128)


def _table_code(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return _lib.SKV_BF16
    if t.dtype == torch.float32:
        return _lib.SKV_F32
    raise ValueError(f"tables and matrices must be bfloat16 or float32, got {t.dtype}")


def _xform(x: torch.Tensor, out: torch.Tensor, cos, sin, matrix) -> torch.Tensor:
    """x / out: [B, S, H, 128] views (unit channel stride); cos / sin [S, 96]; matrix
    [B or 1, S, 4, 4]."""
    if x.dtype != torch.bfloat16 or out.dtype != torch.bfloat16:
        raise ValueError("H3 transforms take bfloat16 features")
    if x.dim() != 4 or x.shape[-1] != 128 or tuple(out.shape) != tuple(x.shape):
        raise ValueError(f"features must be [B, S, H, 128] with a matching out, got "
                         f"{tuple(x.shape)} / {tuple(out.shape)}")
    if x.stride(-1) != 1 or out.stride(-1) != 1:
        raise ValueError("features need unit channel stride")
    for t in (x, out):
        kernels._require_cuda("features", t)
    b, s, h, _ = x.shape
    d = _lib.H3XformDesc(x=x.data_ptr(), x_sb=x.stride(0), x_st=x.stride(1), x_sh=x.stride(2),
                         out=out.data_ptr(), out_sb=out.stride(0), out_st=out.stride(1),
                         out_sh=out.stride(2), batch=b, rows=s, heads=h, head_dim=128)
    keep = []
    if (cos is None) != (sin is None):
        raise ValueError("give cos and sin together")
    if cos is not None:
        if tuple(cos.shape) != (s, ROTARY_CHANNELS) or cos.shape != sin.shape:
            raise ValueError(f"cos / sin must be [{s}, {ROTARY_CHANNELS}], got {tuple(cos.shape)}")
        if cos.dtype != sin.dtype:
            raise ValueError("cos and sin must share a dtype")
        cos = cos if cos.stride(-1) == 1 else cos.contiguous()
        sin = sin if sin.stride() == cos.stride() else sin.contiguous()
        if sin.stride() != cos.stride():
            cos, sin = cos.contiguous(), sin.contiguous()
        for t in (cos, sin):
            kernels._require_cuda("rotary table", t)
        d.cos, d.sin = cos.data_ptr(), sin.data_ptr()
        d.table_dtype, d.table_stride = _table_code(cos), cos.stride(0)
        keep += [cos, sin]
    if matrix is not None:
        if matrix.dim() != 4 or tuple(matrix.shape[1:]) != (s, 4, 4) or matrix.shape[0] not in (1, b):
            raise ValueError(f"matrix must be [{b} or 1, {s}, 4, 4], got {tuple(matrix.shape)}")
        if matrix.stride(-1) != 1 or matrix.stride(-2) != 4:
            matrix = matrix.contiguous()
        kernels._require_cuda("matrix", matrix)
        d.matrix, d.matrix_dtype = matrix.data_ptr(), _table_code(matrix)
        d.matrix_sb = 0 if matrix.shape[0] == 1 else matrix.stride(0)
        d.matrix_st = matrix.stride(1)
        keep.append(matrix)
    lib = _lib.load()
    _lib.check("skv_h3_rope_prope", lib.skv_h3_rope_prope(ctypes.byref(d), kernels._stream(x.device)))
    del keep
    return out


def rope_prope(x: torch.Tensor, cos: torch.Tensor | None, sin: torch.Tensor | None,
               matrix: torch.Tensor | None, out: torch.Tensor | None = None) -> torch.Tensor:
    """BSHD ``x`` [B, S, H, 128] bf16 -> rotate-half MM-RoPE on channels [0, 96) (cos / sin
    [S, 96]) and the camera projection of [96, 128) (matrix [B or 1, S, 4, 4]), one pass
    (fused_prope.py:426-438).  ``out`` may be ``x``."""
    if out is None:
        out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    return _xform(x, out, cos, sin, matrix)


def prope_project(x: torch.Tensor, matrix: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``cat(x[..., :96], project(x[..., 96:128], matrix))`` for ``x`` [B, H, S, 128] (a BHSD
    view, as fused_prope.py:162-167 takes it); returns the BHSD view of BSHD memory."""
    xs = x.transpose(1, 2)
    if out is None:
        o = torch.empty(xs.shape, dtype=x.dtype, device=x.device)
    else:
        o = out.transpose(1, 2)
    _xform(xs, o, None, None, matrix)
    return o.transpose(1, 2)


def logd4_relative_viewmats(viewmats: torch.Tensor) -> torch.Tensor:
    """Each translation t becomes t · log1p(|t|) / (4 |t|) (0 stays 0), evaluated in float32
    (float64 for float64 input) and returned in the input dtype (torch_prope.py:22-40)."""
    work = torch.float64 if viewmats.dtype == torch.float64 else torch.float32
    t = viewmats[..., :3, 3].to(work)
    norm = torch.linalg.vector_norm(t, dim=-1, keepdim=True)
    safe = norm.clamp_min(torch.finfo(work).tiny)
    scale = torch.where(norm > 0, torch.log1p(norm) / (4.0 * safe), torch.zeros_like(norm))
    out = viewmats.clone()
    out[..., :3, 3] = (t * scale).to(viewmats.dtype)
    return out


def suffix_matrices(viewmats: torch.Tensor, ks: torch.Tensor):
    """(Pᵀ, P⁻¹, P) per row with P = lift(Kf) · V for compressed view matrices V and H3's fixed
    focal intrinsics Kf (input intrinsics only give the dtype), in ``viewmats``' dtype
    (torch_prope.py:187-215)."""
    kf = torch.zeros_like(ks)
    kf[..., 0, 0] = WAN_FIXED_FX
    kf[..., 1, 1] = WAN_FIXED_FY
    kf[..., 2, 2] = 1.0
    lift = torch.zeros((*kf.shape[:-2], 4, 4), dtype=kf.dtype, device=kf.device)
    lift[..., :3, :3] = kf
    lift[..., 3, 3] = 1.0
    inv_k = torch.zeros_like(kf)
    inv_k[..., 0, 0] = 1.0 / kf[..., 0, 0]
    inv_k[..., 1, 1] = 1.0 / kf[..., 1, 1]
    inv_k[..., 2, 2] = 1.0
    lift_inv = torch.zeros_like(lift)
    lift_inv[..., :3, :3] = inv_k
    lift_inv[..., 3, 3] = 1.0
    rt = viewmats[..., :3, :3].transpose(-1, -2)
    v_inv = torch.zeros_like(viewmats)
    v_inv[..., :3, :3] = rt
    v_inv[..., :3, 3] = -torch.einsum("...ij,...j->...i", rt, viewmats[..., :3, 3])
    v_inv[..., 3, 3] = 1.0
    p = torch.einsum("...ij,...jk->...ik", lift, viewmats)
    p_inv = torch.einsum("...ij,...jk->...ik", v_inv, lift_inv).to(viewmats.dtype)
    return p.transpose(-1, -2).to(viewmats.dtype), p_inv, p.to(viewmats.dtype)


def prope_qkv_matrices(query_viewmats, query_K, key_viewmats, key_K, dtype=torch.bfloat16):
    """(query matrix Pqᵀ, key / value matrix Pk⁻¹, output matrix Pq) of prope_qkv_separate:
    cameras cast to the features' dtype, logd4-compressed, then ``suffix_matrices``
    (torch_prope.py:218-230)."""
    q_t, _, q_p = suffix_matrices(logd4_relative_viewmats(query_viewmats.to(dtype)), query_K.to(dtype))
    _, k_inv, _ = suffix_matrices(logd4_relative_viewmats(key_viewmats.to(dtype)), key_K.to(dtype))
    return q_t, k_inv, q_p


def prope_qkv_separate(q, k, v, *, query_viewmats, query_K, key_viewmats, key_K):
    """H3's head-sliced PRoPE with separate query and key cameras (torch_prope.py:218-241):
    q / k / v are BHSD [B, H, S, 128] bf16 views; returns (q', k', v', apply_output) with the
    projections of channels [96, 128) done by the HIP kernel."""
    if q.dim() != 4 or k.dim() != 4 or k.shape != v.shape:
        raise ValueError("H3 cached PRoPE requires BHSD queries and equal BHSD keys/values")
    if q.shape[:2] != k.shape[:2] or q.shape[-1] != 128 or k.shape[-1] != 128:
        raise ValueError("H3 cached PRoPE requires matching batch/heads and head_dim=128")
    qm, km, om = prope_qkv_matrices(query_viewmats, query_K, key_viewmats, key_K, q.dtype)
    return (prope_project(q, qm), prope_project(k, km), prope_project(v, km),
            partial(prope_project, matrix=om))
