"""CPU restatement of MiniMax-H3's per-segment transforms — TEST INFRASTRUCTURE ONLY.

H3 attention segments rotate head channels [0, 96) with rotate-half MM-RoPE (cos / sin tables
of the segment's own positions) and project channels [96, 128) with its camera PRoPE: eight
4-vectors per row, q by Pᵀ, k and v by P⁻¹, the attention output by P, where P = lift(Kf) · V'
with V' the logd4-compressed relative view matrix and Kf H3's fixed focal intrinsics
(torch_prope.py:22-48, :187-241; camera.py:15-23).  ``rope_prope`` follows the fused kernel
the reference's rollout runs (fused_prope.py:196-255, whose docstring states it keeps every
bf16 rounding of the eager ``_apply_rotary_emb`` chain; the eager rotary lives in the diffusers
MiniMax-H3 model, a dependency absent here, so the fused kernel's text is what this restates),
``prope_project`` its projection-only kernel (fused_prope.py:30-93), and
``windowed_rollout_attention`` the rollout evaluation of one chunk against its attention window
(sgf_attention.py:580-659: raw prefix / history / chunk keys transformed with the window's
rotary rows and cameras, attention, output projection, raw chunk K/V committed).

Written from reading the reference (not imported, not copied).

Pinning (tests/test_oracle_h3.py):
* ``suffix_matrices`` — the reference's own camera test cases: logd4 of a (3, 4, 0)
  translation is t · log1p(5) / 20 and 0 stays 0 (test_camera.py:50-56); the fixed focal
  intrinsics ignore the input intrinsics (:94-100); Pᵀ on q and P⁻¹ on k keep every 4-vector
  inner product for one camera (:59-80), P (P⁻¹ v) = v for the output map (same test); P⁻¹ P = I
  in float64 on random poses; scores depend on the relative pose only (a rotation applied to
  every camera's world frame leaves them unchanged; a translation-free rotation keeps logd4's
  scale, so the check is exact in float64).
* ``rope_prope`` — cos = 1, sin = 0 and identity matrices return x bit for bit; cos = 0,
  sin = 1 gives (-x2, x1) bit for bit; generic angles preserve every rotated pair's norm and
  compose (rotating by a then b equals rotating by a + b), within bf16 rounding; the
  projection equals a float64 matrix product within one bf16 rounding and is bit-exact against
  an explicit per-element loop in the stated sum order.
* ``windowed_rollout_attention`` / ``memory_kv_attention`` — identity transforms (cos = 1,
  sin = 0, identity matrices) reduce them to segments_ref's windowed_rollout_attention /
  memory_kv_attention exactly; the memory form's per-row transform equals transforming each
  segment's gathered rows with the same rows of the tables (the reference's per-segment
  ``calculate``), checked on a layout with every span.
"""

from __future__ import annotations

import torch

from . import prope_ref as pr
from . import segments_ref as sr

WAN_FIXED_FX = 969.6969696969696 / (960.0 * 2.0)  # camera.py:22
WAN_FIXED_FY = 969.6969696969696 / (540.0 * 2.0)  # camera.py:23
CAM0 = 96   # camera PRoPE channels [96, 128) (camera.py:17-18)
HALF = 48   # rotate-half split of the rotary channels [0, 96) (fused_prope.py:226-231)


def _bf(t: torch.Tensor) -> torch.Tensor:
    """Round to bf16 (nearest even) and back to float32."""
    return t.to(torch.bfloat16).to(torch.float32)


def fixed_focal_intrinsics(ks: torch.Tensor) -> torch.Tensor:
    """H3's fixed focal lengths in place of the input intrinsics (torch_prope.py:43-48), in
    ``ks``'s dtype."""
    out = torch.zeros_like(ks)
    out[..., 0, 0] = WAN_FIXED_FX
    out[..., 1, 1] = WAN_FIXED_FY
    out[..., 2, 2] = 1.0
    return out


def suffix_matrices(viewmats: torch.Tensor, ks: torch.Tensor):
    """(Pᵀ, P⁻¹, P) per row for already-compressed view matrices (torch_prope.py:187-215):
    P = lift(Kn) · V, P⁻¹ = V⁻¹ · lift(Kn⁻¹), Kn the fixed focal intrinsics without a principal
    point; evaluated in ``viewmats``' dtype, as the reference's einsums are."""
    kn = pr.normalised_intrinsics(fixed_focal_intrinsics(ks))
    p = pr.lift_k(kn).to(viewmats.dtype) @ viewmats
    p_inv = pr.invert_se3(viewmats) @ pr.lift_k(pr.invert_k(kn)).to(viewmats.dtype)
    return p.transpose(-1, -2), p_inv, p


def prope_qkv_separate_matrices(query_viewmats, query_ks, key_viewmats, key_ks, dtype):
    """The three matrix sets of prope_qkv_separate (torch_prope.py:218-230): view matrices and
    intrinsics cast to the features' dtype, logd4-compressed, then ``suffix_matrices``; returns
    (query matrix Pqᵀ, key / value matrix Pk⁻¹, output matrix Pq)."""
    qv = pr.transform_relative_viewmats(query_viewmats.to(dtype), "logd4")
    kv = pr.transform_relative_viewmats(key_viewmats.to(dtype), "logd4")
    q_t, _, q_p = suffix_matrices(qv, query_ks.to(dtype))
    _, k_inv, _ = suffix_matrices(kv, key_ks.to(dtype))
    return q_t, k_inv, q_p


def rope_prope(x: torch.Tensor, cos: torch.Tensor | None, sin: torch.Tensor | None,
               matrix: torch.Tensor | None) -> torch.Tensor:
    """x [B, S, H, 128] bf16 -> bf16: rotary on [0, 96) (cos / sin [S, 96], rounded to bf16),
    y1 = bf16(bf16(x1 c1) + bf16(-x2 s1)), y2 = bf16(bf16(x2 c2) + bf16(x1 s2)); projection of
    [96, 128) by matrix [B or 1, S, 4, 4] (rounded to bf16) with the fp32 sum
    ((m0 v0 + m1 v1) + m2 v2) + m3 v3 (fused_prope.py:196-255); None skips a part."""
    xf = x.to(torch.float32)
    out = xf.clone()
    if cos is not None:
        c = _bf(cos.to(torch.float32))[None, :, None, :]
        s = _bf(sin.to(torch.float32))[None, :, None, :]
        x1, x2 = xf[..., :HALF], xf[..., HALF:CAM0]
        out[..., :HALF] = _bf(_bf(x1 * c[..., :HALF]) + _bf(-x2 * s[..., :HALF]))
        out[..., HALF:CAM0] = _bf(_bf(x2 * c[..., HALF:CAM0]) + _bf(x1 * s[..., HALF:CAM0]))
    if matrix is not None:
        b, n, h, _ = x.shape
        m = _bf(matrix.to(torch.float32))[:, :, None, None]  # [B|1, S, 1, 1, 4, 4]
        v = xf[..., CAM0:].reshape(b, n, h, 8, 4)
        y = torch.empty_like(v)
        for i in range(4):
            y[..., i] = ((m[..., i, 0] * v[..., 0] + m[..., i, 1] * v[..., 1])
                         + m[..., i, 2] * v[..., 2]) + m[..., i, 3] * v[..., 3]
        out[..., CAM0:] = _bf(y.reshape(b, n, h, 32))
    return out.to(torch.bfloat16)


def prope_project(x: torch.Tensor, matrix: torch.Tensor) -> torch.Tensor:
    """Channels [0, 96) copied, [96, 128) projected (fused_prope.py:30-93); x [B, S, H, 128]."""
    return rope_prope(x, None, None, matrix)


def windowed_rollout_attention(q, k, v, prefix_k, prefix_v, cache: sr.H3RawKVCache, layer: int,
                               chunk_index: int, *, q_rotary, k_rotary, q_matrix, kv_matrix,
                               out_matrix, commit: bool = False) -> torch.Tensor:
    """One rollout evaluation of a chunk (sgf_attention.py:580-659): keys / values are
    [prefix | history chunks | chunk] raw rows, transformed with ``k_rotary`` (cos, sin rows of
    the whole window) and ``kv_matrix`` (rows of the whole window); the query with ``q_rotary``
    and ``q_matrix``; float64 attention of the bf16 transformed tensors, rounded to bf16; the
    output projected by ``out_matrix``; the raw chunk K/V committed with ``commit``."""
    hist = cache.history(layer, chunk_index)
    keys = torch.cat([prefix_k, *(e[1] for e in hist), k], 1)
    vals = torch.cat([prefix_v, *(e[2] for e in hist), v], 1)
    kt = rope_prope(keys, k_rotary[0], k_rotary[1], kv_matrix)
    vt = prope_project(vals, kv_matrix)
    qt = rope_prope(q, q_rotary[0], q_rotary[1], q_matrix)
    o = sr.attention(qt, kt, vt).to(torch.bfloat16)
    if commit:
        cache.commit(layer, chunk_index, k, v)
    return prope_project(o, out_matrix)


def memory_kv_attention(q, k, v, history_k, history_v, *, text_rows: int, frame_rows: int,
                        n_bank: int, audio_rows: int, rotary, history_rotary, q_matrix,
                        kv_matrix, out_matrix, history_kv_matrix) -> torch.Tensor:
    """MemoryKVAttention.attend with its transforms (memory_kv_attention.py:39-140): every
    packed row [text | anchor | bank | audio | chunk] is rotated and projected with its own
    rotary row and camera in every segment it enters, so the transforms apply per row here
    (q with ``q_matrix``, k / v with ``kv_matrix``, raw history rows with ``history_rotary``
    and ``history_kv_matrix``), then segments_ref's segmented attention, rounded to bf16, then
    the output rows projected by ``out_matrix``."""
    qt = rope_prope(q, rotary[0], rotary[1], q_matrix)
    kt = rope_prope(k, rotary[0], rotary[1], kv_matrix)
    vt = prope_project(v, kv_matrix)
    if history_k.shape[1]:
        hk = rope_prope(history_k, history_rotary[0], history_rotary[1], history_kv_matrix)
        hv = prope_project(history_v, history_kv_matrix)
    else:
        hk, hv = history_k, history_v
    o = sr.memory_kv_attention(qt, kt, vt, hk, hv, text_rows=text_rows, frame_rows=frame_rows,
                               n_bank=n_bank, audio_rows=audio_rows).to(torch.bfloat16)
    return prope_project(o, out_matrix)
