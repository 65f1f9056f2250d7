"""Typed wrappers of the libsolarkv C ABI for torch tensors.

The wrappers only check arguments and pass raw pointers, strides and the current HIP stream;
all arithmetic happens in the HIP kernels.  Pool layouts (per layer):

* K pool ``[n_slots, B, H, Tp, D]`` — keys of a frame, channel-contiguous rows;
* V pool ``[n_slots, B, H, D, Tp]`` — values of a frame, stored transposed;
* scales ``[n_slots, B, H]`` float32 (fp8 pools only), ``absmax / 448`` per (slot, b, h);

with ``Tp = ceil(T / 64) * 64`` and zero padding rows.
"""

from __future__ import annotations

import ctypes
import math
from contextlib import contextmanager
from typing import Sequence

import torch

from . import _lib

HEAD_DIM = 128
TILE = 64

_DTYPE_CODES = {
    torch.float32: _lib.SKV_F32,
    torch.bfloat16: _lib.SKV_BF16,
    torch.float8_e4m3fn: _lib.SKV_FP8_E4M3,
    torch.float16: _lib.SKV_F16,
}


class LaunchTimer:
    """HIP events around kernel launches, recorded on the launching stream.

    ``records[kind]`` is a list of ``(start_event, end_event, work)`` where ``work`` is the
    launch's algorithmic FLOPs (attention) or bytes moved (append / gather).  With ``every=n``
    only launches 0, n, 2n, ... of each kind are bracketed: a timing event waits for the work
    before it, so events around every launch of a rollout add a gap to each launch.
    """

    def __init__(self, every: int = 1):
        self.records: dict[str, list] = {"attention": [], "append": [], "gather": []}
        self.every = max(1, int(every))
        self.seen: dict[str, int] = {k: 0 for k in self.records}

    def sample(self, kind: str) -> bool:
        """Whether this launch of ``kind`` is bracketed (counts the launch)."""
        n = self.seen[kind]
        self.seen[kind] = n + 1
        return n % self.every == 0

    def summary(self, kind: str) -> tuple[int, float, float]:
        """(launches, total milliseconds, total work) of one kernel kind; synchronises."""
        recs = self.records[kind]
        if not recs:
            return 0, 0.0, 0.0
        recs[-1][1].synchronize()
        ms = sum(a.elapsed_time(b) for a, b, _ in recs)
        return len(recs), ms, float(sum(w for _, _, w in recs))


_timer: LaunchTimer | None = None


@contextmanager
def timed_launches(every: int = 1):
    """Within the block, append / gather / attention launches are bracketed by events (every
    ``every``-th launch of each kind, starting with the first)."""
    global _timer
    prev, _timer = _timer, LaunchTimer(every)
    try:
        yield _timer
    finally:
        _timer = prev


def _tic(kind: str):
    if _timer is None or not _timer.sample(kind):
        return None
    ev = torch.cuda.Event(enable_timing=True)
    ev.record()
    return ev


def _toc(kind: str, start, work: float) -> None:
    if start is None or _timer is None:
        return
    ev = torch.cuda.Event(enable_timing=True)
    ev.record()
    _timer.records[kind].append((start, ev, work))


def padded_tokens(frame_tokens: int) -> int:
    return (frame_tokens + TILE - 1) // TILE * TILE


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; expected float32, bfloat16, float16 or float8_e4m3fn")


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_cuda(name: str, t: torch.Tensor) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor (got device {t.device})")


def _token_major(name: str, t: torch.Tensor) -> tuple[int, int, int]:
    """Validate a [B, L, H, D] tensor with unit stride on D; return (sb, st, sh)."""
    _require_cuda(name, t)
    if t.dim() != 4 or t.shape[-1] != HEAD_DIM:
        raise ValueError(f"{name} must be [B, L, H, {HEAD_DIM}], got {tuple(t.shape)}")
    if t.stride(-1) != 1:
        raise ValueError(f"{name} must be contiguous in its last dimension")
    return t.stride(0), t.stride(1), t.stride(2)


def check_pools(kpool: torch.Tensor, vpool: torch.Tensor, frame_tokens: int) -> tuple[int, int, int]:
    """Validate a K/V pool pair; return (n_slots, B, H)."""
    _require_cuda("k_pool", kpool)
    _require_cuda("v_pool", vpool)
    tp = padded_tokens(frame_tokens)
    if kpool.dim() != 5 or vpool.dim() != 5:
        raise ValueError("pools must be 5-D: K [S,B,H,Tp,D], V [S,B,H,D,Tp]")
    s, b, h = kpool.shape[:3]
    if tuple(kpool.shape) != (s, b, h, tp, HEAD_DIM) or tuple(vpool.shape) != (s, b, h, HEAD_DIM, tp):
        raise ValueError(
            f"pool shapes {tuple(kpool.shape)} / {tuple(vpool.shape)} do not match "
            f"K [S,B,H,{tp},{HEAD_DIM}] / V [S,B,H,{HEAD_DIM},{tp}] for frame_tokens={frame_tokens}"
        )
    if not (kpool.is_contiguous() and vpool.is_contiguous()):
        raise ValueError("pools must be contiguous")
    if kpool.dtype != vpool.dtype or kpool.device != vpool.device:
        raise ValueError("K and V pools must share dtype and device")
    return s, b, h


def _scales(kpool, kscale, vscale):
    if kpool.dtype != torch.float8_e4m3fn:
        return None, None
    s, b, h = kpool.shape[:3]
    for name, t in (("k_scale", kscale), ("v_scale", vscale)):
        if t is None:
            raise ValueError(f"fp8 pools need {name}")
        _require_cuda(name, t)
        if t.dtype != torch.float32 or tuple(t.shape) != (s, b, h) or not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous float32 [{s},{b},{h}]")
    return kscale.data_ptr(), vscale.data_ptr()


def _check_rope_hw(kr_pool, kpool, rope_hw, grid_hw, frame_tokens) -> None:
    _require_cuda("kr_pool", kr_pool)
    if kr_pool.shape != kpool.shape or kr_pool.dtype != kpool.dtype or not kr_pool.is_contiguous():
        raise ValueError("kr_pool must be a contiguous tensor shaped and typed like the K pool")
    if grid_hw is None or rope_hw is None:
        raise ValueError("RoPE needs rope_hw and grid_hw")
    gh, gw = int(grid_hw[0]), int(grid_hw[1])
    if gh * gw != frame_tokens:
        raise ValueError(f"grid {gh}x{gw} does not tile a {frame_tokens}-token frame")
    _require_cuda("rope_hw", rope_hw)
    if rope_hw.dtype != torch.float32 or rope_hw.numel() != (gh + gw) * 21 * 2 or not rope_hw.is_contiguous():
        raise ValueError(f"rope_hw must be contiguous float32 with {(gh + gw) * 42} entries")


def rms_rows(x: torch.Tensor, eps: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """Inverse RMS of every token's H x D row of ``x`` [B, L, H, D]: float32 [B, L] with
    ``1 / sqrt(mean(x²) + eps)`` (WanRMSNorm's statistic, model.py:69-84)."""
    lib = _lib.load()
    sb, st, sh = _token_major("x", x)
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"x dtype {x.dtype} unsupported (float32 or bfloat16)")
    b, l, h, _ = x.shape
    if out is None:
        out = torch.empty((b, l), dtype=torch.float32, device=x.device)
    if out.dtype != torch.float32 or tuple(out.shape) != (b, l) or not out.is_contiguous():
        raise ValueError(f"out must be contiguous float32 [{b}, {l}]")
    _lib.check("skv_rms_rows", lib.skv_rms_rows(
        x.data_ptr(), dtype_code(x.dtype), sb, st, sh, b, l, h, HEAD_DIM, float(eps),
        out.data_ptr(), _stream(x.device)))
    return out


def _norm_args(name: str, norm, batch: int, rows: int, heads: int, device):
    """Validate ``(inv_rms [B, >= rows] float32, weight [H*D] float32)``."""
    inv, w = norm
    _require_cuda(f"{name} inv_rms", inv)
    _require_cuda(f"{name} weight", w)
    if (inv.dtype != torch.float32 or inv.dim() != 2 or inv.shape[0] != batch or inv.shape[1] < rows
            or inv.stride(1) != 1):
        raise ValueError(f"{name} inv_rms must be float32 [{batch}, >= {rows}] with unit row stride")
    if w.dtype != torch.float32 or w.numel() != heads * HEAD_DIM or not w.is_contiguous():
        raise ValueError(f"{name} weight must be contiguous float32 with {heads * HEAD_DIM} entries")
    if inv.device != device or w.device != device:
        raise ValueError(f"{name} tensors must be on {device}")
    return inv.data_ptr(), inv.stride(0), w.data_ptr()


_workspaces: dict[tuple[int, int], torch.Tensor] = {}


def workspace(device: torch.device, nbytes: int) -> tuple[int, int, torch.Tensor | None]:
    """(pointer, bytes, tensor) of this device and current stream's scratch tensor, grown to at
    least ``nbytes``.  The kernels' split paths keep their partial results there; launches on one
    stream run in order, so every call on that stream shares it.

    Growing replaces the shared tensor: a launcher that keeps the pointer for later launches must
    also keep the returned tensor alive, or its launches would write into memory the caching
    allocator has handed to another tensor."""
    if nbytes <= 0:
        return 0, 0, None
    key = (device.index if device.index is not None else torch.cuda.current_device(),
           _stream(device))
    t = _workspaces.get(key)
    if t is None or t.numel() < nbytes:
        t = torch.empty(int(nbytes), dtype=torch.uint8, device=device)
        _workspaces[key] = t
    return t.data_ptr(), t.numel(), t


def prepare_append(
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    kpool: torch.Tensor,
    vpool: torch.Tensor,
    dst_slots: Sequence[int],
    *,
    frame_tokens: int,
    src_frame0: int = 0,
    kscale: torch.Tensor | None = None,
    vscale: torch.Tensor | None = None,
    kr_pool: torch.Tensor | None = None,
    rope_hw: torch.Tensor | None = None,
    grid_hw: tuple[int, int] | None = None,
    vr_pool: torch.Tensor | None = None,
    kv_xform: torch.Tensor | None = None,
    k_norm: tuple[torch.Tensor, torch.Tensor] | None = None,
    use_workspace: bool = True,
    kr_scale: torch.Tensor | None = None,
    vr_scale: torch.Tensor | None = None,
):
    """Validate an append once and return a zero-argument launcher that enqueues it on the stream
    current now (repeated launches skip the Python-side checks).

    With ``kr_pool`` (same shape and dtype as ``kpool``), the frames' K is also written there
    with the height/width pairs of RoPE applied (``rope_hw`` from ``rope.spatial_table``,
    ``grid_hw`` = the frame's patch grid).  With ``kv_xform`` (float32 ``[n_frames, B, 4, 4]``,
    the P⁻¹ of each written frame's camera) and ``vr_pool`` (shaped like ``vpool``), PRoPE is
    applied too: ``kr_pool`` gets P⁻¹ on its spatial channel groups and ``vr_pool`` gets P⁻¹ v.
    ``k_norm = (inv_rms, weight)`` stores RMS-normalised K (``rms_rows`` of ``k_new`` and the
    norm's float32 weight); every copy and fp8 code derives from the normalised value.
    ``use_workspace=False`` keeps an fp8 append of few units on the per-unit kernels (no
    scratch); by default it takes the one-pass slice kernel (bf16 sources without ``k_norm``)
    or the tile-grid kernels, with this stream's workspace.

    fp8 pools with ``kr_pool`` (and ``vr_pool``) take float32 ``kr_scale`` (and ``vr_scale``)
    shaped like ``kscale``: each copy is the e4m3 encoding, with its own absmax / 448 per (slot,
    stream, head), of the value a bf16 copy would hold (f32 for f32 sources); the copies need
    the workspace (``use_workspace=True``)."""
    lib = _lib.load()
    n_slots, b, h = check_pools(kpool, vpool, frame_tokens)
    sb, st, sh = _token_major("k_new", k_new)
    if _token_major("v_new", v_new) != (sb, st, sh) or v_new.shape != k_new.shape:
        raise ValueError("k_new and v_new must share shape and strides")
    if k_new.dtype != v_new.dtype:
        raise ValueError("k_new and v_new must share dtype")
    if k_new.shape[0] != b or k_new.shape[2] != h:
        raise ValueError(f"k_new batch/heads {tuple(k_new.shape)} do not match the pool ({b}, {h})")
    n = len(dst_slots)
    if (src_frame0 + n) * frame_tokens > k_new.shape[1]:
        raise ValueError(
            f"frames [{src_frame0}, {src_frame0 + n}) x {frame_tokens} tokens exceed k_new length {k_new.shape[1]}"
        )
    if k_new.device != kpool.device:
        raise ValueError("k_new and pools must be on the same device")
    ks, vs = _scales(kpool, kscale, vscale)
    slots = _lib.int32_array(dst_slots)
    moved = 2 * n * frame_tokens * b * h * HEAD_DIM * (k_new.element_size() + kpool.element_size())
    desc = _lib.AppendDesc(
        k_new=k_new.data_ptr(), v_new=v_new.data_ptr(), src_dtype=dtype_code(k_new.dtype),
        src_sb=sb, src_st=st, src_sh=sh, src_frame0=src_frame0, k_pool=kpool.data_ptr(),
        v_pool=vpool.data_ptr(), k_scale=ks, v_scale=vs, pool_dtype=dtype_code(kpool.dtype),
        n_slots=n_slots, dst_slots=slots, n_frames=n, batch=b, heads=h, head_dim=HEAD_DIM,
        frame_tokens=frame_tokens)
    if kv_xform is not None or vr_pool is not None:
        if kr_pool is None or vr_pool is None or kv_xform is None:
            raise ValueError("PRoPE append needs kr_pool, vr_pool and kv_xform")
        _require_cuda("vr_pool", vr_pool)
        if vr_pool.shape != vpool.shape or vr_pool.dtype != vpool.dtype or not vr_pool.is_contiguous():
            raise ValueError("vr_pool must be a contiguous tensor shaped and typed like the V pool")
        _require_cuda("kv_xform", kv_xform)
        if (kv_xform.dtype != torch.float32 or tuple(kv_xform.shape) != (n, b, 4, 4)
                or not kv_xform.is_contiguous()):
            raise ValueError(f"kv_xform must be contiguous float32 [{n}, {b}, 4, 4]")
        desc.vx_pool, desc.kv_xform = vr_pool.data_ptr(), kv_xform.data_ptr()
        moved += n * frame_tokens * b * h * HEAD_DIM * kpool.element_size()
    if kr_pool is not None:
        _check_rope_hw(kr_pool, kpool, rope_hw, grid_hw, frame_tokens)
        desc.kr_pool, desc.rope_hw = kr_pool.data_ptr(), rope_hw.data_ptr()
        if kpool.dtype == torch.float8_e4m3fn:
            if not use_workspace:
                raise ValueError("fp8 RoPE / PRoPE copies need the workspace (use_workspace=True)")
            named = [("kr_scale", kr_scale)] + ([("vr_scale", vr_scale)] if vr_pool is not None else [])
            for name, t in named:
                if t is None:
                    raise ValueError(f"fp8 copies need {name}")
                _require_cuda(name, t)
                if t.dtype != torch.float32 or t.shape != kscale.shape or not t.is_contiguous():
                    raise ValueError(f"{name} must be contiguous float32 {list(kscale.shape)}")
            desc.kr_scale = kr_scale.data_ptr()
            if vr_pool is not None:
                desc.vx_scale = vr_scale.data_ptr()
        desc.grid_h, desc.grid_w = int(grid_hw[0]), int(grid_hw[1])
        moved += n * frame_tokens * b * h * HEAD_DIM * kpool.element_size()
    if k_norm is not None:
        rms_p, rms_sb, w_p = _norm_args("k_norm", k_norm, b, (src_frame0 + n) * frame_tokens, h,
                                        kpool.device)
        desc.k_inv_rms, desc.k_rms_stride_b, desc.k_norm_weight = rms_p, rms_sb, w_p
    ws_tensor = None
    if use_workspace and kpool.dtype == torch.float8_e4m3fn:
        need = ctypes.c_int64(0)
        _lib.check("skv_append_workspace_size",
                   lib.skv_append_workspace_size(ctypes.byref(desc), ctypes.byref(need)))
        desc.workspace, desc.workspace_bytes, ws_tensor = workspace(kpool.device, need.value)
    args = (ctypes.byref(desc), _stream(kpool.device))
    fn = lib.skv_append_ex

    def launch() -> None:
        t0 = _tic("append")
        _lib.check("skv_append_ex", fn(*args))
        _toc("append", t0, moved)

    launch.bytes_moved = moved
    # the workspace tensor is kept too: a later call that grows this stream's workspace drops
    # the shared reference, and this launcher's descriptor still points at the old block
    launch.keep = (k_new, v_new, kpool, vpool, kscale, vscale, slots, kr_pool, rope_hw, vr_pool,
                   kv_xform, k_norm, kr_scale, vr_scale, desc, args, ws_tensor)
    return launch


def append_frames(
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    kpool: torch.Tensor,
    vpool: torch.Tensor,
    dst_slots: Sequence[int],
    *,
    frame_tokens: int,
    src_frame0: int = 0,
    kscale: torch.Tensor | None = None,
    vscale: torch.Tensor | None = None,
    kr_pool: torch.Tensor | None = None,
    rope_hw: torch.Tensor | None = None,
    grid_hw: tuple[int, int] | None = None,
    vr_pool: torch.Tensor | None = None,
    kv_xform: torch.Tensor | None = None,
    k_norm: tuple[torch.Tensor, torch.Tensor] | None = None,
    use_workspace: bool = True,
    kr_scale: torch.Tensor | None = None,
    vr_scale: torch.Tensor | None = None,
) -> None:
    """Write frames ``src_frame0 + f`` of ``k_new``/``v_new`` ([B, L, H, D]) into ``dst_slots[f]``
    (and, with ``kr_pool``, K with its height/width RoPE pairs rotated into ``kr_pool``; with
    ``kv_xform``, the PRoPE copies; with ``k_norm``, RMS-normalised K; fp8 copies with their
    ``kr_scale`` / ``vr_scale`` — see ``prepare_append``)."""
    prepare_append(k_new, v_new, kpool, vpool, dst_slots, frame_tokens=frame_tokens,
                   src_frame0=src_frame0, kscale=kscale, vscale=vscale, kr_pool=kr_pool,
                   rope_hw=rope_hw, grid_hw=grid_hw, vr_pool=vr_pool, kv_xform=kv_xform,
                   k_norm=k_norm, use_workspace=use_workspace, kr_scale=kr_scale,
                   vr_scale=vr_scale)()


def prepare_gather(
    kpool: torch.Tensor,
    vpool: torch.Tensor,
    slots: Sequence[int],
    *,
    frame_tokens: int,
    k_out: torch.Tensor | None = None,
    v_out: torch.Tensor | None = None,
):
    """Validate a gather once; return (launcher, k_out, v_out).  The launcher enqueues the gather
    on the stream current now."""
    lib = _lib.load()
    n_slots, b, h = check_pools(kpool, vpool, frame_tokens)
    n = len(slots)
    shape = (b, n * frame_tokens, h, HEAD_DIM)
    if k_out is None:
        k_out = torch.empty(shape, dtype=kpool.dtype, device=kpool.device)
    if v_out is None:
        v_out = torch.empty(shape, dtype=kpool.dtype, device=kpool.device)
    for name, t in (("k_out", k_out), ("v_out", v_out)):
        if tuple(t.shape) != shape or t.dtype != kpool.dtype:
            raise ValueError(f"{name} must be {shape} {kpool.dtype}")
    sb, st, sh = _token_major("k_out", k_out)
    if _token_major("v_out", v_out) != (sb, st, sh):
        raise ValueError("k_out and v_out must share strides")
    table = _lib.int32_array(slots)
    args = (
        kpool.data_ptr(), vpool.data_ptr(), dtype_code(kpool.dtype), n_slots, table, n, b, h,
        HEAD_DIM, frame_tokens, k_out.data_ptr(), v_out.data_ptr(), sb, st, sh,
        _stream(kpool.device),
    )
    moved = 2 * 2 * n * frame_tokens * b * h * HEAD_DIM * kpool.element_size()

    def launch() -> None:
        if n == 0:
            return
        t0 = _tic("gather")
        _lib.check("skv_gather", lib.skv_gather(*args))
        _toc("gather", t0, moved)

    launch.bytes_moved = moved
    launch.keep = (kpool, vpool, k_out, v_out, table)
    return launch, k_out, v_out


def gather_frames(
    kpool: torch.Tensor,
    vpool: torch.Tensor,
    slots: Sequence[int],
    *,
    frame_tokens: int,
    k_out: torch.Tensor | None = None,
    v_out: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Materialise pool frames ``slots`` as token-major K, V ``[B, len(slots)*T, H, D]``."""
    launch, k_out, v_out = prepare_gather(kpool, vpool, slots, frame_tokens=frame_tokens,
                                          k_out=k_out, v_out=v_out)
    launch()
    return k_out, v_out


def attention_desc(
    q: torch.Tensor,
    kpool: torch.Tensor,
    vpool: torch.Tensor,
    frame_slots: Sequence[int],
    *,
    frame_tokens: int,
    softmax_scale: float | None = None,
    kscale: torch.Tensor | None = None,
    vscale: torch.Tensor | None = None,
    mask_mode: int = _lib.SKV_MASK_NONE,
    q_pos0: int = 0,
    chunk_tokens: int = 0,
    out: torch.Tensor | None = None,
    rope: tuple[torch.Tensor, tuple[int, int], torch.Tensor] | None = None,
    prope: tuple[torch.Tensor, tuple[int, int], torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
    q_norm: tuple[torch.Tensor, torch.Tensor] | None = None,
    frame_lens: Sequence[int] | None = None,
    segments: Sequence[tuple[int, int]] | None = None,
) -> tuple[_lib.AttentionDesc, torch.Tensor, tuple]:
    """Validate an attention launch and return ``(descriptor, out, keep-alive objects)`` for
    ``skv_attention_ex`` (no workspace set).  Arguments as :func:`attention_frames`."""
    n_slots, b, h = check_pools(kpool, vpool, frame_tokens)
    sb, st, sh = _token_major("q", q)
    if q.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise ValueError(f"q dtype {q.dtype} unsupported (float32, bfloat16 or float16)")
    if (q.dtype == torch.float16) != (kpool.dtype == torch.float16) and not (
            kpool.dtype == torch.float16 and q.dtype == torch.float32):
        raise ValueError("float16 pools take float16 or float32 queries; float16 queries need "
                         "float16 pools")
    if q.shape[0] != b or q.shape[2] != h:
        raise ValueError(f"q batch/heads {tuple(q.shape)} do not match the pool ({b}, {h})")
    if q.device != kpool.device:
        raise ValueError("q and pools must be on the same device")
    if len(frame_slots) == 0:
        raise RuntimeError("attention over an empty key window")
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    if tuple(out.shape) != tuple(q.shape) or out.dtype != q.dtype:
        raise ValueError("out must match q's shape and dtype")
    osb, ost, osh = _token_major("out", out)
    scale = 1.0 / math.sqrt(HEAD_DIM) if softmax_scale is None else float(softmax_scale)
    ks, vs = _scales(kpool, kscale, vscale)
    table = _lib.int32_array(frame_slots)
    d = _lib.AttentionDesc(
        q=q.data_ptr(), q_dtype=dtype_code(q.dtype), q_sb=sb, q_st=st, q_sh=sh,
        k_pool=kpool.data_ptr(), v_pool=vpool.data_ptr(), k_scale=ks, v_scale=vs,
        pool_dtype=dtype_code(kpool.dtype), n_slots=n_slots, frame_slots=table,
        n_frames=len(frame_slots), batch=b, heads=h, head_dim=HEAD_DIM, q_len=q.shape[1],
        frame_tokens=frame_tokens, softmax_scale=scale, mask_mode=mask_mode, q_pos0=q_pos0,
        chunk_tokens=chunk_tokens, out=out.data_ptr(), out_sb=osb, out_st=ost, out_sh=osh)
    keep = [table]
    if q_norm is not None:
        d.q_inv_rms, d.q_rms_stride_b, d.q_norm_weight = _norm_args("q_norm", q_norm, b, q.shape[1],
                                                                    h, q.device)
    if frame_lens is not None:
        if len(frame_lens) != len(frame_slots):
            raise ValueError("frame_lens needs one entry per listed frame")
        flens = _lib.int32_array(frame_lens)
        d.frame_lens = flens
        keep.append(flens)
    if segments is not None:
        if not 1 <= len(segments) <= _lib.SKV_MAX_SEGMENTS:
            raise ValueError(f"1..{_lib.SKV_MAX_SEGMENTS} segments per launch, got {len(segments)}")
        rows = [int(r) for r, _ in segments]
        nfs = [int(f) for _, f in segments]
        if min(rows) < 1 or min(nfs) < 1:
            raise ValueError("every segment needs at least one query row and one frame")
        if sum(rows) != q.shape[1] or sum(nfs) != len(frame_slots):
            raise ValueError(f"segments cover {sum(rows)} rows and {sum(nfs)} frames; q has "
                             f"{q.shape[1]} rows and the list {len(frame_slots)} frames")
        if kpool.dtype != torch.bfloat16 or q.dtype == torch.float16 or mask_mode != _lib.SKV_MASK_NONE:
            raise ValueError("segments need bfloat16 pools, bfloat16 or float32 queries and no mask")
        sr, sf = _lib.int32_array(rows), _lib.int32_array(nfs)
        d.seg_rows, d.seg_frames, d.n_segments = sr, sf, len(segments)
        keep += [sr, sf]
    nq = q.shape[1] // frame_tokens
    if rope is not None and prope is not None:
        raise ValueError("give rope= or prope=, not both")
    if (rope is not None or prope is not None) and segments is not None:
        raise ValueError("segments take no rope= / prope=")
    if rope is not None or prope is not None:
        rhw, ghw = (rope or prope)[0], (rope or prope)[1]
        _check_rope_hw(kpool, kpool, rhw, ghw, frame_tokens)
        if q.shape[1] != nq * frame_tokens:
            raise ValueError(f"RoPE queries must be whole frames (Lq={q.shape[1]})")
        d.rope_hw, d.grid_h, d.grid_w, d.n_qframes = rhw.data_ptr(), int(ghw[0]), int(ghw[1]), nq
    if rope is not None:
        rt = rope[2]
        _require_cuda("rope_t", rt)
        if (tuple(rt.shape) != (nq, len(frame_slots), 22, 2) or rt.dtype != torch.float32
                or not rt.is_contiguous()):
            raise ValueError(f"rope_t must be contiguous float32 [{nq}, {len(frame_slots)}, 22, 2]"
                             f", got {rt.dtype} {tuple(rt.shape)}")
        d.rope_t = rt.data_ptr()
    if prope is not None:
        xt, xs, xo = prope[2], prope[3], prope[4]
        for name, t, shape in (("q_xform_t", xt, (b, len(frame_slots), nq, 11, 4, 4)),
                               ("q_xform_s", xs, (b, nq, 4, 4)), ("out_xform", xo, (b, nq, 4, 4))):
            _require_cuda(name, t)
            if t.dtype != torch.float32 or tuple(t.shape) != shape or not t.is_contiguous():
                raise ValueError(f"{name} must be contiguous float32 {list(shape)}, got "
                                 f"{t.dtype} {tuple(t.shape)}")
        d.q_xform_t, d.q_xform_s, d.out_xform = xt.data_ptr(), xs.data_ptr(), xo.data_ptr()
    return d, out, tuple(keep)


def cu_count(device: torch.device) -> int:
    """Compute units of ``device`` (the split path runs one workgroup per CU)."""
    return torch.cuda.get_device_properties(device).multi_processor_count


def attention_plan(q: torch.Tensor, kpool: torch.Tensor, vpool: torch.Tensor,
                   frame_slots: Sequence[int], *, use_workspace: bool = True,
                   **kw) -> dict[str, int]:
    """The launch :func:`attention_frames` makes for these arguments (``skv_attention_plan``):
    ``waves_per_group``, ``split``, ``n_workgroups``, ``n_qtiles``, ``workspace_bytes``,
    ``key_tiles``."""
    lib = _lib.load()
    d, _, keep = attention_desc(q, kpool, vpool, frame_slots, **kw)
    plan = _lib.LaunchPlan()
    _lib.check("skv_attention_plan", lib.skv_attention_plan(ctypes.byref(d), ctypes.byref(plan)))
    if use_workspace and plan.workspace_bytes > 0:
        d.workspace, d.workspace_bytes, _ = workspace(q.device, plan.workspace_bytes)
        _lib.check("skv_attention_plan", lib.skv_attention_plan(ctypes.byref(d), ctypes.byref(plan)))
    return {name: int(getattr(plan, name)) for name, _ in _lib.LaunchPlan._fields_}


def attention_frames(
    q: torch.Tensor,
    kpool: torch.Tensor,
    vpool: torch.Tensor,
    frame_slots: Sequence[int],
    *,
    frame_tokens: int,
    softmax_scale: float | None = None,
    kscale: torch.Tensor | None = None,
    vscale: torch.Tensor | None = None,
    mask_mode: int = _lib.SKV_MASK_NONE,
    q_pos0: int = 0,
    chunk_tokens: int = 0,
    out: torch.Tensor | None = None,
    rope: tuple[torch.Tensor, tuple[int, int], torch.Tensor] | None = None,
    prope: tuple[torch.Tensor, tuple[int, int], torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
    q_norm: tuple[torch.Tensor, torch.Tensor] | None = None,
    frame_lens: Sequence[int] | None = None,
    segments: Sequence[tuple[int, int]] | None = None,
    use_workspace: bool = True,
) -> torch.Tensor:
    """softmax(q kᵀ·scale) v over the keys of ``frame_slots`` (in order); returns [B, Lq, H, D].

    ``rope = (rope_hw, grid_hw, rope_t)``: ``q`` is pre-RoPE and ``kpool`` is the height/width
    roped K copy; the kernel ropes the queries (``rope_t`` from ``rope.temporal_table`` with one
    row per query frame and one column per entry of ``frame_slots``).

    ``prope = (rope_hw, grid_hw, q_xform_t, q_xform_s, out_xform)``: RoPE then PRoPE; ``kpool`` /
    ``vpool`` are the transformed copies of a PRoPE append and the tables come from
    ``prope.PropeTables`` (float32 ``[B, n_frames, n_qframes, 11, 4, 4]``, ``[B, n_qframes, 4,
    4]`` twice).

    ``q_norm = (inv_rms, weight)``: the kernel RMS-normalises Q at load (``rms_rows`` of ``q``
    and the norm's float32 weight), before RoPE / PRoPE.

    ``frame_lens``: valid keys of each listed frame (``1..frame_tokens``), for windows that mix
    whole frames with shorter spans; keys past a frame's length are masked (mask NONE only).

    ``segments = [(rows, n_frames), ...]``: one launch for several query segments, each over its
    own frame list: segment s is the next ``rows`` query rows and attends the next ``n_frames``
    entries of ``frame_slots`` (and ``frame_lens``).  At most ``SKV_MAX_SEGMENTS``; bfloat16
    pools, bfloat16 or float32 queries, no mask, no RoPE; segments never take the key split.

    Under-filled grids take the balanced key split with this stream's workspace
    (``use_workspace=False`` keeps them on the unsplit kernel)."""
    lib = _lib.load()
    d, out, keep = attention_desc(
        q, kpool, vpool, frame_slots, frame_tokens=frame_tokens, softmax_scale=softmax_scale,
        kscale=kscale, vscale=vscale, mask_mode=mask_mode, q_pos0=q_pos0,
        chunk_tokens=chunk_tokens, out=out, rope=rope, prope=prope, q_norm=q_norm,
        frame_lens=frame_lens, segments=segments)
    if use_workspace:
        plan = _lib.LaunchPlan()
        _lib.check("skv_attention_plan", lib.skv_attention_plan(ctypes.byref(d), ctypes.byref(plan)))
        if plan.workspace_bytes > 0:
            d.workspace, d.workspace_bytes, ws = workspace(q.device, plan.workspace_bytes)
            keep = keep + (ws,)
    t0 = _tic("attention")
    _lib.check("skv_attention_ex", lib.skv_attention_ex(ctypes.byref(d), _stream(q.device)))
    # algorithmic FLOPs: QKᵀ and PV over every key (masking is not discounted)
    if segments is None:
        pairs = q.shape[1] * len(frame_slots) * frame_tokens
    else:
        pairs = sum(r * f for r, f in segments) * frame_tokens
    _toc("attention", t0, 4.0 * d.batch * d.heads * pairs * HEAD_DIM)
    del keep
    return out


def new_pools(
    n_slots: int,
    batch: int,
    heads: int,
    frame_tokens: int,
    dtype: torch.dtype,
    device: torch.device | str,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None, torch.Tensor | None]:
    """Allocate zeroed K/V pools (and fp8 scales) for ``n_slots`` frame slots."""
    tp = padded_tokens(frame_tokens)
    kpool = torch.zeros((n_slots, batch, heads, tp, HEAD_DIM), dtype=dtype, device=device)
    vpool = torch.zeros((n_slots, batch, heads, HEAD_DIM, tp), dtype=dtype, device=device)
    if dtype == torch.float8_e4m3fn:
        kscale = torch.zeros((n_slots, batch, heads), dtype=torch.float32, device=device)
        vscale = torch.zeros((n_slots, batch, heads), dtype=torch.float32, device=device)
    else:
        kscale = vscale = None
    return kpool, vpool, kscale, vscale


_staging: dict[tuple[int, int, torch.dtype], torch.Tensor] = {}


def staging_pools(
    n_slots: int,
    batch: int,
    heads: int,
    frame_tokens: int,
    dtype: torch.dtype,
    device: torch.device,
) -> tuple[torch.Tensor, torch.Tensor]:
    """K/V pools of ``n_slots`` frames over this device and current stream's staging buffer, for
    dense K/V that a call stages and attends at once (the drop-in ``attention``, teacher
    forcing).  The buffer grows on demand and is reused by every such call on the stream; its
    contents are left as they are (not zero-filled): an append writes every row of the slots it
    fills, rows past ``frame_tokens`` as zeros.  Calls on one stream run in order, so a call's
    append waits for the previous call's attention; the buffer stays allocated at its largest
    size (bf16 K+V of a 32768-key window at 12 heads: 201 MB)."""
    if dtype == torch.float8_e4m3fn:
        raise ValueError("staging pools hold bf16, f16 or float32 frames")
    tp = padded_tokens(frame_tokens)
    n = n_slots * batch * heads * tp * HEAD_DIM
    key = (device.index if device.index is not None else torch.cuda.current_device(),
           _stream(device), dtype)
    buf = _staging.get(key)
    if buf is None or buf.numel() < 2 * n:
        buf = torch.empty(2 * n, dtype=dtype, device=device)
        _staging[key] = buf
    kpool = buf[:n].view(n_slots, batch, heads, tp, HEAD_DIM)
    vpool = buf[n : 2 * n].view(n_slots, batch, heads, HEAD_DIM, tp)
    return kpool, vpool
