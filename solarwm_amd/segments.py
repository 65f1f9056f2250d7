"""Segmented attention on the frame-slot kernel: teacher-forcing masks, H3 chunk-list caches and
memory-KV segments.

Each of these reference paths attends query segments to unions of key spans:

* the teacher-forcing block mask over ``[clean | noisy]`` tokens (causal_model.py:337-471): a
  query chunk sees a sink, a bounded run of earlier clean chunks and (noisy) its own chunk;
* H3's rollout window (sgf_attention.py:40-63, :236-258, :580-659): the chunk attends to
  ``[prefix | last <= 5 committed chunks | chunk]`` with the raw chunk K/V kept per layer;
* H3's memory-KV layout (memory_kv_attention.py:39-140): shared, bank, audio and chunk rows,
  each with its own key spans.

Here the key spans live in pool slots (frames of T tokens; spans that are not whole frames use
partly filled slots with per-frame lengths) and each query segment attends its own frame list,
so no mask is materialised and masked-out blocks cost nothing.  Consecutive segments share one
launch of the segmented kernel (up to ``SKV_MAX_SEGMENTS`` segments and ``SKV_MAX_FRAMES``
listed frames per launch; bf16 pools): its grid holds every segment's q-tiles, so short
segments no longer leave the chip idle between launches.  The H3 rotary and camera transforms are applied by the caller (inputs are
post-transform Q/K/V), as the reference applies them before its attention call.
"""

from __future__ import annotations

from typing import Sequence

import torch

from . import _lib, h3, kernels

def attend_segments(q: torch.Tensor, kpool: torch.Tensor, vpool: torch.Tensor,
                    segs: Sequence[tuple[int, Sequence[int], Sequence[int] | None]], *,
                    frame_tokens: int, softmax_scale: float | None = None,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """Attention of consecutive query segments, each over its own frame list: ``segs`` is
    ``[(rows, frame list, frame lengths or None), ...]`` covering ``q``'s rows in order.  Runs of
    consecutive segments go to one launch (``attention_frames(segments=...)``) while they fit the
    launch limits; float32 pools take one launch per segment."""
    if sum(r for r, _, _ in segs) != q.shape[1]:
        raise ValueError(f"segments cover {sum(r for r, _, _ in segs)} rows, q has {q.shape[1]}")
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    T = frame_tokens
    one_launch = kpool.dtype == torch.bfloat16 and q.dtype in (torch.bfloat16, torch.float32)
    groups: list[list[tuple[int, Sequence[int], Sequence[int] | None]]] = []
    n_frames = 0
    for seg in segs:
        if (not groups or not one_launch or len(groups[-1]) == _lib.SKV_MAX_SEGMENTS
                or n_frames + len(seg[1]) > _lib.SKV_MAX_FRAMES):
            groups.append([])
            n_frames = 0
        groups[-1].append(seg)
        n_frames += len(seg[1])
    r0 = 0
    for grp in groups:
        rows = sum(r for r, _, _ in grp)
        frames = [f for _, fr, _ in grp for f in fr]
        lens = None
        if any(ln is not None for _, _, ln in grp):
            lens = [x for _, fr, ln in grp for x in (ln if ln is not None else [T] * len(fr))]
        s = slice(r0, r0 + rows)
        kernels.attention_frames(q[:, s], kpool, vpool, frames, frame_tokens=T,
                                 softmax_scale=softmax_scale, out=out[:, s], frame_lens=lens,
                                 segments=[(r, len(fr)) for r, fr, _ in grp] if len(grp) > 1 else None)
        r0 += rows
    return out


def teacher_forcing_frame_lists(*, num_frames: int, num_frame_per_block: int,
                                max_prior_clean_chunks: int | None = None, sink_size: int = 0):
    """[(first query frame, frame list)] per query chunk of ``[clean | noisy]`` frames (clean
    frames 0..F-1, noisy F..2F-1): the union of the reference's key intervals
    (causal_model.py:434-468) in frames, duplicates removed."""
    F, nb = num_frames, num_frame_per_block
    # the reference's checks, in its order and words (causal_model.py:357-386)
    if nb <= 0:
        raise ValueError(f"num_frame_per_block must be positive, got {nb}")
    if F % nb:
        raise ValueError(f"num_frames={F} must be divisible by num_frame_per_block={nb}")
    sink_size = int(sink_size)
    if sink_size < 0 or sink_size > F:
        raise ValueError(f"sink_size must be in [0, {F}], got {sink_size}")
    if sink_size % nb:
        raise ValueError(f"sink_size={sink_size} must contain whole {nb}-frame chunks")
    chunks = F // nb
    default = max(0, chunks - 1)
    m = default if max_prior_clean_chunks is None else int(max_prior_clean_chunks)
    if not 0 <= m <= default:
        raise ValueError(f"model.max_prior_clean_chunks must be in [0, {default}] for a "
                         f"{chunks}-chunk window, got {m}")
    out = []
    for c in range(chunks):  # clean queries
        frames = set(range(max(0, c - m) * nb if sink_size else 0, (c + 1) * nb))
        frames |= set(range(min(sink_size, (c + 1) * nb)))
        out.append((c * nb, sorted(frames)))
    for c in range(chunks):  # noisy queries: never their own clean chunk
        frames = set(range(min(sink_size, c * nb))) | set(range(max(0, c - m) * nb, c * nb))
        frames |= set(range(F + c * nb, F + (c + 1) * nb))
        out.append((F + c * nb, sorted(frames)))
    return out


def teacher_forcing_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                              num_frames: int, frame_seqlen: int, num_frame_per_block: int,
                              max_prior_clean_chunks: int | None = None, sink_size: int = 0,
                              softmax_scale: float | None = None) -> torch.Tensor:
    """Attention of ``[clean | noisy]`` tokens under the teacher-forcing block mask
    (build_teacher_forcing_block_mask + flex_attention, causal_model.py:337-471 and its
    masked path); q/k/v are [B, 2 * num_frames * frame_seqlen, H, D] in bf16 or float32.
    FlexAttention's padding rows (which only see themselves) are not produced."""
    T = frame_seqlen
    b, L, h, _ = q.shape
    if k.shape != q.shape or v.shape != q.shape or L != 2 * num_frames * T:
        raise ValueError(f"q/k/v must be [B, {2 * num_frames * T}, H, D] and share a shape")
    lists = teacher_forcing_frame_lists(num_frames=num_frames, num_frame_per_block=num_frame_per_block,
                                        max_prior_clean_chunks=max_prior_clean_chunks, sink_size=sink_size)
    kv_dtype = k.dtype if k.dtype in (torch.bfloat16, torch.float32) else torch.bfloat16
    kp, vp = kernels.staging_pools(2 * num_frames, b, h, T, kv_dtype, q.device)
    kernels.append_frames(k.to(kv_dtype), v.to(kv_dtype), kp, vp, list(range(2 * num_frames)),
                          frame_tokens=T)
    qq = q if q.dtype in (torch.bfloat16, torch.float32) else q.to(kv_dtype)
    rows = num_frame_per_block * T  # the lists come in query order: chunk c starts at row c * rows
    out = attend_segments(qq, kp, vp, [(rows, frames, None) for _, frames in lists],
                          frame_tokens=T, softmax_scale=softmax_scale)
    return out.to(q.dtype)


class _SpanWriter:
    """Writes token spans of any length into consecutive slots of a pool (the last slot of a span
    partly filled); returns (slots, lengths)."""

    def __init__(self, kpool: torch.Tensor, vpool: torch.Tensor, frame_tokens: int):
        self.kpool, self.vpool, self.T = kpool, vpool, frame_tokens

    def write(self, k: torch.Tensor, v: torch.Tensor, slots: Sequence[int]) -> list[int]:
        T = self.T
        n = k.shape[1]
        nf = -(-n // T)
        if nf != len(slots):
            raise ValueError(f"a {n}-token span needs {nf} slots, got {len(slots)}")
        if n == 0:
            return []
        whole = n // T
        if whole:
            kernels.append_frames(k, v, self.kpool, self.vpool, list(slots[:whole]), frame_tokens=T)
        lens = [T] * whole
        if n > whole * T:  # the tail goes through a zero-padded frame
            rest = n - whole * T
            pk = torch.zeros((k.shape[0], T, k.shape[2], k.shape[3]), dtype=k.dtype, device=k.device)
            pv = torch.zeros_like(pk)
            pk[:, :rest], pv[:, :rest] = k[:, whole * T :], v[:, whole * T :]
            kernels.append_frames(pk, pv, self.kpool, self.vpool, [slots[whole]], frame_tokens=T)
            lens.append(rest)
        return lens


class ChunkListKVCache:
    """H3's raw chunk-list KV cache (sgf_attention.py:40-63) on frame slots: per layer, the last
    ``window`` committed chunks of ``chunk_frames`` frames; ``history`` demands exactly the
    chunks right before the requested one, as the reference does.  Each layer also has
    ``span_frames`` slots for the per-forward prefix spans (text, anchor, bank, audio rows)."""

    def __init__(self, *, num_layers: int, batch: int, heads: int, frame_tokens: int,
                 chunk_frames: int = 5, window: int = 5, span_frames: int = 8,
                 dtype: torch.dtype = torch.bfloat16, device="cuda"):
        self.T, self.chunk_frames, self.window, self.span_frames = frame_tokens, chunk_frames, window, span_frames
        self.n_chunk_slots = (window + 1) * chunk_frames
        n_slots = self.n_chunk_slots + span_frames
        self.pools = [kernels.new_pools(n_slots, batch, heads, frame_tokens, dtype, device)[:2]
                      for _ in range(num_layers)]
        self.entries: list[list[tuple[int, list[int]]]] = [[] for _ in range(num_layers)]
        self.dtype = dtype

    def clear(self) -> None:
        self.entries = [[] for _ in self.entries]

    def history(self, layer: int, chunk_index: int) -> list[tuple[int, list[int]]]:
        entries = self.entries[layer]
        expected = list(range(max(0, chunk_index - self.window), chunk_index))
        if [e[0] for e in entries] != expected:
            raise RuntimeError(f"H3 KV history differs at layer={layer}, chunk={chunk_index}")
        return entries

    def _staging(self, layer: int) -> list[int]:
        used = {s for _, slots in self.entries[layer] for s in slots}
        free = [s for s in range(self.n_chunk_slots) if s not in used]
        return free[: self.chunk_frames]

    def write_spans(self, layer: int, spans: Sequence[tuple[torch.Tensor, torch.Tensor]]):
        """Store prefix spans (each [B, n, H, D] K and V) in this layer's span slots; returns one
        (slots, lengths) pair per span."""
        kp, vp = self.pools[layer]
        w = _SpanWriter(kp, vp, self.T)
        nxt = self.n_chunk_slots
        out = []
        for k, v in spans:
            nf = -(-k.shape[1] // self.T)
            if nxt + nf > self.n_chunk_slots + self.span_frames:
                raise ValueError(f"prefix spans need more than the cache's {self.span_frames} span frames")
            slots = list(range(nxt, nxt + nf))
            out.append((slots, w.write(k, v, slots)))
            nxt += nf
        return out

    def stage_chunk(self, layer: int, chunk_index: int, k: torch.Tensor, v: torch.Tensor):
        """Append the chunk's raw K/V into free slots; returns (history frames, chunk slots)."""
        hist = self.history(layer, chunk_index)
        if k.shape[1] != self.chunk_frames * self.T:
            raise ValueError(f"a chunk is {self.chunk_frames} frames of {self.T} tokens")
        staging = self._staging(layer)
        kp, vp = self.pools[layer]
        kernels.append_frames(k, v, kp, vp, staging, frame_tokens=self.T)
        return [s for _, slots in hist for s in slots], staging

    def commit_staged(self, layer: int, chunk_index: int, staging: list[int]) -> None:
        self.history(layer, chunk_index)
        self.entries[layer] = [*self.entries[layer], (chunk_index, list(staging))][-self.window :]


def windowed_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cache: ChunkListKVCache,
                       layer: int, chunk_index: int, *, prefix: tuple[torch.Tensor, torch.Tensor] | None = None,
                       commit: bool = False, softmax_scale: float | None = None) -> torch.Tensor:
    """H3 rollout chunk attention (sgf_attention.py:236-258, :580-659): the chunk's queries over
    ``[prefix | history chunks | chunk]``; ``commit`` keeps the chunk's raw K/V as the newest
    history entry (the reference's ``control.cache.commit``)."""
    frames, lens = [], []
    if prefix is not None:
        ((pslots, plens),) = cache.write_spans(layer, [prefix])
        frames += pslots
        lens += plens
    hist, staging = cache.stage_chunk(layer, chunk_index, k, v)
    frames += hist + staging
    lens += [cache.T] * (len(hist) + len(staging))
    kp, vp = cache.pools[layer]
    out = kernels.attention_frames(q, kp, vp, frames, frame_tokens=cache.T,
                                   softmax_scale=softmax_scale, frame_lens=lens)
    if commit:
        cache.commit_staged(layer, chunk_index, staging)
    return out


def memory_kv_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cache: ChunkListKVCache,
                        layer: int, chunk_index: int, *, text_rows: int, n_bank: int,
                        audio_rows: int, commit: bool = False,
                        softmax_scale: float | None = None) -> torch.Tensor:
    """H3 memory-KV attention (MemoryKVAttention.attend, memory_kv_attention.py:39-140) on
    post-transform inputs packed ``[text | anchor frame | bank frames | audio | chunk]``: shared
    rows see the shared rows, bank rows see shared + bank + history, audio rows see shared +
    audio, the chunk sees everything; the chunk's raw K/V are committed with ``commit``."""
    T = cache.T
    chunk_rows = cache.chunk_frames * T
    shared = text_rows + T
    bank_end = shared + n_bank * T
    prefix = bank_end + audio_rows
    if q.shape[1] != prefix + chunk_rows or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("Memory KV packed layout mismatch")
    spans = [(k[:, :text_rows], v[:, :text_rows]), (k[:, text_rows:shared], v[:, text_rows:shared])]
    spans += [(k[:, shared:bank_end], v[:, shared:bank_end]), (k[:, bank_end:prefix], v[:, bank_end:prefix])]
    (ts, tl), (anc, al), (bk, bl), (au, aul) = cache.write_spans(layer, spans)
    hist, staging = cache.stage_chunk(layer, chunk_index, k[:, prefix:], v[:, prefix:])
    kp, vp = cache.pools[layer]
    full = [T] * len(hist)
    segs = [(shared, ts + anc, tl + al)]
    if n_bank:
        segs.append((bank_end - shared, ts + anc + bk + hist, tl + al + bl + full))
    if audio_rows:
        segs.append((audio_rows, ts + anc + au, tl + al + aul))
    segs.append((chunk_rows, ts + anc + bk + au + hist + staging,
                 tl + al + bl + aul + full + [T] * len(staging)))
    out = attend_segments(q, kp, vp, segs, frame_tokens=T, softmax_scale=softmax_scale)
    if commit:
        cache.commit_staged(layer, chunk_index, staging)
    return out


class H3WindowCache:
    """H3's rollout with its own transforms: the raw chunk-list KV cache (H3RawKVCache,
    sgf_attention.py:40-63) and the transformed attention window of the chunk being evaluated
    (the KV window of _windowed_rollout_attention, sgf_attention.py:580-659).

    H3 rotates and projects every key of a chunk's window with positions and cameras of that
    window, so the cache keeps raw K/V (a ring of ``window`` chunks per layer) and builds the
    window's transformed prefix and history frames once per chunk and layer, in pool slots;
    each evaluation of the chunk (denoising steps, the commit pass) transforms only its own
    rows.  The prefix and the tables of a chunk must stay the same over its evaluations, as in
    the reference's KV window; ``invalidate`` forces a rebuild."""

    def __init__(self, *, num_layers: int, batch: int, heads: int, frame_tokens: int,
                 prefix_rows: int, chunk_frames: int = 5, window: int = 5, device="cuda"):
        T = frame_tokens
        self.T, self.cf, self.window, self.P = T, chunk_frames, window, int(prefix_rows)
        self.C = chunk_frames * T
        self.pf = -(-self.P // T)
        # prefix slots: the window's prefix, or the memory layout's four spans (text, anchor,
        # bank, audio), each starting a frame, so up to three more partly filled frames
        self.ns = self.pf + 3
        bf = torch.bfloat16
        shape = (num_layers, window, batch, self.C, heads, 128)
        self.raw_k = torch.empty(shape, dtype=bf, device=device)
        self.raw_v = torch.empty(shape, dtype=bf, device=device)
        self.entries: list[list[tuple[int, int]]] = [[] for _ in range(num_layers)]
        n_slots = self.ns + (window + 1) * chunk_frames
        self.pools = [kernels.new_pools(n_slots, batch, heads, T, bf, device)[:2]
                      for _ in range(num_layers)]
        self.built: list[tuple[str, int] | None] = [None] * num_layers
        rows = max((self.pf + 1) * T, self.C)  # the largest span or chunk, in whole frames
        self._tk = torch.empty((batch, rows, heads, 128), dtype=bf, device=device)
        self._tv = torch.empty_like(self._tk)

    def clear(self) -> None:
        self.entries = [[] for _ in self.entries]
        self.invalidate()

    def invalidate(self) -> None:
        self.built = [None] * len(self.built)

    def history(self, layer: int, chunk_index: int) -> list[tuple[int, int]]:
        entries = self.entries[layer]
        expected = list(range(max(0, chunk_index - self.window), chunk_index))
        if [e[0] for e in entries] != expected:
            raise RuntimeError(f"H3 KV history differs at layer={layer}, chunk={chunk_index}")
        return entries

    def _to_slots(self, layer, k, v, cos, sin, matrix, slots) -> None:
        """Transform raw rows k / v ([B, n, H, 128]) and append them to whole frame slots; rows
        past n in the last slot are zeros (masked by the frame lengths)."""
        n, rows = k.shape[1], len(slots) * self.T
        tk, tv = self._tk[:, :rows], self._tv[:, :rows]
        h3.rope_prope(k, cos, sin, matrix, out=tk[:, :n])
        h3.rope_prope(v, None, None, matrix, out=tv[:, :n])
        if n < rows:
            tk[:, n:].zero_()
            tv[:, n:].zero_()
        kp, vp = self.pools[layer]
        kernels.append_frames(tk, tv, kp, vp, list(slots), frame_tokens=self.T)

    def attend(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layer: int,
               chunk_index: int, *, prefix: tuple[torch.Tensor, torch.Tensor],
               q_rotary: tuple[torch.Tensor, torch.Tensor],
               k_rotary: tuple[torch.Tensor, torch.Tensor], q_matrix: torch.Tensor,
               kv_matrix: torch.Tensor, out_matrix: torch.Tensor, commit: bool = False,
               softmax_scale: float | None = None) -> torch.Tensor:
        """One evaluation of chunk ``chunk_index``: raw chunk rows q / k / v [B, C, H, 128]
        bf16, the raw prefix K / V [B, prefix_rows, H, 128]; ``k_rotary`` (cos, sin) and
        ``kv_matrix`` cover the window's key rows [prefix | history chunks | chunk],
        ``q_rotary``, ``q_matrix`` and ``out_matrix`` the chunk's rows (the reference's kr, qr
        and camera matrices).  Returns the projected attention output [B, C, H, 128]."""
        T, P, C = self.T, self.P, self.C
        if q.shape[1] != C or k.shape != q.shape or v.shape != q.shape:
            raise ValueError(f"q/k/v must be one chunk of {C} rows")
        pk, pv = prefix
        if pk.shape[1] != P or pv.shape != pk.shape:
            raise ValueError(f"the prefix must be {P} rows")
        hist = self.history(layer, chunk_index)
        nh = len(hist)
        total = P + (nh + 1) * C
        kc, ks = k_rotary
        if kc.shape[0] != total or kv_matrix.shape[1] != total:
            raise ValueError(f"k_rotary and kv_matrix need {total} rows (prefix, {nh} history "
                             f"chunks, the chunk), got {kc.shape[0]} / {kv_matrix.shape[1]}")
        pslots = list(range(self.pf))
        hslots, cslots = self._history_slots(nh)
        if self.built[layer] != ("window", chunk_index):
            if P:
                self._to_slots(layer, pk, pv, kc[:P], ks[:P], kv_matrix[:, :P], pslots)
            self._build_history(layer, hist, kc[P:P + nh * C], ks[P:P + nh * C],
                                kv_matrix[:, P:P + nh * C], hslots)
            self.built[layer] = ("window", chunk_index)
        r0 = P + nh * C
        self._to_slots(layer, k, v, kc[r0:], ks[r0:], kv_matrix[:, r0:], cslots)
        qt = h3.rope_prope(q, q_rotary[0], q_rotary[1], q_matrix)
        lens = [T] * (self.pf - 1) + [P - (self.pf - 1) * T] if P else []
        lens += [T] * (len(hslots) + self.cf)
        kp, vp = self.pools[layer]
        out = kernels.attention_frames(qt, kp, vp, pslots + hslots + cslots, frame_tokens=T,
                                       softmax_scale=softmax_scale, frame_lens=lens)
        h3.rope_prope(out, None, None, out_matrix, out=out)
        if commit:
            self._commit(layer, chunk_index, hist, k, v)
        return out

    def _history_slots(self, nh: int) -> tuple[list[int], list[int]]:
        cf, base = self.cf, self.ns
        return ([base + i * cf + j for i in range(nh) for j in range(cf)],
                [base + nh * cf + j for j in range(cf)])

    def _build_history(self, layer, hist, cos, sin, matrix, hslots) -> None:
        """Transform the raw history chunks with the window's rows of the tables into their
        slots (once per chunk and layer)."""
        C, cf = self.C, self.cf
        for i, (_, ring) in enumerate(hist):
            self._to_slots(layer, self.raw_k[layer, ring], self.raw_v[layer, ring],
                           cos[i * C:(i + 1) * C], sin[i * C:(i + 1) * C],
                           matrix[:, i * C:(i + 1) * C], hslots[i * cf:(i + 1) * cf])

    def _commit(self, layer, chunk_index, hist, k, v) -> None:
        """Keep the chunk's raw K/V as the newest history entry (the oldest rolls off)."""
        kept = [*hist, (chunk_index, -1)][-self.window:]
        used = {r for _, r in kept if r >= 0}
        ring = min(r for r in range(self.window) if r not in used)
        self.raw_k[layer, ring].copy_(k)
        self.raw_v[layer, ring].copy_(v)
        self.entries[layer] = [(c, r if r >= 0 else ring) for c, r in kept]

    def attend_memory(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layer: int,
                      chunk_index: int, *, text_rows: int, n_bank: int, audio_rows: int,
                      rotary: tuple[torch.Tensor, torch.Tensor],
                      history_rotary: tuple[torch.Tensor, torch.Tensor] | None,
                      q_matrix: torch.Tensor, kv_matrix: torch.Tensor, out_matrix: torch.Tensor,
                      history_kv_matrix: torch.Tensor | None, commit: bool = False,
                      softmax_scale: float | None = None) -> torch.Tensor:
        """H3 memory-KV attention with its transforms (MemoryKVAttention.attend,
        memory_kv_attention.py:39-140) on raw packed rows ``[text | anchor frame | bank frames
        | audio | chunk]``: every row keeps one rotary row and one camera in every segment it
        enters (``rotary``, ``q_matrix`` / ``kv_matrix`` / ``out_matrix`` per packed row), the
        raw history chunks take ``history_rotary`` and ``history_kv_matrix`` (the window's
        rows; None without history), so each row is transformed once and the segments run as
        one segmented launch; outputs are projected per row.  Shared rows see the shared rows,
        bank rows shared + bank + history, audio rows shared + audio, the chunk everything."""
        T, C = self.T, self.C
        shared = text_rows + T
        bank_end = shared + n_bank * T
        prefix = bank_end + audio_rows
        if q.shape[1] != prefix + C or k.shape != q.shape or v.shape != q.shape:
            raise ValueError("Memory KV packed layout mismatch")
        if rotary[0].shape[0] != prefix + C or kv_matrix.shape[1] != prefix + C:
            raise ValueError(f"rotary and matrices need one row per packed row ({prefix + C})")
        hist = self.history(layer, chunk_index)
        nh = len(hist)
        if nh and (history_rotary is None or history_rotary[0].shape[0] != nh * C
                   or history_kv_matrix is None or history_kv_matrix.shape[1] != nh * C):
            raise ValueError(f"history_rotary and history_kv_matrix need {nh * C} rows")
        cos, sin = rotary
        nxt, spans = 0, []
        for a, b in ((0, text_rows), (text_rows, shared), (shared, bank_end), (bank_end, prefix)):
            nf = -(-(b - a) // T)
            if nf > self.ns - nxt:
                raise ValueError(f"the prefix spans need more than the cache's {self.ns} span "
                                 f"frames (built for {self.P} prefix rows)")
            slots = list(range(nxt, nxt + nf))
            if nf:
                self._to_slots(layer, k[:, a:b], v[:, a:b], cos[a:b], sin[a:b],
                               kv_matrix[:, a:b], slots)
            lens = [T] * (nf - 1) + [(b - a) - (nf - 1) * T] if nf else []
            spans.append((slots, lens))
            nxt += nf
        hslots, cslots = self._history_slots(nh)
        if self.built[layer] != ("memory", chunk_index):
            if nh:
                self._build_history(layer, hist, history_rotary[0], history_rotary[1],
                                    history_kv_matrix, hslots)
            self.built[layer] = ("memory", chunk_index)
        self._to_slots(layer, k[:, prefix:], v[:, prefix:], cos[prefix:], sin[prefix:],
                       kv_matrix[:, prefix:], cslots)
        (ts, tl), (an, al), (bk, bl), (au, aul) = spans
        full = [T] * len(hslots)
        segs = [(shared, ts + an, tl + al)]
        if n_bank:
            segs.append((bank_end - shared, ts + an + bk + hslots, tl + al + bl + full))
        if audio_rows:
            segs.append((audio_rows, ts + an + au, tl + al + aul))
        segs.append((C, ts + an + bk + au + hslots + cslots,
                     tl + al + bl + aul + full + [T] * self.cf))
        qt = h3.rope_prope(q, cos, sin, q_matrix)
        kp, vp = self.pools[layer]
        out = attend_segments(qt, kp, vp, segs, frame_tokens=T, softmax_scale=softmax_scale)
        h3.rope_prope(out, None, None, out_matrix, out=out)
        if commit:
            self._commit(layer, chunk_index, hist, k[:, prefix:], v[:, prefix:])
        return out
