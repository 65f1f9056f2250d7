"""CPU restatement of the segmented attention patterns around the KV cache — TEST
INFRASTRUCTURE ONLY.

* The teacher-forcing mask over ``[clean | noisy]`` tokens
  (solar/backends/wan22/runtime/modeling/causal_model.py:337-471), twice: the per-token rule
  (``attention_mask``, :404-432) and the per-query-segment key intervals the reference builds
  its block mask from (``iter_q_segments``, :434-468).
* H3's raw chunk-list KV cache (solar/backends/minimax_h3/sgf_attention.py:40-63) and the
  window its rollout attends: ``[prefix | last <= 5 committed chunks | current chunk]``
  (sgf_attention.py:236-258, _windowed_rollout_attention :580-659).
* H3's memory-KV segments (solar/backends/minimax_h3/memory_kv_attention.py:39-140): shared
  rows, bank rows, audio rows and the current chunk, each attending to its own key spans.

The rotary and camera transforms of H3 are applied by the reference before attention and are
not part of these functions: inputs are post-transform Q/K/V.

Pinning (tests/test_oracle_segments.py): the dense teacher-forcing mask equals the union of the
segment intervals on many geometries; noisy chunk i never sees clean chunk i; hand cases; the
chunk-list cache keeps exactly the last five chunks and rejects gaps; segmented attention
equals dense attention under the mask built from the same spans.
"""

from __future__ import annotations


import torch

from .wan_cache_ref import attention


# ---------------------------------------------------------------------------------------------
# teacher forcing (causal_model.py:337-471)
# ---------------------------------------------------------------------------------------------
def _tf_geometry(num_frames, frame_seqlen, num_frame_per_block, max_prior_clean_chunks, sink_size):
    if num_frame_per_block <= 0 or num_frames % num_frame_per_block:
        raise ValueError("num_frames must be a positive multiple of num_frame_per_block")
    if not 0 <= sink_size <= num_frames or sink_size % num_frame_per_block:
        raise ValueError("sink_size must be whole chunks inside the window")
    num_chunks = num_frames // num_frame_per_block
    default = max(0, num_chunks - 1)
    m = default if max_prior_clean_chunks is None else int(max_prior_clean_chunks)
    if not 0 <= m <= default:
        raise ValueError(f"max_prior_clean_chunks must be in [0, {default}]")
    return frame_seqlen * num_frame_per_block, num_frames * frame_seqlen, m, sink_size * frame_seqlen


def teacher_forcing_mask(*, num_frames: int, frame_seqlen: int, num_frame_per_block: int,
                         max_prior_clean_chunks: int | None = None, sink_size: int = 0) -> torch.Tensor:
    """Dense bool [L, L] (L = 2 * num_frames * frame_seqlen, True = visible), the per-token rule
    of causal_model.py:404-432 without FlexAttention's padding rows."""
    bs, clean_end, m, sink = _tf_geometry(num_frames, frame_seqlen, num_frame_per_block,
                                          max_prior_clean_chunks, sink_size)
    total = 2 * clean_end
    q = torch.arange(total)[:, None]
    kv = torch.arange(total)[None, :]
    is_clean = q < clean_end
    cc = q // bs
    first = torch.clamp(cc - m, min=0)
    if sink > 0:
        recent = (kv >= first * bs) & (kv < (cc + 1) * bs)
        vis_sink = (kv < sink) & (kv < (cc + 1) * bs)
        clean = is_clean & (vis_sink | recent)
    else:
        clean = is_clean & (kv < (cc + 1) * bs)
    is_noisy = (q >= clean_end) & (q < total)
    nc = (q - clean_end) // bs
    fp = torch.clamp(nc - m, min=0)
    prior_clean = (kv >= fp * bs) & (kv < nc * bs)
    prior_sink = (kv < sink) & (kv < nc * bs)
    ns = clean_end + nc * bs
    own = (kv >= ns) & (kv < ns + bs)
    noisy = is_noisy & (prior_sink | prior_clean | own)
    return (q == kv) | clean | noisy


def teacher_forcing_segments(*, num_frames: int, frame_seqlen: int, num_frame_per_block: int,
                             max_prior_clean_chunks: int | None = None, sink_size: int = 0):
    """[(q_start, q_end, ((k_start, k_end), ...))] per query chunk, the intervals of
    ``iter_q_segments`` (causal_model.py:434-468); empty intervals are dropped."""
    bs, clean_end, m, sink = _tf_geometry(num_frames, frame_seqlen, num_frame_per_block,
                                          max_prior_clean_chunks, sink_size)
    out = []
    for c in range(clean_end // bs):
        if sink > 0:
            iv = ((0, min(sink, (c + 1) * bs)), (max(0, c - m) * bs, (c + 1) * bs))
        else:
            iv = ((0, (c + 1) * bs),)
        out.append((c * bs, (c + 1) * bs, tuple((a, b) for a, b in iv if b > a)))
    for c in range(clean_end // bs):
        iv = ((0, min(sink, c * bs)), (max(0, c - m) * bs, c * bs),
              (clean_end + c * bs, clean_end + (c + 1) * bs))
        out.append((clean_end + c * bs, clean_end + (c + 1) * bs, tuple((a, b) for a, b in iv if b > a)))
    return out


def segment_mask(total: int, segments) -> torch.Tensor:
    """Dense mask of a segment list: row q sees the union of its segment's key intervals."""
    mask = torch.zeros(total, total, dtype=torch.bool)
    for qs, qe, ivs in segments:
        for a, b in ivs:
            mask[qs:qe, a:b] = True
    return mask


def masked_attention(q, k, v, mask, **kw):
    """Dense attention [B, L, H, D] under a [Lq, Lk] bool mask (float64 unless kw say otherwise)."""
    return attention(q, k, v, mask=mask, **kw)


# ---------------------------------------------------------------------------------------------
# H3 raw chunk-list KV cache (sgf_attention.py:40-63) and its rollout window
# ---------------------------------------------------------------------------------------------
class H3RawKVCache:
    """Per layer, the last five committed chunks (index, k, v); history must be the five chunks
    right before the requested one (fewer at the start)."""

    WINDOW = 5

    def __init__(self):
        self.layers: dict[int, list[tuple[int, torch.Tensor, torch.Tensor]]] = {}

    def history(self, layer: int, chunk_index: int):
        entries = self.layers.get(layer, [])
        expected = list(range(max(0, chunk_index - self.WINDOW), chunk_index))
        if [e[0] for e in entries] != expected:
            raise RuntimeError(f"H3 KV history differs at layer={layer}, chunk={chunk_index}")
        return entries

    def commit(self, layer: int, chunk_index: int, key, value):
        entries = self.history(layer, chunk_index)
        self.layers[layer] = [*entries, (chunk_index, key.clone(), value.clone())][-self.WINDOW:]


def windowed_rollout_attention(q, k, v, prefix_k, prefix_v, cache: H3RawKVCache, layer: int,
                               chunk_index: int, *, commit: bool = False, **kw):
    """The rollout chunk segment (sgf_attention.py:236-258): the chunk's queries attend to
    ``cat[prefix, history chunks, current chunk]``; optionally commit the chunk's raw K/V."""
    hist = cache.history(layer, chunk_index)
    keys = torch.cat([prefix_k, *(e[1] for e in hist), k], dim=1)
    values = torch.cat([prefix_v, *(e[2] for e in hist), v], dim=1)
    out = attention(q, keys, values, **kw)
    if commit:
        cache.commit(layer, chunk_index, k, v)
    return out


# ---------------------------------------------------------------------------------------------
# H3 memory-KV segments (memory_kv_attention.py:39-140)
# ---------------------------------------------------------------------------------------------
def memory_kv_segments(*, text_rows: int, frame_rows: int, n_bank: int, audio_rows: int,
                       history_rows: int, chunk_rows: int):
    """Segments of the packed query ``[text | anchor | bank | audio | chunk]`` over the key
    sequence ``[text | anchor | bank | audio | history | chunk]`` (history rows come from the
    cache): shared rows see the shared rows; bank rows see shared, bank and history; audio rows
    see shared and audio; the chunk sees everything.  Returns (q_start, q_end, key intervals)
    in key-sequence coordinates."""
    shared = text_rows + frame_rows
    bank_end = shared + n_bank * frame_rows
    prefix = bank_end + audio_rows
    hist_end = prefix + history_rows
    segs = [(0, shared, ((0, shared),))]
    if n_bank:
        segs.append((shared, bank_end, ((0, bank_end), (prefix, hist_end))))
    if audio_rows:
        segs.append((bank_end, prefix, ((0, shared), (bank_end, prefix))))
    # query rows of the chunk sit after the prefix in the packed query
    segs.append((prefix, prefix + chunk_rows, ((0, hist_end + chunk_rows),)))
    return segs


def memory_kv_attention(q, k, v, history_k, history_v, *, text_rows, frame_rows, n_bank,
                        audio_rows, **kw):
    """The four ``calculate`` calls of MemoryKVAttention.attend on post-transform inputs:
    q/k/v packed [B, prefix + chunk, H, D], history [B, hrows, H, D] from the cache."""
    chunk_rows = q.shape[1] - (text_rows + frame_rows + n_bank * frame_rows + audio_rows)
    prefix = q.shape[1] - chunk_rows
    keys = torch.cat([k[:, :prefix], history_k, k[:, prefix:]], dim=1)
    values = torch.cat([v[:, :prefix], history_v, v[:, prefix:]], dim=1)
    segs = memory_kv_segments(text_rows=text_rows, frame_rows=frame_rows, n_bank=n_bank,
                              audio_rows=audio_rows, history_rows=history_k.shape[1],
                              chunk_rows=chunk_rows)
    outs = []
    for qs, qe, ivs in segs:
        kq = torch.cat([keys[:, a:b] for a, b in ivs], dim=1)
        vq = torch.cat([values[:, a:b] for a, b in ivs], dim=1)
        outs.append(attention(q[:, qs:qe], kq, vq, **kw))
    return torch.cat(outs, dim=1)

