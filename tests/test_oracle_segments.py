"""Pins oracle/segments_ref.py: the teacher-forcing mask's two restatements agree, hand cases,
the H3 chunk-list cache rules and the segment layouts against dense masked attention."""

import pytest
import torch

from oracle import segments_ref as sr

F64 = torch.float64


@pytest.mark.parametrize("F,T,nb,sink,m", [
    (6, 3, 1, 0, None), (6, 3, 2, 2, None), (6, 2, 2, 2, 1), (9, 2, 3, 3, 1), (6, 4, 3, 0, 0),
    (8, 1, 2, 2, 0),
])
def test_tf_mask_equals_segment_intervals(F, T, nb, sink, m):
    kw = dict(num_frames=F, frame_seqlen=T, num_frame_per_block=nb, max_prior_clean_chunks=m,
              sink_size=sink)
    dense = sr.teacher_forcing_mask(**kw)
    segs = sr.teacher_forcing_segments(**kw)
    assert torch.equal(dense, sr.segment_mask(2 * F * T, segs))
    bs, clean_end = nb * T, F * T
    for c in range(F // nb):  # noisy chunk c never sees clean chunk c (no target leak)
        rows = slice(clean_end + c * bs, clean_end + (c + 1) * bs)
        assert not dense[rows, c * bs : (c + 1) * bs].any()
        assert dense[rows, clean_end + c * bs : clean_end + (c + 1) * bs].all()  # sees itself


def test_tf_mask_hand_case():
    """F=3, T=1, one frame per chunk, no sink, full prefix: clean i sees clean 0..i; noisy i sees
    clean 0..i-1 and noisy i."""
    m = sr.teacher_forcing_mask(num_frames=3, frame_seqlen=1, num_frame_per_block=1)
    want = torch.tensor([
        [1, 0, 0, 0, 0, 0],
        [1, 1, 0, 0, 0, 0],
        [1, 1, 1, 0, 0, 0],
        [0, 0, 0, 1, 0, 0],
        [1, 0, 0, 0, 1, 0],
        [1, 1, 0, 0, 0, 1],
    ], dtype=torch.bool)
    assert torch.equal(m, want)
    # a bounded window with a sink: max one prior clean chunk, sink = first chunk
    m = sr.teacher_forcing_mask(num_frames=4, frame_seqlen=1, num_frame_per_block=1,
                                max_prior_clean_chunks=1, sink_size=1)
    assert m[3].tolist() == [True, False, True, True, False, False, False, False]  # sink + recent
    assert m[7].tolist() == [True, False, True, False, False, False, False, True]


def test_tf_geometry_errors():
    with pytest.raises(ValueError):
        sr.teacher_forcing_mask(num_frames=5, frame_seqlen=1, num_frame_per_block=2)
    with pytest.raises(ValueError):
        sr.teacher_forcing_mask(num_frames=4, frame_seqlen=1, num_frame_per_block=2, sink_size=1)
    with pytest.raises(ValueError):
        sr.teacher_forcing_mask(num_frames=4, frame_seqlen=1, num_frame_per_block=1,
                                max_prior_clean_chunks=4)


def _kv(n, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(1, n, 2, 8, generator=g, dtype=F64)


def test_h3_cache_window_and_gaps():
    c = sr.H3RawKVCache()
    assert c.history(0, 0) == []
    for i in range(8):
        c.commit(0, i, _kv(2, i), _kv(2, 100 + i))
    assert [e[0] for e in c.history(0, 8)] == [3, 4, 5, 6, 7]
    with pytest.raises(RuntimeError):
        c.history(0, 7)  # chunk 7 is already committed: the window does not end at 6
    with pytest.raises(RuntimeError):
        c.commit(1, 2, _kv(2, 0), _kv(2, 0))  # layer 1 never saw chunks 0, 1


def test_windowed_attention_is_dense_attention_over_the_window():
    c = sr.H3RawKVCache()
    pk, pv = _kv(3, 1), _kv(3, 2)
    att = dict(round_inputs_to_bf16=False)
    for i in range(3):
        c.commit(0, i, _kv(4, 10 + i), _kv(4, 20 + i))
    q, k, v = _kv(4, 30), _kv(4, 31), _kv(4, 32)
    got = sr.windowed_rollout_attention(q, k, v, pk, pv, c, 0, 3, commit=True, **att)
    keys = torch.cat([pk, _kv(4, 10), _kv(4, 11), _kv(4, 12), k], 1)
    vals = torch.cat([pv, _kv(4, 20), _kv(4, 21), _kv(4, 22), v], 1)
    assert torch.allclose(got, sr.attention(q, keys, vals, **att))
    assert [e[0] for e in c.history(0, 4)] == [0, 1, 2, 3]


@pytest.mark.parametrize("n_bank,audio", [(2, 3), (0, 0), (1, 0)])
def test_memory_kv_segments_match_masked_attention(n_bank, audio):
    text, rows, chunk = 5, 4, 8
    prefix = text + rows + n_bank * rows + audio
    q, k, v = _kv(prefix + chunk, 40), _kv(prefix + chunk, 41), _kv(prefix + chunk, 42)
    hk, hv = _kv(6, 43), _kv(6, 44)
    att = dict(round_inputs_to_bf16=False)
    got = sr.memory_kv_attention(q, k, v, hk, hv, text_rows=text, frame_rows=rows, n_bank=n_bank,
                                 audio_rows=audio, **att)
    keys = torch.cat([k[:, :prefix], hk, k[:, prefix:]], 1)
    vals = torch.cat([v[:, :prefix], hv, v[:, prefix:]], 1)
    segs = sr.memory_kv_segments(text_rows=text, frame_rows=rows, n_bank=n_bank, audio_rows=audio,
                                 history_rows=6, chunk_rows=chunk)
    mask = torch.zeros(prefix + chunk, keys.shape[1], dtype=torch.bool)
    for qs, qe, ivs in segs:
        for a, b in ivs:
            mask[qs:qe, a:b] = True
    assert mask.any(dim=1).all()  # every query row belongs to exactly one segment
    assert torch.allclose(got, sr.masked_attention(q, keys, vals, mask, **att))
    # the shared rows never see the bank, audio, history or the chunk
    assert not mask[: text + rows, text + rows :].any()
