"""GPU parity of segmented attention on the frame-slot kernel against oracle/segments_ref.py:
the teacher-forcing mask (causal_model.py:337-471), H3's chunk-list rollout window
(sgf_attention.py:40-63, :236-258) and H3's memory-KV segments (memory_kv_attention.py:39-140),
including spans that are not whole frames (per-frame key lengths).  Bars: tests/helpers.py."""

import pytest
import torch

from oracle import segments_ref as sr
from solarwm_amd import kernels
from solarwm_amd.segments import (ChunkListKVCache, memory_kv_attention, teacher_forcing_attention,
                                  windowed_attention)

from .helpers import assert_attn_close

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _say(*a):
    print(*a, flush=True)


def _rand(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(BF)


@pytest.mark.parametrize("F,T,nb,sink,m", [(6, 64, 2, 0, None), (6, 64, 2, 2, 1), (9, 100, 3, 3, 1),
                                           (4, 64, 1, 0, 0)])
def test_teacher_forcing_attention(gpu, F, T, nb, sink, m):
    _say("teacher forcing", F, T, nb, sink, m)
    L, H = 2 * F * T, 2
    q, k, v = _rand((1, L, H, 128), 1), _rand((1, L, H, 128), 2), _rand((1, L, H, 128), 3)
    kw = dict(num_frames=F, frame_seqlen=T, num_frame_per_block=nb, max_prior_clean_chunks=m,
              sink_size=sink)
    got = teacher_forcing_attention(q.to(gpu), k.to(gpu), v.to(gpu), **kw)
    want = sr.masked_attention(q, k, v, sr.teacher_forcing_mask(**kw))
    torch.cuda.synchronize()
    assert_attn_close(got, want)


def test_windowed_rollout_with_ragged_prefix(gpu):
    _say("h3 windowed rollout")
    T, H, cf = 64, 2, 5
    cache = ChunkListKVCache(num_layers=2, batch=1, heads=H, frame_tokens=T, chunk_frames=cf,
                             window=5, span_frames=4, device=gpu)
    oc = sr.H3RawKVCache()
    pk, pv = _rand((1, 150, H, 128), 4), _rand((1, 150, H, 128), 5)  # 2 whole frames + 22 rows
    for c in range(8):
        q, k, v = (_rand((1, cf * T, H, 128), 10 * c + i) for i in range(3))
        got = windowed_attention(q.to(gpu), k.to(gpu), v.to(gpu), cache, 1, c,
                                 prefix=(pk.to(gpu), pv.to(gpu)), commit=True)
        want = sr.windowed_rollout_attention(q, k, v, pk, pv, oc, 1, c, commit=True)
        torch.cuda.synchronize()
        assert_attn_close(got, want)
    assert [e[0] for e in cache.history(1, 8)] == [3, 4, 5, 6, 7]
    with pytest.raises(RuntimeError):
        cache.history(0, 3)


@pytest.mark.parametrize("n_bank,audio_rows", [(2, 70), (0, 0)])
def test_memory_kv_attention(gpu, n_bank, audio_rows):
    _say("h3 memory kv", n_bank, audio_rows)
    T, H, cf, text = 64, 2, 5, 100
    cache = ChunkListKVCache(num_layers=1, batch=1, heads=H, frame_tokens=T, chunk_frames=cf,
                             window=5, span_frames=8, device=gpu)
    oc = sr.H3RawKVCache()
    prefix = text + T + n_bank * T + audio_rows
    for c in range(3):
        q, k, v = (_rand((1, prefix + cf * T, H, 128), 100 + 10 * c + i) for i in range(3))
        got = memory_kv_attention(q.to(gpu), k.to(gpu), v.to(gpu), cache, 0, c, text_rows=text,
                                  n_bank=n_bank, audio_rows=audio_rows, commit=True)
        hist = oc.history(0, c)
        hk = torch.cat([e[1] for e in hist], 1) if hist else k[:, :0]
        hv = torch.cat([e[2] for e in hist], 1) if hist else v[:, :0]
        want = sr.memory_kv_attention(q, k, v, hk, hv, text_rows=text, frame_rows=T, n_bank=n_bank,
                                      audio_rows=audio_rows)
        oc.commit(0, c, k[:, prefix:], v[:, prefix:])
        torch.cuda.synchronize()
        assert_attn_close(got, want)


def test_ragged_frames_mask_past_their_length(gpu):
    """frame_lens: keys past a frame's length do not count, even when the slot holds data there."""
    _say("ragged frames")
    T, H = 128, 2
    k, v = _rand((1, 3 * T, H, 128), 20), _rand((1, 3 * T, H, 128), 21)
    q = _rand((1, 200, H, 128), 22)
    kp, vp, _, _ = kernels.new_pools(3, 1, H, T, BF, gpu)
    kernels.append_frames(k.to(gpu), v.to(gpu), kp, vp, [0, 1, 2], frame_tokens=T)
    got = kernels.attention_frames(q.to(gpu), kp, vp, [2, 0, 1], frame_tokens=T, frame_lens=[5, 128, 70])
    keys = torch.cat([k[:, 2 * T : 2 * T + 5], k[:, :T], k[:, T : T + 70]], 1)
    vals = torch.cat([v[:, 2 * T : 2 * T + 5], v[:, :T], v[:, T : T + 70]], 1)
    torch.cuda.synchronize()
    assert_attn_close(got, sr.attention(q, keys, vals))
    with pytest.raises(ValueError):  # ragged frames cannot be combined with the chunk-causal mask
        kernels.attention_frames(q.to(gpu), kp, vp, [0, 1], frame_tokens=T, frame_lens=[5, 128],
                                 mask_mode=1, chunk_tokens=64)
