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


def _segment_case(T, n_seg, seed, ragged):
    """Random consecutive segments: ragged row counts, lists that repeat slots in any order, and
    (``ragged``) frame lengths below T."""
    g = torch.Generator().manual_seed(seed)
    segs = []
    for _ in range(n_seg):
        rows = int(torch.randint(1, 700, (1,), generator=g))
        nf = int(torch.randint(1, 9, (1,), generator=g))
        frames = torch.randint(0, 12, (nf,), generator=g).tolist()
        lens = torch.randint(1, T + 1, (nf,), generator=g).tolist() if ragged else None
        segs.append((rows, frames, lens))
    return segs


@pytest.mark.parametrize("T,qdt,ragged,n_seg", [(64, BF, False, 5), (136, BF, False, 7),
                                                (136, torch.float32, False, 3),
                                                (100, BF, True, 6), (64, torch.float32, True, 4)])
def test_one_launch_for_segments(gpu, T, qdt, ragged, n_seg):
    """attention_frames(segments=...) against the oracle per segment and against one plain launch
    per segment (the unsplit kernel): T = 136 takes packed key tiles, T = 64 / ragged lengths
    frame-aligned ones; rows not multiples of 256 leave partly filled q-tiles in every segment."""
    _say("one launch for segments", T, qdt, ragged, n_seg)
    B, H = 2, 3
    segs = _segment_case(T, n_seg, 1000 + T + n_seg, ragged)
    L = sum(r for r, _, _ in segs)
    k, v = _rand((B, 12 * T, H, 128), 30), _rand((B, 12 * T, H, 128), 31)
    q = _rand((B, L, H, 128), 32).to(qdt)
    kp, vp, _, _ = kernels.new_pools(12, B, H, T, BF, gpu)
    kernels.append_frames(k.to(gpu), v.to(gpu), kp, vp, list(range(12)), frame_tokens=T)
    frames = [f for _, fr, _ in segs for f in fr]
    lens = [x for _, fr, ln in segs for x in (ln or [T] * len(fr))] if ragged else None
    qd = q.to(gpu)
    got = kernels.attention_frames(qd, kp, vp, frames, frame_tokens=T, frame_lens=lens,
                                   segments=[(r, len(fr)) for r, fr, _ in segs])
    per = torch.empty_like(qd)
    r0 = 0
    for rows, fr, ln in segs:
        kernels.attention_frames(qd[:, r0:r0 + rows], kp, vp, fr, frame_tokens=T, frame_lens=ln,
                                 out=per[:, r0:r0 + rows], use_workspace=False)
        r0 += rows
    torch.cuda.synchronize()
    got, per = got.cpu(), per.cpu()
    r0 = 0
    for rows, fr, ln in segs:
        ln = ln or [T] * len(fr)
        keys = torch.cat([k[:, f * T:f * T + n] for f, n in zip(fr, ln)], 1)
        vals = torch.cat([v[:, f * T:f * T + n] for f, n in zip(fr, ln)], 1)
        want = sr.attention(q[:, r0:r0 + rows].float(), keys.float(), vals.float())
        assert_attn_close(got[:, r0:r0 + rows], want)
        r0 += rows
    assert_attn_close(got, per.double(), max_abs=1e-2, mean_abs=5e-4)


def test_segment_groups_beyond_one_launch(gpu):
    """attend_segments splits runs of segments at the launch limits (64 segments, 256 listed
    frames) and keeps float32 pools on one launch per segment; results match one plain launch
    per segment."""
    from solarwm_amd.segments import attend_segments

    _say("segment groups")
    T, H = 64, 2
    g = torch.Generator().manual_seed(77)
    segs = [(int(torch.randint(1, 90, (1,), generator=g)),
             torch.randint(0, 12, (int(torch.randint(1, 12, (1,), generator=g)),), generator=g).tolist(),
             None) for _ in range(90)]
    assert sum(len(f) for _, f, _ in segs) > 256 and len(segs) > 64
    L = sum(r for r, _, _ in segs)
    k, v = _rand((1, 12 * T, H, 128), 40), _rand((1, 12 * T, H, 128), 41)
    q = _rand((1, L, H, 128), 42).to(gpu)
    for dt in (BF, torch.float32):
        kp, vp, _, _ = kernels.new_pools(12, 1, H, T, dt, gpu)
        kernels.append_frames(k.to(gpu).to(dt), v.to(gpu).to(dt), kp, vp, list(range(12)),
                              frame_tokens=T)
        got = attend_segments(q, kp, vp, segs, frame_tokens=T)
        per = torch.empty_like(q)
        r0 = 0
        for rows, fr, _ in segs:
            kernels.attention_frames(q[:, r0:r0 + rows], kp, vp, fr, frame_tokens=T,
                                     out=per[:, r0:r0 + rows], use_workspace=False)
            r0 += rows
        torch.cuda.synchronize()
        assert_attn_close(got, per.cpu().double(), max_abs=1e-2, mean_abs=5e-4)
    with pytest.raises(ValueError, match="segments cover"):
        attend_segments(q[:, :-1], kp, vp, segs, frame_tokens=T)
    with pytest.raises(ValueError, match="bfloat16 pools"):
        kernels.attention_frames(q[:, :10], kp, vp, [0, 1], frame_tokens=T, segments=[(5, 1), (5, 1)])


def test_teacher_forcing_long_rollout(gpu):
    """21 frames in chunks of 3 with a 3-frame sink: 14 segments and 168 listed frames in one
    launch, against the dense-mask oracle."""
    _say("teacher forcing 21 frames")
    F, T, nb, H = 21, 64, 3, 2
    L = 2 * F * T
    q, k, v = _rand((1, L, H, 128), 51), _rand((1, L, H, 128), 52), _rand((1, L, H, 128), 53)
    kw = dict(num_frames=F, frame_seqlen=T, num_frame_per_block=nb, max_prior_clean_chunks=None,
              sink_size=3)
    got = teacher_forcing_attention(q.to(gpu), k.to(gpu), v.to(gpu), **kw)
    want = sr.masked_attention(q, k, v, sr.teacher_forcing_mask(**kw))
    torch.cuda.synchronize()
    assert_attn_close(got, want)
