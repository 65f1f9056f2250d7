"""GPU parity of packed key tiles: with whole bf16 / f16 frames of T = 8k tokens (T not a multiple
of 64), attn_kernel runs its 64-key tiles across frame boundaries (a tile's first keys from the
end of one frame, the rest from the start of the next frame's slot) instead of padding every
frame to whole tiles.  Checked against the float64 oracle (oracle/wan_cache_ref.py attention,
attention.py:141-188 of the reference) with frames stored in shuffled, non-adjacent slots:

* T = 72 (nearly every tile straddles two frames), 200, 136 and C2's 1560, bf16 / f32 queries;
* f16 pools with f16 queries;
* the chunk-causal mask with chunk limits inside straddling tiles;
* the balanced key split over packed tiles (segments that start and end inside straddling tiles);
* a window whose last tile is partial (keys past the window are masked).

Each case asserts through ``skv_attention_plan`` that the launch packs its tiles
(``key_tiles == ceil(n * T / 64)``).  Bars: tests/helpers.py."""

import pytest
import torch

from oracle import wan_cache_ref as ref
from solarwm_amd import _lib, kernels

from .helpers import assert_attn_close

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _rand(shape, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype)


def _pools(k, v, T, dtype, gpu, seed=0):
    """Frames f of dense K/V in shuffled slots with a free slot between most neighbours."""
    B, L, H, _ = k.shape
    n = L // T
    g = torch.Generator().manual_seed(seed)
    slots = torch.randperm(2 * n + 1, generator=g)[:n].tolist()
    kp, vp, _, _ = kernels.new_pools(2 * n + 1, B, H, T, dtype, gpu)
    kd, vd = k.to(gpu), v.to(gpu)
    for f in range(n):
        kernels.append_frames(kd, vd, kp, vp, [slots[f]], frame_tokens=T, src_frame0=f)
    return kp, vp, slots


def _packed(q, kp, vp, slots, T, **kw):
    plan = kernels.attention_plan(q, kp, vp, slots, frame_tokens=T, **kw)
    assert plan["key_tiles"] == -(-len(slots) * T // 64), plan
    return plan


@pytest.mark.parametrize("B,H,Lq,T,n,qdt,pdt", [
    (1, 2, 300, 72, 7, torch.bfloat16, torch.bfloat16),    # 504 keys in 8 tiles, not 14
    (2, 3, 257, 200, 5, torch.bfloat16, torch.bfloat16),
    (1, 2, 1000, 1560, 4, torch.bfloat16, torch.bfloat16),  # C2 frames: 98 tiles, not 100
    (1, 3, 100, 136, 3, torch.float32, torch.bfloat16),
    (1, 2, 300, 72, 7, torch.float16, torch.float16),
    (2, 2, 130, 200, 4, torch.float32, torch.float16),
])
def test_packed_tiles_vs_oracle(gpu, B, H, Lq, T, n, qdt, pdt):
    _say("packed tiles", B, H, Lq, T, n, qdt, pdt)
    q = _rand((B, Lq, H, 128), 1, qdt)
    k, v = _rand((B, n * T, H, 128), 2, pdt), _rand((B, n * T, H, 128), 3, pdt)
    kp, vp, slots = _pools(k, v, T, pdt, gpu)
    qd = q.to(gpu)
    _packed(qd, kp, vp, slots, T)
    out = kernels.attention_frames(qd, kp, vp, slots, frame_tokens=T)
    torch.cuda.synchronize()
    assert out.dtype == qdt
    assert_attn_close(out, ref.attention(q, k.to(qdt), v.to(qdt)))


@pytest.mark.parametrize("clean,noisy,T,per_block", [(2, 2, 136, 2), (1, 3, 200, 3), (3, 3, 72, 3)])
def test_packed_chunk_causal(gpu, clean, noisy, T, per_block):
    """The chunk-causal limits (multiples of T * per_block keys) fall inside straddling tiles."""
    _say("packed chunk-causal", clean, noisy, T, per_block)
    L = (clean + noisy) * T
    q = _rand((1, L, 2, 128), 7, torch.bfloat16)
    k = _rand((1, L, 2, 128), 8, torch.bfloat16)
    v = _rand((1, L, 2, 128), 9, torch.bfloat16)
    dense, _ = ref.inference_window_mask(clean, noisy, T, per_block)
    want = ref.attention(q, k, v, mask=dense[:L, :L])
    kp, vp, slots = _pools(k, v, T, torch.bfloat16, gpu)
    chunk = T * per_block
    for q0 in range(0, L, chunk):  # every block of queries, each against its own limits
        Lq = min(chunk, L - q0)
        qd = q[:, q0 : q0 + Lq].to(gpu)
        kw = dict(mask_mode=_lib.SKV_MASK_CHUNK_CAUSAL, q_pos0=q0, chunk_tokens=chunk)
        _packed(qd, kp, vp, slots, T, **kw)
        got = kernels.attention_frames(qd, kp, vp, slots, frame_tokens=T, **kw)
        torch.cuda.synchronize()
        assert_attn_close(got, want[:, q0 : q0 + Lq])


@pytest.mark.parametrize("H,Lq,T,n", [(16, 200, 72, 60), (2, 256, 1560, 21)])
def test_packed_split(gpu, H, Lq, T, n):
    """Balanced key split over packed tiles: 16 heads x 68 tiles of 72-token frames, and the C2
    window (512 tiles) for two heads; shares start and end inside straddling tiles."""
    _say("packed split", H, Lq, T, n)
    q = _rand((1, Lq, H, 128), 11, torch.bfloat16)
    k, v = _rand((1, n * T, H, 128), 12, torch.bfloat16), _rand((1, n * T, H, 128), 13, torch.bfloat16)
    kp, vp, slots = _pools(k, v, T, torch.bfloat16, gpu)
    qd = q.to(gpu)
    plan = _packed(qd, kp, vp, slots, T)
    assert plan["split"] == 1, plan
    out = kernels.attention_frames(qd, kp, vp, slots, frame_tokens=T)
    plain = kernels.attention_frames(qd, kp, vp, slots, frame_tokens=T, use_workspace=False)
    torch.cuda.synchronize()
    want = ref.attention(q, k, v)
    assert_attn_close(out, want)
    assert_attn_close(plain, want)
