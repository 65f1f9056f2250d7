"""Seeded random shapes for the bf16 / f16 attention kernels against the float64 oracle
(oracle/wan_cache_ref.py attention, attention.py:141-188 of the reference).

Each case draws a frame size (multiples of 8 that pack key tiles across frames, and sizes that do
not, odd ones included: 135 and the release geometry's 405), a window of frames stored in
shuffled slots of a larger pool, a query count (one row, ragged q-tiles, under-filled grids that
take the balanced key split), heads, streams, the pool
dtype and the mask (none, or chunk-causal with the chunk limit anywhere in the window).  The
launch plan's key-tile count is checked against the packing rule, so the cases cover both tile
walks.  Bars: tests/helpers.py."""

import random

import pytest
import torch

from oracle import wan_cache_ref as ref
from solarwm_amd import _lib, kernels

from .helpers import assert_attn_close

pytestmark = pytest.mark.gpu

FRAME_SIZES = [64, 72, 96, 100, 135, 136, 200, 256, 390, 405, 520, 880, 1000, 1560]
Q_LENS = [1, 37, 130, 256, 600, 1170]


def _case(seed):
    r = random.Random(seed)
    T = r.choice(FRAME_SIZES)
    n = r.randint(1, max(1, 12000 // T))
    H = r.choice([1, 2, 3])
    B = r.choice([1, 2])
    Lq = r.choice(Q_LENS)
    pool = r.choice([torch.bfloat16, torch.bfloat16, torch.float16])
    qdt = r.choice([torch.bfloat16, torch.float32]) if pool == torch.bfloat16 else r.choice(
        [torch.float16, torch.float32])
    causal = r.random() < 0.35
    # keep the float64 oracle within about a second
    while Lq * n * T * H * B > 2.5e7 and Lq > 1:
        Lq = Q_LENS[max(0, Q_LENS.index(Lq) - 1)]
    return T, n, H, B, Lq, pool, qdt, causal, r.randrange(1 << 30)


@pytest.mark.parametrize("seed", range(32))
def test_random_shape_vs_oracle(gpu, seed):
    T, n, H, B, Lq, pool, qdt, causal, s = _case(seed)
    print("case", seed, dict(T=T, n=n, H=H, B=B, Lq=Lq, pool=pool, q=qdt, causal=causal), flush=True)
    g = torch.Generator().manual_seed(s)
    q = torch.randn((B, Lq, H, 128), generator=g).to(qdt)
    k = torch.randn((B, n * T, H, 128), generator=g).to(pool)
    v = torch.randn((B, n * T, H, 128), generator=g).to(pool)
    n_slots = n + 3
    slots = torch.randperm(n_slots, generator=g)[:n].tolist()
    kp, vp, _, _ = kernels.new_pools(n_slots, B, H, T, pool, gpu)
    kd, vd = k.to(gpu), v.to(gpu)
    for f in range(n):
        kernels.append_frames(kd, vd, kp, vp, [slots[f]], frame_tokens=T, src_frame0=f)
    kw = {}
    mask = None
    if causal:
        L = n * T
        chunk = T * random.Random(s).randint(1, n)
        q0 = random.Random(s + 1).randint(0, max(0, L - Lq))
        kw = dict(mask_mode=_lib.SKV_MASK_CHUNK_CAUSAL, q_pos0=q0, chunk_tokens=chunk)
        pos = torch.arange(q0, q0 + Lq)[:, None]
        lim = torch.clamp((pos // chunk + 1) * chunk, max=L)
        mask = torch.arange(L)[None, :] < lim
    qd = q.to(gpu)
    plan = kernels.attention_plan(qd, kp, vp, slots, frame_tokens=T, **kw)
    packed = T % 8 == 0 and T % 64 != 0
    want_tiles = -(-n * T // 64) if packed else n * -(-T // 64)
    assert plan["key_tiles"] == want_tiles, plan
    out = kernels.attention_frames(qd, kp, vp, slots, frame_tokens=T, **kw)
    torch.cuda.synchronize()
    assert out.dtype == qdt
    assert_attn_close(out, ref.attention(q, k.to(qdt), v.to(qdt), mask=mask))
