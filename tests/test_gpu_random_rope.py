"""Seeded random shapes for RoPE on load (pre-RoPE caches, a height/width-roped K copy, Q rotated
per key frame) against the oracle's float64 restatement of the reference's window RoPE
(causal_model.py:791-876, :88-197) and attention (attention.py:141-188).

Each case draws a latent grid (frames of gh x gw tokens, most of them not a multiple of 64, so the
last tile of every frame is masked), a set of distinct key-frame positions in shuffled slots,
query-frame positions, heads, the query dtype, and runs with and without the caller workspace (the
launcher may split the keys over all CUs).  Bars: tests/helpers.py."""

import random

import pytest
import torch

from oracle import wan_cache_ref as ref
from solarwm_amd import kernels, rope

from .helpers import assert_attn_close

pytestmark = pytest.mark.gpu

GRIDS = [(8, 8), (6, 11), (10, 10), (13, 7), (15, 26), (30, 52)]


def _case(seed):
    r = random.Random(2000 + seed)
    gh, gw = r.choice(GRIDS)
    T = gh * gw
    n = r.randint(1, max(1, min(12, 9000 // T)))
    kpos = sorted(r.sample(range(n + 4), n))
    nq = r.randint(1, min(3, n))
    qpos = kpos[-nq:]
    H = r.choice([1, 2, 3])
    dtype = r.choice([torch.bfloat16, torch.bfloat16, torch.float32])
    return gh, gw, kpos, qpos, H, dtype, r.randrange(1 << 30)


@pytest.mark.parametrize("seed", range(10))
def test_random_rope_shape_vs_oracle(gpu, seed):
    gh, gw, kpos, qpos, H, dtype, s = _case(seed)
    print("rope case", seed, dict(grid=(gh, gw), kpos=kpos, qpos=qpos, H=H, q=dtype), flush=True)
    T = gh * gw
    n, nq = len(kpos), len(qpos)
    g = torch.Generator().manual_seed(s)
    q = torch.randn((1, nq * T, H, 128), generator=g).to(dtype)
    k = torch.randn((1, n * T, H, 128), generator=g).to(torch.bfloat16)
    v = torch.randn((1, n * T, H, 128), generator=g).to(torch.bfloat16)
    f = ref.wan_rope_freqs()
    want = ref.attention(ref.rope_frames(q, (gh, gw), qpos, f), ref.rope_frames(k, (gh, gw), kpos, f), v)
    cfg = rope.RopeConfig(grid_hw=(gh, gw))
    hw = rope.spatial_table(cfg, gpu)
    slots = torch.randperm(n + 2, generator=g)[:n].tolist()
    kp, vp, _, _ = kernels.new_pools(n + 2, 1, H, T, torch.bfloat16, gpu)
    krp = torch.zeros_like(kp)
    kd, vd = k.to(gpu), v.to(gpu)
    for j in range(n):
        kernels.append_frames(kd, vd, kp, vp, [slots[j]], frame_tokens=T, src_frame0=j,
                              kr_pool=krp, rope_hw=hw, grid_hw=(gh, gw))
    tt = rope.temporal_table(qpos, kpos, cfg, gpu)
    qd = q.to(gpu)
    for ws in (True, False):
        out = kernels.attention_frames(qd, krp, vp, slots, frame_tokens=T, use_workspace=ws,
                                       rope=(hw, (gh, gw), tt))
        torch.cuda.synchronize()
        assert out.dtype == dtype
        assert_attn_close(out, want)
