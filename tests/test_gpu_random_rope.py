"""Seeded random shapes for RoPE on load (pre-RoPE caches, a height/width-roped K copy, Q rotated
per key frame) against the oracle's float64 restatement of the reference's window RoPE
(causal_model.py:791-876, :88-197) and attention (attention.py:141-188).

Each case draws a latent grid (frames of gh x gw tokens, most of them not a multiple of 64, so the
last tile of every frame is masked), a set of distinct key-frame positions in shuffled slots,
query-frame positions, heads, the query dtype, and runs with and without the caller workspace (the
launcher may split the keys over all CUs).  Bars: tests/helpers.py.

fp8 pre-RoPE caches: the same draws with bf16 queries, K/V with or without x20 outlier channels
and, in some cases, the query RMSNorm folded into the load; frames of at least 64 tokens run on
the fp8 matrix cores and are checked against ``fp8_rope_attention`` (the kernel's per-key-frame
e4m3 query, reproduced code for code) with the normalised fp8 bars, shorter frames run the
bf16-decode kernel and are checked against the float64 RoPE path over the decoded copies with the
bars of tests/test_gpu_fp8_rope.py."""

import random

import pytest
import torch

from oracle import wan_cache_ref as ref
from solarwm_amd import kernels, rope

from .helpers import FP8_NORM_MAX, FP8_NORM_MEAN, assert_attn_close

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


FP8_GRIDS = GRIDS + [(5, 9), (4, 12)]  # 45- and 48-token frames: the bf16-decode kernel


def _fp8_case(seed):
    r = random.Random(3000 + seed)
    gh, gw = r.choice(FP8_GRIDS)
    T = gh * gw
    n = r.randint(1, max(1, min(12, 9000 // T)))
    kpos = sorted(r.sample(range(n + 4), n))
    nq = r.randint(1, min(3, n))
    qpos = kpos[-nq:]
    H = r.choice([1, 2, 3])
    return gh, gw, kpos, qpos, H, r.random() < 0.5, r.random() < 0.3, r.randrange(1 << 30)


@pytest.mark.parametrize("seed", range(10))
def test_random_fp8_rope_shape_vs_oracle(gpu, seed):
    from .test_gpu_fp8_rope import FP8_BF16_MAX, FP8_BF16_MEAN

    gh, gw, kpos, qpos, H, outliers, norm, s = _fp8_case(seed)
    print("fp8 rope case", seed, dict(grid=(gh, gw), kpos=kpos, qpos=qpos, H=H, outliers=outliers,
                                      q_norm=norm), flush=True)
    T = gh * gw
    n, nq = len(kpos), len(qpos)
    g = torch.Generator().manual_seed(s)
    q = torch.randn((1, nq * T, H, 128), generator=g).to(torch.bfloat16)
    k = torch.randn((1, n * T, H, 128), generator=g)
    v = torch.randn((1, n * T, H, 128), generator=g)
    if outliers:  # one x20 channel (the data the bf16-decode bars are stated for)
        for x in (k, v):
            x[..., torch.randperm(128, generator=g)[:1]] *= 20.0
    k, v = k.to(torch.bfloat16), v.to(torch.bfloat16)
    cfg = rope.RopeConfig(grid_hw=(gh, gw))
    hw = rope.spatial_table(cfg, gpu)
    slots = torch.randperm(n + 2, generator=g)[:n].tolist()
    kp, vp, ks, vs = kernels.new_pools(n + 2, 1, H, T, torch.float8_e4m3fn, gpu)
    krp, krs = torch.zeros_like(kp), torch.zeros_like(ks)
    kd, vd = k.to(gpu), v.to(gpu)
    for j in range(n):
        kernels.append_frames(kd, vd, kp, vp, [slots[j]], frame_tokens=T, src_frame0=j, kscale=ks,
                              vscale=vs, kr_pool=krp, rope_hw=hw, grid_hw=(gh, gw), kr_scale=krs)
    tt = rope.temporal_table(qpos, kpos, cfg, gpu)
    qd = q.to(gpu)
    args = dict(frame_tokens=T, kscale=krs, vscale=vs, rope=(hw, (gh, gw), tt))
    qq = q
    if norm:  # the query as the kernel normalises it: bf16((q * inv_rms) * w), fp32 products
        w = (torch.rand(H * 128, generator=g) + 0.5).to(torch.bfloat16).float()
        inv = kernels.rms_rows(qd, 1e-6)
        args["q_norm"] = (inv, w.to(gpu))
        qq = ((q.float() * inv.cpu()[..., None, None]) * w.view(H, 128)).to(torch.bfloat16)
    f = ref.wan_rope_freqs()
    v_eff = ref.fp8_fake_quant_frames(v.float(), T).double()
    if T >= 64:
        want = ref.fp8_rope_attention(qq, ref.fp8_rope_copy_decoded(k, (gh, gw), f, T), v_eff,
                                      (gh, gw), qpos, kpos, T)
        bars = (FP8_NORM_MAX, FP8_NORM_MEAN)
    else:
        want = ref.attention(ref.rope_frames(qq, (gh, gw), qpos, f),
                             ref.rope_frames(ref.fp8_rope_copy_effective(k, (gh, gw), f, T),
                                             (gh, gw), kpos, f), v_eff)
        bars = (FP8_BF16_MAX, FP8_BF16_MEAN)
    rms_v = v_eff.pow(2).mean(dim=1, keepdim=True).sqrt().clamp_min(1e-6)
    for ws in (True, False):
        out = kernels.attention_frames(qd, krp, vp, slots, use_workspace=ws, **args)
        if T < 64:  # the bf16-decode kernel: bit-identical to the bf16 kernel on decoded pools
            dec = dict(args, kscale=None, vscale=None)
            base = kernels.attention_frames(qd, (krp.float() * krs[..., None, None]).to(torch.bfloat16),
                                            (vp.float() * vs[..., None, None]).to(torch.bfloat16),
                                            slots, use_workspace=ws, **dec)
            assert torch.equal(out, base)
        torch.cuda.synchronize()
        assert out.dtype == torch.bfloat16 and torch.isfinite(out).all()
        e = (out.cpu().double() - want).abs() / rms_v
        print(f"  workspace {ws}: normalised max {float(e.max()):.3e} mean {float(e.mean()):.3e}",
              flush=True)
        assert float(e.max()) <= bars[0] and float(e.mean()) <= bars[1]
