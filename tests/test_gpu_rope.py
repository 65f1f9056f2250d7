"""GPU parity of RoPE on load (pre-RoPE caches) against the oracle's float64 restatement of the
reference's window RoPE (causal_model.py:791-876, :88-197).

Bars: raw pools bit-exact; the height/width-roped K copy within one bf16 rounding of the float64
rotation; attention within the bf16 bars of tests/helpers.py.
"""

import pytest
import torch

from oracle import wan_cache_ref as ref
from solarwm_amd import apply_cache_updates, attend_cached, kernels, make_kv_cache_allocator, rope

from .helpers import assert_attn_close

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _say(*a):
    print(*a, flush=True)


def _rand(shape, seed, dtype=BF):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype)


@pytest.mark.parametrize("gh,gw", [(8, 8), (10, 10), (30, 52)])
def test_append_rope_copy(gpu, gh, gw):
    _say("append rope", gh, gw)
    T, H = gh * gw, 3
    k, v = _rand((1, 2 * T, H, 128), 1), _rand((1, 2 * T, H, 128), 2)
    cfg = rope.RopeConfig(grid_hw=(gh, gw))
    hw = rope.spatial_table(cfg, gpu)
    kp, vp, _, _ = kernels.new_pools(4, 1, H, T, BF, gpu)
    krp = torch.full_like(kp, 7.0)
    kernels.append_frames(k.to(gpu), v.to(gpu), kp, vp, [2, 0], frame_tokens=T, kr_pool=krp,
                          rope_hw=hw, grid_hw=(gh, gw))
    torch.cuda.synchronize()
    f = ref.wan_rope_freqs()
    Tp = kernels.padded_tokens(T)
    for i, s in enumerate([2, 0]):
        frame = k[:, i * T : (i + 1) * T]
        assert torch.equal(kp[s, :, :, :T].permute(0, 2, 1, 3).cpu(), frame)  # raw K untouched
        want = ref.rope_frames(frame, (gh, gw), [0], f).float()  # temporal position 0
        got = krp[s, :, :, :T].permute(0, 2, 1, 3).cpu().float()
        diff = (got - want).abs()
        assert bool((diff <= want.abs() * 2.0**-7 + 1e-30).all()), float(diff.max())
        assert float((diff > 0).float().mean()) < 0.01
        assert torch.equal(got[..., :44], frame[..., :44].float())  # temporal pairs unrotated
        if Tp > T:
            assert krp[s, :, :, T:].abs().sum() == 0


@pytest.mark.parametrize(
    "gh,gw,kpos,qpos,dtype",
    [(8, 8, [0, 4, 5, 6, 7], [6, 7], BF), (10, 10, [0, 1, 2, 3, 4, 5], [3, 4, 5], BF),
     (6, 11, [3, 0, 9], [2], torch.float32), (30, 52, [0, 18, 19, 20], [18, 19, 20], BF)],
)
def test_attention_rope_vs_oracle(gpu, gh, gw, kpos, qpos, dtype):
    _say("attention rope", gh, gw, kpos, qpos, dtype)
    T, H = gh * gw, 2
    n, nq = len(kpos), len(qpos)
    q = _rand((1, nq * T, H, 128), 3, dtype)
    k, v = _rand((1, n * T, H, 128), 4), _rand((1, n * T, H, 128), 5)
    f = ref.wan_rope_freqs()
    want = ref.attention(ref.rope_frames(q, (gh, gw), qpos, f), ref.rope_frames(k, (gh, gw), kpos, f), v)
    cfg = rope.RopeConfig(grid_hw=(gh, gw))
    hw = rope.spatial_table(cfg, gpu)
    g = torch.Generator().manual_seed(6)
    slots = torch.randperm(n + 2, generator=g)[:n].tolist()
    kp, vp, _, _ = kernels.new_pools(n + 2, 1, H, T, BF, gpu)
    krp = torch.zeros_like(kp)
    for j in range(n):
        kernels.append_frames(k.to(gpu), v.to(gpu), kp, vp, [slots[j]], frame_tokens=T,
                              src_frame0=j, kr_pool=krp, rope_hw=hw, grid_hw=(gh, gw))
    out = kernels.attention_frames(q.to(gpu), krp, vp, slots, frame_tokens=T,
                                   rope=(hw, (gh, gw), rope.temporal_table(qpos, kpos, cfg, gpu)))
    torch.cuda.synchronize()
    assert out.dtype == dtype
    assert_attn_close(out, want)


@pytest.mark.parametrize(
    "sink,cap,gh,gw,chunks,echo,rtf",
    [(1, 6, 8, 8, 5, True, None), (0, 5, 10, 10, 4, True, None), (1, 5, 8, 8, 4, False, 4),
     (1, 21, 30, 52, 2, True, None)],
)
def test_cached_rollout_rope_vs_oracle(gpu, sink, cap, gh, gw, chunks, echo, rtf):
    """Pre-RoPE cached rollout (2 passes per chunk, commit on the second): every pass within the
    attention bars of the oracle with the reference's window RoPE, and the committed cache holds
    the raw K/V bit-exact."""
    _say("rollout rope", sink, cap, gh, gw, chunks, echo, rtf)
    T, H, nb = gh * gw, 2, 2
    cfg = rope.RopeConfig(grid_hw=(gh, gw), use_echorope=echo, rope_train_frames=rtf)
    cache = make_kv_cache_allocator(
        num_layers=1, num_heads=H, head_dim=128, frame_sequence_length=T, local_attn_size=cap,
        sink_size=sink, num_frame_per_block=nb, rope=cfg)(1, dtype=BF, device=gpu)[0]
    oc = ref.allocate_kv_cache(num_layers=1, batch_size=1, cache_tokens=cap * T, num_heads=H,
                               head_dim=128, dtype=BF)[0]
    orope = {"freqs": ref.wan_rope_freqs(), "grid_hw": (gh, gw), "use_echorope": echo,
             "rope_train_frames": rtf}
    seed = 10
    for c in range(chunks):
        for commit in (False, True):
            seed += 1
            q, k, v = (_rand((1, nb * T, H, 128), seed * 3 + i) for i in range(3))
            start = c * nb * T
            x, info = attend_cached(q.to(gpu), k.to(gpu), v.to(gpu), cache, start)
            want, oinfo = ref.cached_self_attention(
                q, k, v, oc, current_start=start, frame_seqlen=T, sink_size=sink,
                local_attn_size=cap, rope=orope)
            torch.cuda.synchronize()
            assert_attn_close(x, want)
            if commit:
                apply_cache_updates([cache], [(0, info)])
                ref.apply_cache_updates([oc], [(0, oinfo)])
    assert torch.equal(cache["k"].cpu(), oc["k"]) and torch.equal(cache["v"].cpu(), oc["v"])
