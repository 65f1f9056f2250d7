"""GPU parity of fused PRoPE on the cached path against the oracle's float64 restatement of the
reference (RoPE then PRoPE, causal_model.py:1170-1199 -> camera_prope.py:93-261; camera cache
causal_model.py:1948-2075).

Bars: raw pools and camera metadata bit-exact; the transformed K/V copies within one bf16
rounding of the float64 transform.  Attention: camera transforms make the outputs up to ~2x
larger than plain attention's and every transformed operand is bf16, so the bar is the
reference's own arithmetic (bf16 matrices applied to bf16 features, emulated on the CPU) on the
same pass: against the float64 restatement, our mean and 99.9th-percentile errors stay within
1.25x of the reference's and our largest error within 2.5x of its largest (or within the plain
bf16 bars of tests/helpers.py, whichever is looser).
"""

import pytest
import torch

from oracle import prope_ref as pr
from oracle import wan_cache_ref as ref
from solarwm_amd import (PropeConfig, RopeConfig, apply_cache_updates, attend_cached,
                         commit_camera_cache, kernels, make_kv_cache_allocator, rope,
                         stage_camera_cache)

from .cameras import per_token, trajectory
from .helpers import MAX_ABS, MEAN_ABS

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _say(*a):
    print(*a, flush=True)


def _rand(shape, seed, dtype=BF):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype)


def _errors(got, want):
    """(max, 99.9th percentile, mean) of |got - want|."""
    d = (got.double() - want.double()).abs().flatten()
    return float(d.max()), float(d.kthvalue(max(1, int(d.numel() * 0.999))).values), float(d.mean())


def _within_bf16(got, want):
    """|got - want| <= 2^-8 |want| + 1e-5: one bf16 rounding of an fp32 evaluation."""
    d = (got.double() - want.double()).abs()
    return bool((d <= want.double().abs() * 2.0**-8 + 1e-5).all()), float(d.max())


@pytest.mark.parametrize("gh,gw,B", [(8, 8, 1), (10, 10, 2), (30, 52, 1)])
def test_append_prope_copies(gpu, gh, gw, B):
    _say("append prope", gh, gw, B)
    T, H = gh * gw, 3
    k, v = _rand((B, 2 * T, H, 128), 1), _rand((B, 2 * T, H, 128), 2)
    vm, ks = trajectory(B, 2, seed=4, t_scale=0.8)
    _, _, pinv = pr.projection_matrices(vm.double(), ks.double())  # [B, 2, 4, 4]
    hw = rope.spatial_table(RopeConfig(grid_hw=(gh, gw)), gpu)
    kp, vp, _, _ = kernels.new_pools(4, B, H, T, BF, gpu)
    kx, vx = torch.full_like(kp, 7.0), torch.full_like(vp, 7.0)
    xf = pinv.transpose(0, 1).to(torch.float32).contiguous().to(gpu)  # [2, B, 4, 4]
    kernels.append_frames(k.to(gpu), v.to(gpu), kp, vp, [2, 0], frame_tokens=T, kr_pool=kx,
                          rope_hw=hw, grid_hw=(gh, gw), vr_pool=vx, kv_xform=xf)
    torch.cuda.synchronize()
    f = ref.wan_rope_freqs()
    Tp = kernels.padded_tokens(T)
    for i, s in enumerate([2, 0]):
        kf, vf = k[:, i * T : (i + 1) * T], v[:, i * T : (i + 1) * T]
        assert torch.equal(kp[s, :, :, :T].permute(0, 2, 1, 3).cpu(), kf)
        assert torch.equal(vp[s, :, :, :, :T].permute(0, 3, 1, 2).cpu(), vf)
        m = pinv[:, i][:, None].expand(B, T, 4, 4)  # per token of frame i
        want_k = pr.apply_tiled(ref.rope_frames(kf.double(), (gh, gw), [0], f), m)
        got_k = kx[s, :, :, :T].permute(0, 2, 1, 3).cpu()
        assert torch.equal(got_k[..., :44], kf[..., :44])  # temporal groups stay raw
        ok, err = _within_bf16(got_k[..., 44:], want_k[..., 44:])
        assert ok, ("kx", i, err)
        want_v = pr.apply_tiled(vf.double(), m)
        ok, err = _within_bf16(vx[s, :, :, :, :T].permute(0, 3, 1, 2).cpu(), want_v)
        assert ok, ("vx", i, err)
        if Tp > T:
            assert kx[s, :, :, T:].abs().sum() == 0 and vx[s, ..., T:].abs().sum() == 0


@pytest.mark.parametrize(
    "sink,cap,gh,gw,chunks,echo,rtf,transform,B",
    [(1, 6, 8, 8, 5, True, None, "linear", 1),
     (0, 5, 10, 10, 4, True, None, "logd4", 2),
     (1, 5, 8, 8, 4, False, 4, "linear", 1),
     (1, 21, 30, 52, 2, True, None, "linear", 1)],
)
def test_cached_rollout_prope_vs_oracle(gpu, sink, cap, gh, gw, chunks, echo, rtf, transform, B):
    """Camera-conditioned rollout (2 passes per chunk, commit on the second): every pass within
    the attention bars of the oracle's RoPE-then-PRoPE attention, the committed cache holds the
    raw K/V bit-exact and layer 0's camera metadata equals the oracle's camera cache."""
    _say("rollout prope", sink, cap, gh, gw, chunks, echo, rtf, transform, B)
    T, H, nb = gh * gw, 2, 2
    cfg = RopeConfig(grid_hw=(gh, gw), use_echorope=echo, rope_train_frames=rtf)
    caches = make_kv_cache_allocator(
        num_layers=1, num_heads=H, head_dim=128, frame_sequence_length=T, local_attn_size=cap,
        sink_size=sink, num_frame_per_block=nb, rope=cfg,
        prope=PropeConfig(camera_translation_transform=transform))(B, dtype=BF, device=gpu)
    oc = ref.allocate_kv_cache(num_layers=1, batch_size=B, cache_tokens=cap * T, num_heads=H,
                               head_dim=128, dtype=BF)
    orope = {"freqs": ref.wan_rope_freqs(), "grid_hw": (gh, gw), "use_echorope": echo,
             "rope_train_frames": rtf}
    vm, ks = trajectory(B, chunks * nb, seed=21, t_scale=0.6)
    vm_tok, ks_tok = per_token(vm, T), per_token(ks, T)
    vm_dev, ks_dev = vm_tok.to(gpu), ks_tok.to(gpu)
    seed = 30
    for c in range(chunks):
        for commit in (False, True):
            seed += 1
            q, k, v = (_rand((B, nb * T, H, 128), seed * 3 + i) for i in range(3))
            start = c * nb * T
            cp = stage_camera_cache(caches, vm_dev, ks_dev, start, nb * T)
            x, info = attend_cached(q.to(gpu), k.to(gpu), v.to(gpu), caches[0], start, camera=cp)
            cq, ck, tv, tk, oupd = pr.stage_fused_camera_cache(
                oc, cam_viewmats=vm_tok, cam_ks=ks_tok, current_start=start, num_new_tokens=nb * T,
                frame_seqlen=T, sink_size=sink, local_attn_size=cap)
            cams = {"q_viewmats": cq, "q_ks": ck, "kv_viewmats": tv, "kv_ks": tk,
                    "transform": transform}
            args = dict(current_start=start, frame_seqlen=T, sink_size=sink, local_attn_size=cap,
                        rope=orope)
            want, oinfo = ref.cached_self_attention(q, k, v, oc[0], prope=cams, **args)
            # the reference's own rounding on the same pass (the cache is only read here)
            want_ref, _ = ref.cached_self_attention(q, k, v, oc[0], prope=dict(cams, emulate_bf16=True),
                                                    **args)
            torch.cuda.synchronize()
            assert torch.isfinite(x).all()
            e_ours, e_ref = _errors(x.cpu(), want), _errors(want_ref, want)
            _say(f"  chunk {c} commit {commit}: (max, p99.9, mean) ours "
                 f"{tuple(f'{e:.2e}' for e in e_ours)} reference {tuple(f'{e:.2e}' for e in e_ref)}")
            assert e_ours[0] <= max(MAX_ABS, 2.5 * e_ref[0]), "max"
            assert e_ours[1] <= max(MAX_ABS / 2, 1.25 * e_ref[1]), "p99.9"
            assert e_ours[2] <= max(MEAN_ABS, 1.25 * e_ref[2]), "mean"
            if commit:
                apply_cache_updates(caches, [(0, info)])
                commit_camera_cache(cp)
                ref.apply_cache_updates(oc, [(0, oinfo)])
                pr.commit_fused_camera_cache(oupd)
    c0 = caches[0]
    assert torch.equal(c0["k"].cpu(), oc[0]["k"]) and torch.equal(c0["v"].cpu(), oc[0]["v"])
    meta, st = c0["_fused_prope_camera_metadata"], oc[0][pr.STATE_KEY]
    assert torch.equal(meta["viewmats"].cpu(), st["viewmats"]) and torch.equal(meta["K"].cpu(), st["K"])


def test_prope_without_cameras_after_camera_history_raises(gpu):
    T, nb = 64, 1
    caches = make_kv_cache_allocator(
        num_layers=1, num_heads=1, head_dim=128, frame_sequence_length=T, local_attn_size=3,
        num_frame_per_block=nb, rope=RopeConfig(grid_hw=(8, 8)), prope=PropeConfig())(
            1, dtype=BF, device=gpu)
    vm, ks = trajectory(1, 2, seed=2)
    q = _rand((1, T, 1, 128), 1).to(gpu)
    cp = stage_camera_cache(caches, vm.to(gpu), ks.to(gpu), 0, T, per_frame=True)
    _, info = attend_cached(q, q, q, caches[0], 0, camera=cp)
    apply_cache_updates(caches, [(0, info)])
    with pytest.raises(ValueError, match="camera="):
        attend_cached(q, q, q, caches[0], T)
