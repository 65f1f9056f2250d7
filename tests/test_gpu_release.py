"""The reference's shipped inference geometry on the GPU against the oracle.

configs/solar_wm/wan22_ti2v_5b/infer_stage2_sgf_81f.yaml:16-27 with architectures/ti2v_5b.json:
latent 30 x 54 -> 2x2 patches -> 405 tokens per frame (grid 15 x 27, an odd frame size: every
frame's 448-row slot ends in 43 masked padding keys), 24 heads x 128, chunks of 3 frames, an
18-frame cache with no sink, rolling eviction, window RoPE without EchoRoPE (rope_train_frames
21) and fused PRoPE with the linear translation transform.  8 chunks (the release's 7 plus one
more eviction), a ``none`` pass then a commit pass each.

Checks: every pass's attention on two of the 24 heads against the oracle's float64 RoPE-then-
PRoPE attention (heads are independent and share every rotation, so the oracle runs on those
heads only), with the bars of tests/test_gpu_prope.py (the reference's own bf16 arithmetic on the
same pass sets the scale); the committed raw cache of all 24 heads bit-exact against an all-head
oracle after every commit; layer 0's camera metadata equal to the oracle's camera cache.
"""

import pytest
import torch

from oracle import prope_ref as pr
from oracle import wan_cache_ref as ref
from solarwm_amd import (PropeConfig, RopeConfig, apply_cache_updates, attend_cached,
                         commit_camera_cache, make_kv_cache_allocator, stage_camera_cache)

from .cameras import per_token, trajectory
from .helpers import MAX_ABS, MEAN_ABS

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _say(*a):
    print(*a, flush=True)


def _errors(got, want):
    d = (got.double() - want.double()).abs().flatten()
    return float(d.max()), float(d.kthvalue(max(1, int(d.numel() * 0.999))).values), float(d.mean())


def test_release_geometry_rollout(gpu):
    gh, gw, H, nb, cap, sink, chunks = 15, 27, 24, 3, 18, 0, 8
    T, Lq = gh * gw, nb * gh * gw
    hs = [0, 23]
    _say("release geometry", dict(T=T, H=H, cap=cap, sink=sink, chunks=chunks))
    rcfg = RopeConfig(grid_hw=(gh, gw), use_echorope=False, rope_train_frames=21)
    caches = make_kv_cache_allocator(
        num_layers=1, num_heads=H, head_dim=128, frame_sequence_length=T, local_attn_size=cap,
        sink_size=sink, num_frame_per_block=nb, rope=rcfg,
        prope=PropeConfig(camera_translation_transform="linear"))(1, dtype=BF, device=gpu)
    o_sub = ref.allocate_kv_cache(num_layers=1, batch_size=1, cache_tokens=cap * T,
                                  num_heads=len(hs), head_dim=128, dtype=BF)
    o_all = ref.allocate_kv_cache(num_layers=1, batch_size=1, cache_tokens=cap * T, num_heads=H,
                                  head_dim=128, dtype=BF)
    orope = {"freqs": ref.wan_rope_freqs(), "grid_hw": (gh, gw), "use_echorope": False,
             "rope_train_frames": 21}
    vm, ks = trajectory(1, chunks * nb, seed=405, t_scale=0.7)
    vm_tok, ks_tok = per_token(vm, T), per_token(ks, T)
    vm_dev, ks_dev = vm_tok.to(gpu), ks_tok.to(gpu)
    g = torch.Generator().manual_seed(405)
    for c in range(chunks):
        start = c * Lq
        for commit in (False, True):
            q, k, v = (torch.randn((1, Lq, H, 128), generator=g).to(BF) for _ in range(3))
            cp = stage_camera_cache(caches, vm_dev, ks_dev, start, Lq)
            x, info = attend_cached(q.to(gpu), k.to(gpu), v.to(gpu), caches[0], start, camera=cp)
            cq, ck, tv, tk, oupd = pr.stage_fused_camera_cache(
                o_sub, cam_viewmats=vm_tok, cam_ks=ks_tok, current_start=start,
                num_new_tokens=Lq, frame_seqlen=T, sink_size=sink, local_attn_size=cap)
            cams = {"q_viewmats": cq, "q_ks": ck, "kv_viewmats": tv, "kv_ks": tk,
                    "transform": "linear"}
            args = dict(current_start=start, frame_seqlen=T, sink_size=sink, local_attn_size=cap,
                        rope=orope)
            qs, ksub, vsub = q[:, :, hs], k[:, :, hs], v[:, :, hs]
            want, oinfo = ref.cached_self_attention(qs, ksub, vsub, o_sub[0], prope=cams, **args)
            want_ref, _ = ref.cached_self_attention(qs, ksub, vsub, o_sub[0],
                                                    prope=dict(cams, emulate_bf16=True), **args)
            _, ainfo = ref.cached_self_attention(
                q, k, v, o_all[0], current_start=start, frame_seqlen=T, sink_size=sink,
                local_attn_size=cap, attn_fn=lambda *a: torch.zeros(0))
            torch.cuda.synchronize()
            got = x[:, :, hs].cpu()
            assert torch.isfinite(got).all()
            e_ours, e_ref = _errors(got, want), _errors(want_ref, want)
            _say(f"  chunk {c} commit {commit}: (max, p99.9, mean) ours "
                 f"{tuple(f'{e:.2e}' for e in e_ours)} reference {tuple(f'{e:.2e}' for e in e_ref)}")
            assert e_ours[0] <= max(MAX_ABS, 2.5 * e_ref[0]), "max"
            assert e_ours[1] <= max(MAX_ABS / 2, 1.25 * e_ref[1]), "p99.9"
            assert e_ours[2] <= max(MEAN_ABS, 1.25 * e_ref[2]), "mean"
            if commit:
                apply_cache_updates(caches, [(0, info)])
                commit_camera_cache(cp)
                ref.apply_cache_updates(o_sub, [(0, oinfo)])
                ref.apply_cache_updates(o_all, [(0, ainfo)])
                pr.commit_fused_camera_cache(oupd)
                c0 = caches[0]
                gk, gv = c0["k"].cpu(), c0["v"].cpu()
                assert torch.equal(gk, o_all[0]["k"]) and torch.equal(gv, o_all[0]["v"]), c
                assert int(c0["local_end_index"][0]) == int(o_all[0]["local_end_index"][0])
                assert int(c0["global_end_index"][0]) == int(o_all[0]["global_end_index"][0])
    assert int(caches[0]["local_end_index"][0]) == cap * T  # evicted at chunks 6 and 7
    meta, st = caches[0]["_fused_prope_camera_metadata"], o_sub[0][pr.STATE_KEY]
    assert torch.equal(meta["viewmats"].cpu(), st["viewmats"])
    assert torch.equal(meta["K"].cpu(), st["K"])
