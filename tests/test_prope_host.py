"""Host logic of fused PRoPE (solarwm_amd/prope.py) on the CPU: the camera store follows the
oracle's camera cache through rolling / direct / recompute passes, and the per-pass tables give
the oracle's RoPE-then-PRoPE scores (no kernel runs here)."""

import pytest
import torch

from oracle import prope_ref as pr
from oracle import wan_cache_ref as ref
from solarwm_amd import PropeConfig, RopeConfig, make_kv_cache_allocator, stage_camera_cache

from .cameras import per_token, trajectory

F64 = torch.float64


def _drive(cache, start, n_tokens, commit, sink_recache=False):
    """One layer's pass through the slot table only (what attend_cached does around the kernels)."""
    plan, temp, staging, window = cache.plan(start, n_tokens, sink_recache)
    upd = cache.stage(plan, temp)
    if commit:
        cache.commit(upd, plan.current_end, plan.local_end_index)
    return plan, window


def _oracle_scores(q, k, qpos, kpos, vq, kq, vk, kk, transform):
    """(P_qᵀ R_q q)·(P_k⁻¹ R_k k) over the temporal channels 0..43, one token per frame."""
    f = ref.wan_rope_freqs()
    rq = ref.rope_frames(q[None, :, None], (1, 1), qpos, f)[0, :, 0]  # [nq, 128]
    rk = ref.rope_frames(k[None, :, None], (1, 1), kpos, f)[0, :, 0]  # [nk, 128]
    _, pq_t, _ = pr.projection_matrices(pr.transform_relative_viewmats(vq, transform), kq)
    _, _, pk_inv = pr.projection_matrices(pr.transform_relative_viewmats(vk, transform), kk)
    tq = pr.apply_tiled(rq[None, :, None], pq_t[None])[0, :, 0, :44]
    tk = pr.apply_tiled(rk[None, :, None], pk_inv[None])[0, :, 0, :44]
    return tq @ tk.T  # [nq, nk]


@pytest.mark.parametrize("sink,cap,nb,schedule,transform,echo", [
    (1, 6, 2, [0, 2, 4, 6, 8], "linear", True),
    (0, 5, 1, [0, 1, 2, 3, 4, 5], "logd4", True),
    (1, 5, 2, [0, 2, 2, 4, 6], "linear", False),  # a recompute pass at frame 2
])
def test_camera_pass_tables_and_store(sink, cap, nb, schedule, transform, echo):
    T, B = 64, 2
    cfg = RopeConfig(grid_hw=(8, 8), use_echorope=echo)
    caches = make_kv_cache_allocator(
        num_layers=1, num_heads=1, head_dim=128, frame_sequence_length=T, local_attn_size=cap,
        sink_size=sink, num_frame_per_block=nb, rope=cfg,
        prope=PropeConfig(camera_translation_transform=transform))(B, dtype=torch.bfloat16, device="cpu")
    c0 = caches[0]
    n_frames = max(schedule) + nb
    vm, ks = trajectory(B, n_frames, seed=3, t_scale=0.8)
    vm_tok, ks_tok = per_token(vm, T), per_token(ks, T)
    odict = ref.allocate_kv_cache(num_layers=1, batch_size=B, cache_tokens=cap * T, num_heads=1,
                                  head_dim=4, dtype=torch.float32)
    g = torch.Generator().manual_seed(5)
    for start_f in schedule:
        for commit in (False, True):
            start = start_f * T
            cp = stage_camera_cache(caches, vm_tok, ks_tok, start, nb * T)
            _, _, tv, tk, oupd = pr.stage_fused_camera_cache(
                odict, cam_viewmats=vm_tok, cam_ks=ks_tok, current_start=start,
                num_new_tokens=nb * T, frame_seqlen=T, sink_size=sink, local_attn_size=cap)
            plan, window = _drive(c0, start, nb * T, commit)
            assert cp.window == tuple(window)
            # per-frame cameras of the visible window, from the oracle's staged camera rows
            wv = pr.visible_cameras(tv, list(plan.window))[:, ::T]
            wk = pr.visible_cameras(tk, list(plan.window))[:, ::T]
            nk = len(window)
            ns = (plan.window[0][1] - plan.window[0][0]) // T if sink > 0 else 0
            pos = ref.rope_positions(num_sink_frames=ns, num_local_frames=nk - ns, num_new_frames=nb,
                                     use_echorope=echo, max_attention_size=cap * T, frame_seqlen=T,
                                     current_start_frame=start_f, sink_branch=sink > 0)
            qpos = list(range(pos["q_start"], pos["q_start"] + nb))
            kpos = list(range(ns)) + list(range(pos["local_start"], pos["local_start"] + nk - ns))
            for b in range(B):
                vq, kq = vm[b, start_f : start_f + nb].double(), ks[b, start_f : start_f + nb].double()
                q = torch.randn(nb, 128, generator=g, dtype=F64)
                k = torch.randn(nk, 128, generator=g, dtype=F64)
                want = _oracle_scores(q, k, qpos, kpos, vq, kq, wv[b].double(), wk[b].double(), transform)
                w = cp.q_xform_t[b].double()  # [nk, nb, 11, 4, 4]
                qg = q[:, :44].reshape(nb, 11, 4)
                kg = k[:, :44].reshape(nk, 11, 4)
                got = torch.einsum("jfgim,fgm,jgi->fj", w, qg, kg)
                assert torch.allclose(got, want, rtol=1e-5, atol=1e-5 * float(want.abs().max())), (start_f, b)
                p, pt, pinv = pr.projection_matrices(pr.transform_relative_viewmats(vq, transform), kq)
                assert torch.allclose(cp.q_xform_s[b].double(), pt, atol=1e-6)
                assert torch.allclose(cp.out_xform[b].double(), p, atol=1e-6)
            if commit:
                pr.commit_fused_camera_cache(oupd)
                odict[0]["global_end_index"].fill_(plan.current_end)
                odict[0]["local_end_index"].fill_(plan.local_end_index)
                meta = c0["_fused_prope_camera_metadata"]
                st = odict[0][pr.STATE_KEY]
                assert torch.equal(meta["viewmats"], st["viewmats"]) and torch.equal(meta["K"], st["K"])


def test_written_frames_take_their_cameras_inverse():
    T, B, nb = 64, 1, 2
    caches = make_kv_cache_allocator(
        num_layers=2, num_heads=1, head_dim=128, frame_sequence_length=T, local_attn_size=4,
        sink_size=0, num_frame_per_block=nb, rope=RopeConfig(grid_hw=(8, 8)),
        prope=PropeConfig())(B, dtype=torch.bfloat16, device="cpu")
    vm, ks = trajectory(B, 4, seed=8)
    cp = stage_camera_cache(caches, vm, ks, 2 * T, nb * T, per_frame=True)
    _, _, pinv = pr.projection_matrices(vm[0, 2:4].double(), ks[0, 2:4].double())
    assert torch.allclose(cp.kv_xform[:, 0].double(), pinv, atol=1e-6)
    # both layers share the store; only layer 0 exposes the reference's key
    assert caches[1].camera is caches[0].camera
    assert "_fused_prope_camera_metadata" in caches[0] and "_fused_prope_camera_metadata" not in caches[1]


def test_camera_errors():
    T = 64
    alloc = make_kv_cache_allocator(
        num_layers=1, num_heads=1, head_dim=128, frame_sequence_length=T, local_attn_size=4,
        num_frame_per_block=1, rope=RopeConfig(grid_hw=(8, 8)), prope=PropeConfig())
    caches = alloc(1, dtype=torch.bfloat16, device="cpu")
    vm, ks = trajectory(1, 3, seed=9)
    tok = per_token(vm, T)
    tok[0, 1] = torch.eye(4)  # a camera that changes inside frame 0
    with pytest.raises(ValueError, match="one camera per latent frame"):
        stage_camera_cache(caches, tok, per_token(ks, T), 0, T)
    with pytest.raises(ValueError, match="both viewmats and K"):
        stage_camera_cache(caches, vm, None, 0, T, per_frame=True)
    # K/V history written without cameras cannot be camera-conditioned later (reference rule)
    _drive(caches[0], 0, T, commit=True)
    with pytest.raises(RuntimeError, match="without shared camera metadata"):
        stage_camera_cache(caches, vm, ks, T, T, per_frame=True)
    with pytest.raises(ValueError):
        PropeConfig(camera_translation_transform="cubic")
    with pytest.raises(ValueError, match="at least 64"):
        make_kv_cache_allocator(num_layers=1, num_heads=1, head_dim=128, frame_sequence_length=4,
                                local_attn_size=4, rope=RopeConfig(grid_hw=(2, 2)),
                                prope=PropeConfig())(1, dtype=torch.bfloat16, device="cpu")
    with pytest.raises(ValueError, match="rope="):
        make_kv_cache_allocator(num_layers=1, num_heads=1, head_dim=128, frame_sequence_length=T,
                                local_attn_size=4, prope=PropeConfig())(1, dtype=torch.bfloat16,
                                                                        device="cpu")
