"""Pins oracle/prope_ref.py (fused PRoPE restatement) by algebra, closed forms and invariants."""

import math

import pytest
import torch

from oracle import prope_ref as pr
from oracle import wan_cache_ref as ref

F64 = torch.float64
FX, FY = 969.6969696969696 / 1920.0, 969.6969696969696 / 1080.0  # the data path's intrinsics


def rand_se3(n, seed, t_scale=1.0, angle=math.pi):
    """[n, 4, 4] float64 rigid transforms: random axis, rotation angle up to ``angle``."""
    g = torch.Generator().manual_seed(seed)
    axis = torch.randn(n, 3, generator=g, dtype=F64)
    axis = axis / axis.norm(dim=-1, keepdim=True)
    th = (torch.rand(n, generator=g, dtype=F64) * 2 - 1) * angle
    kx = torch.zeros(n, 3, 3, dtype=F64)
    kx[:, 0, 1], kx[:, 0, 2], kx[:, 1, 2] = -axis[:, 2], axis[:, 1], -axis[:, 0]
    kx = kx - kx.transpose(1, 2)
    rot = torch.eye(3, dtype=F64) + th.sin()[:, None, None] * kx + (1 - th.cos())[:, None, None] * kx @ kx
    m = torch.zeros(n, 4, 4, dtype=F64)
    m[:, :3, :3] = rot
    m[:, :3, 3] = torch.randn(n, 3, generator=g, dtype=F64) * t_scale
    m[:, 3, 3] = 1.0
    return m


def intrinsics(n, fx=FX, fy=FY, cx=0.5, cy=0.5):
    k = torch.zeros(n, 3, 3, dtype=F64)
    k[:, 0, 0], k[:, 1, 1], k[:, 0, 2], k[:, 1, 2], k[:, 2, 2] = fx, fy, cx, cy, 1.0
    return k


def test_se3_and_intrinsics_inverses():
    m = rand_se3(16, 1, t_scale=3.0)
    eye4 = torch.eye(4, dtype=F64).expand(16, 4, 4)
    assert torch.allclose(m @ pr.invert_se3(m), eye4, atol=1e-12)
    assert torch.allclose(pr.invert_se3(m) @ m, eye4, atol=1e-12)
    k = intrinsics(16, fx=0.7, fy=1.3, cx=0.4, cy=0.6)
    assert torch.allclose(pr.invert_k(k) @ k, torch.eye(3, dtype=F64).expand(16, 3, 3), atol=1e-12)
    lifted = pr.lift_k(k)
    assert torch.equal(lifted[:, :3, :3], k) and torch.equal(lifted[:, 3], torch.tensor([0.0, 0, 0, 1], dtype=F64).expand(16, 4))


def test_projection_matrices():
    v = rand_se3(8, 2, t_scale=2.0)
    k = intrinsics(8)
    p, pt, pinv = pr.projection_matrices(v, k)
    assert torch.allclose(p @ pinv, torch.eye(4, dtype=F64).expand(8, 4, 4), atol=1e-12)
    assert torch.equal(pt, p.transpose(-1, -2))
    # P = diag(fx, fy, 1, 1) V: the principal point is dropped
    assert torch.allclose(p, torch.diag(torch.tensor([FX, FY, 1.0, 1.0], dtype=F64)) @ v, atol=1e-15)
    p2, _, _ = pr.projection_matrices(v, intrinsics(8, cx=0.1, cy=0.9))
    assert torch.equal(p, p2)
    # GTA branch: no intrinsics -> P = V
    pg, _, pginv = pr.projection_matrices(v, None)
    assert torch.equal(pg, v) and torch.allclose(pginv, torch.linalg.inv(v), atol=1e-12)


def test_translation_transforms():
    v = torch.eye(4, dtype=torch.float32).repeat(3, 1, 1)
    v[0, :3, 3] = torch.tensor([3.0, 4.0, 0.0])
    v[1, :3, :3] = torch.tensor([[0.0, -1, 0], [1, 0, 0], [0, 0, 1]])
    v[1, :3, 3] = torch.tensor([0.0, 0.0, -2.0])
    assert pr.transform_relative_viewmats(v, "linear") is v
    out = pr.transform_relative_viewmats(v, "logd4")
    s = math.log1p(5.0) / 20.0
    assert torch.allclose(out[0, :3, 3], torch.tensor([3 * s, 4 * s, 0.0]), rtol=1e-6)
    assert torch.allclose(out[1, :3, 3], torch.tensor([0.0, 0.0, -math.log1p(2.0) / 4.0]), rtol=1e-6)
    assert torch.equal(out[2], v[2])  # zero translation stays zero
    assert torch.equal(out[:, :3, :3], v[:, :3, :3]) and torch.equal(out[:, 3], v[:, 3])
    with pytest.raises(ValueError):
        pr.transform_relative_viewmats(v, "cubic")


def test_apply_tiled_matches_loops():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 3, 2, 8, generator=g, dtype=F64)
    m = torch.randn(2, 3, 4, 4, generator=g, dtype=F64)
    got = pr.apply_tiled(x, m)
    want = torch.zeros_like(x)
    for b in range(2):
        for l in range(3):
            for h in range(2):
                for grp in range(2):
                    for i in range(4):
                        want[b, l, h, 4 * grp + i] = sum(
                            float(m[b, l, i, j]) * float(x[b, l, h, 4 * grp + j]) for j in range(4))
    assert torch.allclose(got, want, atol=1e-12)


def _qkv(lq, lk, seed, h=2, d=16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(1, lq, h, d, generator=g, dtype=F64),
            torch.randn(1, lk, h, d, generator=g, dtype=F64),
            torch.randn(1, lk, h, d, generator=g, dtype=F64))


def _f64_attention(q, k, v):
    return ref.attention(q, k, v, round_inputs_to_bf16=False)


def test_identity_cameras_change_nothing():
    q, k, v = _qkv(3, 5, 4)
    eye = torch.eye(4, dtype=F64).expand(1, 3, 4, 4)
    eyek = torch.eye(4, dtype=F64).expand(1, 5, 4, 4)
    qo, ko, vo, out_fn = pr.prope_qkv_separate(
        q, k, v, q_viewmats=eye, q_ks=torch.eye(3, dtype=F64).expand(1, 3, 3, 3),
        kv_viewmats=eyek, kv_ks=torch.eye(3, dtype=F64).expand(1, 5, 3, 3))
    assert torch.equal(qo, q) and torch.equal(ko, k) and torch.equal(vo, v)
    assert torch.equal(out_fn(q), q)


@pytest.mark.parametrize("transform", ["linear", "logd4"])
def test_one_camera_everywhere_is_plain_attention(transform):
    """Pq Pk⁻¹ = I and P (Σ p P⁻¹ v) = Σ p v: PRoPE attention with a single camera equals plain
    attention exactly (pins Pᵀ on q, P⁻¹ on k and v, P on the output)."""
    q, k, v = _qkv(6, 10, 5)
    cam = rand_se3(1, 6, t_scale=1.5)
    kq = intrinsics(1)
    x = pr.fused_prope_attention(
        q, k, v, q_viewmats=cam.expand(1, 6, 4, 4), q_ks=kq.expand(1, 6, 3, 3),
        kv_viewmats=cam.expand(1, 10, 4, 4), kv_ks=kq.expand(1, 10, 3, 3),
        attn_fn=_f64_attention, transform=transform)
    assert torch.allclose(x, _f64_attention(q, k, v), atol=1e-10)


def test_scores_depend_on_relative_pose_only():
    """A common world change G (V -> V G for every camera) leaves Pq Pk⁻¹, hence every score and
    the mapped-back output, unchanged; different per-token poses do change the scores."""
    q, k, v = _qkv(4, 7, 7)
    cq, ck = rand_se3(4, 8, t_scale=1.0)[None], rand_se3(7, 9, t_scale=1.0)[None]
    kq, kk = intrinsics(4)[None], intrinsics(7)[None]
    gw = rand_se3(1, 10, t_scale=2.0)[0]

    def run(cq_, ck_):
        qo, ko, _, _ = pr.prope_qkv_separate(q, k, v, q_viewmats=cq_, q_ks=kq, kv_viewmats=ck_, kv_ks=kk)
        s = torch.einsum("blhd,bmhd->bhlm", qo, ko)
        x = pr.fused_prope_attention(q, k, v, q_viewmats=cq_, q_ks=kq, kv_viewmats=ck_, kv_ks=kk,
                                     attn_fn=_f64_attention)
        return s, x

    s0, x0 = run(cq, ck)
    s1, x1 = run(cq @ gw, ck @ gw)
    assert torch.allclose(s0, s1, atol=1e-9) and torch.allclose(x0, x1, atol=1e-9)
    plain = torch.einsum("blhd,bmhd->bhlm", q, k)
    assert float((s0 - plain).abs().max()) > 1e-2


def test_reference_rounding_within_attention_bars():
    """The reference applies bf16 matrices to bf16 features; its result stays within the bf16
    attention bars of the float64 restatement for realistic cameras (the data path's intrinsics,
    rotations up to 30 degrees, translations up to ~2)."""
    from .helpers import MAX_ABS, MEAN_ABS

    g = torch.Generator().manual_seed(11)
    lq, lk, h = 64, 256, 2
    q, k, v = (torch.randn(1, n, h, 128, generator=g).to(torch.bfloat16) for n in (lq, lk, lk))
    cq = rand_se3(1, 12, t_scale=0.7, angle=math.pi / 6).expand(lq, 4, 4)[None].float()
    ck = torch.repeat_interleave(rand_se3(4, 13, t_scale=0.7, angle=math.pi / 6), lk // 4, 0)[None].float()
    kq, kk = intrinsics(lq)[None].float(), intrinsics(lk)[None].float()
    args = dict(q_viewmats=cq, q_ks=kq, kv_viewmats=ck, kv_ks=kk, attn_fn=ref.attention)
    exact = pr.fused_prope_attention(q, k, v, **args)
    emul = pr.fused_prope_attention(q, k, v, emulate_bf16=True, **args)
    d = (emul.double() - exact.double()).abs()
    print(f"reference rounding vs float64: max {float(d.max()):.2e} mean {float(d.mean()):.2e}")
    assert float(d.max()) <= MAX_ABS and float(d.mean()) <= MEAN_ABS


def _labelled(lq, first_id, h=1, d=4):
    """K/V whose channel 0 is the global token id; cameras whose translation x is that id."""
    ids = torch.arange(first_id, first_id + lq, dtype=torch.float32)
    x = torch.zeros(1, lq, h, d)
    x[..., 0] = ids[None, :, None]
    cam = torch.eye(4).repeat(1, lq, 1, 1)
    cam[0, :, 0, 3] = ids
    ks = torch.zeros(1, lq, 3, 3)
    ks[0, :, 0, 0] = ids
    return x, cam, ks


@pytest.mark.parametrize("sink,cap,nb,schedule", [
    (1, 5, 2, [0, 2, 4, 6, 8, 10]),
    (0, 4, 1, [0, 1, 2, 3, 4, 5, 6]),
    (1, 6, 2, [0, 2, 2, 4, 6, 6, 8]),  # repeated starts are recompute passes
])
def test_camera_cache_follows_kv_rows(sink, cap, nb, schedule):
    """Token-labelled K and cameras: after every committed pass the camera cache holds, row for
    row, the ids the K cache holds; a ``none`` pass changes neither; staging touches nothing."""
    T = 3
    kvc = ref.allocate_kv_cache(num_layers=1, batch_size=1, cache_tokens=cap * T, num_heads=1,
                                head_dim=4, dtype=torch.float32)
    for start_f in schedule:
        for policy in ("none", "commit"):
            start = start_f * T
            x, cam, ks = _labelled(nb * T, start)
            before = [t.clone() for t in (kvc[0]["k"], )]
            cur_v, cur_k, tv, tk, upd = pr.stage_fused_camera_cache(
                kvc, cam_viewmats=cam, cam_ks=ks, current_start=start, num_new_tokens=nb * T,
                frame_seqlen=T, sink_size=sink, local_attn_size=cap)
            state_before = kvc[0][pr.STATE_KEY]["viewmats"].clone()
            _, info = ref.cached_self_attention(x, x, x, kvc[0], current_start=start, frame_seqlen=T,
                                                sink_size=sink, local_attn_size=cap)
            assert torch.equal(kvc[0][pr.STATE_KEY]["viewmats"], state_before)
            if policy == "commit":
                ref.apply_cache_updates(kvc, [(0, info)])
                pr.commit_fused_camera_cache(upd)
                st = kvc[0][pr.STATE_KEY]
                assert torch.equal(st["viewmats"][0, :, 0, 3], kvc[0]["k"][0, :, 0, 0])
                assert torch.equal(st["K"][0, :, 0, 0], kvc[0]["k"][0, :, 0, 0])
            else:
                assert torch.equal(kvc[0]["k"], before[0])


def test_camera_cache_rejects_history_without_metadata():
    T = 2
    kvc = ref.allocate_kv_cache(num_layers=1, batch_size=1, cache_tokens=4 * T, num_heads=1,
                                head_dim=4, dtype=torch.float32)
    kvc[0]["local_end_index"].fill_(T)
    kvc[0]["global_end_index"].fill_(T)
    x, cam, ks = _labelled(T, T)
    with pytest.raises(RuntimeError):
        pr.stage_fused_camera_cache(kvc, cam_viewmats=cam, cam_ks=ks, current_start=T,
                                    num_new_tokens=T, frame_seqlen=T, sink_size=0, local_attn_size=4)
    with pytest.raises(ValueError):
        pr.slice_current_camera_tokens(cam, current_start=5 * T, num_new_tokens=T + 1)
    full = torch.arange(10.0).view(1, 10, 1, 1)
    assert torch.equal(pr.slice_current_camera_tokens(full, current_start=4, num_new_tokens=3), full[:, 4:7])


# ---------------------------------------------------------------------------------------------
# the PRoPE self-attention branch with its own cache (causal_model.py:1296-1525)
# ---------------------------------------------------------------------------------------------
def _labelled_chunk(start, n, heads=1):
    ids = torch.arange(start, start + n, dtype=F64)
    return ids.view(1, n, 1, 1).expand(1, n, heads, 4).clone()


def _frame_ids(k_labels, T):
    row = k_labels[0, :, 0, 0]
    return [int(row[f * T]) // T for f in range(row.shape[0] // T)]


def test_branch_with_identity_cameras_is_the_main_cache_with_immediate_commit():
    """Identity cameras: the branch's cache rows are the raw token ids, committed by the branch
    forward itself; the C1 known answer (390-token frames, chunk 3, 21-frame cache, sink 1,
    10 chunks x (none, commit)) comes out of its cache."""
    T, chunk_f, cap_f, sink_f = 390, 3, 21, 1
    Lq = chunk_f * T
    cache = ref.allocate_kv_cache(1, 1, cap_f * T, 1, 4, F64)[0]
    eye = torch.eye(4, dtype=F64).expand(1, Lq, 4, 4)
    seen = []

    def rec(q, k, v):
        seen.append(k[0, :, 0, 0].clone())
        return torch.zeros_like(q)

    for c in range(10):
        for policy in ("none", "commit_detached"):
            before = {key: val.clone() for key, val in cache.items()}
            x = _labelled_chunk(c * Lq, Lq)
            pr.prope_branch_forward(x, x, x, cache, viewmats=eye, ks=None, current_start=c * Lq,
                                    frame_seqlen=T, sink_size=sink_f, local_attn_size=cap_f,
                                    cache_update_policy=policy, attn_fn=rec)
            if policy == "none":
                assert all(torch.equal(before[k], cache[k]) for k in before)
            else:
                assert int(cache["global_end_index"]) == (c + 1) * Lq
    lk = [len(s) for s in seen[1::2]]
    assert lk == [1170, 2340, 3510, 4680, 5850, 7020, 8190, 8190, 8190, 8190]
    assert _frame_ids(cache["k"], T) == [0] + list(range(10, 30))


def _f64_attention(q, k, v):
    return ref.attention(q, k, v, round_inputs_to_bf16=False)


def _branch_rollout(cams_fn, n_chunks=3, T=8, H=2, cap_f=5, sink_f=1, seed=0):
    g = torch.Generator().manual_seed(seed)
    Lq = 2 * T
    cache = ref.allocate_kv_cache(1, 1, cap_f * T, H, 128, F64)[0]
    outs = []
    for c in range(n_chunks):
        q, k, v = (torch.randn(1, Lq, H, 128, generator=g, dtype=F64) for _ in range(3))
        vm, kk = cams_fn(c, Lq)
        outs.append(pr.prope_branch_forward(
            q, k, v, cache, viewmats=vm, ks=kk, current_start=c * Lq, frame_seqlen=T,
            sink_size=sink_f, local_attn_size=cap_f, attn_fn=_f64_attention))
    return outs, cache


def test_branch_with_one_camera_for_every_token_is_plain_cached_attention():
    """One camera P for all tokens: (Pᵀq)·(P⁻¹k) = q·k and P Σ p P⁻¹v = Σ p v, so the branch's
    outputs equal the main branch's cached attention on the raw inputs."""
    cam = rand_se3(1, 7, t_scale=2.0)
    kk = intrinsics(1)
    outs, _ = _branch_rollout(lambda c, L: (cam.expand(1, L, 4, 4), kk.expand(1, L, 3, 3)))
    g = torch.Generator().manual_seed(0)
    T, Lq, cache = 8, 16, ref.allocate_kv_cache(1, 1, 40, 2, 128, F64)[0]
    for c in range(3):
        q, k, v = (torch.randn(1, Lq, 2, 128, generator=g, dtype=F64) for _ in range(3))
        want, upd = ref.cached_self_attention(q, k, v, cache, current_start=c * Lq, frame_seqlen=T,
                                              sink_size=1, local_attn_size=5,
                                              attn_fn=_f64_attention)
        ref.apply_cache_updates([cache], [(0, upd)])
        assert torch.allclose(outs[c], want, atol=1e-10), c


def test_branch_is_invariant_to_a_common_world_change():
    """Scores and outputs depend on relative poses only (linear translation mode): moving every
    camera by one world transform leaves every output unchanged, while different poses per frame
    do change them."""
    poses = rand_se3(16, 11, t_scale=1.5, angle=0.4)
    world = rand_se3(1, 12, t_scale=3.0)[0]
    kk = intrinsics(1)

    def cams(moved):
        def fn(c, L):
            per_frame = poses[2 * c : 2 * c + 2] @ (world if moved else torch.eye(4, dtype=F64))
            return per_frame.repeat_interleave(L // 2, dim=0)[None], kk.expand(1, L, 3, 3)
        return fn

    a, _ = _branch_rollout(cams(False))
    b, _ = _branch_rollout(cams(True))
    flat, _ = _branch_rollout(lambda c, L: (torch.eye(4, dtype=F64).expand(1, L, 4, 4), kk.expand(1, L, 3, 3)))
    for x, y, z in zip(a, b, flat):
        assert torch.allclose(x, y, atol=1e-9)
    assert not torch.allclose(a[-1], flat[-1], atol=1e-3)
