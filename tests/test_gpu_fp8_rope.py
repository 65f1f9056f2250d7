"""GPU parity of fp8 caches on the pre-RoPE (RoPE on load) and fused-PRoPE paths.

An fp8 pre-RoPE cache keeps the raw frames as e4m3 codes with per-(slot, stream, head) scales, as
the post-RoPE fp8 cache does, plus fp8 copies the attention reads: K with its height/width RoPE
pairs rotated (and, camera-aware, P⁻¹ on K's spatial groups and P⁻¹ v), each with its own scales.
RoPE on load over frames of at least 64 tokens runs the fp8-MFMA kernel: the query's spatial
pairs are turned once, its temporal pairs per key frame, and it is quantised per row to e4m3 with
a bound no turn exceeds.  Shorter frames and fused PRoPE run the bf16 kernel, which decodes each
staged tile to bf16 with its frame's scale and multiplies in bf16.

Bars:
* raw codes and scales bit-exact against the oracle quantisation of the raw frames;
* copy codes and scales bit-exact against the e4m3 quantisation of the bf16 (f32) copies the
  bf16 / f32 append writes for the same source (those copies are pinned against float64 in
  tests/test_gpu_rope.py and tests/test_gpu_prope.py);
* fp8-MFMA attention against ``fp8_rope_attention`` (the per-key-frame e4m3 query of the
  kernel's contract, reproduced code for code, over the decoded copy; float64 softmax; pinned in
  tests/test_oracle.py) with the normalised bars of the post-RoPE fp8 kernel (tests/helpers.py),
  and on N(0,1) data against the float64 RoPE oracle with the north-star fp8 bars;
* bf16-decode attention (frames under 64 tokens) bit-identical to the bf16 kernel over bf16
  pools holding the decoded values bf16(code x scale), in the same launch shape, and against the
  oracle's float64 RoPE (and PRoPE) path run on the effective inputs of the decoded copies
  (``fp8_rope_copy_effective``, ``prope_ref.fp8_prope_copies_effective``, pinned in
  tests/test_oracle.py): what remains is bf16 arithmetic (error divided by each channel's V RMS;
  K/V carry 1% x20 outlier channels, whose sharper logits put it above the N(0,1) bars).
"""

import pytest
import torch

from oracle import prope_ref as pr
from oracle import wan_cache_ref as ref
from solarwm_amd import (PropeConfig, RopeConfig, apply_cache_updates, attend_cached,
                         commit_camera_cache, kernels, make_kv_cache_allocator, rope,
                         stage_camera_cache)

from .cameras import per_token, trajectory
from .helpers import (FP8_MAX_ABS, FP8_MEAN_ABS, FP8_NORM_MAX, FP8_NORM_MEAN, MAX_ABS, MEAN_ABS,
                      assert_attn_close)

pytestmark = pytest.mark.gpu

# Normalised error (divided by each channel's V RMS) of the bf16-decode kernel (frames under 64
# tokens) over the decoded fp8 frames against the float64 oracle, on K/V with x20 outlier
# channels.  The kernel rounds the query to bf16 after turning its temporal pairs per key frame,
# the oracle rounds the turned key instead; on an outlier key channel that rounding moves a logit
# by up to ~0.03, so the largest output errors reach ~0.06-0.08 while the mean stays at the bf16
# level (1.1e-3 to 2.2e-3 over these tests and the random shapes of test_gpu_random_rope.py).
# The bf16 kernel over the same decoded pools measures the same errors (its outputs are
# bit-identical, checked below).  A frame decoded with another frame's scale (1.25x or 2x)
# measures 0.3-4.5 (tests/helpers.py).
FP8_BF16_MAX, FP8_BF16_MEAN = 0.1, 3e-3

BF = torch.bfloat16
F8 = torch.float8_e4m3fn


def _say(*a):
    print(*a, flush=True)


def _outlier(shape, seed, dtype=BF):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g)
    x[..., torch.randperm(shape[-1], generator=g)[: max(1, shape[-1] // 100)]] *= 20.0
    return x.to(dtype)


def _frames(pool, s, T, vt):
    """[B, H, T, D] of slot s of a pool (V pools stored transposed)."""
    x = pool[s]
    return x[..., :T].transpose(-1, -2) if vt else x[:, :, :T]


def _assert_codes(pool, scale, slot, want_frame, T, vt):
    codes, sc = ref.fp8_quantize(want_frame)
    got = _frames(pool, slot, T, vt).cpu()
    assert torch.equal(got.view(torch.uint8), codes.view(torch.uint8))
    assert torch.equal(scale[slot].cpu(), sc)
    pad = pool[slot][..., T:] if vt else pool[slot][:, :, T:]
    assert int(pad.view(torch.uint8).count_nonzero()) == 0


@pytest.mark.parametrize("B,H,gh,gw,src,prope", [
    (1, 3, 8, 8, BF, False),        # few units: one-pass raw kernel, then the copies' tile grids
    (4, 12, 30, 52, BF, False),     # C5's chunk
    (2, 2, 10, 10, torch.float32, False),
    (16, 24, 8, 8, BF, False),      # 2304 units: per-unit raw kernels, then the copies
    (1, 3, 8, 8, BF, True),
    (2, 3, 10, 10, BF, True),
    (4, 12, 30, 52, BF, True),
])
def test_fp8_append_copies(gpu, B, H, gh, gw, src, prope):
    T = gh * gw
    _say("fp8 append copies", B, H, gh, gw, src, "prope" if prope else "rope")
    k, v = _outlier((B, 3 * T, H, 128), 1, src), _outlier((B, 3 * T, H, 128), 2, src)
    kd, vd = k.to(gpu), v.to(gpu)
    cfg = RopeConfig(grid_hw=(gh, gw))
    hw = rope.spatial_table(cfg, gpu)
    slots = [4, 1, 2]
    xf = None
    if prope:
        vm, ks = trajectory(B, 3, seed=9, t_scale=0.8)
        _, _, pinv = pr.projection_matrices(vm.double(), ks.double())
        xf = pinv.transpose(0, 1).to(torch.float32).contiguous().to(gpu)  # [3, B, 4, 4]
    # fp8 pools and copies (stale bytes everywhere first)
    kp, vp, ks8, vs8 = kernels.new_pools(6, B, H, T, F8, gpu)
    krp = torch.empty_like(kp)
    vrp = torch.empty_like(vp) if prope else None
    for t in (kp, vp, krp) + ((vrp,) if prope else ()):
        t.view(torch.uint8).fill_(0x55)
    krs = torch.full_like(ks8, 7.0)
    vrs = torch.full_like(vs8, 7.0) if prope else None
    kernels.append_frames(kd, vd, kp, vp, slots, frame_tokens=T, kscale=ks8, vscale=vs8,
                          kr_pool=krp, rope_hw=hw, grid_hw=(gh, gw), vr_pool=vrp, kv_xform=xf,
                          kr_scale=krs, vr_scale=vrs)
    # the bf16 / f32 copies of the same source
    rdt = BF if src == BF else torch.float32
    bkp, bvp, _, _ = kernels.new_pools(6, B, H, T, rdt, gpu)
    bkr = torch.zeros_like(bkp)
    bvr = torch.zeros_like(bvp) if prope else None
    kernels.append_frames(kd, vd, bkp, bvp, slots, frame_tokens=T, kr_pool=bkr, rope_hw=hw,
                          grid_hw=(gh, gw), vr_pool=bvr, kv_xform=xf)
    torch.cuda.synchronize()
    for f, s in enumerate(slots):
        raw_k = k[:, f * T : (f + 1) * T].permute(0, 2, 1, 3)
        raw_v = v[:, f * T : (f + 1) * T].permute(0, 2, 1, 3)
        _assert_codes(kp, ks8, s, raw_k, T, False)
        _assert_codes(vp, vs8, s, raw_v, T, True)
        _assert_codes(krp, krs, s, _frames(bkr, s, T, False).cpu(), T, False)
        if prope:
            _assert_codes(vrp, vrs, s, _frames(bvr, s, T, True).cpu(), T, True)
    assert int(krp[0].view(torch.uint8).ne(0x55).sum()) == 0  # slots not written stay stale
    assert float(krs[0].max()) == 7.0


def _rope_pools(k, v, B, H, gh, gw, n, slots, gpu):
    T = gh * gw
    hw = rope.spatial_table(RopeConfig(grid_hw=(gh, gw)), gpu)
    kp, vp, ks8, vs8 = kernels.new_pools(n + 2, B, H, T, F8, gpu)
    krp, krs = torch.zeros_like(kp), torch.zeros_like(ks8)
    kd, vd = k.to(gpu), v.to(gpu)
    for j in range(n):
        kernels.append_frames(kd, vd, kp, vp, [slots[j]], frame_tokens=T, src_frame0=j,
                              kscale=ks8, vscale=vs8, kr_pool=krp, rope_hw=hw, grid_hw=(gh, gw),
                              kr_scale=krs)
    return hw, krp, krs, vp, vs8


@pytest.mark.parametrize("B,H,gh,gw,kpos,qpos,split", [
    (1, 2, 8, 8, [0, 4, 5, 6, 7], [6, 7], False),
    (2, 3, 10, 10, [0, 1, 2, 3, 4, 5], [3, 4, 5], False),
    (1, 2, 30, 52, [0, 1, 2, 3, 4, 5], [5], True),  # one frame of queries: the balanced split
    (1, 2, 4, 8, [0, 2, 3, 4, 5, 6], [5, 6], False),  # 32-token frames: the bf16-decode kernel
])
def test_fp8_attention_rope_vs_oracle(gpu, B, H, gh, gw, kpos, qpos, split):
    T = gh * gw
    n, nq = len(kpos), len(qpos)
    _say("fp8 attention rope", B, H, gh, gw, kpos, qpos)
    g = torch.Generator().manual_seed(12)
    q = torch.randn((B, nq * T, H, 128), generator=g).to(BF)
    k, v = _outlier((B, n * T, H, 128), 13), _outlier((B, n * T, H, 128), 14)
    f = ref.wan_rope_freqs()
    v_eff = ref.fp8_fake_quant_frames(v.float(), T).double()
    if T >= 64:  # the fp8-MFMA kernel's own quantised query over the decoded copy
        want = ref.fp8_rope_attention(q, ref.fp8_rope_copy_decoded(k, (gh, gw), f, T), v_eff,
                                      (gh, gw), qpos, kpos, T)
        bar_max, bar_mean = FP8_NORM_MAX, FP8_NORM_MEAN
    else:
        k_eff = ref.fp8_rope_copy_effective(k, (gh, gw), f, T)
        want = ref.attention(ref.rope_frames(q, (gh, gw), qpos, f),
                             ref.rope_frames(k_eff, (gh, gw), kpos, f), v_eff)
        bar_max, bar_mean = FP8_BF16_MAX, FP8_BF16_MEAN
    slots = torch.randperm(n + 2, generator=g)[:n].tolist()
    hw, krp, krs, vp, vs8 = _rope_pools(k, v, B, H, gh, gw, n, slots, gpu)
    qd = q.to(gpu)
    rt = (hw, (gh, gw), rope.temporal_table(qpos, kpos, RopeConfig(grid_hw=(gh, gw)), gpu))
    args = dict(frame_tokens=T, kscale=krs, vscale=vs8, rope=rt)
    plan = kernels.attention_plan(qd, krp, vp, slots, **args)
    assert (plan["split"] > 0) == split, plan
    outs = [kernels.attention_frames(qd, krp, vp, slots, **args)]
    if split:
        outs.append(kernels.attention_frames(qd, krp, vp, slots, use_workspace=False, **args))
    refs = []
    if T < 64:
        # the bf16 kernel over bf16 pools holding the decoded values bf16(code x scale): the
        # bf16-decode instances stage each tile to exactly these values and run the same products
        kdec = (krp.float() * krs[..., None, None]).to(BF)
        vdec = (vp.float() * vs8[..., None, None]).to(BF)
        refs = [kernels.attention_frames(qd, kdec, vdec, slots, frame_tokens=T, rope=rt,
                                         use_workspace=ws) for ws in ((True, False) if split else (True,))]
    torch.cuda.synchronize()
    rms_v = v_eff.pow(2).mean(dim=1, keepdim=True).sqrt()
    for i, out in enumerate(outs):
        assert out.dtype == BF and torch.isfinite(out).all()
        mode = "split" if split and i == 0 else "unsplit"
        e = (out.cpu().double() - want.double()).abs() / rms_v
        _say(f"  {mode}: normalised error max {float(e.max()):.3e} mean {float(e.mean()):.3e}")
        if refs:
            assert torch.equal(out, refs[i]), mode  # same launch shape, same arithmetic
        assert float(e.max()) <= bar_max and float(e.mean()) <= bar_mean


def test_fp8_rope_split_segment_ending_on_its_largest_logit(gpu):
    """Regression: balanced-split segments whose last key tile holds their rows' largest logit.

    With these inputs (N(0,1), one frame of queries over 6 key frames, 256 workgroups over 14
    q-tiles x 150 tiles) the segment of workgroup 211 covers tiles 80..88 of (head 1, q-tile 4)
    and row 36 of that q-tile meets its largest logit (log2 units 7.7 against 2.4 before) in
    tile 88.  Its probabilities then overflow e4m3 and the row-sum product turns NaN, which must
    send the wave to the rare path before the last PV product.  The read of that row sum once
    came 2 issue slots after the product on the path that skips the mask block (too early for an
    8-pass product), so the wave kept the previous tile's sum and rows 36 and 52 (which share the
    row-sum product's column) came out NaN.  Every row of the split and unsplit launches is
    checked against the quantisation-exact oracle."""
    B, H, gh, gw, kpos, qpos = 1, 2, 30, 52, [0, 1, 2, 3, 4, 5], [5]
    T, n = gh * gw, len(kpos)
    _say("fp8 rope split, segment ending on its largest logit")
    g = torch.Generator().manual_seed(12)
    q = torch.randn((B, T, H, 128), generator=g).to(BF)
    k = torch.randn((B, n * T, H, 128), generator=g).to(BF)
    v = torch.randn((B, n * T, H, 128), generator=g).to(BF)
    f = ref.wan_rope_freqs()
    v_eff = ref.fp8_fake_quant_frames(v.float(), T).double()
    want = ref.fp8_rope_attention(q, ref.fp8_rope_copy_decoded(k, (gh, gw), f, T), v_eff,
                                  (gh, gw), qpos, kpos, T)
    slots = list(range(n))
    hw, krp, krs, vp, vs8 = _rope_pools(k, v, B, H, gh, gw, n, slots, gpu)
    rt = (hw, (gh, gw), rope.temporal_table(qpos, kpos, RopeConfig(grid_hw=(gh, gw)), gpu))
    args = dict(frame_tokens=T, kscale=krs, vscale=vs8, rope=rt)
    plan = kernels.attention_plan(q.to(gpu), krp, vp, slots, **args)
    assert plan["split"] > 0, plan
    outs = [kernels.attention_frames(q.to(gpu), krp, vp, slots, use_workspace=ws, **args)
            for ws in (True, False)]
    torch.cuda.synchronize()
    rms_v = v_eff.pow(2).mean(dim=1, keepdim=True).sqrt()
    for mode, out in zip(("split", "unsplit"), outs):
        assert torch.isfinite(out).all(), (mode, (~torch.isfinite(out)).nonzero()[:4].tolist())
        e = (out.cpu().double() - want).abs() / rms_v
        _say(f"  {mode}: normalised error max {float(e.max()):.3e} mean {float(e.mean()):.3e}; "
             f"rows 1060, 1076 of head 1 max {float(e[0, [1060, 1076], 1].max()):.3e}")
        assert float(e.max()) <= FP8_NORM_MAX and float(e.mean()) <= FP8_NORM_MEAN, mode


@pytest.mark.parametrize("B,H,gh,gw,kpos,qpos", [
    (1, 2, 30, 52, [0, 1, 2, 3, 4, 5], [5]),
    (2, 3, 10, 10, [0, 1, 2, 3, 4, 5, 6, 7], [6, 7]),
])
def test_fp8_attention_rope_unit_scale_vs_bf16_oracle(gpu, B, H, gh, gw, kpos, qpos):
    """N(0,1) Q/K/V: RoPE on load over an fp8 cache meets the north-star fp8 bar against the
    float64 RoPE oracle over the bf16 inputs (query, key and probability roundings included)."""
    T = gh * gw
    n, nq = len(kpos), len(qpos)
    _say("fp8 attention rope unit scale", B, H, gh, gw, kpos, qpos)
    g = torch.Generator().manual_seed(15)
    q, k, v = (torch.randn((B, L * T, H, 128), generator=g).to(BF) for L in (nq, n, n))
    f = ref.wan_rope_freqs()
    want = ref.attention(ref.rope_frames(q, (gh, gw), qpos, f), ref.rope_frames(k, (gh, gw), kpos, f),
                         v, compute_dtype=torch.float32)
    slots = list(range(n))
    hw, krp, krs, vp, vs8 = _rope_pools(k, v, B, H, gh, gw, n, slots, gpu)
    rt = (hw, (gh, gw), rope.temporal_table(qpos, kpos, RopeConfig(grid_hw=(gh, gw)), gpu))
    out = kernels.attention_frames(q.to(gpu), krp, vp, slots, frame_tokens=T, kscale=krs,
                                   vscale=vs8, rope=rt)
    torch.cuda.synchronize()
    assert_attn_close(out, want, FP8_MAX_ABS, FP8_MEAN_ABS)


def _oracle_cache(B, cap, T, H, dtype):
    return ref.allocate_kv_cache(num_layers=1, batch_size=B, cache_tokens=cap * T, num_heads=H,
                                 head_dim=128, dtype=dtype)


@pytest.mark.parametrize("sink,cap,gh,gw,nb,chunks,echo,rtf,B,H", [
    (1, 6, 8, 8, 2, 5, True, None, 2, 3),
    (0, 5, 10, 10, 2, 4, True, None, 1, 2),
    (1, 5, 8, 8, 2, 4, False, 4, 1, 2),
    (0, 18, 15, 27, 3, 7, False, 21, 1, 2),  # the release geometry's RoPE (no sink, odd T)
])
def test_fp8_rope_rollout_vs_oracle(gpu, sink, cap, gh, gw, nb, chunks, echo, rtf, B, H):
    """Pre-RoPE fp8 rollout (2 passes per chunk, commit on the second): every pass against the
    oracle's window with the fp8-MFMA kernel's quantised query (``fp8_rope_attention`` at the
    window's RoPE positions) over the decoded copies; the committed raw codes and scales equal
    the oracle quantisation of the oracle's raw bf16 cache."""
    T = gh * gw
    _say("fp8 rollout rope", sink, cap, gh, gw, nb, chunks, echo, rtf, B, H)
    cfg = RopeConfig(grid_hw=(gh, gw), use_echorope=echo, rope_train_frames=rtf)
    cache = make_kv_cache_allocator(
        num_layers=1, num_heads=H, head_dim=128, frame_sequence_length=T, local_attn_size=cap,
        sink_size=sink, num_frame_per_block=nb, rope=cfg, cache_dtype=F8)(B, dtype=BF, device=gpu)[0]
    o_eff = _oracle_cache(B, cap, T, H, torch.float64)[0]
    o_raw = _oracle_cache(B, cap, T, H, BF)[0]
    f = ref.wan_rope_freqs()
    orope = {"freqs": f, "grid_hw": (gh, gw), "use_echorope": echo, "rope_train_frames": rtf}
    g = torch.Generator().manual_seed(20)
    for c in range(chunks):
        for commit in (False, True):
            q = torch.randn((B, nb * T, H, 128), generator=g).to(BF)
            k = _outlier((B, nb * T, H, 128), 100 + 2 * c + commit)
            v = _outlier((B, nb * T, H, 128), 200 + 2 * c + commit)
            start = c * nb * T
            x, info = attend_cached(q.to(gpu), k.to(gpu), v.to(gpu), cache, start)
            k_eff = ref.fp8_rope_copy_effective(k, (gh, gw), f, T)
            v_eff = ref.fp8_fake_quant_frames(v.float(), T).double()
            args = dict(current_start=start, frame_seqlen=T, sink_size=sink, local_attn_size=cap)
            seen = {}

            def attend(qq, kk, vv, qp, kp):  # the window's copy: spatial pairs turned, temporal raw
                seen["v"] = vv
                kc = ref.rope_frames(kk, (gh, gw), [0] * (kk.shape[1] // T), f)
                return ref.fp8_rope_attention(qq, kc, vv, (gh, gw), qp, kp, T)

            want, oinfo = ref.cached_self_attention(q, k_eff, v_eff, o_eff,
                                                    rope=dict(orope, attend=attend), **args)
            _, rinfo = ref.cached_self_attention(q, k, v, o_raw, attn_fn=lambda *a: torch.zeros(0),
                                                 **args)
            torch.cuda.synchronize()
            rms_v = seen["v"].double().pow(2).mean(dim=1, keepdim=True).sqrt()
            e = (x.cpu().double() - want.double()).abs() / rms_v
            _say(f"  chunk {c} commit {commit}: normalised max {float(e.max()):.3e} "
                 f"mean {float(e.mean()):.3e}")
            assert torch.isfinite(x).all()
            assert float(e.max()) <= FP8_NORM_MAX and float(e.mean()) <= FP8_NORM_MEAN
            if commit:
                apply_cache_updates([cache], [(0, info)])
                ref.apply_cache_updates([o_eff], [(0, oinfo)])
                ref.apply_cache_updates([o_raw], [(0, rinfo)])
    for p in range(cap):
        slot = cache.table[p]
        _assert_codes(cache.kpool, cache.kscale, slot,
                      o_raw["k"][:, p * T : (p + 1) * T].permute(0, 2, 1, 3), T, False)
        _assert_codes(cache.vpool, cache.vscale, slot,
                      o_raw["v"][:, p * T : (p + 1) * T].permute(0, 2, 1, 3), T, True)


def _errors(got, want):
    d = (got.double() - want.double()).abs().flatten()
    return float(d.max()), float(d.kthvalue(max(1, int(d.numel() * 0.999))).values), float(d.mean())


@pytest.mark.parametrize("sink,cap,gh,gw,chunks,transform,B", [
    (1, 6, 8, 8, 5, "linear", 1),
    (0, 5, 10, 10, 4, "logd4", 2),
])
def test_fp8_prope_rollout_vs_oracle(gpu, sink, cap, gh, gw, chunks, transform, B):
    """Camera-aware fp8 rollout (2 passes per chunk, commit on the second): each pass against the
    oracle's RoPE-then-PRoPE over the effective inputs of the decoded copies, with the bars of
    tests/test_gpu_prope.py (the reference's own bf16 arithmetic on the same inputs sets them);
    layer 0's camera metadata equals the oracle's camera cache."""
    T, H, nb = gh * gw, 2, 2
    _say("fp8 rollout prope", sink, cap, gh, gw, chunks, transform, B)
    cfg = RopeConfig(grid_hw=(gh, gw))
    caches = make_kv_cache_allocator(
        num_layers=1, num_heads=H, head_dim=128, frame_sequence_length=T, local_attn_size=cap,
        sink_size=sink, num_frame_per_block=nb, rope=cfg, cache_dtype=F8,
        prope=PropeConfig(camera_translation_transform=transform))(B, dtype=BF, device=gpu)
    oc = _oracle_cache(B, cap, T, H, torch.float64)
    f = ref.wan_rope_freqs()
    orope = {"freqs": f, "grid_hw": (gh, gw), "use_echorope": True, "rope_train_frames": None}
    vm, ks = trajectory(B, chunks * nb, seed=31, t_scale=0.6)
    vm_tok, ks_tok = per_token(vm, T), per_token(ks, T)
    vm_dev, ks_dev = vm_tok.to(gpu), ks_tok.to(gpu)
    g = torch.Generator().manual_seed(32)
    for c in range(chunks):
        for commit in (False, True):
            start = c * nb * T
            rows = slice(start, start + nb * T)
            q = torch.randn((B, nb * T, H, 128), generator=g).to(BF)
            k = _outlier((B, nb * T, H, 128), 300 + 2 * c + commit)
            v = _outlier((B, nb * T, H, 128), 400 + 2 * c + commit)
            cp = stage_camera_cache(caches, vm_dev, ks_dev, start, nb * T)
            x, info = attend_cached(q.to(gpu), k.to(gpu), v.to(gpu), caches[0], start, camera=cp)
            _, _, p_inv = pr.projection_matrices(
                pr.transform_relative_viewmats(vm_tok[:, rows].double(), transform),
                ks_tok[:, rows].double())
            k_eff, v_eff = pr.fp8_prope_copies_effective(k, v, p_inv, (gh, gw), f, T)
            cq, ck, tv, tk, oupd = pr.stage_fused_camera_cache(
                oc, cam_viewmats=vm_tok, cam_ks=ks_tok, current_start=start,
                num_new_tokens=nb * T, frame_seqlen=T, sink_size=sink, local_attn_size=cap)
            cams = {"q_viewmats": cq, "q_ks": ck, "kv_viewmats": tv, "kv_ks": tk,
                    "transform": transform}
            args = dict(current_start=start, frame_seqlen=T, sink_size=sink, local_attn_size=cap,
                        rope=orope)
            want, oinfo = ref.cached_self_attention(q, k_eff, v_eff, oc[0], prope=cams, **args)
            want_ref, _ = ref.cached_self_attention(q, k_eff.to(BF), v_eff.to(BF), oc[0],
                                                    prope=dict(cams, emulate_bf16=True), **args)
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
    meta, st = caches[0]["_fused_prope_camera_metadata"], oc[0][pr.STATE_KEY]
    assert torch.equal(meta["viewmats"].cpu(), st["viewmats"]) and torch.equal(meta["K"].cpu(), st["K"])
