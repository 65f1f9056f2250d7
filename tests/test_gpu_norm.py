"""GPU parity of the commit-path fusion: q/k RMSNorm folded into the append and the attention
Q load, and the cross-attention cache, against the oracle (WanRMSNorm causal_model.py:908-910,
model.py:69-84; WanCrossAttention model.py:152-184).

Bars: the inverse RMS within 1e-5 relative of float64; normalised K within one bf16 rounding of
the float64 norm (the kernels evaluate x * rms * w in fp32 and round once; the reference's
in-dtype bf16 sequence rounds about four times); raw V bit-exact; fp8 codes and scales
bit-exact against the oracle's quantisation of the normalised bf16 K the same append writes;
attention within the bf16 bars of tests/helpers.py.
"""

from types import SimpleNamespace

import pytest
import torch

from oracle import wan_cache_ref as ref
from solarwm_amd import (RopeConfig, apply_cache_updates, attend_cached, cross_attend, kernels,
                         make_crossattn_cache_allocator, make_kv_cache_allocator, rope)

from .helpers import assert_attn_close

pytestmark = pytest.mark.gpu

BF = torch.bfloat16
EPS = 1e-6


def _say(*a):
    print(*a, flush=True)


def _rand(shape, seed, dtype=BF, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def _weight(n, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.rand(n, generator=g) + 0.5


def _rows_scaled(shape, seed, dtype=BF):
    """Rows with RMS spread over two decades, so the per-token statistic matters."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g) * torch.exp(torch.randn(shape[0], shape[1], 1, 1, generator=g) * 1.2)
    return x.to(dtype)


def _within_bf16(got, want):
    d = (got.double() - want.double()).abs()
    return bool((d <= want.double().abs() * 2.0**-8 + 1e-6).all()), float(d.max())


@pytest.mark.parametrize("dtype", [BF, torch.float32])
@pytest.mark.parametrize("wide", [False, True])
def test_rms_rows_vs_f64(gpu, dtype, wide):
    _say("rms rows", dtype, wide)
    B, L, H = 2, 300, 12
    x = _rows_scaled((B, L, H + 2 if wide else H, 128), 1, dtype)[:, :, :H]
    xd = x.to(gpu)
    got = kernels.rms_rows(xd, EPS).cpu().double()
    xf = x.double().reshape(B, L, H * 128)
    want = 1.0 / torch.sqrt(xf.pow(2).mean(-1) + EPS)
    assert torch.allclose(got, want, rtol=1e-5, atol=0)


@pytest.mark.parametrize("use_rope", [False, True])
def test_append_norm_bf16(gpu, use_rope):
    _say("append norm bf16", use_rope)
    gh, gw = 30, 52
    T, H, B = gh * gw, 4, 2
    k, v = _rows_scaled((B, 2 * T, H, 128), 2), _rand((B, 2 * T, H, 128), 3)
    w = _weight(H * 128, 4)
    kd = k.to(gpu)
    inv = kernels.rms_rows(kd, EPS)
    kp, vp, _, _ = kernels.new_pools(3, B, H, T, BF, gpu)
    extra = {}
    if use_rope:
        hw = rope.spatial_table(RopeConfig(grid_hw=(gh, gw)), gpu)
        extra = dict(kr_pool=torch.zeros_like(kp), rope_hw=hw, grid_hw=(gh, gw))
    kernels.append_frames(kd, v.to(gpu), kp, vp, [2, 0], frame_tokens=T,
                          k_norm=(inv, w.to(gpu)), **extra)
    torch.cuda.synchronize()
    want = ref.norm_heads(k, w, EPS)
    for i, s in enumerate([2, 0]):
        got = kp[s, :, :, :T].permute(0, 2, 1, 3).cpu()
        ok, err = _within_bf16(got, want[:, i * T : (i + 1) * T])
        assert ok, (i, err)
        assert torch.equal(vp[s, :, :, :, :T].permute(0, 3, 1, 2).cpu(), v[:, i * T : (i + 1) * T])
        if use_rope:  # the RoPE copy derives from the stored normalised value
            rk = ref.rope_frames(got.double(), (gh, gw), [0], ref.wan_rope_freqs())
            ok, err = _within_bf16(extra["kr_pool"][s, :, :, :T].permute(0, 2, 1, 3).cpu(), rk)
            assert ok, ("rope copy", i, err)


@pytest.mark.parametrize("src,T,B,H", [(BF, 1560, 1, 3), (BF, 100, 1, 3), (BF, 1700, 1, 3),
                                       (torch.float32, 390, 1, 3), (BF, 1560, 4, 128),
                                       (BF, 100, 4, 128), (torch.float32, 390, 4, 128)])
def test_append_norm_fp8_codes(gpu, src, T, B, H):
    """fp8 codes and scales of a normalised append equal the oracle's quantisation of the
    normalised K the bf16 append writes.  B=1, H=3 (6 units) runs the tile-split kernels;
    B=4, H=128 (1024 units, 4 per CU) one workgroup per unit: the on-chip kernel with register
    and LDS tiles, with register tiles only, and the two-pass kernel (f32 source)."""
    _say("append norm fp8", src, T, B, H)
    k, v = _rows_scaled((B, T, H, 128), 5, src), _rand((B, T, H, 128), 6, src)
    w = _weight(H * 128, 7)
    kd, vd = k.to(gpu), v.to(gpu)
    norm = (kernels.rms_rows(kd, EPS), w.to(gpu))
    kp, vp, _, _ = kernels.new_pools(1, B, H, T, src, gpu)
    kernels.append_frames(kd, vd, kp, vp, [0], frame_tokens=T, k_norm=norm)
    k8, v8, ks, vs = kernels.new_pools(2, B, H, T, torch.float8_e4m3fn, gpu)
    kernels.append_frames(kd, vd, k8, v8, [1], frame_tokens=T, kscale=ks, vscale=vs, k_norm=norm)
    torch.cuda.synchronize()
    kn = kp[0, :, :, :T].cpu()  # [B, H, T, D] normalised K as the bf16 / f32 pool holds it
    codes, scale = ref.fp8_quantize(kn)
    assert torch.equal(k8[1, :, :, :T].cpu().view(torch.uint8), codes.view(torch.uint8))
    assert torch.equal(ks[1].cpu(), scale)
    codes, scale = ref.fp8_quantize(v.permute(0, 2, 1, 3))
    assert torch.equal(v8[1, ..., :T].cpu().transpose(-1, -2).view(torch.uint8), codes.view(torch.uint8))
    assert torch.equal(vs[1].cpu(), scale)


@pytest.mark.parametrize("pool", [BF, torch.float8_e4m3fn])
def test_attention_q_norm(gpu, pool):
    _say("attention q norm", pool)
    B, H, T, n, Lq = 1, 2, 256, 3, 300
    q = _rows_scaled((B, Lq, H, 128), 8)
    k, v = _rand((B, n * T, H, 128), 9), _rand((B, n * T, H, 128), 10)
    w = _weight(H * 128, 11)
    kp, vp, ks, vs = kernels.new_pools(n, B, H, T, pool, gpu)
    for f in range(n):
        kernels.append_frames(k.to(gpu), v.to(gpu), kp, vp, [f], frame_tokens=T, src_frame0=f,
                              kscale=ks, vscale=vs)
    qd = q.to(gpu)
    got = kernels.attention_frames(qd, kp, vp, list(range(n)), frame_tokens=T, kscale=ks,
                                   vscale=vs, q_norm=(kernels.rms_rows(qd, EPS), w.to(gpu)))
    qn = ref.norm_heads(q, w, EPS)
    if pool == BF:
        assert_attn_close(got, ref.attention(qn, k, v))
    else:  # same kernel fed the normalised bf16 Q directly
        base = kernels.attention_frames(qn.to(BF).to(gpu), kp, vp, list(range(n)), frame_tokens=T,
                                        kscale=ks, vscale=vs)
        assert float((got.float() - base.float()).abs().max()) < 2e-2


@pytest.mark.parametrize("use_rope", [False, True])
def test_cached_rollout_with_norms(gpu, use_rope):
    """attend_cached with the raw projections and the layer's norm modules vs the oracle fed
    norm_q(q) / norm_k(k): every pass within the bars; the cache's V bit-exact and its K within
    one bf16 rounding of the float64 norm."""
    _say("rollout norms", use_rope)
    gh, gw = 8, 8
    T, H, nb, sink, cap, chunks = gh * gw, 2, 2, 1, 6, 5
    nq = SimpleNamespace(weight=_weight(H * 128, 12).to(BF), eps=EPS)
    nk = SimpleNamespace(weight=_weight(H * 128, 13).to(BF), eps=EPS)
    cfg = RopeConfig(grid_hw=(gh, gw)) if use_rope else None
    cache = make_kv_cache_allocator(num_layers=1, num_heads=H, head_dim=128, frame_sequence_length=T,
                                    local_attn_size=cap, sink_size=sink, num_frame_per_block=nb,
                                    rope=cfg)(1, dtype=BF, device=gpu)[0]
    oc = ref.allocate_kv_cache(num_layers=1, batch_size=1, cache_tokens=cap * T, num_heads=H,
                               head_dim=128, dtype=BF)[0]
    orope = ({"freqs": ref.wan_rope_freqs(), "grid_hw": (gh, gw), "use_echorope": True,
              "rope_train_frames": None} if use_rope else None)
    seed = 50
    for c in range(chunks):
        for commit in (False, True):
            seed += 1
            q, k = _rows_scaled((1, nb * T, H, 128), seed * 3), _rows_scaled((1, nb * T, H, 128), seed * 3 + 1)
            v = _rand((1, nb * T, H, 128), seed * 3 + 2)
            x, info = attend_cached(q.to(gpu), k.to(gpu), v.to(gpu), cache, c * nb * T,
                                    norm_q=nq, norm_k=nk)
            qn = ref.norm_heads(q, nq.weight.float(), EPS).to(BF)
            kn = ref.norm_heads(k, nk.weight.float(), EPS).to(BF)
            want, oinfo = ref.cached_self_attention(qn, kn, v, oc, current_start=c * nb * T,
                                                    frame_seqlen=T, sink_size=sink,
                                                    local_attn_size=cap, rope=orope)
            torch.cuda.synchronize()
            assert_attn_close(x, want)
            if commit:
                apply_cache_updates([cache], [(0, info)])
                ref.apply_cache_updates([oc], [(0, oinfo)])
    assert torch.equal(cache["v"].cpu(), oc["v"])
    # both caches hold a bf16 rounding of (nearly) the same normalised value: one ulp apart at most
    d = (cache["k"].cpu().double() - oc["k"].double()).abs()
    assert bool((d <= oc["k"].double().abs() * 2.0**-7 + 1e-6).all()), float(d.max())


def test_cross_attention_cache(gpu):
    _say("cross attention cache")
    B, H, L1, L2 = 2, 3, 700, 512
    alloc = make_crossattn_cache_allocator(num_layers=2, num_heads=H, head_dim=128)
    caches = alloc(B, dtype=BF, device=gpu)
    nq = SimpleNamespace(weight=_weight(H * 128, 20), eps=EPS)
    nk = SimpleNamespace(weight=_weight(H * 128, 21), eps=EPS)
    q = _rows_scaled((B, L1, H, 128), 22)
    ck, cv = _rows_scaled((B, L2, H, 128), 23), _rand((B, L2, H, 128), 24)
    ck2, cv2 = _rand((B, L2, H, 128), 25), _rand((B, L2, H, 128), 26)
    assert not caches[0]["is_init"]
    x1 = cross_attend(q.to(gpu), ck.to(gpu), cv.to(gpu), caches[0], norm_q=nq, norm_k=nk)
    x2 = cross_attend(q.to(gpu), ck2.to(gpu), cv2.to(gpu), caches[0], norm_q=nq, norm_k=nk)
    torch.cuda.synchronize()
    oc = {"k": None, "v": None, "is_init": False}
    want = ref.cross_attention(q, ck, cv, oc, norm_q=lambda t: ref.norm_heads(t, nq.weight, EPS),
                               norm_k=lambda t: ref.norm_heads(t, nk.weight, EPS))
    assert caches[0]["is_init"] and not caches[1]["is_init"]
    assert torch.equal(x1, x2)  # the second context is ignored, as in the reference
    assert_attn_close(x1, want)
    assert torch.equal(caches[0]["v"].cpu(), cv)
    ok, err = _within_bf16(caches[0]["k"].cpu(), ref.norm_heads(ck, nk.weight, EPS))
    assert ok, err
    with pytest.raises(NotImplementedError):
        cross_attend(q.to(gpu), None, None, caches[0], context_lens=torch.tensor([5, 6]))
