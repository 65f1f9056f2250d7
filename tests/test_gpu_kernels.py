"""GPU parity of the append / gather / attention kernels against the CPU oracle.

Bars: integer/byte movement bit-exact; attention within 2e-2 max-abs and 1e-3 mean-abs error
(bf16 operands, fp32 accumulation) of the oracle's float64 SDPA on the same bf16-rounded inputs.
"""

import pytest
import torch

from oracle import wan_cache_ref as ref
from solarwm_amd import _lib, kernels
from solarwm_amd.attention import attention, chunk_causal_attention

from .helpers import assert_attn_close

pytestmark = pytest.mark.gpu



def _say(*a):
    print(*a, flush=True)


def _rand(shape, seed, dtype=torch.float32, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,H,T", [(1, 12, 390), (2, 3, 100), (1, 2, 64), (1, 1, 1560)])
def test_append_gather_roundtrip_and_layout(gpu, dtype, B, H, T):
    _say("append/gather", dtype, B, H, T)
    n_slots, n_new = 7, 3
    # strided source: K and V are views into one packed [B, L, 3, H, D] tensor
    packed = _rand((B, n_new * T, 3, H, 128), seed=T + H, dtype=dtype).to(gpu)
    k_src, v_src = packed[:, :, 1], packed[:, :, 2]
    kpool, vpool, _, _ = kernels.new_pools(n_slots, B, H, T, dtype, gpu)
    vpool.fill_(7)  # padding rows must come back as zeros after an append
    slots = [5, 0, 3]
    kernels.append_frames(k_src, v_src, kpool, vpool, slots, frame_tokens=T)
    torch.cuda.synchronize()
    Tp = kernels.padded_tokens(T)
    for f, s in enumerate(slots):
        want_k = k_src[:, f * T : (f + 1) * T].permute(0, 2, 1, 3)  # [B, H, T, D]
        want_v = v_src[:, f * T : (f + 1) * T].permute(0, 2, 1, 3)
        assert torch.equal(kpool[s, :, :, :T], want_k)
        assert torch.equal(vpool[s, :, :, :, :T], want_v.transpose(-1, -2))
        if Tp > T:
            assert kpool[s, :, :, T:].abs().sum() == 0 and vpool[s, :, :, :, T:].abs().sum() == 0
    order = [3, 5, 0, 5]
    gk, gv = kernels.gather_frames(kpool, vpool, order, frame_tokens=T)
    torch.cuda.synchronize()
    for j, s in enumerate(order):
        f = slots.index(s)
        assert torch.equal(gk[:, j * T : (j + 1) * T], k_src[:, f * T : (f + 1) * T])
        assert torch.equal(gv[:, j * T : (j + 1) * T], v_src[:, f * T : (f + 1) * T])


@pytest.mark.parametrize("src_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,H,T,wide", [(1, 12, 1560, False), (4, 2, 390, False),
                                        (1, 3, 100, False), (2, 2, 1560, True),
                                        (1, 2, 1700, False), (1, 2, 1153, True),
                                        (4, 64, 100, False), (4, 64, 1700, True)])
def test_fp8_append_matches_oracle(gpu, src_dtype, B, H, T, wide):
    """Chunks with fewer than 4 (frame, batch, head, K|V) units per CU go through the tile-split
    kernels; the B=4, H=64 cases (1024 units) through one workgroup per unit: the on-chip
    kernel for frames of up to 25 tiles from bf16 sources, the two-pass kernel for longer
    frames and f32 sources.  ``wide``: the source is a head slice of a wider tensor (token
    stride > H * 128)."""
    _say("fp8 append", src_dtype, B, H, T, wide)
    x = _rand((B, 2 * T, H + 3 if wide else H, 128), seed=11, dtype=torch.float32)[:, :, :H]
    g = torch.Generator().manual_seed(12)
    outlier = torch.randperm(128, generator=g)[:2]
    x[..., outlier] *= 20.0
    x[0, :T, 0] = 0.0  # an all-zero (frame, head): scale 0, codes 0
    x = x.to(src_dtype)
    v = (x * -0.5).to(src_dtype)
    kpool, vpool, ks, vs = kernels.new_pools(4, B, H, T, torch.float8_e4m3fn, gpu)
    kpool.view(torch.uint8).fill_(0x55), vpool.view(torch.uint8).fill_(0x55)  # stale slots
    xd, vd = x.to(gpu), v.to(gpu)
    if wide:  # keep the head-slice strides on the device
        xd, vd = (torch.zeros((B, 2 * T, H + 3, 128), dtype=src_dtype, device=gpu)[:, :, :H]
                  for _ in range(2))
        xd.copy_(x), vd.copy_(v)
        assert xd.stride(1) == (H + 3) * 128
    kernels.append_frames(xd, vd, kpool, vpool, [2, 1], frame_tokens=T, kscale=ks, vscale=vs)
    torch.cuda.synchronize()
    for f, s in enumerate([2, 1]):
        for src, pool, sc, vt in ((x, kpool, ks, False), (v, vpool, vs, True)):
            frame = src[:, f * T : (f + 1) * T].permute(0, 2, 1, 3)  # [B, H, T, D]
            codes, scale = ref.fp8_quantize(frame)
            got = pool[s].cpu()
            got = got[..., :T].transpose(-1, -2) if vt else got[:, :, :T]
            assert torch.equal(got.view(torch.uint8), codes.view(torch.uint8)), (f, vt)
            assert torch.equal(sc[s].cpu(), scale), (f, vt)
            pad = pool[s][..., T:] if vt else pool[s][:, :, T:]
            assert int(pad.view(torch.uint8).count_nonzero()) == 0, (f, vt)  # rows T..Tp-1


@pytest.mark.parametrize("B,T,forced", [(4, 1560, False), (3, 1560, False), (2, 1560, False),
                                        (4, 1000, False), (1, 1560, False), (4, 1560, True),
                                        (1, 1560, True)])
def test_fp8_append_one_pass_slices(gpu, monkeypatch, B, T, forced):
    """Config-5 chunks (3 frames x B streams x 12 heads) take the one-pass kernel, whose slices
    are 4 / 3 / 2 / 3 / 1 tiles long here (T=1000: a 40-row last tile inside the last slice).
    Codes and scales equal the oracle's and the per-unit kernels', stale slot bytes and padding
    rows are overwritten.  Unforced, every unit completes within the wait (workspace flag word
    0); ``forced`` sets the wait bound to 0 from the host, so workgroups that find their unit
    incomplete take the fallback (re-read the whole unit) and the results must not change."""
    H, nf = 12, 3
    _say("fp8 append one pass", B, H, T, nf, "forced fallback" if forced else "")
    if forced:
        monkeypatch.setenv("SOLARKV_SLICE_WAIT_US", "0")
    g = torch.Generator().manual_seed(40 + B)
    x = torch.randn((B, nf * T, H, 128), generator=g)
    x[..., torch.randperm(128, generator=g)[:3]] *= 25.0
    x[0, T : 2 * T, 5] = 0.0  # an all-zero (frame, head) in the middle frame
    x[B - 1, 2 * T - 1, 7, 3] = 900.0  # the absmax sits in the frame's last row
    x = x.to(torch.bfloat16)
    v = (x.float() * 0.75 - 0.1).to(torch.bfloat16)
    xd, vd = x.to(gpu), v.to(gpu)
    slots = [4, 0, 2]
    outs = []
    for use_ws in (True, False):
        kpool, vpool, ks, vs = kernels.new_pools(6, B, H, T, torch.float8_e4m3fn, gpu)
        kpool.view(torch.uint8).fill_(0x55), vpool.view(torch.uint8).fill_(0x55)
        ks.fill_(7.0), vs.fill_(7.0)
        kernels.append_frames(xd, vd, kpool, vpool, slots, frame_tokens=T, kscale=ks, vscale=vs,
                              use_workspace=use_ws)
        torch.cuda.synchronize()
        if use_ws:  # word 0 of this stream's workspace: the one-pass kernel's fallback flag
            ws = kernels._workspaces[(gpu.index or 0, kernels._stream(gpu))]
            flag = int(ws[:8].view(torch.int64).item())
            assert flag == (1 if forced else 0), \
                f"fallback flag {flag:#x} (not 0/1: the one-pass kernel was not taken)"
        outs.append([t.cpu() for t in (kpool, vpool, ks, vs)])
    for a, b in zip(*outs):
        assert torch.equal(a.view(torch.uint8) if a.dtype != torch.float32 else a,
                           b.view(torch.uint8) if b.dtype != torch.float32 else b)
    kpool, vpool, ks, vs = outs[0]
    for f, s in enumerate(slots):
        for src, pool, sc, vt in ((x, kpool, ks, False), (v, vpool, vs, True)):
            frame = src[:, f * T : (f + 1) * T].permute(0, 2, 1, 3)
            codes, scale = ref.fp8_quantize(frame)
            got = pool[s]
            got = got[..., :T].transpose(-1, -2) if vt else got[:, :, :T]
            assert torch.equal(got.view(torch.uint8), codes.view(torch.uint8)), (f, vt)
            assert torch.equal(sc[s], scale), (f, vt)
            pad = pool[s][..., T:] if vt else pool[s][:, :, T:]
            assert int(pad.view(torch.uint8).count_nonzero()) == 0, (f, vt)
    assert torch.equal(kpool[1].view(torch.uint8), torch.full_like(kpool[1].view(torch.uint8), 0x55))


def test_kept_fp8_append_outlives_workspace_growth(gpu):
    """A kept fp8 append launcher (few units: the one-pass kernel with this stream's workspace)
    must hold its workspace block.  An attention launch that takes the split grows the stream's
    workspace in between; a sentinel of the old block's size is then allocated, and the kept
    launcher runs again: the sentinel is untouched and the codes still match the oracle."""
    B, H, T, nf = 4, 12, 1560, 3
    _say("kept fp8 append across workspace growth", B, H, T, nf)
    g = torch.Generator().manual_seed(90)
    x = torch.randn((B, nf * T, H, 128), generator=g)
    x[..., torch.randperm(128, generator=g)[:2]] *= 20.0
    x = x.to(torch.bfloat16)
    v = (x.float() * 0.5).to(torch.bfloat16)
    kpool, vpool, ks, vs = kernels.new_pools(5, B, H, T, torch.float8_e4m3fn, gpu)
    slots = [3, 0, 4]
    key = (gpu.index or 0, kernels._stream(gpu))
    torch.cuda.synchronize()
    kernels._workspaces.pop(key, None)  # start from no workspace (earlier tests grew it)
    launch = kernels.prepare_append(x.to(gpu), v.to(gpu), kpool, vpool, slots, frame_tokens=T,
                                    kscale=ks, vscale=vs)
    desc = next(o for o in launch.keep if isinstance(o, _lib.AppendDesc))
    ws_small = launch.keep[-1]
    assert ws_small is not None and desc.workspace == ws_small.data_ptr()
    small_bytes = ws_small.numel()
    del ws_small  # from here on only the launcher holds the block
    launch()
    # grow the workspace: one frame of queries over 6 frames splits over every CU
    qa = _rand((1, T, 12, 128), 91, torch.bfloat16).to(gpu)
    ka = _rand((1, 6 * T, 12, 128), 92, torch.bfloat16)
    apool, bpool, aslots = _pool_from(ka, ka, T, torch.bfloat16, gpu)
    plan = kernels.attention_plan(qa, apool, bpool, aslots, frame_tokens=T)
    assert plan["split"] >= 1 and plan["workspace_bytes"] > desc.workspace_bytes, plan
    kernels.attention_frames(qa, apool, bpool, aslots, frame_tokens=T)
    torch.cuda.synchronize()
    assert kernels._workspaces[key].data_ptr() != desc.workspace  # the stream's was replaced
    sentinel = torch.full((small_bytes,), 0xA5, dtype=torch.uint8, device=gpu)
    kpool.view(torch.uint8).fill_(0x55), vpool.view(torch.uint8).fill_(0x55)
    launch()
    torch.cuda.synchronize()
    assert int((sentinel != 0xA5).sum()) == 0, "the kept launcher wrote into a freed workspace"
    for f, s in enumerate(slots):
        for src, pool, sc, vt in ((x, kpool, ks, False), (v, vpool, vs, True)):
            codes, scale = ref.fp8_quantize(src[:, f * T : (f + 1) * T].permute(0, 2, 1, 3))
            got = pool[s].cpu()
            got = got[..., :T].transpose(-1, -2) if vt else got[:, :, :T]
            assert torch.equal(got.view(torch.uint8), codes.view(torch.uint8)), (f, vt)
            assert torch.equal(sc[s].cpu(), scale), (f, vt)


def _pool_from(k, v, T, dtype, device, perm_seed=0):
    """Store dense K/V [B, n*T, H, D] frame by frame in shuffled slots; return pools + order."""
    B, L, H, _ = k.shape
    n = L // T
    g = torch.Generator().manual_seed(perm_seed)
    n_slots = n + 2
    slots = torch.randperm(n_slots, generator=g)[:n].tolist()
    kpool, vpool, _, _ = kernels.new_pools(n_slots, B, H, T, dtype, device)
    kd, vd = k.to(device), v.to(device)
    for f in range(n):
        kernels.append_frames(kd, vd, kpool, vpool, [slots[f]], frame_tokens=T, src_frame0=f)
    return kpool, vpool, slots


@pytest.mark.parametrize(
    "B,H,Lq,T,n,dtype",
    [(1, 2, 128, 64, 2, torch.bfloat16), (1, 3, 200, 100, 5, torch.bfloat16),
     (2, 2, 390, 390, 4, torch.float32), (1, 12, 1170, 390, 6, torch.bfloat16),
     (1, 1, 37, 1560, 3, torch.bfloat16), (1, 4, 1, 70, 2, torch.bfloat16),
     (1, 24, 2640, 880, 3, torch.bfloat16)],  # last: config-3 shape, runs 4-wave workgroups
)
def test_attention_frames_vs_oracle(gpu, B, H, Lq, T, n, dtype):
    _say("attention", B, H, Lq, T, n, dtype)
    q = _rand((B, Lq, H, 128), 1, dtype)
    k = _rand((B, n * T, H, 128), 2, dtype)
    v = _rand((B, n * T, H, 128), 3, dtype)
    kpool, vpool, slots = _pool_from(k, v, T, dtype, gpu)
    out = kernels.attention_frames(q.to(gpu), kpool, vpool, slots, frame_tokens=T)
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.shape == q.shape
    assert_attn_close(out, ref.attention(q, k, v))


def test_attention_sharp_and_scaled_logits(gpu):
    """Large logits (peaked softmax) and a non-default softmax_scale."""
    q = _rand((1, 256, 2, 128), 4, torch.bfloat16, scale=3.0)
    k = _rand((1, 640, 2, 128), 5, torch.bfloat16, scale=3.0)
    v = _rand((1, 640, 2, 128), 6, torch.bfloat16)
    kpool, vpool, slots = _pool_from(k, v, 160, torch.bfloat16, gpu)
    for scale in (None, 0.02):
        out = kernels.attention_frames(q.to(gpu), kpool, vpool, slots, frame_tokens=160,
                                       softmax_scale=scale)
        torch.cuda.synchronize()
        assert_attn_close(out, ref.attention(q, k, v, softmax_scale=scale))


def test_attention_late_max_for_some_queries(gpu):
    """Row maxima that jump late in the window for a few queries only, so inside one wave some
    lanes keep their probabilities and others raise their max and recompute the tile."""
    T, n = 96, 8
    q = _rand((1, 320, 2, 128), 21, torch.float32)
    k = _rand((1, n * T, 2, 128), 22, torch.float32)
    v = _rand((1, n * T, 2, 128), 23, torch.float32)
    g = torch.Generator().manual_seed(24)
    picks = torch.randperm(320, generator=g)[:20]
    for j, qi in enumerate(picks.tolist()):
        key = (n - 1 - j % 3) * T + 5 * j % T  # keys in the last three frames
        # logit ~20 log2 units above the others: the partial sum crosses 2^8
        k[0, key, j % 2] = 0.5 * k[0, key, j % 2] + 1.2 * q[0, qi, j % 2]
    q, k, v = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
    kpool, vpool, slots = _pool_from(k, v, T, torch.bfloat16, gpu)
    out = kernels.attention_frames(q.to(gpu), kpool, vpool, slots, frame_tokens=T)
    torch.cuda.synchronize()
    assert_attn_close(out, ref.attention(q, k, v))


@pytest.mark.parametrize("clean,noisy,T,per_block", [(2, 1, 100, 1), (3, 3, 64, 3), (0, 3, 50, 3),
                                                      (6, 3, 130, 3)])
def test_chunk_causal_vs_oracle_mask(gpu, clean, noisy, T, per_block):
    _say("chunk-causal", clean, noisy, T, per_block)
    L = (clean + noisy) * T
    q = _rand((1, L, 2, 128), 7, torch.bfloat16)
    k = _rand((1, L, 2, 128), 8, torch.bfloat16)
    v = _rand((1, L, 2, 128), 9, torch.bfloat16)
    dense, _ = ref.inference_window_mask(clean, noisy, T, per_block)
    want = ref.attention(q, k, v, mask=dense[:L, :L])
    got = chunk_causal_attention(q.to(gpu), k.to(gpu), v.to(gpu), chunk_tokens=T * per_block)
    torch.cuda.synchronize()
    assert_attn_close(got, want)
    # the same mask through the frame table, queries = the last chunk only (q_pos0 offset)
    Lq = T * per_block
    kpool, vpool, slots = _pool_from(k, v, T, torch.bfloat16, gpu)
    got2 = kernels.attention_frames(
        q[:, L - Lq :].to(gpu), kpool, vpool, slots, frame_tokens=T,
        mask_mode=_lib.SKV_MASK_CHUNK_CAUSAL, q_pos0=L - Lq, chunk_tokens=Lq,
    )
    torch.cuda.synchronize()
    assert_attn_close(got2, want[:, L - Lq :])


def test_dropin_attention_signature(gpu):
    q = _rand((2, 300, 3, 128), 10, torch.float32)
    k = _rand((2, 500, 3, 128), 11, torch.float32)
    v = _rand((2, 500, 3, 128), 12, torch.float32)
    out = attention(q.to(gpu), k.to(gpu), v.to(gpu))
    torch.cuda.synchronize()
    assert out.dtype == torch.float32  # flash path keeps q's dtype (attention.py:138)
    assert_attn_close(out, ref.attention(q, k, v))
    ql = torch.tensor([300, 120])
    kl = torch.tensor([77, 500])
    out = attention(q.to(gpu), k.to(gpu), v.to(gpu), q_lens=ql, k_lens=kl)
    torch.cuda.synchronize()
    assert_attn_close(out[0], ref.attention(q[:1], k[:1, :77], v[:1, :77])[0])
    assert_attn_close(out[1, :120], ref.attention(q[1:, :120], k[1:], v[1:])[0])
    assert out[1, 120:].abs().sum() == 0


def test_dropin_attention_reuses_staging_without_zero_fill(gpu):
    """attention() stages dense K/V in this stream's reused buffer, which it never zero-fills: a
    first call grows the buffer, the buffer is then filled with NaN, and a smaller call whose
    390-key window leaves 58 padding rows in its slot must still match the oracle (the append
    writes every row of the slot) without reallocating the buffer."""
    q1, k1, v1 = (_rand((1, L, 3, 128), 80 + i, torch.bfloat16) for i, L in enumerate((300, 1000, 1000)))
    out1 = attention(q1.to(gpu), k1.to(gpu), v1.to(gpu))
    torch.cuda.synchronize()
    assert_attn_close(out1, ref.attention(q1, k1, v1))
    key = (gpu.index or 0, kernels._stream(gpu), torch.bfloat16)
    buf = kernels._staging[key]
    buf.fill_(float("nan"))
    q2, k2, v2 = (_rand((2, L, 2, 128), 90 + i, torch.bfloat16) for i, L in enumerate((100, 390, 390)))
    out2 = attention(q2.to(gpu), k2.to(gpu), v2.to(gpu))
    torch.cuda.synchronize()
    assert kernels._staging[key] is buf
    assert_attn_close(out2, ref.attention(q2, k2, v2))


def test_full_size_closed_form_identical_keys(gpu):
    """C2 shape (Lq 4680, 21 frames x 1560 keys, 12 heads): with every key equal, softmax is
    uniform and the output is the mean of V over all 32760 keys."""
    T, n, H = 1560, 21, 12
    q = torch.randn(1, 4680, H, 128, device=gpu, dtype=torch.bfloat16)
    k = torch.randn(1, 1, H, 128, device=gpu, dtype=torch.bfloat16).expand(1, n * T, H, 128).contiguous()
    v = torch.randn(1, n * T, H, 128, device=gpu, dtype=torch.bfloat16)
    kpool, vpool, _, _ = kernels.new_pools(n + 3, 1, H, T, torch.bfloat16, gpu)
    slots = list(range(n + 3))[3:][::-1]
    for f in range(n):
        kernels.append_frames(k, v, kpool, vpool, [slots[f]], frame_tokens=T, src_frame0=f)
    out = kernels.attention_frames(q, kpool, vpool, slots, frame_tokens=T)
    want = v.double().mean(dim=1, keepdim=True)
    torch.cuda.synchronize()
    err = (out.double() - want).abs()
    assert float(err.max()) < 2e-4, float(err.max())


def test_attention_is_deterministic(gpu):
    q = _rand((1, 700, 4, 128), 20, torch.bfloat16).to(gpu)
    k = _rand((1, 1560, 4, 128), 21, torch.bfloat16)
    kpool, vpool, slots = _pool_from(k, k * 0.5, 390, torch.bfloat16, gpu)
    a = kernels.attention_frames(q, kpool, vpool, slots, frame_tokens=390)
    b = kernels.attention_frames(q, kpool, vpool, slots, frame_tokens=390)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_empty_window_raises(gpu):
    kpool, vpool, _, _ = kernels.new_pools(2, 1, 1, 64, torch.bfloat16, gpu)
    q = torch.zeros(1, 4, 1, 128, device=gpu, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="empty key window"):
        kernels.attention_frames(q, kpool, vpool, [], frame_tokens=64)
    with pytest.raises(ValueError, match="outside"):
        kernels.attention_frames(q, kpool, vpool, [5], frame_tokens=64)


# ---------------------------------------------------------------------------------------------
# fp8-e4m3 cache (BASELINE config 5 semantics): per-(slot, stream, head) absmax/448 scales;
# attention error measured against the oracle on the original bf16 K/V.
# ---------------------------------------------------------------------------------------------
def _fp8_pool_from(k, v, T, device, perm_seed=0):
    B, L, H, _ = k.shape
    n = L // T
    g = torch.Generator().manual_seed(perm_seed)
    slots = torch.randperm(n + 2, generator=g)[:n].tolist()
    kpool, vpool, ks, vs = kernels.new_pools(n + 2, B, H, T, torch.float8_e4m3fn, device)
    kd, vd = k.to(device), v.to(device)
    for f in range(n):
        kernels.append_frames(kd, vd, kpool, vpool, [slots[f]], frame_tokens=T, src_frame0=f,
                              kscale=ks, vscale=vs)
    return kpool, vpool, ks, vs, slots


def _outlier_kv(shape, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g)
    ch = torch.randperm(shape[-1], generator=g)[: max(1, shape[-1] // 100)]
    x[..., ch] *= 20.0  # 1% of channels are x20 outliers
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("B,H,Lq,T,n", [
    (4, 3, 390, 390, 21), (1, 12, 1170, 390, 6), (2, 1, 37, 1560, 2), (1, 24, 2640, 880, 7),
    pytest.param(1, 12, 1170, 390, 3, marks=pytest.mark.skip(
        reason="quantisation floor: over a 1170-key window the e4m3 cache itself (the "
               "quantisation-aware oracle, no kernel) is 3.3e-2 max-abs from the bf16 oracle, "
               "above the 3e-2 bar; tests/test_oracle.py::test_fp8_quantisation_floor_short_window "
               "measures it and test_fp8_attention_outliers_vs_quantised_oracle bounds the "
               "kernel's own error")),
])
def test_fp8_attention_unit_scale_vs_bf16_oracle(gpu, B, H, Lq, T, n):
    """N(0,1) K/V: the fp8 cache path meets the north-star fp8 bar (stated for the 21-frame
    config-5 window) against the bf16 oracle on windows of 2340 to 8190 keys."""
    _say("fp8 attention unit scale", B, H, Lq, T, n)
    from .helpers import FP8_MAX_ABS, FP8_MEAN_ABS

    q = _rand((B, Lq, H, 128), 31, torch.bfloat16)
    k = _rand((B, n * T, H, 128), 32, torch.bfloat16)
    v = _rand((B, n * T, H, 128), 33, torch.bfloat16)
    kpool, vpool, ks, vs, slots = _fp8_pool_from(k, v, T, gpu)
    out = kernels.attention_frames(q.to(gpu), kpool, vpool, slots, frame_tokens=T, kscale=ks,
                                   vscale=vs)
    torch.cuda.synchronize()
    want = ref.attention(q, k, v, compute_dtype=torch.float32)
    assert_attn_close(out, want, FP8_MAX_ABS, FP8_MEAN_ABS)


def assert_fp8_close_normalised(got, q, k, v, T, mask=None):
    """Outlier data: compare with the quantisation-aware oracle (fp8 cache frames and fp8 query
    rows decoded, fp64 softmax) and normalise the error by each channel's V RMS; what remains is
    the fp8 rounding of P and fp32 accumulation.  The mean bar is FP8_NORM_MEAN, or the margin
    times the error that P's rounding alone causes on the case where that is larger (few rows
    over few effective keys)."""
    from .helpers import FP8_NORM_MAX, FP8_NORM_MEAN, FP8_P_ROUNDING_MARGIN, fp8_p_rounding_error

    want = ref.attention(ref.fp8_fake_quant_rows(q), ref.fp8_fake_quant_frames(k.float(), T),
                         ref.fp8_fake_quant_frames(v.float(), T), mask=mask,
                         round_inputs_to_bf16=False).double()
    rms_v = v.double().pow(2).mean(dim=1, keepdim=True).sqrt().clamp_min(1e-6)
    got = got.detach().cpu().double()
    assert torch.isfinite(got).all()
    e = (got - want).abs() / rms_v
    e_p = float(fp8_p_rounding_error(q, k, v, T, mask=mask).mean())
    bar_mean = max(FP8_NORM_MEAN, FP8_P_ROUNDING_MARGIN * e_p)
    _say(f"fp8 normalised error: max {float(e.max()):.3e} mean {float(e.mean()):.3e} "
         f"(P rounding alone: mean {e_p:.3e})")
    assert float(e.max()) <= FP8_NORM_MAX, f"normalised max error {float(e.max()):.3e}"
    assert float(e.mean()) <= bar_mean, f"normalised mean error {float(e.mean()):.3e} > {bar_mean:.3e}"


@pytest.mark.parametrize("B,H,Lq,T,n", [(1, 2, 256, 130, 4), (4, 3, 390, 390, 3), (1, 12, 1170, 390, 6),
                                        (2, 1, 37, 1560, 2)])
def test_fp8_attention_outliers_vs_quantised_oracle(gpu, B, H, Lq, T, n):
    _say("fp8 attention outliers", B, H, Lq, T, n)
    q = _rand((B, Lq, H, 128), 31, torch.bfloat16)
    k = _outlier_kv((B, n * T, H, 128), 32)
    v = _outlier_kv((B, n * T, H, 128), 33)
    kpool, vpool, ks, vs, slots = _fp8_pool_from(k, v, T, gpu)
    out = kernels.attention_frames(q.to(gpu), kpool, vpool, slots, frame_tokens=T, kscale=ks,
                                   vscale=vs)
    torch.cuda.synchronize()
    assert_fp8_close_normalised(out, q, k, v, T)


def test_fp8_chunk_causal_and_zero_frames(gpu):
    T, n = 100, 6
    q = _rand((1, n * T, 2, 128), 41, torch.bfloat16)
    k = _outlier_kv((1, n * T, 2, 128), 42)
    v = _outlier_kv((1, n * T, 2, 128), 43)
    k[:, 2 * T : 3 * T] = 0  # an all-zero K frame (scale 0) and V frame
    v[:, 4 * T : 5 * T] = 0
    kpool, vpool, ks, vs, slots = _fp8_pool_from(k, v, T, gpu)
    dense, _ = ref.inference_window_mask(0, n, T, 2)
    got = kernels.attention_frames(q.to(gpu), kpool, vpool, slots, frame_tokens=T, kscale=ks,
                                   vscale=vs, mask_mode=_lib.SKV_MASK_CHUNK_CAUSAL,
                                   chunk_tokens=2 * T)
    torch.cuda.synchronize()
    assert_fp8_close_normalised(got, q, k, v, T, mask=dense[: n * T, : n * T])
