"""Shared assertions for the GPU parity tests."""

import torch

# Bars for bf16 attention (fp32 accumulation) against the float64 oracle.
MAX_ABS, MEAN_ABS = 2e-2, 1e-3
# Bar for attention over an fp8-e4m3 cache against the bf16-cache oracle (N(0,1) K/V).
FP8_MAX_ABS, FP8_MEAN_ABS = 3e-2, 3e-3
# fp8 cache with outlier channels: error against the quantisation-aware oracle (the cache's e4m3
# K/V frames and per-row e4m3 queries decoded, float64 softmax) divided by each channel's V RMS
# (e4m3 keeps 3 mantissa bits, so absolute errors scale with the channel).  What remains is the
# kernel's own arithmetic, mostly the e4m3 rounding of P: measured on MI355X at most 0.167 max and
# 5.4e-3 mean over every fp8 GPU test (windows of 2 to 21 frames, the C5 shape included).  One
# frame decoded with 1.25x or 2x its scale measures 0.31 to 4.5 max (tests/test_oracle.py plants
# it), so these bars reject a kernel that mixes up frame scales.
FP8_NORM_MAX, FP8_NORM_MEAN = 0.25, 8e-3
# A single query row whose softmax rests on a dozen keys averages the e4m3 rounding of P over
# few terms, so the rounding alone can pass FP8_NORM_MEAN (one such random case: 9.2e-3 from P's
# rounding alone, 8.4e-3 measured).  The mean bar of such a case is FP8_P_ROUNDING_MARGIN times
# what fp8_p_rounding_error gives on it, where that is larger.
FP8_P_ROUNDING_MARGIN = 1.25


def fp8_p_rounding_error(q, k, v, frame_tokens, mask=None):
    """Normalised error that the e4m3 rounding of P alone causes on a case (CPU, float64).

    The quantisation-aware attention (fp8 query rows and K/V frames decoded) is evaluated twice:
    with P unrounded, and with P stored as the fp8 kernel stores it, e4m3(p * sv_f * G) with
    p = exp(s - row max), sv_f the V frame's absmax / 448 per stream and head, G = 28 / the
    largest sv_f of the window (an all-zero V frame keeps p unscaled), and O = sum(pq v) /
    sum(pq).  Returns |difference| divided by each channel's V RMS, the normalisation of the
    fp8 parity bars.  q: [B, Lq, H, D]; k, v: [B, n * frame_tokens, H, D]; mask: [Lq, L] bool
    (True = attend) or None."""
    from oracle import wan_cache_ref as ref

    T = frame_tokens
    B, L, H, D = v.shape
    n = L // T
    qh = ref.fp8_fake_quant_rows(q.float()).double()
    kh = ref.fp8_fake_quant_frames(k.float(), T).double()
    vh = ref.fp8_fake_quant_frames(v.float(), T).double()
    sv = v.double().reshape(B, n, T, H, D).abs().amax(dim=(2, 4)) / 448.0  # [B, n, H]
    smax = sv.amax(dim=1, keepdim=True)
    g = torch.where(smax > 0, 28.0 / smax.clamp_min(1e-30), torch.ones_like(smax))
    pv = sv * g
    pv = torch.where(pv > 0, pv, torch.ones_like(pv))
    pvk = pv.permute(0, 2, 1).repeat_interleave(T, dim=2)[:, :, None, :]  # [B, H, 1, L]
    s = torch.einsum("bqhd,bkhd->bhqk", qh, kh) * D ** -0.5
    if mask is not None:
        s = s.masked_fill(~mask.to(torch.bool), float("-inf"))
    p = torch.exp(s - s.amax(-1, keepdim=True))
    pq = (p * pvk).float().to(torch.float8_e4m3fn).double() / pvk
    exact = torch.einsum("bhqk,bkhd->bqhd", p, vh) / p.sum(-1).permute(0, 2, 1)[..., None]
    rounded = torch.einsum("bhqk,bkhd->bqhd", pq, vh) / pq.sum(-1).permute(0, 2, 1)[..., None]
    rms_v = v.double().pow(2).mean(dim=1, keepdim=True).sqrt().clamp_min(1e-6)
    return (rounded - exact).abs() / rms_v


def assert_attn_close(got, want, max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    got = got.detach().cpu()
    assert torch.isfinite(got).all(), "non-finite attention output"
    err = (got.double() - want.double()).abs()
    assert float(err.max()) <= max_abs, f"max-abs error {float(err.max()):.3e} > {max_abs}"
    assert float(err.mean()) <= mean_abs, f"mean-abs error {float(err.mean()):.3e} > {mean_abs}"
