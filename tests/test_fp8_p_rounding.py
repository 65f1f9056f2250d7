"""Pins of tests/helpers.fp8_p_rounding_error, which sizes the mean bar of the fp8 parity tests
for cases that average P's e4m3 rounding over few keys (CPU only)."""

import math

import torch

from oracle import wan_cache_ref as ref

from .helpers import fp8_p_rounding_error


def _e4m3(x: float) -> float:
    return float(torch.tensor([x], dtype=torch.float32).to(torch.float8_e4m3fn).float())


def _brute(q, k, v, T, mask):
    """The same quantity element by element: per stream b, head h and query row i."""
    B, L, H, D = v.shape
    n = L // T
    qh = ref.fp8_fake_quant_rows(q.float()).double()
    kh = ref.fp8_fake_quant_frames(k.float(), T).double()
    vh = ref.fp8_fake_quant_frames(v.float(), T).double()
    out = torch.zeros(B, q.shape[1], H, D, dtype=torch.float64)
    for b in range(B):
        for h in range(H):
            sv = [float(v[b, f * T:(f + 1) * T, h].float().abs().max()) / 448.0 for f in range(n)]
            g = 28.0 / max(sv) if max(sv) > 0 else 1.0
            pv = [x * g if x * g > 0 else 1.0 for x in sv]
            rms = [math.sqrt(float(v[b, :, h, d].double().pow(2).mean())) for d in range(D)]
            for i in range(q.shape[1]):
                keys = [j for j in range(L) if mask is None or bool(mask[i, j])]
                s = {j: float(qh[b, i, h] @ kh[b, j, h]) / math.sqrt(D) for j in keys}
                m = max(s.values())
                p = {j: math.exp(s[j] - m) for j in keys}
                pq = {j: _e4m3(p[j] * pv[j // T]) / pv[j // T] for j in keys}
                for d in range(D):
                    exact = sum(p[j] * float(vh[b, j, h, d]) for j in keys) / sum(p.values())
                    rounded = sum(pq[j] * float(vh[b, j, h, d]) for j in keys) / sum(pq.values())
                    out[b, i, h, d] = abs(rounded - exact) / max(rms[d], 1e-6)
    return out


def test_matches_an_element_by_element_restatement():
    g = torch.Generator().manual_seed(3)
    B, H, T, n, Lq, D = 2, 2, 5, 3, 3, 8
    q = torch.randn(B, Lq, H, D, generator=g) * 2.0
    k = (torch.randn(B, n * T, H, D, generator=g) * 1.5).bfloat16()
    v = torch.randn(B, n * T, H, D, generator=g).bfloat16()
    v[1, T:2 * T, 0] = 0  # an all-zero V frame keeps its P unscaled
    v[0, 2 * T:, 1] *= 8  # frames of different V scales, so G and sv_f matter
    mask = torch.ones(Lq, n * T, dtype=torch.bool)
    mask[0, 2 * T:] = False
    for m in (None, mask):
        got = fp8_p_rounding_error(q, k, v, T, mask=m)
        want = _brute(q, k, v, T, m)
        assert torch.allclose(got, want, rtol=1e-9, atol=1e-12), float((got - want).abs().max())
        assert float(got.max()) > 0  # the rounding is visible at this size


def test_invariant_under_power_of_two_v_scaling():
    g = torch.Generator().manual_seed(4)
    q = torch.randn(1, 4, 2, 128, generator=g)
    k = torch.randn(1, 3 * 64, 2, 128, generator=g).bfloat16()
    v = torch.randn(1, 3 * 64, 2, 128, generator=g).bfloat16()
    a = fp8_p_rounding_error(q, k, v, 64)
    b = fp8_p_rounding_error(q, k, v * 4, 64)
    assert torch.allclose(a, b, rtol=1e-9, atol=1e-15)


def test_few_effective_keys_round_worse_than_many():
    g = torch.Generator().manual_seed(5)
    k = torch.randn(1, 4 * 390, 1, 128, generator=g).bfloat16()
    v = torch.randn(1, 4 * 390, 1, 128, generator=g).bfloat16()
    q = torch.randn(1, 1, 1, 128, generator=g)
    flat = float(fp8_p_rounding_error(q * 0.05, k, v, 390).mean())   # ~1560 effective keys
    peaky = float(fp8_p_rounding_error(q * 6.0, k, v, 390).mean())   # a handful
    assert flat < 2e-3 < peaky
