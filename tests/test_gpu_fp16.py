"""fp16 attention (the reference's ``attention(..., dtype=torch.float16)``, attention.py:46-138):
f16 inputs, or fp32 inputs with dtype=float16, run the attention kernel on f16 pools with f16
MFMAs.  Bars: within 2e-2 max-abs / 1e-3 mean-abs of float64 SDPA on the f16 inputs, and
clearly below what the bf16 path makes of the same inputs (so the arithmetic is f16, not a bf16
fallback); f16 append / gather bit-exact.
"""

import pytest
import torch

from oracle import wan_cache_ref as ref
from solarwm_amd import kernels
from solarwm_amd.attention import attention

from .helpers import assert_attn_close

pytestmark = pytest.mark.gpu

F16 = torch.float16


def _say(*a):
    print(*a, flush=True)


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g) * scale


def _f64_ref(q, k, v):
    return ref.attention(q.double(), k.double(), v.double(), round_inputs_to_bf16=False)


@pytest.mark.parametrize("B,H,Lq,Lk", [(1, 2, 256, 640), (2, 3, 100, 390), (1, 12, 1560, 4680)])
def test_fp16_attention_vs_float64(gpu, B, H, Lq, Lk):
    _say("fp16 attention", B, H, Lq, Lk)
    q, k, v = (_rand((B, L, H, 128), 50 + i).to(F16) for i, L in enumerate((Lq, Lk, Lk)))
    out = attention(q.to(gpu), k.to(gpu), v.to(gpu))
    torch.cuda.synchronize()
    assert out.dtype == F16
    want = _f64_ref(q, k, v)
    assert_attn_close(out, want)
    # the same inputs through the bf16 path: its error is several times the f16 path's
    out_bf = attention(q.float().to(gpu), k.float().to(gpu), v.float().to(gpu))
    e16 = float((out.cpu().double() - want).abs().mean())
    ebf = float((out_bf.cpu().double() - want).abs().mean())
    _say(f"  mean error f16 {e16:.3e}, bf16 {ebf:.3e}")
    assert e16 < ebf / 3


def test_fp16_dtype_argument_casts_fp32_inputs(gpu):
    """fp32 inputs with dtype=float16 compute in f16 (attention.py:69-73) and return fp32."""
    q, k, v = (_rand((1, L, 4, 128), 60 + i) for i, L in enumerate((300, 700, 700)))
    got = attention(q.to(gpu), k.to(gpu), v.to(gpu), dtype=F16)
    via16 = attention(q.to(F16).to(gpu), k.to(F16).to(gpu), v.to(F16).to(gpu))
    torch.cuda.synchronize()
    assert got.dtype == torch.float32
    assert torch.equal(got.cpu(), via16.float().cpu())
    assert_attn_close(got, _f64_ref(q.to(F16), k.to(F16), v.to(F16)))


def test_fp16_varlen_and_q_scale(gpu):
    q, k, v = (_rand((2, L, 3, 128), 70 + i).to(F16) for i, L in enumerate((200, 500, 500)))
    ql, kl = torch.tensor([200, 77]), torch.tensor([500, 301])
    out = attention(q.to(gpu), k.to(gpu), v.to(gpu), q_lens=ql, k_lens=kl, q_scale=0.5)
    torch.cuda.synchronize()
    for b in range(2):
        qs = (q[b : b + 1, : ql[b]].float() * 0.5).to(F16)
        want = _f64_ref(qs, k[b : b + 1, : kl[b]], v[b : b + 1, : kl[b]])
        assert_attn_close(out[b : b + 1, : ql[b]], want)
        assert int(out[b, ql[b]:].count_nonzero()) == 0


def test_fp16_split_and_chunk_causal(gpu):
    """One frame of queries over a long window takes the balanced key split (f16 instance);
    the chunk-causal mask runs unsplit."""
    T, n, H = 1560, 21, 12
    q = _rand((1, T, H, 128), 80).to(F16)
    k, v = (_rand((1, n * T, H, 128), 81 + i).to(F16) for i in range(2))
    kp, vp, _, _ = kernels.new_pools(n, 1, H, T, F16, gpu)
    for f in range(n):
        kernels.append_frames(k.to(gpu), v.to(gpu), kp, vp, [f], frame_tokens=T, src_frame0=f)
    plan = kernels.attention_plan(q.to(gpu), kp, vp, list(range(n)), frame_tokens=T)
    assert plan["split"] == 1
    out = kernels.attention_frames(q.to(gpu), kp, vp, list(range(n)), frame_tokens=T)
    torch.cuda.synchronize()
    hs = slice(0, 2)
    assert_attn_close(out[:, :, hs], _f64_ref(q[:, :, hs], k[:, :, hs], v[:, :, hs]))
    from solarwm_amd.attention import chunk_causal_attention
    Tc, L = 100, 600  # 2 clean + 4 noisy frames of 100 tokens, chunks of 2 frames
    qc = _rand((1, L, 2, 128), 90).to(F16)
    kc, vc = (_rand((1, L, 2, 128), 91 + i).to(F16) for i in range(2))
    got = chunk_causal_attention(qc.to(gpu), kc.to(gpu), vc.to(gpu), chunk_tokens=2 * Tc)
    torch.cuda.synchronize()
    dense, _ = ref.inference_window_mask(2, 4, Tc, 2)
    want = ref.attention(qc.double(), kc.double(), vc.double(), mask=dense[:L, :L],
                         round_inputs_to_bf16=False)
    assert got.dtype == F16
    assert_attn_close(got, want)


def test_fp16_append_gather_bit_exact(gpu):
    B, H, T = 2, 3, 390
    k = _rand((B, 2 * T, H, 128), 95).to(F16)
    v = _rand((B, 2 * T, H, 128), 96).to(F16)
    k[0, 5, 1, 7] = float("inf")
    v[1, 9, 2, 3] = -65504.0
    kp, vp, _, _ = kernels.new_pools(4, B, H, T, F16, gpu)
    kernels.append_frames(k.to(gpu), v.to(gpu), kp, vp, [3, 1], frame_tokens=T)
    gk, gv = kernels.gather_frames(kp, vp, [3, 1], frame_tokens=T)
    torch.cuda.synchronize()
    assert gk.dtype == F16
    assert torch.equal(gk.cpu().view(torch.int16), k.view(torch.int16))
    assert torch.equal(gv.cpu().view(torch.int16), v.view(torch.int16))
    with pytest.raises(ValueError):  # f16 pools take plain appends only
        kernels.append_frames(k.to(gpu), v.to(gpu), kp, vp, [0], frame_tokens=T,
                              k_norm=(torch.ones(B, 2 * T, device=gpu),
                                      torch.ones(H * 128, device=gpu)))
