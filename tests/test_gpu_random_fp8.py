"""Seeded random shapes for the fp8-e4m3 attention kernel against the quantisation-aware oracle
(oracle/wan_cache_ref.py: fp8 frames and query rows decoded, float64 softmax; the reference's
attention is attention.py:141-188, the cache format causal_model.py:2894-2914).

Each case draws a frame size (one-tile frames, where every step of the kernel opens a key
frame and changes the P scale, up to C5's 1560), a window of frames in shuffled slots, a query
count, heads, streams, the query dtype, the data (N(0,1) or 1% of channels x20, sometimes an
all-zero K or V frame) and the mask (none, or chunk-causal), and runs each case twice: with the
caller workspace (the launcher may take the balanced split, whose instances sum P on the VALU)
and without it (the unsplit instances, which sum P on the matrix core).  Bars: tests/helpers.py
(normalised by each channel's V RMS)."""

import random

import pytest
import torch

from oracle import wan_cache_ref as ref
from solarwm_amd import _lib, kernels

from .test_gpu_kernels import _outlier_kv, assert_fp8_close_normalised

pytestmark = pytest.mark.gpu

FRAME_SIZES = [64, 72, 100, 130, 390, 880, 1560]
Q_LENS = [1, 37, 130, 256, 600, 1170]


def _case(seed):
    r = random.Random(1000 + seed)
    T = r.choice(FRAME_SIZES)
    n = r.randint(1, max(1, min(30, 9000 // T)))
    H = r.choice([1, 2, 3])
    B = r.choice([1, 2, 4])
    Lq = r.choice(Q_LENS)
    qdt = r.choice([torch.bfloat16, torch.bfloat16, torch.float32])
    outliers = r.random() < 0.5
    zero = r.choice([None, None, "k", "v"]) if n > 1 else None
    causal = r.random() < 0.3
    while Lq * n * T * H * B > 2.0e7 and Lq > 1:  # keep the float64 oracle within a second
        Lq = Q_LENS[max(0, Q_LENS.index(Lq) - 1)]
    return T, n, H, B, Lq, qdt, outliers, zero, causal, r.randrange(1 << 30)


# 20209: one query row over 4680 keys with outlier channels and an all-zero V frame, whose
# softmax rests on about 12 keys (the mean bar then follows P's rounding, tests/helpers.py)
@pytest.mark.parametrize("seed", [*range(16), 20209])
def test_random_fp8_shape_vs_quantised_oracle(gpu, seed):
    T, n, H, B, Lq, qdt, outliers, zero, causal, s = _case(seed)
    print("fp8 case", seed, dict(T=T, n=n, H=H, B=B, Lq=Lq, q=qdt, outliers=outliers, zero=zero,
                                 causal=causal), flush=True)
    g = torch.Generator().manual_seed(s)
    q = torch.randn((B, Lq, H, 128), generator=g).to(qdt)
    if outliers:
        k = _outlier_kv((B, n * T, H, 128), s + 1)
        v = _outlier_kv((B, n * T, H, 128), s + 2)
    else:
        k = torch.randn((B, n * T, H, 128), generator=g).to(torch.bfloat16)
        v = torch.randn((B, n * T, H, 128), generator=g).to(torch.bfloat16)
    if zero is not None:
        f = random.Random(s).randrange(n)
        (k if zero == "k" else v)[:, f * T : (f + 1) * T] = 0
    slots = torch.randperm(n + 2, generator=g)[:n].tolist()
    kp, vp, ks, vs = kernels.new_pools(n + 2, B, H, T, torch.float8_e4m3fn, gpu)
    kd, vd = k.to(gpu), v.to(gpu)
    for f in range(n):
        kernels.append_frames(kd, vd, kp, vp, [slots[f]], frame_tokens=T, src_frame0=f,
                              kscale=ks, vscale=vs)
    kw, mask = {}, None
    if causal:
        L = n * T
        chunk = T * random.Random(s).randint(1, n)
        q0 = random.Random(s + 1).randint(0, max(0, L - Lq))
        kw = dict(mask_mode=_lib.SKV_MASK_CHUNK_CAUSAL, q_pos0=q0, chunk_tokens=chunk)
        pos = torch.arange(q0, q0 + Lq)[:, None]
        lim = torch.clamp((pos // chunk + 1) * chunk, max=L)
        mask = torch.arange(L)[None, :] < lim
    qd = q.to(gpu)
    for ws in (True, False):
        out = kernels.attention_frames(qd, kp, vp, slots, frame_tokens=T, kscale=ks, vscale=vs,
                                       use_workspace=ws, **kw)
        torch.cuda.synchronize()
        assert out.dtype == qdt
        print("  workspace", ws, flush=True)
        assert_fp8_close_normalised(out.float(), q.float(), k, v, T, mask=mask)
