"""GPU parity of the balanced key split of the attention kernels (one workgroup per CU over
equal shares of the (q-tile, key tile) units, split q-tiles merged by a second kernel) against
the float64 oracle (oracle/wan_cache_ref.py attention, attention.py:141-188 of the reference).

The launcher takes the split when the unsplit grid would leave most CUs idle: every case below
has few q-tiles over a long key window, so it does.  Cases: a q-tile shared by many
workgroups (each gets about four key tiles), float queries with a ragged last q-tile, frames
with short valid spans so some workgroups see only masked keys, and the C2 window with a query
count that leaves most of the last q-tile empty.  Bars: tests/helpers.py."""

import pytest
import torch

from oracle import segments_ref as sr
from oracle import wan_cache_ref as ref
from solarwm_amd import kernels

from .helpers import assert_attn_close

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _say(*a):
    print(*a, flush=True)


def _rand(shape, seed, dtype=BF):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype)


def _pools(k, v, T, gpu, seed=0):
    B, L, H, _ = k.shape
    n = L // T
    g = torch.Generator().manual_seed(seed)
    slots = torch.randperm(n + 2, generator=g)[:n].tolist()
    kp, vp, _, _ = kernels.new_pools(n + 2, B, H, T, BF, gpu)
    for f in range(n):
        kernels.append_frames(k.to(gpu), v.to(gpu), kp, vp, [slots[f]], frame_tokens=T, src_frame0=f)
    return kp, vp, slots


@pytest.mark.parametrize("B,H,Lq,T,n,dtype", [
    (1, 2, 256, 1560, 21, BF),              # 2 q-tiles x 525 key tiles over 256 workgroups
    (2, 3, 300, 390, 14, torch.float32),    # float Q/O, last q-tile 44 of 256 rows
    (1, 4, 1000, 1560, 8, BF),              # C2 frame size, 4 q-tiles per head
])
def test_split_vs_oracle(gpu, B, H, Lq, T, n, dtype):
    _say("split attention", B, H, Lq, T, n, dtype)
    q = _rand((B, Lq, H, 128), 1, dtype)
    k, v = _rand((B, n * T, H, 128), 2), _rand((B, n * T, H, 128), 3)
    kp, vp, slots = _pools(k, v, T, gpu)
    plan = kernels.attention_plan(q.to(gpu), kp, vp, slots, frame_tokens=T)
    assert plan["split"] == 1 and plan["n_workgroups"] == kernels.cu_count(gpu), plan
    out = kernels.attention_frames(q.to(gpu), kp, vp, slots, frame_tokens=T)
    plain = kernels.attention_frames(q.to(gpu), kp, vp, slots, frame_tokens=T, use_workspace=False)
    torch.cuda.synchronize()
    assert out.dtype == dtype
    want = ref.attention(q, k.to(dtype), v.to(dtype))
    assert_attn_close(out, want)
    assert_attn_close(plain, want)


def test_split_ragged_frames_with_fully_masked_shares(gpu):
    """Frames keep 5..70 of 1560 keys: most key tiles are wholly masked, so many workgroups'
    shares hold no visible key (max -inf, sum 0) and the merge must skip them."""
    T, n, H = 1560, 21, 2
    lens = [5, 70, 1560, 64, 65, 1] + [7] * (n - 6)
    k, v = _rand((1, n * T, H, 128), 4), _rand((1, n * T, H, 128), 5)
    q = _rand((1, 256, H, 128), 6)
    kp, vp, slots = _pools(k, v, T, gpu, seed=1)
    out = kernels.attention_frames(q.to(gpu), kp, vp, slots, frame_tokens=T, frame_lens=lens)
    keys = torch.cat([k[:, j * T : j * T + lens[j]] for j in range(n)], 1)
    vals = torch.cat([v[:, j * T : j * T + lens[j]] for j in range(n)], 1)
    torch.cuda.synchronize()
    assert_attn_close(out, sr.attention(q, keys, vals))


def test_split_is_deterministic_and_strided_output(gpu):
    """Same inputs twice give identical bits; an output view with padded strides is written
    only inside the view."""
    T, n, H, Lq = 1560, 6, 4, 700
    q = _rand((1, Lq, H, 128), 7).to(gpu)
    k = _rand((1, n * T, H, 128), 8)
    kp, vp, slots = _pools(k, k * 0.5, T, gpu)
    a = kernels.attention_frames(q, kp, vp, slots, frame_tokens=T)
    b = kernels.attention_frames(q, kp, vp, slots, frame_tokens=T)
    big = torch.full((1, Lq, H, 160), 7.0, device=gpu, dtype=BF)
    c = kernels.attention_frames(q, kp, vp, slots, frame_tokens=T, out=big[..., :128])
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(a, c)
    assert bool((big[..., 128:] == 7.0).all())


def test_split_float32_pools(gpu):
    """The split path on fp32 pools (the config-1 cache dtype): 2 q-tiles x 4 heads over 21
    frames of 390 tokens."""
    B, H, Lq, T, n = 1, 4, 512, 390, 21
    q = _rand((B, Lq, H, 128), 30, torch.float32)
    k, v = _rand((B, n * T, H, 128), 31, torch.float32), _rand((B, n * T, H, 128), 32, torch.float32)
    g = torch.Generator().manual_seed(3)
    slots = torch.randperm(n + 2, generator=g)[:n].tolist()
    kp, vp, _, _ = kernels.new_pools(n + 2, B, H, T, torch.float32, gpu)
    for f in range(n):
        kernels.append_frames(k.to(gpu), v.to(gpu), kp, vp, [slots[f]], frame_tokens=T, src_frame0=f)
    out = kernels.attention_frames(q.to(gpu), kp, vp, slots, frame_tokens=T)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32
    assert_attn_close(out, ref.attention(q, k, v))


def test_split_with_q_norm(gpu):
    """Q RMSNorm at load on the split path: equal to the oracle's attention of the normalised
    queries (WanRMSNorm's statistic, model.py:69-84)."""
    B, H, Lq, T, n, eps = 1, 2, 300, 1560, 21, 1e-6
    g = torch.Generator().manual_seed(40)
    q = (torch.randn(B, Lq, H, 128, generator=g) *
         torch.exp(torch.randn(B, Lq, 1, 1, generator=g) * 1.2)).to(BF)
    w = torch.rand(H * 128, generator=g) + 0.5
    k, v = _rand((B, n * T, H, 128), 41), _rand((B, n * T, H, 128), 42)
    kp, vp, slots = _pools(k, v, T, gpu, seed=2)
    qd = q.to(gpu)
    got = kernels.attention_frames(qd, kp, vp, slots, frame_tokens=T,
                                   q_norm=(kernels.rms_rows(qd, eps), w.to(gpu)))
    torch.cuda.synchronize()
    assert_attn_close(got, ref.attention(ref.norm_heads(q, w, eps), k, v))


def test_split_fp8_ragged_and_zero_frames(gpu):
    """The split path of the fp8 cache kernel: frames keep 1..1560 of their keys (shares with no
    visible key), one K frame and one V frame are all zero (scale 0), and 1% of the channels
    are x20 outliers.  Compared with the quantisation-aware oracle (fp8 frames and query rows
    decoded, fp64 softmax); the error is divided by each channel's V RMS."""
    from .helpers import FP8_NORM_MAX, FP8_NORM_MEAN

    T, n, H, Lq = 1560, 21, 2, 256  # 2 q-tiles x 525 key tiles over 256 workgroups
    _say("split fp8 attention", H, Lq, T, n)
    lens = [5, 70, 1560, 64, 65, 1, 1560, 900] + [7] * (n - 8)
    g = torch.Generator().manual_seed(50)
    k = torch.randn(1, n * T, H, 128, generator=g)
    v = torch.randn(1, n * T, H, 128, generator=g)
    ch = torch.randperm(128, generator=g)[:2]
    k[..., ch] *= 20.0
    v[..., ch] *= 20.0
    k[:, 2 * T : 3 * T] = 0
    v[:, 6 * T : 7 * T] = 0
    k, v = k.to(BF), v.to(BF)
    q = _rand((1, Lq, H, 128), 51)
    g = torch.Generator().manual_seed(5)
    slots = torch.randperm(n + 2, generator=g)[:n].tolist()
    kp, vp, ks, vs = kernels.new_pools(n + 2, 1, H, T, torch.float8_e4m3fn, gpu)
    kd, vd = k.to(gpu), v.to(gpu)
    for f in range(n):
        kernels.append_frames(kd, vd, kp, vp, [slots[f]], frame_tokens=T, src_frame0=f,
                              kscale=ks, vscale=vs)
    got = kernels.attention_frames(q.to(gpu), kp, vp, slots, frame_tokens=T, kscale=ks,
                                   vscale=vs, frame_lens=lens)
    again = kernels.attention_frames(q.to(gpu), kp, vp, slots, frame_tokens=T, kscale=ks,
                                     vscale=vs, frame_lens=lens)
    torch.cuda.synchronize()
    assert torch.equal(got, again)
    kq = ref.fp8_fake_quant_frames(k.float(), T)
    vq = ref.fp8_fake_quant_frames(v.float(), T)
    keys = torch.cat([kq[:, j * T : j * T + lens[j]] for j in range(n)], 1)
    vals = torch.cat([vq[:, j * T : j * T + lens[j]] for j in range(n)], 1)
    want = ref.attention(ref.fp8_fake_quant_rows(q), keys, vals, round_inputs_to_bf16=False).double()
    rms_v = torch.cat([v[:, j * T : j * T + lens[j]] for j in range(n)], 1).double()
    rms_v = rms_v.pow(2).mean(dim=1, keepdim=True).sqrt().clamp_min(1e-6)
    got = got.cpu().double()
    assert torch.isfinite(got).all()
    e = (got - want).abs() / rms_v
    assert float(e.max()) <= FP8_NORM_MAX, f"normalised max error {float(e.max()):.3e}"
    assert float(e.mean()) <= FP8_NORM_MEAN, f"normalised mean error {float(e.mean()):.3e}"
