"""GPU parity of the tail split (launch plan ``split == 2``) on bf16 and f16 pools.

A grid of one full round of 8-wave workgroups plus a partly filled one runs the full round
unsplit, then spreads the last round's q-tiles over every CU and merges their partial records.
Shape B=4, H=3, Lq=7836: 31 q-tiles per (stream, head), 372 in all = 256 + 116 on MI355X's 256
CUs, the last q-tile ragged (156 of 256 rows).  Every output row is checked against the float64
oracle and against the unsplit kernel (``use_workspace=False``).
"""

import pytest
import torch

from oracle import wan_cache_ref as ref
from solarwm_amd import kernels

from .helpers import assert_attn_close

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _rand(shape, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype)


@pytest.mark.parametrize("T,nf,dtype,packed", [
    (880, 3, torch.bfloat16, True),    # key tiles packed across frames (T % 8 == 0)
    (390, 6, torch.bfloat16, False),   # frame-aligned tiles, padding keys masked
    (880, 3, torch.float16, True),     # f16 pools and MFMAs, packed
])
def test_tail_split_every_row(gpu, T, nf, dtype, packed):
    B, H, Lq = 4, 3, 7836
    _say("tail split", B, H, Lq, T, nf, dtype)
    q = _rand((B, Lq, H, 128), 70, dtype)
    k = _rand((B, nf * T, H, 128), 71, dtype)
    v = _rand((B, nf * T, H, 128), 72, dtype)
    g = torch.Generator().manual_seed(73)
    slots = torch.randperm(nf + 2, generator=g)[:nf].tolist()
    kpool, vpool, _, _ = kernels.new_pools(nf + 2, B, H, T, dtype, gpu)
    kd, vd = k.to(gpu), v.to(gpu)
    for f in range(nf):
        kernels.append_frames(kd, vd, kpool, vpool, [slots[f]], frame_tokens=T, src_frame0=f)
    qd = q.to(gpu)
    if kernels.cu_count(gpu) != 256:
        pytest.skip("the shape is sized for 256 CUs")
    plan = kernels.attention_plan(qd, kpool, vpool, slots, frame_tokens=T)
    assert plan["split"] == 2 and plan["n_qtiles"] == 372, plan
    want_tiles = -(-nf * T // 64) if packed else nf * -(-T // 64)
    assert plan["key_tiles"] == want_tiles, plan
    got = kernels.attention_frames(qd, kpool, vpool, slots, frame_tokens=T)
    plain = kernels.attention_frames(qd, kpool, vpool, slots, frame_tokens=T, use_workspace=False)
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    gap = float((got.float() - plain.float()).abs().max())
    _say(f"  split vs unsplit max {gap:.3e}")
    assert gap <= 4e-3, gap  # same products, partial sums merged in another order
    if dtype == torch.float16:
        want = ref.attention(q.double(), k.double(), v.double(), round_inputs_to_bf16=False)
    else:
        want = ref.attention(q, k, v)
    assert_attn_close(got, want)
    assert_attn_close(plain, want)
