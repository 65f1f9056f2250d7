"""skv_attention_ex_noalloc (the entry point that allocates nothing) against skv_attention_ex
with a caller workspace, through the C ABI: two calls in a row on split-taking shapes, the
second smaller, so the second reads a static scratch that still holds the first call's
records; plus a launch that does not split and the argument checks."""

import ctypes

import pytest
import torch

from solarwm_amd import _lib, kernels

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _say(*a):
    print(*a, flush=True)


def _case(gpu, B, H, Lq, T, n, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Lq, H, 128, generator=g).to(BF).to(gpu)
    k = torch.randn(B, n * T, H, 128, generator=g).to(BF).to(gpu)
    v = torch.randn(B, n * T, H, 128, generator=g).to(BF).to(gpu)
    kp, vp, _, _ = kernels.new_pools(n + 2, B, H, T, BF, gpu)
    slots = list(range(2, n + 2))[::-1]
    for f in range(n):
        kernels.append_frames(k, v, kp, vp, [slots[f]], frame_tokens=T, src_frame0=f)
    return q, kp, vp, slots


def _both(gpu, q, kp, vp, slots, T, expect_split):
    lib = _lib.load()
    stream = torch.cuda.current_stream(gpu).cuda_stream
    # existing entry point, caller workspace
    d, ref_out, keep = kernels.attention_desc(q, kp, vp, slots, frame_tokens=T)
    plan = _lib.LaunchPlan()
    _lib.check("plan", lib.skv_attention_plan(ctypes.byref(d), ctypes.byref(plan)))
    assert plan.workspace_bytes <= _lib.SKV_NOALLOC_SCRATCH_BYTES
    assert (plan.workspace_bytes > 0) == expect_split, plan.workspace_bytes
    ws = torch.empty(max(plan.workspace_bytes, 1), dtype=torch.uint8, device=gpu)
    if plan.workspace_bytes:
        d.workspace, d.workspace_bytes = ws.data_ptr(), plan.workspace_bytes
    _lib.check("skv_attention_ex", lib.skv_attention_ex(ctypes.byref(d), stream))
    # the no-allocation entry point
    d2, out, keep2 = kernels.attention_desc(q, kp, vp, slots, frame_tokens=T)
    _lib.check("skv_attention_ex_noalloc", lib.skv_attention_ex_noalloc(ctypes.byref(d2), stream))
    torch.cuda.synchronize()
    return ref_out, out


def test_noalloc_matches_workspace_entry_point_on_two_calls(gpu):
    big = (1, 4, 1000, 1560, 21)  # 16 q-tiles over 525 key tiles: split on 256 CUs
    small = (1, 2, 256, 1560, 21)  # fewer heads and queries: 2 q-tiles, still split
    for i, (B, H, Lq, T, n) in enumerate((big, small)):
        _say("noalloc call", i, "B H Lq T n =", B, H, Lq, T, n)
        q, kp, vp, slots = _case(gpu, B, H, Lq, T, n, 100 + i)
        want, got = _both(gpu, q, kp, vp, slots, T, expect_split=True)
        assert torch.isfinite(got).all()
        assert torch.equal(got, want), float((got.float() - want.float()).abs().max())


def test_noalloc_unsplit_launch_and_argument_checks(gpu):
    lib = _lib.load()
    _say("noalloc unsplit C2-like launch")
    q, kp, vp, slots = _case(gpu, 1, 12, 4680, 1560, 3, 7)  # 228 workgroups: no split
    want, got = _both(gpu, q, kp, vp, slots, 1560, expect_split=False)
    assert torch.equal(got, want)
    d, _, keep = kernels.attention_desc(q, kp, vp, slots, frame_tokens=1560)
    d.workspace, d.workspace_bytes = q.data_ptr(), 64
    assert lib.skv_attention_ex_noalloc(ctypes.byref(d), None) == _lib.SKV_E_ARG
    assert b"static scratch" in lib.skv_last_error()
    assert lib.skv_attention_ex_noalloc(None, None) == _lib.SKV_E_ARG
