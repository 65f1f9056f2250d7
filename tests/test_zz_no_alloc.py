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


def test_noalloc_under_graph_capture(gpu):
    """skv_noalloc_init, then skv_attention_ex_noalloc captured in a HIP graph on a split-taking
    shape.  Before each of three replays an eager no-allocation call on another split shape
    overwrites the static scratch; every replay equals skv_attention_ex with a workspace."""
    lib = _lib.load()
    _lib.check("skv_noalloc_init", lib.skv_noalloc_init())
    _lib.check("skv_noalloc_init", lib.skv_noalloc_init())  # idempotent
    _say("noalloc graph capture")
    q, kp, vp, slots = _case(gpu, 1, 4, 1000, 1560, 21, 300)
    want, _ = _both(gpu, q, kp, vp, slots, 1560, expect_split=True)
    q2, kp2, vp2, slots2 = _case(gpu, 1, 2, 256, 1560, 21, 301)
    d, out, keep = kernels.attention_desc(q, kp, vp, slots, frame_tokens=1560)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.graph(graph, stream=side):
        st = lib.skv_attention_ex_noalloc(ctypes.byref(d), side.cuda_stream)
    assert st == _lib.SKV_OK, lib.skv_last_error()
    torch.cuda.synchronize()
    for i in range(3):
        out.fill_(float("nan"))
        want2, got2 = _both(gpu, q2, kp2, vp2, slots2, 1560, expect_split=True)
        assert torch.equal(got2, want2)
        graph.replay()
        torch.cuda.synchronize()
        _say("  replay", i)
        assert torch.equal(out, want), (i, float((out.float() - want.float()).abs().max()))


_CHILD = r"""
import ctypes, sys
import torch
sys.path.insert(0, sys.argv[1])
from solarwm_amd import _lib, kernels
lib = _lib.load()
gpu = torch.device("cuda:0")
g = torch.Generator().manual_seed(5)
B, H, Lq, T, n = 1, 4, 1000, 1560, 21
q = torch.randn(B, Lq, H, 128, generator=g).bfloat16().to(gpu)
k = torch.randn(B, n * T, H, 128, generator=g).bfloat16().to(gpu)
kp, vp, _, _ = kernels.new_pools(n + 2, B, H, T, torch.bfloat16, gpu)
slots = list(range(2, n + 2))
for f in range(n):
    kernels.append_frames(k, k, kp, vp, [slots[f]], frame_tokens=T, src_frame0=f)
want = kernels.attention_frames(q, kp, vp, slots, frame_tokens=T)
d, out, keep = kernels.attention_desc(q, kp, vp, slots, frame_tokens=T)
side = torch.cuda.Stream(gpu)
side.wait_stream(torch.cuda.current_stream(gpu))
torch.cuda.synchronize()
print("child: capture before set-up", flush=True)
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph, stream=side):
    st = lib.skv_attention_ex_noalloc(ctypes.byref(d), side.cuda_stream)
assert st == _lib.SKV_E_UNSUPPORTED, st
assert b"skv_noalloc_init" in lib.skv_last_error(), lib.skv_last_error()
print("child: set up, capture, replay", flush=True)
assert lib.skv_noalloc_init() == _lib.SKV_OK, lib.skv_last_error()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph, stream=side):
    st = lib.skv_attention_ex_noalloc(ctypes.byref(d), side.cuda_stream)
assert st == _lib.SKV_OK, lib.skv_last_error()
for _ in range(2):
    out.fill_(float("nan"))
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want)
print("child: done", flush=True)
"""


def test_noalloc_capture_needs_set_up_and_process_exits_cleanly(gpu, tmp_path):
    """In a fresh process (no scratch set up on the device yet): a captured call returns
    SKV_E_UNSUPPORTED naming skv_noalloc_init and records nothing; after skv_noalloc_init the
    captured call replays correctly.  The child then exits normally: the library's code objects
    (its three translation units, the static scratch placed) are unregistered by the runtime's
    exit handlers without a fault (exit status 0)."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    script = tmp_path / "child.py"
    script.write_text(_CHILD)
    _say("noalloc child process")
    res = subprocess.run([sys.executable, "-u", str(script), root], capture_output=True,
                         text=True, timeout=240)
    _say(res.stdout[-2000:], res.stderr[-2000:])
    assert res.returncode == 0, res.returncode
    assert "child: done" in res.stdout
