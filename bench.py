#!/usr/bin/env python3
"""Benchmark of the block-causal KV-cache inference path on one MI355X.

Workload (Wan2.1-1.3B shape): 30 layers, 12 heads x 128, 1560 tokens per
latent frame, chunks of 3 frames (4680 queries), a 21-frame (32760-token) cache per layer with a
1-frame sink and rolling eviction, 27 chunks.  One step = one chunk of the reference sampler
(solar/backends/wan22/runtime/stage2.py:674-760): 4 denoising passes with
cache_update_policy "none" and 1 commit pass, each pass running the cached self-attention of all
30 layers (append of the chunk into staging slots + attention over sink | window | chunk) and
the commit pass advancing every layer's slot table.  Projections/FFN are outside the path.

Printed JSON (one line): value = latent frames/s of K timed steady-state chunks (3 frames per
chunk), each attending over the full 21-frame window: the chunks that fill the window run first,
untimed, so the figure does not depend on K; configured_run = the 27 chunks of BASELINE's run
from an empty cache, ramp-up included, beside it.  roofline = the attention kernel's algorithmic
TFLOP/s (4*Lq*Lk*H*D per launch, from HIP events around every 7th launch in the timed region)
against dense bf16 MFMA peak; cpu_baseline = the
reference op sequence (clone, memmove, slice-assign, cat, bf16 SDPA) restated on the host CPU
for one steady-state layer pass, extrapolated; reference_gpu = the same op sequence with
PyTorch-ROCm on the GPU (SDPA flash backend) over the same chunks.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

CONFIGS = {
    "c2": dict(workload="wan2.1-1.3b", layers=30, heads=12, T=1560, chunk_f=3, cap_f=21,
               sink_f=1, chunks=27, batch=1, cache="bf16", grid=(30, 52)),
    "c3": dict(workload="wan2.2-5b", layers=30, heads=24, T=880, chunk_f=3, cap_f=21,
               sink_f=1, chunks=40, batch=1, cache="bf16", grid=(22, 40)),
    "c5": dict(workload="wan2.1-1.3b fp8-e4m3 kv, 4 streams", layers=30, heads=12, T=1560,
               chunk_f=3, cap_f=21, sink_f=1, chunks=27, batch=4, cache="fp8", grid=(30, 52)),
    # the reference's shipped inference (configs/solar_wm/wan22_ti2v_5b/infer_stage2_sgf_81f.yaml:
    # 16-27 with architectures/ti2v_5b.json): 30 layers, 24 heads, 405-token frames (grid 15 x 27),
    # 3-frame chunks, 18-frame cache without a sink, window RoPE without EchoRoPE frozen at 21
    # training frames, fused PRoPE with linear translations; 21 output frames = 7 chunks
    "release": dict(workload="wan2.2-ti2v-5b release inference", layers=30, heads=24, T=405,
                    chunk_f=3, cap_f=18, sink_f=0, chunks=7, batch=1, cache="bf16", grid=(15, 27),
                    echorope=False, rope_train_frames=21, translation="linear"),
}
# grid: the latent patch grid of one frame (480x832 video -> 60x104 latent -> 2x2 patches; the
# 5B model's 16x VAE: 704x1280 -> 44x80 -> 22x40), used by the pre-RoPE (RoPE on load) legs
# config 4: 33B-class memory path (one GPU holds one layer's 256-slot bank: 8.4 GB; all 48
# layers would need 403 GB)
C4 = dict(workload="33b-class memory path", layers=48, heads=40, T=1560, chunk_f=3, cap_f=21,
          sink_f=1, bank=256, mem_frames=8)
PASSES = ["none"] * 4 + ["commit"]  # stage2.py:683-760: NFE4 then a t=0 commit forward
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
FP8_PEAK_TFLOPS = 5000.0  # MI355X dense fp8 MFMA
CPU_PASSES = 5  # timed CPU baseline layer passes per thread count (after one warm-up pass)
HBM_PEAK_GBPS = 8000.0
# HBM bytes per steady-state attention launch (Lq 4680 x Lk 32760, H12) measured with rocprofv3
# on `bench.py --probe`: FETCH_SIZE x2.0 (337.45 MB) + WRITE_SIZE x1.0 (14.38 MB); the scale
# factors are what the same counters read for a 1 GiB device copy.  Counters cannot be read
# from inside the process, so the figure is recorded here for the config it was measured on.
# Config 5 (one attention call = the unsplit launch, the tail-split launch and the merge, as
# the roofline's achieved figure is per call): 591.0 + 473.0 + 49.9 MB read, 48.5 + 68.2 +
# 9.1 MB written (profiles/attn_fp8_c5_counters.txt).
ATTN_TRAFFIC_BYTES = {"c2": 351.83e6, "c5": 1239.7e6}
ATTN_TRAFFIC_FILES = {"c2": "profiles/attn_kernel_c2_traffic.txt",
                      "c5": "profiles/attn_fp8_c5_counters.txt"}
ATTN_TRAFFIC_SOURCE = ("recorded constant, not measured in this run: rocprofv3 --pmc FETCH_SIZE "
                       "and WRITE_SIZE runs of `bench.py --probe --config {cfg}` ({file})")
# Launch timing inside the timed rollout: HIP events around every 7th launch of each kind
# (7 is coprime with the 150 launches of a chunk, so the samples rotate over layers and
# passes).  A timing event waits for the work before it; events around every launch cost
# 2-3% of the rollout's wall time.
EVENT_EVERY = 7


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_inputs(cfg, device, seed=1234, outliers=False):
    """Per-layer bf16 Q/K/V of one chunk, N(0,1); with ``outliers`` 1% of K/V channels x20
    (BASELINE config 5)."""
    import torch

    g = torch.Generator(device=device).manual_seed(seed)
    Lq = cfg["chunk_f"] * cfg["T"]
    shape = (cfg["batch"], Lq, cfg["heads"], 128)
    ch = torch.randperm(128, generator=g, device=device)[:2] if outliers else None
    out = []
    for _ in range(cfg["layers"]):
        q, k, v = (torch.randn(shape, generator=g, device=device, dtype=torch.bfloat16) for _ in range(3))
        if ch is not None:
            k[..., ch] *= 20
            v[..., ch] *= 20
        out.append((q, k, v))
    return out


def _rope_config(cfg):
    from solarwm_amd import RopeConfig

    return RopeConfig(grid_hw=cfg["grid"], use_echorope=cfg.get("echorope", True),
                      rope_train_frames=cfg.get("rope_train_frames"))


def make_caches(cfg, device, rope=False, prope=False):
    import torch

    from solarwm_amd import PropeConfig, make_kv_cache_allocator

    alloc = make_kv_cache_allocator(
        num_layers=cfg["layers"], num_heads=cfg["heads"], head_dim=128,
        frame_sequence_length=cfg["T"], local_attn_size=cfg["cap_f"], sink_size=cfg["sink_f"],
        num_frame_per_block=cfg["chunk_f"],
        cache_dtype=torch.float8_e4m3fn if cfg["cache"] == "fp8" else None,
        rope=_rope_config(cfg) if rope or prope else None,
        prope=PropeConfig(camera_translation_transform=cfg.get("translation", "linear")) if prope else None,
    )
    return alloc(cfg["batch"], dtype=torch.bfloat16, device=device)


def camera_trajectory(cfg, frames, device, seed=11):
    """Per-latent-frame cameras [B, F, 4, 4] / [B, F, 3, 3] (float32): a slow pan (yaw up to
    ~0.05 rad per frame) with a forward walk, and the data path's intrinsics
    (data.py:516-530: fx = 969.7/1920, fy = 969.7/1080, principal point 0.5)."""
    import torch

    g = torch.Generator().manual_seed(seed)
    B = cfg["batch"]
    yaw = torch.cumsum(torch.rand(B, frames, generator=g, dtype=torch.float64) * 0.05, dim=1)
    v = torch.zeros(B, frames, 4, 4, dtype=torch.float64)
    v[..., 0, 0], v[..., 0, 2] = yaw.cos(), yaw.sin()
    v[..., 2, 0], v[..., 2, 2] = -yaw.sin(), yaw.cos()
    v[..., 1, 1] = v[..., 3, 3] = 1.0
    v[..., 2, 3] = -0.1 * torch.arange(frames, dtype=torch.float64)
    k = torch.zeros(B, frames, 3, 3, dtype=torch.float64)
    k[..., 0, 0], k[..., 1, 1] = 969.6969696969696 / 1920.0, 969.6969696969696 / 1080.0
    k[..., 0, 2] = k[..., 1, 2] = 0.5
    k[..., 2, 2] = 1.0
    return v.float().to(device), k.float().to(device)


def timed_rollout(cfg, inputs, caches, chunk_ids, cams=None, n_none=len(PASSES) - 1):
    """Run chunks with HIP events around every EVENT_EVERY-th launch of each kind; returns the
    measured figures."""
    import torch

    from solarwm_amd import kernels

    chunk_ids = list(chunk_ids)
    marks = []  # HIP events at chunk boundaries (no synchronisation inside the rollout)

    def mark(_c=None):
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        marks.append(ev)

    with kernels.timed_launches(EVENT_EVERY) as tm:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        mark()
        run_ours(cfg, inputs, caches, chunk_ids, cams, on_chunk=mark, n_none=n_none)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    chunk_ms = [a.elapsed_time(b) for a, b in zip(marks[:-1], marks[1:])]
    # chunks whose window is full (cap_f frames visible): chunk c sees min((c+1)*chunk_f, cap_f)
    full_from = max(0, -(-cfg["cap_f"] // cfg["chunk_f"]) - 1)
    steady_ms = [ms for c, ms in zip(chunk_ids, chunk_ms) if c >= full_from]
    n_attn, attn_ms, attn_flops = tm.summary("attention")
    n_app, app_ms, app_bytes = tm.summary("append")
    recs = tm.records["attention"]
    top = max(w for _, _, w in recs)
    steady = [r for r in recs if r[2] == top]
    st_ms = sum(a.elapsed_time(b) for a, b, _ in steady) / len(steady)
    n = len(list(chunk_ids))
    return {
        "wall_s": wall,
        "chunks": n,
        "frames_per_s": cfg["chunk_f"] * cfg["batch"] * n / wall,
        "attn_launches": n_attn,
        "attn_avg_ms": attn_ms / n_attn,
        "attn_tflops": attn_flops / (attn_ms / 1e3) / 1e12,
        "attn_steady_ms": st_ms,
        "attn_steady_tflops": top / (st_ms / 1e3) / 1e12,
        "append_gbps": app_bytes / (app_ms / 1e3) / 1e9,
        "append_avg_us": app_ms / n_app * 1e3,
        "chunk_ms": chunk_ms,
        "steady_chunks": len(steady_ms),
        "steady_frames_per_s": (cfg["chunk_f"] * cfg["batch"] * len(steady_ms) / (sum(steady_ms) / 1e3)
                                if steady_ms else None),
    }


def run_ours(cfg, inputs, caches, chunk_ids, cams=None, on_chunk=None, n_none=len(PASSES) - 1):
    """Our path over chunks, in the sampler's pass order (``driver.rollout_passes``: ``n_none``
    ``none`` passes, 4 by default, then the commit pass per chunk) with ``driver.cached_forward``'s block loop and
    deferred commit; ``cams`` (per-frame viewmats, K) stages one fused-PRoPE camera pass per
    forward for all layers.  ``on_chunk(c)`` runs after each chunk's commit pass is enqueued."""
    from solarwm_amd import attend_cached, driver, stage_camera_cache

    T, Lq = cfg["T"], cfg["chunk_f"] * cfg["T"]
    chunk_ids = list(chunk_ids)
    outs = [None] * cfg["layers"]
    if not chunk_ids:
        return
    n_frames = (max(chunk_ids) + 1) * cfg["chunk_f"]
    plan = [p for p in driver.rollout_passes(n_frames, cfg["chunk_f"], T, n_none)
            if p.chunk in set(chunk_ids)]
    for p in plan:
        cp = None
        if cams is not None:
            cp = stage_camera_cache(caches, cams[0], cams[1], p.current_start, Lq, per_frame=True)

        def block(layer, cache, p=p, cp=cp):
            q, k, v = inputs[layer]
            x, info = attend_cached(q, k, v, cache, p.current_start, out=outs[layer], camera=cp)
            outs[layer] = x
            return x, info

        driver.cached_forward(caches, block, cache_update_policy=p.policy, camera=cp)
        if p.policy != driver.NONE and on_chunk is not None:
            on_chunk(p.chunk)


def _ref_rope_frames(x, grid, positions, freqs):
    """The reference's window RoPE of one part of the window (echorope_apply,
    causal_model.py:88-197): float64 complex multiply by the table rows of each frame's temporal
    position and each token's (h, w), cast back to x's dtype."""
    import torch

    gh, gw = grid
    B, L, n, D = x.shape
    F = len(positions)
    if F == 0:  # an empty part of the window (no sink frames)
        return x
    ct, ch, cw = 22, 21, 21
    ft, fh, fw = freqs.split([ct, ch, cw], dim=1)
    pos = torch.tensor(list(positions), dtype=torch.long, device=x.device)
    f_all = torch.cat([ft[pos].view(F, 1, 1, ct).expand(F, gh, gw, ct),
                       fh[:gh].view(1, gh, 1, ch).expand(F, gh, gw, ch),
                       fw[:gw].view(1, 1, gw, cw).expand(F, gh, gw, cw)], dim=-1).reshape(L, 1, -1)
    xc = torch.view_as_complex(x.to(torch.float64).reshape(B, L, n, D // 2, 2))
    return torch.view_as_real(xc * f_all).reshape(B, L, n, D).to(x.dtype)


def _ref_freqs(device):
    """Wan's complex RoPE table (model.py:28-35, causal_model.py:1855-1866) on the GPU."""
    import torch

    def params(dim):
        inv = 1.0 / torch.pow(torch.tensor(10000.0, dtype=torch.float64),
                              torch.arange(0, dim, 2, dtype=torch.float64) / dim)
        ang = torch.outer(torch.arange(1024, dtype=torch.float64), inv)
        return torch.polar(torch.ones_like(ang), ang)

    return torch.cat([params(44), params(42), params(42)], dim=1).to(device)


def _ref_projection(viewmats, ks):
    """The reference's per-token PRoPE matrices in float32 (camera_prope.py:206-231,
    :307-338): P = lift(K_norm) V, P⁻¹ = V⁻¹ lift(K_norm⁻¹)."""
    import torch

    kn = torch.zeros_like(ks)
    kn[..., 0, 0], kn[..., 1, 1], kn[..., 2, 2] = ks[..., 0, 0], ks[..., 1, 1], 1.0
    lift = torch.zeros(ks.shape[:-2] + (4, 4), dtype=ks.dtype, device=ks.device)
    lift[..., :3, :3] = kn
    lift[..., 3, 3] = 1.0
    kinv = torch.zeros_like(ks)
    kinv[..., 0, 0], kinv[..., 1, 1], kinv[..., 2, 2] = 1.0 / kn[..., 0, 0], 1.0 / kn[..., 1, 1], 1.0
    lift_inv = torch.zeros_like(lift)
    lift_inv[..., :3, :3] = kinv
    lift_inv[..., 3, 3] = 1.0
    rt = viewmats[..., :3, :3].transpose(-1, -2)
    vinv = torch.zeros_like(viewmats)
    vinv[..., :3, :3] = rt
    vinv[..., :3, 3] = -torch.einsum("...ij,...j->...i", rt, viewmats[..., :3, 3])
    vinv[..., 3, 3] = 1.0
    p = torch.einsum("...ij,...jk->...ik", lift, viewmats)
    return p, torch.einsum("...ij,...jk->...ik", vinv, lift_inv)


def _ref_tiled(feats, mats):
    """_apply_tiled_projmat's per-ray branch (camera_prope.py:234-256) on [B, L, H, D]:
    matrix cast to the features' dtype, one 4x4 per token over every 4-channel group."""
    import torch

    B, L, H, D = feats.shape
    f = feats.transpose(1, 2).reshape(B, H, L, D // 4, 4)
    out = torch.einsum("btij,bntpj->bntpi", mats.to(feats.dtype), f)
    return out.reshape(B, H, L, D).transpose(1, 2)


def reference_gpu_step(cfg, inputs, dense, chunk_ids, rope=False, cams=None):
    """The reference's per-layer op sequence on the GPU with PyTorch-ROCm: clone the cache,
    memmove the non-sink window, slice-assign the chunk, cat sink|local, SDPA; deferred commit
    repeats memmove + assign (causal_model.py:1028-1226, :2856-2921).  With ``rope`` the cache
    is pre-RoPE and the sink, local window and queries are re-roped in float64 every pass
    (_rope_sink_local_and_query, causal_model.py:791-876).  With ``cams`` (per-frame viewmats, K)
    the fused PRoPE mode runs too: the camera cache is staged once per forward
    (causal_model.py:1948-2066: clone, roll, write) and every layer builds per-token P / P⁻¹ of
    its window and applies them with bf16 einsums (causal_model.py:1170-1199 ->
    camera_prope.py:93-256)."""
    import torch
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from solarwm_amd.rope import positions as rope_positions

    freqs = _ref_freqs(inputs[0][0].device) if rope else None
    rcfg = _rope_config(cfg) if rope else None

    T, Lq = cfg["T"], cfg["chunk_f"] * cfg["T"]
    sink = cfg["sink_f"] * T
    cap = cfg["cap_f"] * T
    for c in chunk_ids:
        cs = c * Lq
        for policy in PASSES:
            ups = []
            if cams is not None:
                st0 = dense[0]
                cv = cams[0][:, cs // T : cs // T + Lq // T].repeat_interleave(T, dim=1)
                ck = cams[1][:, cs // T : cs // T + Lq // T].repeat_interleave(T, dim=1)
                tcv, tck = st0["cv"].clone(), st0["ck"].clone()
                ge, le = st0["g"], st0["l"]
                if cs + Lq > ge and Lq + le > cap:
                    ev = Lq + le - cap
                    ro = le - ev - sink
                    nle = le + cs + Lq - ge - ev
                    tcv[:, sink : sink + ro] = tcv[:, sink + ev : sink + ev + ro].clone()
                    tck[:, sink : sink + ro] = tck[:, sink + ev : sink + ev + ro].clone()
                else:
                    nle = le + cs + Lq - ge
                tcv[:, nle - Lq : nle] = cv
                tck[:, nle - Lq : nle] = ck
            for layer, (q, k, v) in enumerate(inputs):
                st = dense[layer]
                ge, le = st["g"], st["l"]
                ce = cs + Lq
                tk = st["k"].clone()
                tv = st["v"].clone()
                if ce > ge and Lq + le > cap:
                    ev = Lq + le - cap
                    ro = le - ev - sink
                    nle = le + ce - ge - ev
                    tk[:, sink : sink + ro] = tk[:, sink + ev : sink + ev + ro].clone()
                    tv[:, sink : sink + ro] = tv[:, sink + ev : sink + ev + ro].clone()
                else:
                    ev = ro = 0
                    nle = le + ce - ge
                ls = nle - Lq
                tk[:, ls:nle] = k
                tv[:, ls:nle] = v
                a_s = min(sink, nle)
                lsw = max(sink, nle - (cap - sink))
                k_sink, k_loc, qr = tk[:, :a_s], tk[:, lsw:nle], q
                if rope:
                    qpos, kpos = rope_positions(
                        rcfg, num_sink_frames=a_s // T, num_local_frames=(nle - lsw) // T,
                        num_new_frames=Lq // T, max_attention_size=cap, frame_tokens=T,
                        current_start_frame=cs // T, sink_branch=True)
                    qr = _ref_rope_frames(q, cfg["grid"], qpos, freqs)
                    k_sink = _ref_rope_frames(k_sink, cfg["grid"], kpos[: a_s // T], freqs)
                    k_loc = _ref_rope_frames(k_loc, cfg["grid"], kpos[a_s // T :], freqs)
                kc = torch.cat([k_sink, k_loc], dim=1)
                vc = torch.cat([tv[:, :a_s], tv[:, lsw:nle]], dim=1)
                if cams is not None:
                    wv = torch.cat([tcv[:, :a_s], tcv[:, lsw:nle]], dim=1)
                    wk = torch.cat([tck[:, :a_s], tck[:, lsw:nle]], dim=1)
                    p_q, _ = _ref_projection(cv, ck)
                    _, p_kinv = _ref_projection(wv, wk)
                    qr = _ref_tiled(qr, p_q.transpose(-1, -2))
                    kc, vc = _ref_tiled(kc, p_kinv), _ref_tiled(vc, p_kinv)
                with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                    x = torch.nn.functional.scaled_dot_product_attention(
                        qr.transpose(1, 2).contiguous(), kc.transpose(1, 2).contiguous(),
                        vc.transpose(1, 2).contiguous(),
                    ).transpose(1, 2).contiguous()
                if cams is not None:
                    x = _ref_tiled(x, p_q)
                ups.append((layer, ev, ro, ls, nle, ce, k, v))
                del x
            if policy != "none":
                for layer, ev, ro, ls, nle, ce, k, v in ups:
                    st = dense[layer]
                    if ro > 0:
                        st["k"][:, sink : sink + ro] = st["k"][:, sink + ev : sink + ev + ro].clone()
                        st["v"][:, sink : sink + ro] = st["v"][:, sink + ev : sink + ev + ro].clone()
                    st["k"][:, ls:nle] = k
                    st["v"][:, ls:nle] = v
                    st["g"], st["l"] = ce, nle
                if cams is not None:
                    dense[0]["cv"].copy_(tcv)
                    dense[0]["ck"].copy_(tck)


def _host_cores():
    """(cores this process may run on, os.cpu_count())."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return avail, os.cpu_count() or 1


def cpu_baseline(cfg):
    """Reference op sequence on the host CPU (the oracle's restatement, bf16 SDPA as the
    reference's fallback, attention.py:172-188): one steady-state C2 layer pass (rolling eviction
    over a full cache), extrapolated to frames/s of the 30-layer, 5-pass chunk.  Timed with the
    thread count torch starts with (the box's CPU share, OMP_NUM_THREADS) and with os.cpu_count()
    threads, each after one untimed warm-up pass, as the median of CPU_PASSES timed passes; the
    faster thread count is reported."""
    import torch

    from oracle import wan_cache_ref as ref

    T, Lq, H = cfg["T"], cfg["chunk_f"] * cfg["T"], cfg["heads"]
    cap = cfg["cap_f"] * T
    g = torch.Generator().manual_seed(7)
    cache = ref.allocate_kv_cache(1, cfg["batch"], cap, H, 128, torch.bfloat16)
    cache[0]["k"].copy_(torch.randn(cache[0]["k"].shape, generator=g).bfloat16())
    cache[0]["v"].copy_(torch.randn(cache[0]["v"].shape, generator=g).bfloat16())
    cache[0]["global_end_index"].fill_(cap)
    cache[0]["local_end_index"].fill_(cap)
    q, k, v = (torch.randn(cfg["batch"], Lq, H, 128, generator=g).bfloat16() for _ in range(3))
    avail, total = _host_cores()
    start_threads = torch.get_num_threads()
    times, samples = {}, {}
    for threads in sorted({start_threads, total}):
        torch.set_num_threads(threads)
        runs = []
        for i in range(CPU_PASSES + 1):  # the first pass warms the allocator and the thread pool
            t0 = time.perf_counter()
            ref.cached_self_attention(
                q, k, v, cache[0], current_start=cap, frame_seqlen=T, sink_size=cfg["sink_f"],
                local_attn_size=cfg["cap_f"], attn_fn=ref.sdpa_fallback_attention,
            )
            if i:
                runs.append(time.perf_counter() - t0)
        samples[threads] = runs
        times[threads] = sorted(runs)[len(runs) // 2]
    torch.set_num_threads(start_threads)
    best = min(times, key=times.get)
    dt = times[best]
    per_chunk = dt * cfg["layers"] * len(PASSES)
    return {
        "value": round(cfg["chunk_f"] / per_chunk, 6),
        "unit": "latent frames/s",
        "cores": best,
        "kind": "port",
        "sample": (
            f"steady-state layer passes (Lq={Lq}, Lk={cap}, H={H}, rolling eviction) of the "
            f"reference op sequence: median {dt:.2f} s of {CPU_PASSES} timed passes after a "
            f"warm-up, {best} threads, x{cfg['layers']} layers x{len(PASSES)} passes"
        ),
        "seconds_by_threads": {str(t): round(x, 3) for t, x in times.items()},
        "passes_by_threads": {str(t): [round(x, 3) for x in r] for t, r in samples.items()},
        "host_cpu_count": total,
        "host_cores_available": avail,
    }


def cpu_c1_end_to_end():
    """BASELINE config 1 end to end on the host CPU: the oracle's restatement of the reference
    cache branch (fp32, H12 x 128, 390 tokens/frame, chunks of 3 frames, 21-frame cache with a
    1-frame sink, 10 chunks x 2 passes, commit on the 2nd, one layer, float32 SDPA), timed with
    the starting thread count and with os.cpu_count() threads."""
    import torch

    from oracle import wan_cache_ref as ref

    T, chunk_f, cap_f, sink_f, H = 390, 3, 21, 1, 12
    Lq = chunk_f * T
    g = torch.Generator().manual_seed(1)
    data = [[tuple(torch.randn(1, Lq, H, 128, generator=g) * 128 ** -0.5 for _ in range(3))
             for _ in range(2)] for _ in range(10)]

    def inputs(c, p, layer):
        return data[c][p]

    avail, total = _host_cores()
    start_threads = torch.get_num_threads()
    times = {}
    for threads in sorted({start_threads, total}):
        torch.set_num_threads(threads)
        cache = ref.allocate_kv_cache(1, 1, cap_f * T, H, 128, torch.float32)
        t0 = time.perf_counter()
        ref.rollout(10, ["none", "commit"], Lq, inputs, cache, frame_seqlen=T, sink_size=sink_f,
                    local_attn_size=cap_f,
                    attn_fn=lambda q, k, v: ref.attention(q, k, v, compute_dtype=torch.float32,
                                                          round_inputs_to_bf16=False))
        times[threads] = time.perf_counter() - t0
    torch.set_num_threads(start_threads)
    best = min(times, key=times.get)
    return {
        "value": round(30 / times[best], 4),
        "unit": "latent frames/s",
        "cores": best,
        "kind": "port",
        "sample": "config 1 end to end: 10 chunks x 2 passes (30 latent frames), 1 layer, fp32",
        "seconds_by_threads": {str(t): round(x, 3) for t, x in times.items()},
        "host_cpu_count": total,
        "host_cores_available": avail,
    }


def _back_to_back_ms(launch, iters):
    """Average milliseconds per launch of a prepared launcher (arguments validated once, so the
    host issues launches faster than the kernels run) issued back to back on the current stream
    between one pair of HIP events."""
    import torch

    launch()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        launch()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


def append_bandwidth(cfg, device, iters=48, min_source_bytes=768 << 20):
    """One chunk's append (chunk_f frames of K and V, the config's batch and heads) into staging
    slots, launched back to back.  Launches rotate over enough distinct source chunks (at least
    10, and at least 768 MB of K/V, three times the 256 MB MALL) that every source is read cold
    from HBM.  Algorithmic bytes = K+V read + write."""
    import torch

    from solarwm_amd import kernels

    T, H, B, nf = cfg["T"], cfg["heads"], cfg["batch"], cfg["chunk_f"]
    dt = torch.bfloat16 if cfg["cache"] == "bf16" else torch.float8_e4m3fn
    g = torch.Generator(device=device).manual_seed(5)
    chunk_bytes = 2 * B * nf * T * H * 128 * 2
    n_src = max(10, -(-min_source_bytes // chunk_bytes))
    kpool, vpool, ks, vs = kernels.new_pools(cfg["cap_f"] + nf, B, H, T, dt, device)
    dst = list(range(cfg["cap_f"], cfg["cap_f"] + nf))
    launches = []
    for _ in range(n_src):
        k = torch.randn(B, nf * T, H, 128, generator=g, device=device, dtype=torch.bfloat16)
        v = torch.randn(B, nf * T, H, 128, generator=g, device=device, dtype=torch.bfloat16)
        launches.append(kernels.prepare_append(k, v, kpool, vpool, dst, frame_tokens=T,
                                               kscale=ks, vscale=vs))
    it = iter(range(1 << 30))

    def launch():
        launches[next(it) % n_src]()

    ms = _back_to_back_ms(launch, iters)
    moved = launches[0].bytes_moved
    del kpool, vpool, launches
    # the same bytes as one plain device copy (torch copy_ of the chunk's K+V bytes from the
    # same rotating cold sources): what a transfer of this size reaches on this GPU
    flat = torch.empty(chunk_bytes // 2, dtype=torch.bfloat16, device=device)
    srcs = [torch.randn(chunk_bytes // 2, generator=g, device=device, dtype=torch.bfloat16)
            for _ in range(n_src)]
    it2 = iter(range(1 << 30))
    copy_ms = _back_to_back_ms(lambda: flat.copy_(srcs[next(it2) % n_src]), iters)
    del flat, srcs
    torch.cuda.empty_cache()
    return moved / (ms / 1e3) / 1e9, ms, n_src, n_src * chunk_bytes, 2 * chunk_bytes / (copy_ms / 1e3) / 1e9


def gather_bandwidth(device, iters=24):
    """Config-4 memory-bank gather: every launch materialises its own 8 seeded frames
    (randperm(256)[:8] per launch, as each chunk draws) of a 256-slot bank (H=40, 1560 tokens per
    frame) token-major, launched back to back; algorithmic bytes = K+V read + write."""
    import torch

    from solarwm_amd import kernels

    T, H, n_bank = 1560, 40, 256
    kpool, vpool, _, _ = kernels.new_pools(n_bank, 1, H, T, torch.bfloat16, device)
    kpool.normal_()
    vpool.normal_()
    g = torch.Generator().manual_seed(4)
    ko = torch.empty(1, 8 * T, H, 128, dtype=torch.bfloat16, device=device)
    vo = torch.empty_like(ko)
    launches = []
    for _ in range(iters + 1):
        idx = torch.randperm(n_bank, generator=g)[:8].tolist()
        launches.append(kernels.prepare_gather(kpool, vpool, idx, frame_tokens=T, k_out=ko,
                                               v_out=vo)[0])
    it = iter(range(1 << 30))

    def launch():
        launches[next(it) % len(launches)]()

    ms = _back_to_back_ms(launch, iters)
    moved = launches[0].bytes_moved
    del kpool, vpool, ko, vo, launches
    torch.cuda.empty_cache()
    # the same bytes as one plain device copy (torch copy_ of 255.6 MB), three source /
    # destination pairs in rotation (767 MB each side, three times the 256 MB MALL) so that
    # neither the reads nor the rewrites are served from the cache
    n = moved // 4  # bf16 elements per side: K+V of 8 frames
    gd = torch.Generator(device=device).manual_seed(6)
    pairs = [(torch.randn(n, generator=gd, device=device, dtype=torch.bfloat16),
              torch.empty(n, device=device, dtype=torch.bfloat16)) for _ in range(3)]
    it2 = iter(range(1 << 30))

    def copy():
        src, dst = pairs[next(it2) % 3]
        dst.copy_(src)

    copy_ms = _back_to_back_ms(copy, iters)
    del pairs
    torch.cuda.empty_cache()
    return moved / (ms / 1e3) / 1e9, ms, moved / (copy_ms / 1e3) / 1e9


def eviction_latency(cfg, iters=2000):
    """Eviction is slot-table arithmetic on the host (causal_model.py:1054-1067 memmove and
    2863-2921 commit replaced by a permutation of frame slots): time one layer's plan + stage +
    commit in steady state (full window, rolling eviction of chunk_f frames), and report the
    reference's clone + memmove bytes per layer and pass that it replaces."""
    from solarwm_amd.cache import CacheGeometry, SlotTable

    T, H, cap, sink, chunk = cfg["T"], cfg["heads"], cfg["cap_f"], cfg["sink_f"], cfg["chunk_f"]
    geom = CacheGeometry(batch=cfg["batch"], heads=H, head_dim=128, frame_tokens=T,
                         capacity_frames=cap, sink_frames=sink, staging_frames=chunk)
    tab = SlotTable(geom)
    Lq = chunk * T
    start = 0
    for _ in range(-(-cap // chunk) + 2):  # fill the window, then roll twice
        p, temp, _, _ = tab.plan(start, Lq)
        tab.commit(tab.stage(p, temp), p.current_end, p.local_end_index)
        start += Lq
    rolled = None
    t0 = time.perf_counter()
    for _ in range(iters):
        p, temp, _, _ = tab.plan(start, Lq)
        tab.commit(tab.stage(p, temp), p.current_end, p.local_end_index)
        rolled = p.num_rolled_tokens
        start += Lq
    us = (time.perf_counter() - t0) / iters * 1e6
    elem = cfg["batch"] * H * 128 * 2  # bytes per token of K (or V), bf16
    clone = 2 * 2 * cap * T * elem     # read + write of K and V
    memmove = 2 * 2 * rolled * elem    # read + write of the rolled tokens of K and V
    return {
        "host_us_per_layer_pass": round(us, 2),
        "device_bytes": 0,
        "reference_bytes_avoided_per_layer_pass": clone + memmove,
        "reference_clone_bytes": clone,
        "reference_memmove_bytes": memmove,
        "note": "plan + stage + commit of one layer's slot table in steady state (rolling "
                f"eviction of {chunk} frames); no bytes move on the GPU",
    }


def probe(cfg, device, iters=20):
    """Short fixed sequence for hardware-counter runs (rocprofv3 --pmc): a plain device copy of
    exactly 1 GiB (the FETCH_SIZE / WRITE_SIZE calibration), then steady-state launches of the
    append kernel (one chunk of Lq tokens per launch, rotating over 10 cold source chunks as in
    the rollout, where each layer appends its own freshly projected K/V), the attention kernel
    (Lq x the full window; fp8 pools for config 5) and, for config 2, the config-4 memory-bank
    gather (8 seeded frames of a 256-slot bank per launch, H=40, fresh indices every launch)."""
    import torch

    from solarwm_amd import kernels

    src = torch.empty(1 << 29, dtype=torch.int16, device=device).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)  # 1 GiB read + 1 GiB written per launch
    torch.cuda.synchronize()
    del src, dst
    T, Lq, H, B = cfg["T"], cfg["chunk_f"] * cfg["T"], cfg["heads"], cfg["batch"]
    n = cfg["cap_f"]
    fp8 = cfg["cache"] == "fp8"
    dt = torch.float8_e4m3fn if fp8 else torch.bfloat16
    kpool, vpool, ks, vs = kernels.new_pools(n + cfg["chunk_f"], B, H, T, dt, device)
    srcs = make_inputs(dict(cfg, layers=10), device, outliers=fp8)
    q, k, v = srcs[0]
    for f in range(n):
        kernels.append_frames(k, v, kpool, vpool, [f], frame_tokens=T,
                              src_frame0=f % cfg["chunk_f"], kscale=ks, vscale=vs)
    slots = list(range(n))
    appends = [kernels.prepare_append(kk, vv, kpool, vpool, [n, n + 1, n + 2], frame_tokens=T,
                                      kscale=ks, vscale=vs) for _, kk, vv in srcs]
    for i in range(iters):
        appends[i % len(appends)]()
    for _ in range(iters):
        kernels.attention_frames(q, kpool, vpool, slots, frame_tokens=T, kscale=ks, vscale=vs)
    torch.cuda.synchronize()
    del kpool, vpool, srcs, appends
    torch.cuda.empty_cache()
    msg = (f"[probe] copy 1 GiB x3, append x{iters} ({Lq} tokens, 10 rotating sources), attention "
           f"x{iters} (B{B} H{H} Lq {Lq}, Lk {n * T}, {cfg['cache']} pools)")
    if cfg is CONFIGS["c2"]:
        Tb, Hb, n_bank = C4["T"], C4["heads"], C4["bank"]
        bk, bv, _, _ = kernels.new_pools(n_bank, 1, Hb, Tb, torch.bfloat16, device)
        g = torch.Generator().manual_seed(4)
        ko = torch.empty(1, C4["mem_frames"] * Tb, Hb, 128, dtype=torch.bfloat16, device=device)
        vo = torch.empty_like(ko)
        for _ in range(iters):
            idx = torch.randperm(n_bank, generator=g)[:C4["mem_frames"]].tolist()
            kernels.prepare_gather(bk, bv, idx, frame_tokens=Tb, k_out=ko, v_out=vo)[0]()
        torch.cuda.synchronize()
        msg += f", gather x{iters} ({C4['mem_frames']} of {n_bank} frames, H{Hb}, fresh indices)"
    log(msg)


def four_pass_leg(device):
    """The config-2 rollout with 4 passes per chunk, the 4th committing (3 ``none`` + 1 commit:
    the NFE-4 count of BASELINE's configs with the cache written on the last denoising step),
    beside the headline's reference-faithful 4 ``none`` + 1 commit (stage2.py:683-760)."""
    import torch

    cfg = CONFIGS["c2"]
    inputs = make_inputs(cfg, device)
    caches = make_caches(cfg, device)
    run_ours(cfg, inputs, caches, range(2), n_none=3)  # warmup, then back to an empty cache
    torch.cuda.synchronize()
    for c in caches:
        c.reset()
    torch.cuda.synchronize()
    st = timed_rollout(cfg, inputs, caches, range(cfg["chunks"]), n_none=3)
    del inputs, caches
    torch.cuda.empty_cache()
    return {
        "frames_per_s": round(st["frames_per_s"], 4),
        "steady_frames_per_s": round(st["steady_frames_per_s"], 4) if st["steady_frames_per_s"] else None,
        "attn_tflops": round(st["attn_tflops"], 1),
        "workload": f"{cfg['workload']}: {cfg['chunks']} chunks x (3 none + 1 commit) passes, "
                    f"{cfg['layers']} layers",
    }


def steady_state(name, device, fill=7, timed=3, rope=False, prope=False):
    """Configs 3 and 5 (and config 2 with RoPE on load): fill the 21-frame window (chunks
    0..fill-1, untimed), then time `timed` steady-state chunks (4 none + 1 commit passes over all
    layers)."""
    import torch

    cfg = CONFIGS[name]
    inputs = make_inputs(cfg, device, outliers=cfg["cache"] == "fp8")
    caches = make_caches(cfg, device, rope=rope, prope=prope)
    cams = camera_trajectory(cfg, (fill + timed) * cfg["chunk_f"], device) if prope else None
    run_ours(cfg, inputs, caches, range(fill), cams)
    st = timed_rollout(cfg, inputs, caches, range(fill, fill + timed), cams)
    st["workload"] = (
        f"{cfg['workload']}: {cfg['layers']} layers, H{cfg['heads']}xD128, {cfg['T']} tok/frame, "
        f"Lq {cfg['chunk_f'] * cfg['T']}, window {cfg['cap_f'] * cfg['T']} keys, batch "
        f"{cfg['batch']}, {cfg['cache']} cache{', pre-RoPE cache (RoPE on load)' if rope else ''}"
        f"{', pre-RoPE camera-aware cache (RoPE + fused PRoPE on load)' if prope else ''}; "
        f"chunks {fill}..{fill + timed - 1} (steady state)"
    )
    del inputs, caches
    torch.cuda.empty_cache()
    return st


def c2_rope(device, fill=7, timed=2, prope=False, name="c2"):
    """Config 2 (or ``name``) with a pre-RoPE cache, as the reference keeps it: ours (RoPE
    applied on load by the kernels) against the reference op sequence that re-ropes the window
    in float64 every pass, both over steady-state chunks.  ``prope``: the fused-PRoPE camera
    mode on top (one camera per latent frame, a slow pan), against the reference's per-layer
    per-token camera matrices and bf16 einsums."""
    import torch

    ours = steady_state(name, device, fill=fill, timed=timed, rope=True, prope=prope)
    cfg = CONFIGS[name]
    inputs = make_inputs(cfg, device)
    T = cfg["T"]
    # the reference's caches start full (global = local end = the 21-frame window), the state
    # after `fill` chunks; the timed chunks then evict and re-rope exactly as in steady state
    full = cfg["cap_f"] * T
    dense = [
        {"k": torch.zeros(cfg["batch"], full, cfg["heads"], 128, dtype=torch.bfloat16, device=device),
         "v": torch.zeros(cfg["batch"], full, cfg["heads"], 128, dtype=torch.bfloat16, device=device),
         "g": fill * cfg["chunk_f"] * T, "l": full}
        for _ in range(cfg["layers"])
    ]
    cams = None
    if prope:
        cams = camera_trajectory(cfg, (fill + 1 + timed) * cfg["chunk_f"], device)
        # camera cache rows of the full window: valid matrices (frame 0's camera)
        dense[0]["cv"] = cams[0][:, :1].expand(-1, full, -1, -1).contiguous()
        dense[0]["ck"] = cams[1][:, :1].expand(-1, full, -1, -1).contiguous()
    reference_gpu_step(cfg, inputs, dense, range(fill, fill + 1), rope=True, cams=cams)  # warm
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    reference_gpu_step(cfg, inputs, dense, range(fill + 1, fill + 1 + timed), rope=True, cams=cams)
    torch.cuda.synchronize()
    rfps = cfg["chunk_f"] * timed / (time.perf_counter() - t0)
    del dense, inputs
    torch.cuda.empty_cache()
    return {
        "frames_per_s": round(ours["frames_per_s"], 4),
        "attn_tflops": round(ours["attn_tflops"], 1),
        "attn_avg_ms": round(ours["attn_avg_ms"], 4),
        "reference_gpu_frames_per_s": round(rfps, 4),
        "speedup": round(ours["frames_per_s"] / rfps, 3),
        "workload": ours["workload"],
        "note": ("reference = the same op sequence with its float64 window re-rope per pass"
                 + (" and per-layer per-token PRoPE matrices applied by bf16 einsums" if prope else "")),
    }


def commit_path(device, iters=20):
    """Config 2, one layer in steady state: what q/k RMSNorm (causal_model.py:908-910) costs on
    our path (norms folded into the append and the attention Q load, plus two inverse-RMS
    passes) against the reference's in-dtype bf16 norm_q + norm_k (WanRMSNorm, model.py:69-84)
    on the same tensors; and cross-attention over the cached 512-token text context (ours: the
    attention kernel with Q normalised at load; reference: norm_q + flash SDPA over the cached
    K/V, model.py:152-184)."""
    from types import SimpleNamespace

    import torch
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from solarwm_amd import attend_cached, cross_attend, make_crossattn_cache_allocator

    cfg = dict(CONFIGS["c2"], layers=1)
    T, Lq, H = cfg["T"], cfg["chunk_f"] * cfg["T"], cfg["heads"]
    inputs = make_inputs(cfg, device)
    q, k, v = inputs[0]
    g = torch.Generator(device=device).manual_seed(3)
    norm = [SimpleNamespace(weight=(torch.rand(H * 128, generator=g, device=device) + 0.5).bfloat16(),
                            eps=1e-6) for _ in range(2)]

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / iters * 1e3  # us

    caches = make_caches(cfg, device)
    run_ours(cfg, inputs, caches, range(7))
    start = 7 * Lq
    plain = timed(lambda: attend_cached(q, k, v, caches[0], start))
    fused = timed(lambda: attend_cached(q, k, v, caches[0], start, norm_q=norm[0], norm_k=norm[1]))

    def ref_norms():
        for x, n in ((q, norm[0]), (k, norm[1])):
            xf = x.reshape(cfg["batch"], Lq, H * 128)
            (xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + n.eps)).type_as(xf) * n.weight

    ref_norm = timed(ref_norms)
    del caches
    xc = make_crossattn_cache_allocator(num_layers=1, num_heads=H, head_dim=128)(
        cfg["batch"], dtype=torch.bfloat16, device=device)[0]
    ck = torch.randn(cfg["batch"], 512, H, 128, generator=g, device=device, dtype=torch.bfloat16)
    cv = torch.randn_like(ck)
    cross_attend(q, ck, cv, xc, norm_q=norm[0], norm_k=norm[1])
    ours_x = timed(lambda: cross_attend(q, None, None, xc, norm_q=norm[0]))
    kt, vt = ck.transpose(1, 2).contiguous(), cv.transpose(1, 2).contiguous()

    def ref_cross():
        qf = q.reshape(cfg["batch"], Lq, H * 128)
        qn = ((qf * torch.rsqrt(qf.pow(2).mean(dim=-1, keepdim=True) + 1e-6)).type_as(qf)
              * norm[0].weight).view(cfg["batch"], Lq, H, 128)
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            torch.nn.functional.scaled_dot_product_attention(qn.transpose(1, 2).contiguous(), kt, vt)

    ref_x = timed(ref_cross)
    del inputs, xc
    torch.cuda.empty_cache()
    return {
        "layer_pass_us": round(plain, 1),
        "layer_pass_with_qk_norm_us": round(fused, 1),
        "our_qk_norm_cost_us": round(fused - plain, 1),
        "reference_qk_norm_us": round(ref_norm, 1),
        "cross_attention_us": round(ours_x, 1),
        "reference_cross_attention_us": round(ref_x, 1),
        "workload": f"config 2 layer in steady state (Lq {Lq}, window {cfg['cap_f'] * T} keys, H{H}); "
                    f"cross-attention Lq {Lq} over 512 cached context tokens",
    }


def single_frame_leg(device, iters=20):
    """One frame of queries per block (num_frame_per_block = 1: Lq = 1560) over the config-2
    window (21 frames x 1560 keys, H12).  The unsplit grid would be 7 q-tiles x 12 heads = 84
    workgroups on 256 CUs, so the launcher splits the key range over every CU (one workgroup per
    CU, partials merged by a second kernel).  Reference: flash SDPA on the already-materialised
    window (its cat/clone copies are not counted)."""
    import torch
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from solarwm_amd import kernels

    T, H, n, Lq = 1560, 12, 21, 1560
    g = torch.Generator(device=device).manual_seed(11)
    q = torch.randn(1, Lq, H, 128, generator=g, device=device, dtype=torch.bfloat16)
    k = torch.randn(1, n * T, H, 128, generator=g, device=device, dtype=torch.bfloat16)
    v = torch.randn(1, n * T, H, 128, generator=g, device=device, dtype=torch.bfloat16)
    kp, vp, _, _ = kernels.new_pools(n, 1, H, T, torch.bfloat16, device)
    kernels.append_frames(k, v, kp, vp, list(range(n)), frame_tokens=T)
    slots = list(range(n))

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / iters

    ours = timed(lambda: kernels.attention_frames(q, kp, vp, slots, frame_tokens=T))
    qt, kt, vt = (x.transpose(1, 2).contiguous() for x in (q, k, v))

    def ref():
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            torch.nn.functional.scaled_dot_product_attention(qt, kt, vt)

    ref_ms = timed(ref)
    flops = 4.0 * Lq * n * T * H * 128
    del q, k, v, kp, vp, qt, kt, vt
    torch.cuda.empty_cache()
    return {
        "attn_ms": round(ours, 4),
        "attn_tflops": round(flops / (ours / 1e3) / 1e12, 1),
        "reference_ms": round(ref_ms, 4),
        "reference_tflops": round(flops / (ref_ms / 1e3) / 1e12, 1),
        "speedup": round(ref_ms / ours, 2),
        "workload": f"one frame of queries (Lq {Lq}) over {n} x {T} cached keys, H{H}, bf16; "
                    "key range split over all CUs (84 q-tile workgroups unsplit)",
    }


def segments_leg(device, iters=5):
    """Segmented attention at the config-2 head shape (H12, 1560 tok/frame):
    * teacher forcing over [clean | noisy] x 6 frames (2 chunks of 3, sink 1 chunk, 1 prior clean
      chunk; causal_model.py:337-471): ours (one segmented launch: every query chunk over its
      own frame list; one launch per chunk timed beside it) vs the reference's op, FlexAttention with a block mask of the same rule
      (causal_model.py:984-989; torch.compile'd, timed after compiling), and vs SDPA with the
      dense boolean mask (its fallback);
    * H3 rollout window (sgf_attention.py:236-258): a 5-frame chunk over a 1000-token prefix,
      5 history chunks and itself: ours (chunk-list cache, ragged prefix) vs torch.cat + flash
      SDPA.
    FLOPs count visible keys only."""
    import torch
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from solarwm_amd.segments import (ChunkListKVCache, attend_segments, teacher_forcing_attention,
                                      teacher_forcing_frame_lists, windowed_attention)

    T, H = 1560, 12
    g = torch.Generator(device=device).manual_seed(9)

    def rnd(*shape):
        return torch.randn(*shape, generator=g, device=device, dtype=torch.bfloat16)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / iters

    F, nb = 6, 3
    kw = dict(num_frames=F, frame_seqlen=T, num_frame_per_block=nb, max_prior_clean_chunks=1,
              sink_size=3)
    L = 2 * F * T
    q, k, v = rnd(1, L, H, 128), rnd(1, L, H, 128), rnd(1, L, H, 128)
    lists = teacher_forcing_frame_lists(**{x: kw[x] for x in ("num_frames", "num_frame_per_block",
                                                               "max_prior_clean_chunks", "sink_size")})
    tf_flops = sum(4.0 * nb * T * len(fr) * T * H * 128 for _, fr in lists)
    ours_tf = timed(lambda: teacher_forcing_attention(q, k, v, **kw))
    # the same attention as one launch per query chunk (the segments' frame lists over the same
    # staged pools)
    from solarwm_amd import kernels

    kp, vp = kernels.staging_pools(2 * F, 1, H, T, torch.bfloat16, device)
    kernels.append_frames(k, v, kp, vp, list(range(2 * F)), frame_tokens=T)
    o_per = torch.empty_like(q)

    def per_chunk():
        for f0, frames in lists:
            s = slice(f0 * T, (f0 + nb) * T)
            kernels.attention_frames(q[:, s], kp, vp, frames, frame_tokens=T, out=o_per[:, s])

    per_tf = timed(per_chunk)
    o_one = torch.empty_like(q)
    segs = [(nb * T, frames, None) for _, frames in lists]
    one_tf = timed(lambda: attend_segments(q, kp, vp, segs, frame_tokens=T, out=o_one))
    torch.cuda.synchronize()
    tf_launch_diff = float((o_one.float() - o_per.float()).abs().max())
    # the dense mask of the same rule, built on the host from the frame lists
    mask = torch.zeros(L, L, dtype=torch.bool)
    for f0, frames in lists:
        for fr in frames:
            mask[f0 * T : (f0 + nb) * T, fr * T : (fr + 1) * T] = True
    mask = mask.to(device)
    qt, kt, vt = (x.transpose(1, 2).contiguous() for x in (q, k, v))
    sdpa_tf = timed(lambda: torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask))
    flex_tf, flex_note = None, None
    try:
        from torch.nn.attention.flex_attention import create_block_mask, flex_attention

        allowed = torch.zeros(2 * F // nb, 2 * F, dtype=torch.bool)
        for f0, frames in lists:
            for fr in frames:
                allowed[f0 // nb, fr] = True
        allowed = allowed.to(device)

        def mask_mod(b, h, q_idx, kv_idx):
            return allowed[q_idx // (nb * T), kv_idx // T]

        block_mask = create_block_mask(mask_mod, 1, 1, L, L, device=device)
        flex = torch.compile(flex_attention, dynamic=False)
        flex_tf = timed(lambda: flex(qt, kt, vt, block_mask=block_mask))
    except Exception as e:  # the baseline only: report why it is missing
        flex_note = f"FlexAttention unavailable: {type(e).__name__}: {str(e)[:160]}"
    ref_tf = flex_tf if flex_tf is not None else sdpa_tf
    del mask, qt, kt, vt, q, k, v, o_per, o_one

    cf, P = 5, 1000
    cache = ChunkListKVCache(num_layers=1, batch=1, heads=H, frame_tokens=T, chunk_frames=cf,
                             window=5, span_frames=1, device=device)
    pk, pv = rnd(1, P, H, 128), rnd(1, P, H, 128)
    for c in range(5):
        windowed_attention(rnd(1, cf * T, H, 128), rnd(1, cf * T, H, 128), rnd(1, cf * T, H, 128),
                           cache, 0, c, prefix=(pk, pv), commit=True)
    q, k, v = rnd(1, cf * T, H, 128), rnd(1, cf * T, H, 128), rnd(1, cf * T, H, 128)
    ours_w = timed(lambda: windowed_attention(q, k, v, cache, 0, 5, prefix=(pk, pv)))
    hist = [(rnd(1, cf * T, H, 128), rnd(1, cf * T, H, 128)) for _ in range(5)]

    def ref_window():
        keys = torch.cat([pk, *(a for a, _ in hist), k], 1)
        vals = torch.cat([pv, *(b for _, b in hist), v], 1)
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            torch.nn.functional.scaled_dot_product_attention(
                q.transpose(1, 2).contiguous(), keys.transpose(1, 2).contiguous(),
                vals.transpose(1, 2).contiguous())

    ref_w = timed(ref_window)
    w_flops = 4.0 * cf * T * (P + 6 * cf * T) * H * 128
    del cache, hist, q, k, v, pk, pv
    torch.cuda.empty_cache()
    out = {
        "teacher_forcing_ms": round(ours_tf, 3),
        "teacher_forcing_tflops": round(tf_flops / (ours_tf / 1e3) / 1e12, 1),
        "teacher_forcing_reference_ms": round(ref_tf, 3),
        "teacher_forcing_reference": "flex_attention + block mask" if flex_tf is not None else "SDPA + dense mask",
        "teacher_forcing_speedup": round(ref_tf / ours_tf, 2),
        "teacher_forcing_sdpa_dense_mask_ms": round(sdpa_tf, 3),
        "teacher_forcing_attention_ms": round(one_tf, 3),
        "teacher_forcing_per_chunk_launches_ms": round(per_tf, 3),
        "teacher_forcing_launch_max_abs_diff": tf_launch_diff,
        "h3_window_ms": round(ours_w, 3),
        "h3_window_tflops": round(w_flops / (ours_w / 1e3) / 1e12, 1),
        "h3_window_reference_ms": round(ref_w, 3),
        "h3_window_speedup": round(ref_w / ours_w, 2),
        "workload": (f"teacher forcing [clean|noisy] 2x{F} frames x {T} tok, H{H}, chunks of {nb}, "
                     f"sink 1 chunk, 1 prior chunk (reference: FlexAttention with the block mask); H3 window "
                     f"{cf}-frame chunk over {P} prefix + 5 history chunks (reference: cat + flash SDPA)"),
    }
    if flex_note:
        out["teacher_forcing_note"] = flex_note
    return out


def h3_leg(device, iters=20):
    """H3's transforms (H12 x 128, 1560-token frames, a 5-frame chunk over a 1000-row prefix
    and 5 history chunks, the segments leg's window):
    * ``skv_h3_rope_prope`` over the window's 47800 key rows (rotary + camera projection), bytes
      = read + write of the rows (tables and matrices excluded), cold sources (three rotating
      inputs over the 256 MB MALL), vs the same transform as the reference's eager torch ops
      (rotate-half in bf16, per-row 4x4 einsum, cat: sgf_attention.py:199-203 with
      torch_prope.py:79-93);
    * one evaluation of a chunk through H3WindowCache with its window already built (the four
      denoising evaluations after the first): transforms of the chunk's q / k / v, their append,
      attention over the window, the output projection."""
    import torch

    from solarwm_amd import h3
    from solarwm_amd.segments import H3WindowCache

    T, H, cf, P = 1560, 12, 5, 1000
    C = cf * T
    rows = P + 6 * C
    g = torch.Generator(device=device).manual_seed(33)
    bf = torch.bfloat16
    xs = [torch.randn(1, rows, H, 128, generator=g, device=device, dtype=bf) for _ in range(3)]
    outs = [torch.empty_like(x) for x in xs]
    theta = torch.rand(rows, 48, generator=g, device=device) * 20.0
    cos = torch.cat([theta.cos(), theta.cos()], 1).to(bf)
    sin = torch.cat([theta.sin(), theta.sin()], 1).to(bf)
    m = (torch.randn(1, rows, 4, 4, generator=g, device=device) * 0.6).to(bf)
    it = iter(range(1 << 30))

    def ours():
        i = next(it) % 3
        h3.rope_prope(xs[i], cos, sin, m, out=outs[i])

    ms = _back_to_back_ms(ours, iters)
    nbytes = 2 * rows * H * 128 * 2

    def eager():
        x = xs[next(it) % 3]
        x1, x2 = x[..., :48], x[..., 48:96]
        c, s_ = cos[None, :, None], sin[None, :, None]
        rot = torch.cat([x1 * c[..., :48] - x2 * s_[..., :48], x2 * c[..., 48:] + x1 * s_[..., 48:]], -1)
        cam = torch.einsum("bsij,bshpj->bshpi", m, x[..., 96:].reshape(1, rows, H, 8, 4))
        torch.cat([rot, cam.reshape(1, rows, H, 32)], -1)

    eager_ms = _back_to_back_ms(eager, iters)
    del xs, outs
    torch.cuda.empty_cache()
    cache = H3WindowCache(num_layers=1, batch=1, heads=H, frame_tokens=T, prefix_rows=P,
                          chunk_frames=cf, window=5, device=device)
    rnd = lambda *sh: torch.randn(*sh, generator=g, device=device, dtype=bf)  # noqa: E731
    pk, pv = rnd(1, P, H, 128), rnd(1, P, H, 128)
    qrot = (cos[:C], sin[:C])
    qm = m[:, :C]
    for c in range(5):
        total = P + (c + 1) * C
        cache.attend(rnd(1, C, H, 128), rnd(1, C, H, 128), rnd(1, C, H, 128), 0, c, prefix=(pk, pv),
                     q_rotary=qrot, k_rotary=(cos[:total], sin[:total]), q_matrix=qm,
                     kv_matrix=m[:, :total], out_matrix=qm, commit=True)
    q, k, v = rnd(1, C, H, 128), rnd(1, C, H, 128), rnd(1, C, H, 128)

    def evaluate():
        cache.attend(q, k, v, 0, 5, prefix=(pk, pv), q_rotary=qrot, k_rotary=(cos, sin),
                     q_matrix=qm, kv_matrix=m, out_matrix=qm)

    eval_ms = _back_to_back_ms(evaluate, 5)
    flops = 4.0 * C * rows * H * 128
    del cache
    torch.cuda.empty_cache()
    return {
        "rope_prope_us": round(ms * 1e3, 1),
        "rope_prope_gbps": round(nbytes / (ms / 1e3) / 1e9, 1),
        "rope_prope_hbm_frac": round(nbytes / (ms / 1e3) / 8e12, 4),
        "rope_prope_eager_torch_us": round(eager_ms * 1e3, 1),
        "rope_prope_speedup": round(eager_ms / ms, 2),
        "window_evaluation_ms": round(eval_ms, 3),
        "window_evaluation_tflops": round(flops / (eval_ms / 1e3) / 1e12, 1),
        "workload": (f"H{H} x 128, {T}-token frames, {cf}-frame chunk over a {P}-row prefix and "
                     f"5 history chunks ({rows} key rows); bf16"),
    }


def c5_quality(device, hs=slice(4, 6), rows=slice(1500, 1756)):
    """Config 5 cache memory and attention error on one steady-state layer pass, attributed:
    the fp8-cache output against the bf16-cache output splits into what the e4m3 cache itself
    costs (the bf16 kernel over the fp8 cache's frames decoded to bf16, against the bf16 cache)
    and what the fp8 kernel adds (the fp8 kernel against that decoded-cache bf16 run: Q rows and
    P in e4m3 inside the kernel).  4 streams, 1% x20 outlier channels, Lk 32760; errors over all
    rows and heads, normalised by each channel's V RMS where marked."""
    import torch

    from solarwm_amd import attend_cached, kernels

    cfg = dict(CONFIGS["c5"], layers=1)
    T, Lq = cfg["T"], cfg["chunk_f"] * cfg["T"]
    inputs = make_inputs(cfg, device, outliers=True)
    outs, mem, keep = {}, {}, {}
    start = 7 * Lq
    for cache in ("fp8", "bf16"):
        c = dict(cfg, cache=cache)
        caches = make_caches(c, device)
        run_ours(c, inputs, caches, range(7))
        q, k, v = inputs[0]
        x, _ = attend_cached(q, k, v, caches[0], start)
        outs[cache] = x.float()
        kp = caches[0].kpool
        live = cfg["cap_f"] * kp[0].numel() * kp.element_size() * 2  # K+V of the live window
        if caches[0].kscale is not None:
            live += 2 * cfg["cap_f"] * caches[0].kscale[0].numel() * 4
        mem[cache] = live
        keep[cache] = caches[0]
        del caches
    # the fp8 cache's window (plus the chunk in its staging slots) decoded to bf16 pools
    c8 = keep["fp8"]
    window = c8.plan(start, Lq)[3]
    kd = (c8.kpool.float() * c8.kscale[..., None, None]).to(torch.bfloat16)
    vd = (c8.vpool.float() * c8.vscale[..., None, None]).to(torch.bfloat16)
    q = inputs[0][0]
    outs["decoded"] = kernels.attention_frames(q, kd, vd, window, frame_tokens=T).float()
    torch.cuda.synchronize()
    v = inputs[0][2].float()
    rms_v = v.pow(2).mean(dim=1, keepdim=True).sqrt()

    def err(a, b):
        e = (outs[a] - outs[b]).abs()
        return {"max_abs": float(e.max()), "mean_abs": float(e.mean()),
                "normalised_max": float((e / rms_v).max()),
                "normalised_mean": float((e / rms_v).mean())}

    alone = err("decoded", "bf16")
    whole = err("fp8", "bf16")
    res = {
        "north_star_fp8_bar": {
            "max_abs": 3e-2,
            "met": whole["max_abs"] <= 3e-2,
            "fp8_cache_max_abs": whole["max_abs"],
            "e4m3_cache_alone_max_abs": alone["max_abs"],
            "note": "unmet by the quantisation recipe itself: one absmax/448 scale per (head, "
                    "frame) leaves the x20 outlier channels' e4m3 steps far above 3e-2, and the "
                    "bf16 kernel over the decoded fp8 cache (no fp8 arithmetic) already misses "
                    "the bar by the e4m3_cache_alone figure; the tests bound the kernel's own "
                    "error against the quantisation-aware oracle instead",
        },
        "cache_bytes_per_layer_bf16": mem["bf16"],
        "cache_bytes_per_layer_fp8": mem["fp8"],
        "memory_saved_pct": round(100 * (1 - mem["fp8"] / mem["bf16"]), 2),
        "fp8_vs_bf16_cache": whole,
        "e4m3_cache_alone": alone,
        "fp8_kernel_arithmetic": err("fp8", "decoded"),
        "note": "fp8_vs_bf16_cache = e4m3_cache_alone (bf16 kernel over decoded fp8 frames vs the "
                "bf16 cache) + fp8_kernel_arithmetic (fp8 kernel vs that decoded run); the "
                "largest absolute errors sit on the x20 outlier channels",
    }
    del keep, kd, vd, inputs
    torch.cuda.empty_cache()
    return res


def sharp_logits_leg(device, gains=(1.0, 2.0, 4.0), iters=10):
    """How the bf16 kernel's speculative row max (probabilities against a running max that is
    raised only when a tile's partial sum exceeds 2^8) behaves on sharper logits: one C2
    steady-state launch (Lq 4680 over 32760 keys, H12) with Q scaled by each gain (logit standard
    deviation = gain), and with the first frame's keys made 3x larger (a sink frame that
    dominates the softmax)."""
    import torch

    from solarwm_amd import kernels

    cfg = CONFIGS["c2"]
    T, Lq, H, n = cfg["T"], cfg["chunk_f"] * cfg["T"], cfg["heads"], cfg["cap_f"]
    g = torch.Generator(device=device).manual_seed(21)
    kp, vp, _, _ = kernels.new_pools(n, 1, H, T, torch.bfloat16, device)
    k = torch.randn(1, n * T, H, 128, generator=g, device=device, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    q0 = torch.randn(1, Lq, H, 128, generator=g, device=device, dtype=torch.bfloat16)
    for f in range(n):
        kernels.append_frames(k, v, kp, vp, [f], frame_tokens=T, src_frame0=f)
    slots = list(range(n))
    out = torch.empty_like(q0)

    def ms_for(q):
        for _ in range(2):
            kernels.attention_frames(q, kp, vp, slots, frame_tokens=T, out=out)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            kernels.attention_frames(q, kp, vp, slots, frame_tokens=T, out=out)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / iters

    res = {f"q_x{gn:g}_ms": round(ms_for((q0.float() * gn).to(torch.bfloat16)), 4) for gn in gains}
    kernels.append_frames((k.float() * 3).to(torch.bfloat16), v, kp, vp, [0], frame_tokens=T)
    res["sink_frame_keys_x3_ms"] = round(ms_for(q0), 4)
    del kp, vp, k, v
    torch.cuda.empty_cache()
    return res


def c4_memory_path(device, timed_chunks=3):
    """Config 4 at its real per-layer shape: 40 heads, 1560 tok/frame, a 256-slot memory bank
    per layer; each chunk attends 8 seeded bank frames ahead of the 21-frame live window
    (45240 keys) straight from the slot table.  One layer is timed and extrapolated to 48."""
    import torch

    from solarwm_amd import apply_cache_updates, attend_cached, kernels
    from solarwm_amd.cache import CacheGeometry, SlotKVCache

    c = C4
    geom = CacheGeometry(batch=1, heads=c["heads"], head_dim=128, frame_tokens=c["T"],
                         capacity_frames=c["cap_f"], sink_frames=c["sink_f"],
                         staging_frames=c["chunk_f"], bank_frames=c["bank"])
    cache = SlotKVCache(geom, dtype=torch.bfloat16, device=device)
    b0 = geom.bank_slot0
    cache.kpool[b0:].normal_()
    cache.vpool[b0:].normal_()
    q, k, v = make_inputs(dict(c, layers=1, batch=1), device)[0]
    Lq = c["chunk_f"] * c["T"]
    for ch in range(7):  # fill the live window
        _, upd = attend_cached(q, k, v, cache, ch * Lq)
        apply_cache_updates([cache], [(0, upd)])
    g = torch.Generator().manual_seed(11)
    out = torch.empty_like(q)
    with kernels.timed_launches() as tm:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for ch in range(7, 7 + timed_chunks):
            idx = torch.randperm(c["bank"], generator=g)[: c["mem_frames"]].tolist()
            for policy in PASSES:
                _, upd = attend_cached(q, k, v, cache, ch * Lq, memory_frames=idx, out=out)
                if policy != "none":
                    apply_cache_updates([cache], [(0, upd)])
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    n, ms, flops = tm.summary("attention")
    per_pass = wall / (timed_chunks * len(PASSES))
    del cache
    torch.cuda.empty_cache()
    return {
        "workload": "33B-class memory path: H40xD128, 1560 tok/frame, Lq 4680, 8 of 256 bank "
                    "frames + 21-frame window (45240 keys), one layer timed, x48 extrapolated",
        "frames_per_s_48_layers_extrapolated": round(c["chunk_f"] / (per_pass * c["layers"] * len(PASSES)), 4),
        "layer_pass_ms": round(per_pass * 1e3, 3),
        "attn_tflops": round(flops / (ms / 1e3) / 1e12, 1),
        "attn_avg_ms": round(ms / n, 3),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="chunks timed (default: all)")
    ap.add_argument("--warmup", type=int, default=2, help="untimed warmup chunks")
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--no-baselines", action="store_true", help="skip CPU / reference-GPU legs")
    ap.add_argument("--no-aux", action="store_true",
                    help="skip the steady-state legs of configs 3, 4 and 5")
    ap.add_argument("--probe", action="store_true",
                    help="run the fixed counter-collection sequence instead of the benchmark")
    args = ap.parse_args()
    if args.gpus != 1:
        print(
            f"bench.py: --gpus {args.gpus} is not supported; this build measures one GPU "
            "(the path shards by head across GPUs, see the design notes)", file=sys.stderr,
        )
        sys.exit(2)

    import torch

    from solarwm_amd import kernels

    cfg = CONFIGS[args.config]
    if args.probe:
        probe(cfg, torch.device("cuda:0"))
        return
    K = cfg["chunks"] if args.steps is None else args.steps
    W = args.warmup
    dev = torch.device("cuda:0")
    T, Lq = cfg["T"], cfg["chunk_f"] * cfg["T"]
    log(f"[bench] config {args.config}: {cfg}; timed chunks {K}, warmup {W}")
    inputs = make_inputs(cfg, dev, outliers=cfg["cache"] == "fp8")
    caches = make_caches(cfg, dev)

    # warmup on its own rollout, then reset every cache to the empty state
    run_ours(cfg, inputs, caches, range(W))
    torch.cuda.synchronize()
    for c in caches:
        c.reset()
    torch.cuda.synchronize()
    log("[bench] warmup done")

    # steady state: fill the window untimed (chunks 0..full_from-1, whose windows are still
    # growing), then time K chunks whose attention sees the whole cache window; the result no
    # longer depends on how many ramp-up chunks a short --steps run includes
    full_from = max(0, -(-cfg["cap_f"] // cfg["chunk_f"]) - 1)
    run_ours(cfg, inputs, caches, range(full_from))
    torch.cuda.synchronize()
    timed_ids = range(full_from, full_from + K)
    st = timed_rollout(cfg, inputs, caches, timed_ids)
    wall, fps = st["wall_s"], st["frames_per_s"]
    achieved = st["attn_tflops"]
    log(f"[bench] chunk ms: {[round(x, 2) for x in st['chunk_ms']]}")
    # the configured run beside it: chunks 0..chunks-1 from an empty cache, ramp-up included
    for c in caches:
        c.reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run_ours(cfg, inputs, caches, range(cfg["chunks"]))
    torch.cuda.synchronize()
    full_wall = time.perf_counter() - t0
    full_fps = cfg["chunk_f"] * cfg["batch"] * cfg["chunks"] / full_wall
    log(f"[bench] configured run: {cfg['chunks']} chunks from an empty cache in {full_wall:.3f} s "
        f"-> {full_fps:.3f} latent frames/s")
    log(f"[bench] ours: {wall:.3f} s for {K} steady chunks -> {fps:.3f} latent frames/s; attention "
        f"{st['attn_launches']} timed launches avg {st['attn_avg_ms']:.3f} ms, {achieved:.1f} TFLOP/s "
        f"(steady {st['attn_steady_ms']:.3f} ms, {st['attn_steady_tflops']:.1f} TFLOP/s); "
        f"append {st['append_gbps']:.0f} GB/s")

    peak = BF16_PEAK_TFLOPS if cfg["cache"] == "bf16" else FP8_PEAK_TFLOPS
    result = {
        "metric": "latent frames/s per 30-layer stack",
        "value": round(fps, 4),
        "unit": "latent frames/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(wall / K * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if cfg["cache"] == "bf16" else "fp8-e4m3 K/V, bf16 Q/O",
        "data": "synthetic: seeded N(0,1) bf16 Q/K/V per layer, resident in HBM before timing"
                + ("; 1% of K/V channels x20" if cfg["cache"] == "fp8" else ""),
        "config": {
            "workload": (
                f"{cfg['workload']} kv-cache rollout: {cfg['layers']} layers, H{cfg['heads']}xD128, "
                f"{T} tok/frame, chunk {cfg['chunk_f']} frames (Lq {Lq}), cache {cfg['cap_f']} "
                f"frames ({cfg['cap_f'] * T} tokens), sink {cfg['sink_f']} frame, steady state: "
                f"chunks {full_from}..{full_from + K - 1} (full window; chunks 0..{full_from - 1} "
                "fill it untimed) x (4 none + 1 commit) passes"
            ),
            "batch": cfg["batch"],
            "layers": cfg["layers"],
            "passes_per_chunk": len(PASSES),
        },
        "roofline": {
            "bound": "mfma",
            "kernel": ("skv::attn_kernel<8, bf16, bf16, 0, false, true> (8-wave groups, key tiles "
                       "packed across frames)") if cfg["cache"] == "bf16" else "skv::attn_fp8_kernel<8, bf16>",
            "achieved": round(achieved, 2),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4),
            "traffic": ATTN_TRAFFIC_BYTES.get(args.config),
            "traffic_per": ("steady-state launch (Lk = cache window), rocprofv3 FETCH_SIZE + WRITE_SIZE"
                            if cfg["cache"] == "bf16" else
                            "steady-state call (Lk = cache window): unsplit launch + tail-split "
                            "launch + merge, rocprofv3 FETCH_SIZE + WRITE_SIZE"),
            "traffic_source": (ATTN_TRAFFIC_SOURCE.format(cfg=args.config,
                                                          file=ATTN_TRAFFIC_FILES[args.config])
                               if args.config in ATTN_TRAFFIC_FILES else None),
            "launches_timed": st["attn_launches"],
            "timed_every": EVENT_EVERY,
            "avg_launch_ms": round(st["attn_avg_ms"], 4),
            "steady_state": {"Lk": cfg["cap_f"] * T, "avg_launch_ms": round(st["attn_steady_ms"], 4),
                             "achieved": round(st["attn_steady_tflops"], 2)},
        },
        "attn_mfma_util_pct": round(100 * achieved / peak, 2),
        "configured_run": {
            "frames_per_s": round(full_fps, 4),
            "chunks": cfg["chunks"],
            "wall_s": round(full_wall, 4),
            "note": f"BASELINE's run length: chunks 0..{cfg['chunks'] - 1} from an empty cache "
                    f"(the first {full_from} see growing windows), wall clock, no launch events",
        },
        "append_in_rollout": {
            "gbps": round(st["append_gbps"], 1),
            "avg_launch_us": round(st["append_avg_us"], 2),
            "note": f"HIP events around every {EVENT_EVERY}th append inside the rollout; they include the host enqueue gap",
        },
    }

    app_gbps, app_ms, n_src, src_bytes, copy_gbps = append_bandwidth(cfg, dev)
    result["append_gbps"] = round(app_gbps, 1)
    result["append_frac_hbm"] = round(app_gbps / HBM_PEAK_GBPS, 4)
    result["append_avg_launch_us"] = round(app_ms * 1e3, 2)
    result["append_sources"] = f"{n_src} rotating source chunks, {src_bytes / 1e6:.0f} MB (read cold)"
    result["append_copy_ceiling_gbps"] = round(copy_gbps, 1)
    result["append_copy_ceiling_note"] = ("torch copy_ of the same K+V bytes from the same cold "
                                          "sources: the rate a transfer of this size reaches")
    log(f"[bench] append ({cfg['chunk_f']} frames, back to back, {n_src} cold sources): "
        f"{app_gbps:.0f} GB/s, {app_ms * 1e3:.1f} us")

    gbps, g_ms, g_copy = gather_bandwidth(dev)
    result["gather_gbps"] = round(gbps, 1)
    result["gather_frac_hbm"] = round(gbps / HBM_PEAK_GBPS, 4)
    result["gather_avg_launch_us"] = round(g_ms * 1e3, 2)
    result["gather_copy_ceiling_gbps"] = round(g_copy, 1)
    result["gather_copy_ceiling_note"] = ("torch copy_ of the same 255.6 MB, three cold source / "
                                          "destination pairs in rotation")
    result["append_gather_target_note"] = (
        "north-star target 70% of HBM peak: a plain device copy of the append's bytes reaches "
        "append_copy_ceiling_gbps and of the gather's gather_copy_ceiling_gbps on this GPU")
    log(f"[bench] gather (C4 bank, 8 of 256 frames, fresh indices per launch): {gbps:.0f} GB/s, "
        f"{g_ms * 1e3:.1f} us; same-size copy {g_copy:.0f} GB/s")
    result["eviction"] = eviction_latency(cfg)
    log(f"[bench] eviction: {result['eviction']['host_us_per_layer_pass']} us host per layer pass, "
        f"{result['eviction']['reference_bytes_avoided_per_layer_pass'] / 1e6:.1f} MB of reference "
        "clone + memmove avoided")

    if not args.no_baselines:
        del caches
        torch.cuda.empty_cache()
        dense = [
            {"k": torch.zeros(cfg["batch"], cfg["cap_f"] * T, cfg["heads"], 128, dtype=torch.bfloat16, device=dev),
             "v": torch.zeros(cfg["batch"], cfg["cap_f"] * T, cfg["heads"], 128, dtype=torch.bfloat16, device=dev),
             "g": 0, "l": 0}
            for _ in range(cfg["layers"])
        ]
        reference_gpu_step(cfg, inputs, dense, range(1))
        for d in dense:
            d["k"].zero_()
            d["v"].zero_()
            d["g"] = d["l"] = 0
        torch.cuda.synchronize()
        reference_gpu_step(cfg, inputs, dense, range(full_from))  # fill, untimed
        torch.cuda.synchronize()
        log("[bench] reference GPU path: timing")
        t0 = time.perf_counter()
        reference_gpu_step(cfg, inputs, dense, timed_ids)
        torch.cuda.synchronize()
        rwall = time.perf_counter() - t0
        rfps = cfg["chunk_f"] * K / rwall
        result["reference_gpu"] = {
            "value": round(rfps, 4),
            "unit": "latent frames/s",
            "kind": "reference op sequence on PyTorch-ROCm (clone, memmove, cat, SDPA flash)",
            "chunks": f"{full_from}..{full_from + K - 1} (the same steady-state chunks)",
            "speedup": round(fps / rfps, 3),
        }
        log(f"[bench] reference GPU: {rwall:.3f} s -> {rfps:.3f} frames/s; speedup {fps / rfps:.2f}x")
        del dense
        log("[bench] CPU baseline: timing one layer pass")
        result["cpu_baseline"] = cpu_baseline(cfg)
        log(f"[bench] CPU baseline: {result['cpu_baseline']}")
        log("[bench] CPU baseline: config 1 end to end")
        result["cpu_baseline_c1"] = cpu_c1_end_to_end()
        log(f"[bench] CPU baseline c1: {result['cpu_baseline_c1']}")
    else:
        result["cpu_baseline"] = None
    del inputs
    caches = None
    torch.cuda.empty_cache()
    if not args.no_aux and args.config == "c2":
        aux = {}
        for name in ("c3", "c5"):
            log(f"[bench] aux {name}: steady state")
            r = steady_state(name, dev)
            aux[name] = {k2: (round(v2, 4) if isinstance(v2, float) else v2) for k2, v2 in r.items()}
            log(f"[bench] aux {name}: {aux[name]}")
        aux["c2_four_passes"] = four_pass_leg(dev)
        log(f"[bench] aux c2_four_passes: {aux['c2_four_passes']}")
        log("[bench] aux c2 with RoPE on load")
        aux["c2_rope"] = c2_rope(dev)
        log(f"[bench] aux c2_rope: {aux['c2_rope']}")
        aux["c2_prope"] = c2_rope(dev, prope=True)
        log(f"[bench] aux c2_prope: {aux['c2_prope']}")
        log("[bench] aux release: the reference's shipped inference geometry")
        aux["release"] = c2_rope(dev, fill=6, timed=2, prope=True, name="release")
        log(f"[bench] aux release: {aux['release']}")
        notes = {"c5_rope": "fp8 raw frames plus an fp8 RoPE copy of K; attn_fp8_kernel turns "
                            "the query's temporal pairs per key frame and multiplies e4m3 codes",
                 "c5_prope": "fp8 raw frames plus fp8 PRoPE copies; the attention decodes each "
                             "staged tile to bf16 and multiplies in bf16"}
        for name, kw in (("c5_rope", dict(rope=True)), ("c5_prope", dict(prope=True))):
            log(f"[bench] aux {name}: fp8 cache with RoPE on load")
            r = steady_state("c5", dev, timed=2, **kw)
            aux[name] = {"frames_per_s": round(r["frames_per_s"], 4),
                         "attn_tflops": round(r["attn_tflops"], 1),
                         "attn_avg_ms": round(r["attn_avg_ms"], 4),
                         # c5_rope multiplies e4m3 codes (fp8 peak); c5_prope bf16 (bf16 peak)
                         ("attn_frac_fp8_peak" if name == "c5_rope" else "attn_frac_bf16_peak"):
                             round(r["attn_tflops"] / (FP8_PEAK_TFLOPS if name == "c5_rope"
                                                      else BF16_PEAK_TFLOPS), 4),
                         "append_avg_us": round(r["append_avg_us"], 2),
                         "workload": r["workload"],
                         "note": notes[name]}
            log(f"[bench] aux {name}: {aux[name]}")
        aux["commit_path"] = commit_path(dev)
        log(f"[bench] aux commit_path: {aux['commit_path']}")
        aux["segments"] = segments_leg(dev)
        log(f"[bench] aux segments: {aux['segments']}")
        aux["h3"] = h3_leg(dev)
        log(f"[bench] aux h3: {aux['h3']}")
        aux["single_frame"] = single_frame_leg(dev)
        log(f"[bench] aux single_frame: {aux['single_frame']}")
        aux["sharp_logits"] = sharp_logits_leg(dev)
        log(f"[bench] aux sharp_logits: {aux['sharp_logits']}")
        log("[bench] aux c5: fp8 vs bf16 quality")
        aux["c5"]["quality"] = c5_quality(dev)
        log(f"[bench] aux c5 quality: {aux['c5']['quality']}")
        log("[bench] aux c4: memory path")
        aux["c4"] = c4_memory_path(dev)
        aux["c4"]["gather_gbps"] = result["gather_gbps"]
        log(f"[bench] aux c4: {aux['c4']}")
        result["aux"] = aux
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
