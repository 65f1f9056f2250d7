#!/usr/bin/env python3
"""Benchmark of the block-causal KV-cache inference path on one MI355X.

Workload (Wan2.1-1.3B shape): 30 layers, 12 heads x 128, 1560 tokens per
latent frame, chunks of 3 frames (4680 queries), a 21-frame (32760-token) cache per layer with a
1-frame sink and rolling eviction, 27 chunks.  One step = one chunk of the reference sampler
(solar/backends/wan22/runtime/stage2.py:674-760): 4 denoising passes with
cache_update_policy "none" and 1 commit pass, each pass running the cached self-attention of all
30 layers (append of the chunk into staging slots + attention over sink | window | chunk) and
the commit pass advancing every layer's slot table.  Projections/FFN are outside the path.

Printed JSON (one line): value = latent frames/s of the timed chunks (3 frames per chunk);
roofline = the attention kernel's algorithmic TFLOP/s (4*Lq*Lk*H*D per launch, from HIP events
around every launch in the timed region) against dense bf16 MFMA peak; cpu_baseline = the
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
               sink_f=1, chunks=27, batch=1),
    "c3": dict(workload="wan2.2-5b", layers=30, heads=24, T=880, chunk_f=3, cap_f=21,
               sink_f=1, chunks=40, batch=1),
}
PASSES = ["none"] * 4 + ["commit"]  # stage2.py:683-760: NFE4 then a t=0 commit forward
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
HBM_PEAK_GBPS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_inputs(cfg, device, seed=1234):
    import torch

    g = torch.Generator(device=device).manual_seed(seed)
    Lq = cfg["chunk_f"] * cfg["T"]
    shape = (cfg["batch"], Lq, cfg["heads"], 128)
    return [
        tuple(torch.randn(shape, generator=g, device=device, dtype=torch.bfloat16) for _ in range(3))
        for _ in range(cfg["layers"])
    ]


def run_ours(cfg, inputs, caches, chunk_ids):
    from solarwm_amd import apply_cache_updates, attend_cached

    Lq = cfg["chunk_f"] * cfg["T"]
    outs = [None] * cfg["layers"]
    for c in chunk_ids:
        for policy in PASSES:
            infos = []
            for layer, (q, k, v) in enumerate(inputs):
                x, upd = attend_cached(q, k, v, caches[layer], c * Lq, out=outs[layer])
                outs[layer] = x
                infos.append((layer, upd))
            if policy != "none":
                apply_cache_updates(caches, infos)


def reference_gpu_step(cfg, inputs, dense, chunk_ids):
    """The reference's per-layer op sequence on the GPU with PyTorch-ROCm: clone the cache,
    memmove the non-sink window, slice-assign the chunk, cat sink|local, SDPA; deferred commit
    repeats memmove + assign (causal_model.py:1028-1226, :2856-2921)."""
    import torch
    from torch.nn.attention import SDPBackend, sdpa_kernel

    T, Lq = cfg["T"], cfg["chunk_f"] * cfg["T"]
    sink = cfg["sink_f"] * T
    cap = cfg["cap_f"] * T
    for c in chunk_ids:
        cs = c * Lq
        for policy in PASSES:
            ups = []
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
                kc = torch.cat([tk[:, :a_s], tk[:, lsw:nle]], dim=1)
                vc = torch.cat([tv[:, :a_s], tv[:, lsw:nle]], dim=1)
                with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                    x = torch.nn.functional.scaled_dot_product_attention(
                        q.transpose(1, 2).contiguous(), kc.transpose(1, 2).contiguous(),
                        vc.transpose(1, 2).contiguous(),
                    ).transpose(1, 2).contiguous()
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


def cpu_baseline(cfg):
    """Reference op sequence on the host CPU (oracle restatement, bf16 SDPA as the reference's
    fallback): one steady-state layer pass (rolling eviction over a full cache), extrapolated to
    frames/s of the 30-layer, 5-pass chunk."""
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
    t0 = time.perf_counter()
    ref.cached_self_attention(
        q, k, v, cache[0], current_start=cap, frame_seqlen=T, sink_size=cfg["sink_f"],
        local_attn_size=cfg["cap_f"], attn_fn=ref.sdpa_fallback_attention,
    )
    dt = time.perf_counter() - t0
    per_chunk = dt * cfg["layers"] * len(PASSES)
    return {
        "value": round(cfg["chunk_f"] / per_chunk, 6),
        "unit": "latent frames/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (
            f"1 steady-state layer pass (Lq={Lq}, Lk={cap}, H={H}, rolling eviction) of the "
            f"reference op sequence in {dt:.2f} s, x{cfg['layers']} layers x{len(PASSES)} passes"
        ),
    }


def gather_bandwidth(device, iters=10):
    """Config-4 memory-bank gather: 8 seeded frames of a 256-slot bank (H=40, 1560 tokens per
    frame) materialised token-major; algorithmic bytes = K+V read + write."""
    import torch

    from solarwm_amd import kernels

    T, H, n_bank = 1560, 40, 256
    kpool, vpool, _, _ = kernels.new_pools(n_bank, 1, H, T, torch.bfloat16, device)
    kpool.normal_()
    vpool.normal_()
    g = torch.Generator().manual_seed(4)
    idx = torch.randperm(n_bank, generator=g)[:8].tolist()
    ko = torch.empty(1, 8 * T, H, 128, dtype=torch.bfloat16, device=device)
    vo = torch.empty_like(ko)
    kernels.gather_frames(kpool, vpool, idx, frame_tokens=T, k_out=ko, v_out=vo)
    with kernels.timed_launches() as tm:
        for _ in range(iters):
            kernels.gather_frames(kpool, vpool, idx, frame_tokens=T, k_out=ko, v_out=vo)
    n, ms, moved = tm.summary("gather")
    del kpool, vpool
    return moved / (ms / 1e3) / 1e9, ms / n


def probe(cfg, device, iters=20):
    """Short fixed sequence for hardware-counter runs (rocprofv3 --pmc): a plain device copy of
    exactly 1 GiB (the FETCH_SIZE / WRITE_SIZE calibration), then steady-state launches of the
    append kernel (one chunk, Lq tokens) and the attention kernel (Lq x full window)."""
    import torch

    from solarwm_amd import kernels

    src = torch.empty(1 << 29, dtype=torch.int16, device=device).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)  # 1 GiB read + 1 GiB written per launch
    torch.cuda.synchronize()
    del src, dst
    T, Lq, H = cfg["T"], cfg["chunk_f"] * cfg["T"], cfg["heads"]
    n = cfg["cap_f"]
    kpool, vpool, _, _ = kernels.new_pools(n + cfg["chunk_f"], cfg["batch"], H, T, torch.bfloat16, device)
    q, k, v = make_inputs(dict(cfg, layers=1), device)[0]
    for f in range(n):
        kernels.append_frames(k, v, kpool, vpool, [f], frame_tokens=T, src_frame0=f % cfg["chunk_f"])
    slots = list(range(n))
    for _ in range(iters):
        kernels.append_frames(k, v, kpool, vpool, [n, n + 1, n + 2], frame_tokens=T)
    for _ in range(iters):
        kernels.attention_frames(q, kpool, vpool, slots, frame_tokens=T)
    torch.cuda.synchronize()
    log(f"[probe] copy 1 GiB x3, append x{iters} ({Lq} tokens), attention x{iters} (Lq {Lq}, Lk {n * T})")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="chunks timed (default: all)")
    ap.add_argument("--warmup", type=int, default=2, help="untimed warmup chunks")
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--no-baselines", action="store_true", help="skip CPU / reference-GPU legs")
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

    from solarwm_amd import kernels, make_kv_cache_allocator

    cfg = CONFIGS[args.config]
    if args.probe:
        probe(cfg, torch.device("cuda:0"))
        return
    K = cfg["chunks"] if args.steps is None else args.steps
    W = args.warmup
    dev = torch.device("cuda:0")
    T, Lq = cfg["T"], cfg["chunk_f"] * cfg["T"]
    log(f"[bench] config {args.config}: {cfg}; timed chunks {K}, warmup {W}")
    inputs = make_inputs(cfg, dev)
    alloc = make_kv_cache_allocator(
        num_layers=cfg["layers"], num_heads=cfg["heads"], head_dim=128, frame_sequence_length=T,
        local_attn_size=cfg["cap_f"], sink_size=cfg["sink_f"], num_frame_per_block=cfg["chunk_f"],
    )
    caches = alloc(cfg["batch"], dtype=torch.bfloat16, device=dev)

    # warmup on its own rollout, then reset every cache to the empty state
    run_ours(cfg, inputs, caches, range(W))
    torch.cuda.synchronize()
    for c in caches:
        c.reset()
    torch.cuda.synchronize()
    log("[bench] warmup done")

    with kernels.timed_launches() as tm:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        run_ours(cfg, inputs, caches, range(K))
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    wall = t1 - t0
    fps = cfg["chunk_f"] * K / wall
    n_attn, attn_ms, attn_flops = tm.summary("attention")
    n_app, app_ms, app_bytes = tm.summary("append")
    steady = [r for r in tm.records["attention"] if r[2] == max(w for _, _, w in tm.records["attention"])]
    st_ms = sum(a.elapsed_time(b) for a, b, _ in steady) / len(steady)
    st_tflops = steady[0][2] / (st_ms / 1e3) / 1e12
    achieved = attn_flops / (attn_ms / 1e3) / 1e12
    log(f"[bench] ours: {wall:.3f} s for {K} chunks -> {fps:.3f} latent frames/s; attention "
        f"{n_attn} launches avg {attn_ms / n_attn:.3f} ms, {achieved:.1f} TFLOP/s "
        f"(steady {st_ms:.3f} ms, {st_tflops:.1f} TFLOP/s); append {app_bytes / (app_ms / 1e3) / 1e9:.0f} GB/s")

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
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) bf16 Q/K/V per layer, resident in HBM before timing",
        "config": {
            "workload": (
                f"{cfg['workload']} kv-cache rollout: {cfg['layers']} layers, H{cfg['heads']}xD128, "
                f"{T} tok/frame, chunk {cfg['chunk_f']} frames (Lq {Lq}), cache {cfg['cap_f']} "
                f"frames ({cfg['cap_f'] * T} tokens), sink {cfg['sink_f']} frame, chunks 0..{K - 1} "
                "x (4 none + 1 commit) passes"
            ),
            "batch": cfg["batch"],
            "layers": cfg["layers"],
            "passes_per_chunk": len(PASSES),
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "attn_kernel<bf16,bf16>",
            "achieved": round(achieved, 2),
            "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
            "traffic": None,
            "launches": n_attn,
            "avg_launch_ms": round(attn_ms / n_attn, 4),
            "steady_state": {"Lk": cfg["cap_f"] * T, "avg_launch_ms": round(st_ms, 4),
                             "achieved": round(st_tflops, 2)},
        },
        "attn_mfma_util_pct": round(100 * achieved / BF16_PEAK_TFLOPS, 2),
        "append_gbps": round(app_bytes / (app_ms / 1e3) / 1e9, 1),
        "append_frac_hbm": round(app_bytes / (app_ms / 1e3) / 1e9 / HBM_PEAK_GBPS, 4),
        "append_avg_launch_us": round(app_ms / n_app * 1e3, 2),
    }
    del tm

    gbps, g_ms = gather_bandwidth(dev)
    result["gather_gbps"] = round(gbps, 1)
    result["gather_frac_hbm"] = round(gbps / HBM_PEAK_GBPS, 4)
    log(f"[bench] gather (C4 bank, 8 of 256 frames): {gbps:.0f} GB/s, {g_ms * 1e3:.1f} us")

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
        for st in dense:
            st["k"].zero_(); st["v"].zero_(); st["g"] = st["l"] = 0
        torch.cuda.synchronize()
        log("[bench] reference GPU path: timing")
        t0 = time.perf_counter()
        reference_gpu_step(cfg, inputs, dense, range(K))
        torch.cuda.synchronize()
        rwall = time.perf_counter() - t0
        rfps = cfg["chunk_f"] * K / rwall
        result["reference_gpu"] = {
            "value": round(rfps, 4),
            "unit": "latent frames/s",
            "kind": "reference op sequence on PyTorch-ROCm (clone, memmove, cat, SDPA flash)",
            "speedup": round(fps / rfps, 3),
        }
        log(f"[bench] reference GPU: {rwall:.3f} s -> {rfps:.3f} frames/s; speedup {fps / rfps:.2f}x")
        del dense
        log("[bench] CPU baseline: timing one layer pass")
        result["cpu_baseline"] = cpu_baseline(cfg)
        log(f"[bench] CPU baseline: {result['cpu_baseline']}")
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
