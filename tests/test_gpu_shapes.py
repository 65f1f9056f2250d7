"""The kernel instances the benchmark runs, at the benchmark's shapes, against the oracle.

* C3 (Wan2.2-5B shape: H24, 880-token frames, Lq 2640 over the full 21-frame window): the
  launcher takes the balanced key split on 8-wave workgroups (asserted through
  ``skv_attention_plan``); checked on a head/row subset against the float64 oracle.
* C4 (33B memory path: H40, 1560-token frames, 8 frames of a 256-slot memory bank ahead of the
  21 live frames after eviction): the plain 8-wave kernel over 29 frames on 4.6 GB pools
  (frame-aligned tiles), through ``attend_cached`` with ``memory_frames``, against
  ``cached_self_attention(memory_k=...)`` (memory_kv_attention.py:97-137 places the bank ahead of
  the window); the bank gather bit-exact at H40 (memory_retrieval.py:79-86).
* C5 (fp8-e4m3 cache, 4 streams, H12, 1560-token frames, 1% x20 outlier channels, eviction
  done): ``attn_fp8_kernel`` on its 912-workgroup grid through ``attend_cached``, against the
  quantisation-aware oracle (the cache's fp8 K/V frames and the per-row fp8 query decoded,
  float64 softmax) with the normalised bars of tests/helpers.py; the committed codes and scales
  equal the oracle quantisation of its bf16 cache.

Reference ops: causal_model.py:1135-1226 (window), attention.py:141-188 (attention).
"""

import pytest
import torch

from oracle import wan_cache_ref as ref
from solarwm_amd import apply_cache_updates, attend_cached, kernels, make_kv_cache_allocator

from .helpers import FP8_NORM_MAX, FP8_NORM_MEAN, assert_attn_close

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _say(*a):
    print(*a, flush=True)


def _qkv(seed, shape, outliers=None):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(shape, generator=g) for _ in range(3))
    if outliers is not None:
        k[..., outliers] *= 20.0
        v[..., outliers] *= 20.0
    return q.to(BF), k.to(BF), v.to(BF)


def test_c3_full_window_takes_the_split(gpu):
    T, nf, H, Lq = 880, 21, 24, 2640
    _say("C3 full window", H, Lq, nf, T)
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, Lq, H, 128, generator=g).to(BF)
    k = torch.randn(1, nf * T, H, 128, generator=g).to(BF)
    v = torch.randn(1, nf * T, H, 128, generator=g).to(BF)
    kp, vp, _, _ = kernels.new_pools(nf + 3, 1, H, T, BF, gpu)
    slots = list(range(3, nf + 3))[::-1]  # frames in non-contiguous slot order
    kd, vd = k.to(gpu), v.to(gpu)
    for f in range(nf):
        kernels.append_frames(kd, vd, kp, vp, [slots[f]], frame_tokens=T, src_frame0=f)
    qd = q.to(gpu)
    plan = kernels.attention_plan(qd, kp, vp, slots, frame_tokens=T)
    assert (plan["split"], plan["waves_per_group"], plan["n_workgroups"]) == (1, 8, 256), plan
    out = kernels.attention_frames(qd, kp, vp, slots, frame_tokens=T)
    unsplit = kernels.attention_frames(qd, kp, vp, slots, frame_tokens=T, use_workspace=False)
    torch.cuda.synchronize()
    for hs, rows in ((slice(0, 2), slice(0, 256)), (slice(22, 24), slice(2384, 2640)),
                     (slice(11, 12), slice(1200, 1500))):
        want = ref.attention(q[:, rows, hs], k[:, :, hs], v[:, :, hs], compute_dtype=torch.float32)
        assert_attn_close(out[:, rows, hs], want)
        assert_attn_close(unsplit[:, rows, hs], want)


def test_c4_full_bank_and_live_window(gpu):
    """The benchmark's C4 layer: a 256-slot memory bank beside the 21 live frames (pools of
    280 slots x H40 x 1600 rows: 4.6 GB each, past the packed walk's 4 GB bound, so the plan
    keeps frame-aligned tiles and 64-bit slot bases).  The bank is generated on the GPU and
    copied whole to the host; 8 seeded bank frames are gathered bit-exactly (skv_gather against
    the oracle's gather over the host copy) and attended ahead of the window after eviction."""
    T, H, cap, sink, chunk_f, bank_n = 1560, 40, 21, 1, 3, 256
    Lq = chunk_f * T
    _say("C4 window: 8 of a 256-slot bank + 21 live frames", H, T)
    alloc = make_kv_cache_allocator(num_layers=1, num_heads=H, head_dim=128,
                                    frame_sequence_length=T, local_attn_size=cap, sink_size=sink,
                                    num_frame_per_block=chunk_f, bank_frames=bank_n)
    cache = alloc(1, dtype=BF, device=gpu)[0]
    assert cache.kpool.numel() * 2 > 1 << 32, cache.kpool.shape
    oracle = ref.allocate_kv_cache(1, 1, cap * T, H, 128, BF)
    gd = torch.Generator(device=gpu).manual_seed(44)
    bank_k = torch.randn(1, bank_n * T, H, 128, generator=gd, device=gpu, dtype=BF)
    bank_v = torch.randn(1, bank_n * T, H, 128, generator=gd, device=gpu, dtype=BF)
    for f0 in range(0, bank_n, 64):  # at most 64 frames per append
        cache.write_bank(list(range(f0, f0 + 64)), bank_k[:, f0 * T : (f0 + 64) * T],
                         bank_v[:, f0 * T : (f0 + 64) * T])
    torch.cuda.synchronize()
    bank_k_host, bank_v_host = bank_k.cpu(), bank_v.cpu()
    del bank_k, bank_v
    g = torch.Generator().manual_seed(45)
    # 7 seeded indices drawn without replacement, plus the last entry, whose slot starts past
    # the pool's first 4 GB (bank slots follow the 24 live and staging slots, 16.4 MB apart)
    idx = torch.randperm(bank_n - 1, generator=g)[:7].tolist() + [bank_n - 1]
    assert cache.bank_slots([bank_n - 1])[0] * cache.kpool[0].numel() * 2 > 1 << 32
    mem_k, mem_v = ref.memory_gather(bank_k_host, idx, T), ref.memory_gather(bank_v_host, idx, T)
    del bank_k_host, bank_v_host
    gk, gv = kernels.gather_frames(cache.kpool, cache.vpool, cache.bank_slots(idx), frame_tokens=T)
    torch.cuda.synchronize()
    assert torch.equal(gk.cpu(), mem_k) and torch.equal(gv.cpu(), mem_v)
    del gk, gv
    checks = ((slice(17, 19), slice(3000, 3256)), (slice(38, 40), slice(4608, 4680)),
              (slice(0, 1), slice(0, 256)))

    for c in range(8):  # chunk 7 evicts frames 1..3
        q, k, v = _qkv(400 + c, (1, Lq, H, 128))
        mem = idx if c == 7 else None
        x, upd = attend_cached(q.to(gpu), k.to(gpu), v.to(gpu), cache, c * Lq, memory_frames=mem)
        if c == 7:
            frames = cache.bank_slots(idx) + cache.plan(c * Lq, Lq)[3]
            plan = kernels.attention_plan(q.to(gpu), cache.kpool, cache.vpool, frames,
                                          frame_tokens=T)
            assert len(frames) == 29 and (plan["split"], plan["n_workgroups"]) == (0, 760), plan
            assert plan["key_tiles"] == 29 * 25, plan  # frame-aligned: pools past 4 GB
            seen = {}

            def keep(qq, kk, vv):
                seen["k"], seen["v"] = kk, vv
                return torch.zeros(0)

            _, oupd = ref.cached_self_attention(
                q, k, v, oracle[0], current_start=c * Lq, frame_seqlen=T, sink_size=sink,
                local_attn_size=cap, memory_k=mem_k, memory_v=mem_v, attn_fn=keep)
            assert seen["k"].shape[1] == 29 * T
            torch.cuda.synchronize()
            for hs, rows in checks:
                want = ref.attention(q[:, rows, hs], seen["k"][:, :, hs], seen["v"][:, :, hs],
                                     compute_dtype=torch.float32)
                assert_attn_close(x[:, rows, hs], want)
        else:
            _, oupd = ref.cached_self_attention(
                q, k, v, oracle[0], current_start=c * Lq, frame_seqlen=T, sink_size=sink,
                local_attn_size=cap, attn_fn=lambda q, k, v: torch.zeros(0))
        apply_cache_updates([cache], [(0, upd)])
        ref.apply_cache_updates(oracle, [(0, oupd)])
    assert cache.local_end == cap * T
    lk, lv = cache.logical_kv()
    torch.cuda.synchronize()
    assert torch.equal(lk.cpu(), oracle[0]["k"]) and torch.equal(lv.cpu(), oracle[0]["v"])


def fp8_normalised_errors(got, q, k, v, T):
    """(max, mean) of |got - quantisation-aware oracle| / (each channel's V RMS over the window)
    for q [B, Lq, H, D] against the window k, v [B, Lk, H, D]."""
    want = ref.attention(ref.fp8_fake_quant_rows(q), ref.fp8_fake_quant_frames(k.float(), T),
                         ref.fp8_fake_quant_frames(v.float(), T), round_inputs_to_bf16=False)
    rms_v = v.double().pow(2).mean(dim=1, keepdim=True).sqrt().clamp_min(1e-6)
    e = (got.detach().cpu().double() - want.double()).abs() / rms_v
    return float(e.max()), float(e.mean())


def test_c5_fp8_full_shape_after_eviction(gpu):
    B, H, T, cap, sink, chunk_f = 4, 12, 1560, 21, 1, 3
    Lq = chunk_f * T
    _say("C5 fp8 full shape", B, H, T)
    alloc = make_kv_cache_allocator(num_layers=1, num_heads=H, head_dim=128,
                                    frame_sequence_length=T, local_attn_size=cap, sink_size=sink,
                                    num_frame_per_block=chunk_f, cache_dtype=torch.float8_e4m3fn)
    cache = alloc(B, dtype=BF, device=gpu)[0]
    oracle = ref.allocate_kv_cache(1, B, cap * T, H, 128, BF)
    ch = torch.randperm(128, generator=torch.Generator().manual_seed(5))[:2]  # 1% of channels
    # row blocks: a middle q-tile on two heads, the last (ragged, 72-row) q-tile on every head
    # and the first on two more; the launch runs 3 full rounds unsplit and splits the last
    # round's 144 q-tiles (the tail) over every CU, so both kinds are checked
    checks = ((slice(4, 6), slice(1500, 1756)), (slice(0, 12), slice(4608, 4680)),
              (slice(10, 12), slice(0, 256)))
    errs = []
    for c in range(8):  # chunks 0..6 fill the 21 frames, chunk 7 evicts frames 1..3
        policies = ("none", "commit") if c == 7 else ("commit",)
        for policy in policies:
            q, k, v = _qkv(500 + 10 * c + len(errs), (B, Lq, H, 128), outliers=ch)
            x, upd = attend_cached(q.to(gpu), k.to(gpu), v.to(gpu), cache, c * Lq)
            seen = {}

            def sub(qq, kk, vv):
                seen["k"], seen["v"] = kk, vv
                return torch.zeros(0)

            _, oupd = ref.cached_self_attention(
                q, k, v, oracle[0], current_start=c * Lq, frame_seqlen=T, sink_size=sink,
                local_attn_size=cap, attn_fn=sub if c == 7 else (lambda *a: torch.zeros(0)))
            if c == 7:
                assert seen["k"].shape[1] == cap * T
                torch.cuda.synchronize()
                for hs, rows in checks:
                    e = fp8_normalised_errors(x[:, rows, hs], q[:, rows, hs], seen["k"][:, :, hs],
                                              seen["v"][:, :, hs], T)
                    _say(f"C5 fp8 {policy} heads {hs.start}..{hs.stop - 1} rows {rows.start}.."
                         f"{rows.stop - 1}: normalised max {e[0]:.3e} mean {e[1]:.3e}")
                    errs.append(e)
            if policy == "commit":
                apply_cache_updates([cache], [(0, upd)])
                ref.apply_cache_updates(oracle, [(0, oupd)])
    for mx, mean in errs:
        assert mx <= FP8_NORM_MAX and mean <= FP8_NORM_MEAN, errs
    # committed codes and scales: the oracle quantisation of its bf16 cache, after eviction
    for p in (0, 1, 10, 20):
        slot = cache.table[p]
        frame = oracle[0]["k"][:, p * T : (p + 1) * T].permute(0, 2, 1, 3)  # [B, H, T, D]
        codes, scale = ref.fp8_quantize(frame)
        assert torch.equal(cache.kpool[slot, :, :, :T].cpu().view(torch.uint8),
                           codes.view(torch.uint8)), p
        assert torch.equal(cache.kscale[slot].cpu(), scale), p
