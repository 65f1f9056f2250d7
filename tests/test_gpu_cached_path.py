"""End-to-end parity of the cached path (SlotKVCache + attend_cached + apply_cache_updates)
against the oracle's restatement of the reference (clone, memmove, slice-assign, cat, SDPA).

Cache state must be bit-exact after every commit (the gathered logical cache equals the oracle's
dense cache, stale rows included) and every pass's attention output within the bf16 tolerance.
"""

import pytest
import torch

from oracle import wan_cache_ref as ref
from solarwm_amd import apply_cache_updates, attend_cached, make_kv_cache_allocator

from .helpers import assert_attn_close

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _inputs(seed, shape, dtype, scale):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(shape, generator=g) * scale).to(dtype) for _ in range(3)]


def _run(gpu, *, layers, H, T, chunk_f, cap_f, sink_f, n_chunks, passes, dtype, scale,
         head_subset=None, q_rows=None, check_every_pass=True):
    Lq = chunk_f * T
    alloc = make_kv_cache_allocator(
        num_layers=layers, num_heads=H, head_dim=128, frame_sequence_length=T,
        local_attn_size=cap_f, sink_size=sink_f, num_frame_per_block=chunk_f,
    )
    caches = alloc(1, dtype=dtype, device=gpu)
    oracle = ref.allocate_kv_cache(layers, 1, cap_f * T, H, 128, dtype)

    def sub_attn(q, k, v):
        hs = slice(None) if head_subset is None else head_subset
        rows = slice(None) if q_rows is None else q_rows
        return ref.attention(q[:, rows, hs], k[:, :, hs], v[:, :, hs], compute_dtype=torch.float32)

    for c in range(n_chunks):
        start = c * Lq
        for p, policy in enumerate(passes):
            _say(f"chunk {c} pass {p} ({policy})")
            infos, oinfos = [], []
            for layer in range(layers):
                seed = 1000 * c + 10 * p + layer
                q, k, v = _inputs(seed, (1, Lq, H, 128), dtype, scale)
                x, upd = attend_cached(q.to(gpu), k.to(gpu), v.to(gpu), caches[layer], start)
                infos.append((layer, upd))
                want, oupd = ref.cached_self_attention(
                    q, k, v, oracle[layer], current_start=start, frame_seqlen=T, sink_size=sink_f,
                    local_attn_size=cap_f, attn_fn=sub_attn if check_every_pass or policy != "none"
                    else (lambda q, k, v: torch.zeros(0)),
                )
                oinfos.append((layer, oupd))
                assert (upd[0], upd[1]) == (oupd[0], oupd[1])
                if want.numel():
                    hs = slice(None) if head_subset is None else head_subset
                    rows = slice(None) if q_rows is None else q_rows
                    torch.cuda.synchronize()
                    assert_attn_close(x[:, rows, hs], want)
            if policy != "none":
                apply_cache_updates(caches, infos)
                ref.apply_cache_updates(oracle, oinfos)
                for layer in range(layers):
                    gk, gv = caches[layer].logical_kv()
                    torch.cuda.synchronize()
                    assert torch.equal(gk.cpu(), oracle[layer]["k"]), f"K cache differs c={c}"
                    assert torch.equal(gv.cpu(), oracle[layer]["v"]), f"V cache differs c={c}"
                    assert int(caches[layer]["global_end_index"]) == int(oracle[layer]["global_end_index"])
                    assert int(caches[layer]["local_end_index"]) == int(oracle[layer]["local_end_index"])


def test_c1_full_run(gpu):
    """BASELINE config 1 at full size: fp32, H=12, 390 tokens/frame, chunk 3 frames, 21-frame
    cache with a 1-frame sink, 10 chunks x 2 passes (commit on the 2nd), Q/K/V ~ N(0,1)/sqrt(128)."""
    _run(gpu, layers=1, H=12, T=390, chunk_f=3, cap_f=21, sink_f=1, n_chunks=10,
         passes=["none", "commit"], dtype=torch.float32, scale=128 ** -0.5)


def test_small_multi_layer_nfe4(gpu):
    """Reference NFE4 pattern (4 x none + commit) over 3 layers, no sink, eviction from chunk 3."""
    _run(gpu, layers=3, H=2, T=64, chunk_f=2, cap_f=5, sink_f=0, n_chunks=6,
         passes=["none"] * 4 + ["commit"], dtype=torch.bfloat16, scale=1.0)


@pytest.mark.slow
def test_c2_shape_first_eight_chunks(gpu):
    """Wan2.1-1.3B shape (1560 tokens/frame, 12 heads, Lq 4680, 21-frame cache, 1 sink frame)
    for 8 chunks (eviction starts at chunk 7): cache bit-exact after every commit; attention
    checked on 2 heads x 256 query rows of the commit pass of every chunk."""
    _run(gpu, layers=1, H=12, T=1560, chunk_f=3, cap_f=21, sink_f=1, n_chunks=8,
         passes=["none", "commit"], dtype=torch.bfloat16, scale=1.0,
         head_subset=slice(5, 7), q_rows=slice(1000, 1256), check_every_pass=False)


def test_memory_bank_frames_fused(gpu):
    """Config-4 semantics at reduced size: 8 bank frames chosen by a seeded permutation are
    attended ahead of the live window without being copied; bank frames read back bit-exact."""
    T, H, bank_n = 130, 4, 24
    alloc = make_kv_cache_allocator(
        num_layers=1, num_heads=H, head_dim=128, frame_sequence_length=T, local_attn_size=7,
        sink_size=1, num_frame_per_block=3, bank_frames=bank_n,
    )
    cache = alloc(1, dtype=torch.bfloat16, device=gpu)[0]
    g = torch.Generator().manual_seed(5)
    bank_k = torch.randn(1, bank_n * T, H, 128, generator=g).bfloat16()
    bank_v = torch.randn(1, bank_n * T, H, 128, generator=g).bfloat16()
    cache.write_bank(list(range(bank_n)), bank_k.to(gpu), bank_v.to(gpu))
    oracle = ref.allocate_kv_cache(1, 1, 7 * T, H, 128, torch.bfloat16)
    from solarwm_amd import kernels

    for c in range(4):
        idx = torch.randperm(bank_n, generator=g)[:8].tolist()
        mk = ref.memory_gather(bank_k, idx, T)
        mv = ref.memory_gather(bank_v, idx, T)
        gk, gv = kernels.gather_frames(cache.kpool, cache.vpool, cache.bank_slots(idx),
                                       frame_tokens=T)
        torch.cuda.synchronize()
        assert torch.equal(gk.cpu(), mk) and torch.equal(gv.cpu(), mv)
        q, k, v = _inputs(77 + c, (1, 3 * T, H, 128), torch.bfloat16, 1.0)
        x, upd = attend_cached(q.to(gpu), k.to(gpu), v.to(gpu), cache, c * 3 * T,
                               memory_frames=idx)
        want, oupd = ref.cached_self_attention(
            q, k, v, oracle[0], current_start=c * 3 * T, frame_seqlen=T, sink_size=1,
            local_attn_size=7, memory_k=mk, memory_v=mv,
        )
        torch.cuda.synchronize()
        assert_attn_close(x, want)
        apply_cache_updates([cache], [(0, upd)])
        ref.apply_cache_updates(oracle, [(0, oupd)])


def test_fp8_cache_rollout_vs_bf16_oracle(gpu):
    """Config-5 semantics at reduced size: 4 independent streams, fp8-e4m3 cache with
    per-(frame, head) scales, K/V with 1% x20 outlier channels; the committed cache holds exactly
    the oracle's quantisation of its bf16 cache, and each pass's attention matches the
    quantisation-aware oracle (fp8 frames and query rows decoded) within the normalised fp8 bar."""
    from .helpers import FP8_NORM_MAX, FP8_NORM_MEAN

    T, H, chunk_f, cap_f, sink_f, B = 130, 3, 3, 7, 1, 4
    Lq = chunk_f * T
    alloc = make_kv_cache_allocator(
        num_layers=1, num_heads=H, head_dim=128, frame_sequence_length=T, local_attn_size=cap_f,
        sink_size=sink_f, num_frame_per_block=chunk_f, cache_dtype=torch.float8_e4m3fn,
    )
    cache = alloc(B, dtype=torch.bfloat16, device=gpu)[0]
    oracle = ref.allocate_kv_cache(1, B, cap_f * T, H, 128, torch.bfloat16)
    g = torch.Generator().manual_seed(9)
    ch = torch.randperm(128, generator=g)[:2]

    def qaware(q, k, v):
        return ref.attention(ref.fp8_fake_quant_rows(q), ref.fp8_fake_quant_frames(k.float(), T),
                             ref.fp8_fake_quant_frames(v.float(), T), round_inputs_to_bf16=False)

    for c in range(5):
        for policy in ("none", "commit"):
            q = torch.randn(B, Lq, H, 128, generator=g).bfloat16()
            k = torch.randn(B, Lq, H, 128, generator=g)
            v = torch.randn(B, Lq, H, 128, generator=g)
            k[..., ch] *= 20
            v[..., ch] *= 20
            k, v = k.bfloat16(), v.bfloat16()
            x, upd = attend_cached(q.to(gpu), k.to(gpu), v.to(gpu), cache, c * Lq)
            seen = {}

            def attn(qq, kk, vv):
                seen["v"] = vv
                return qaware(qq, kk, vv)

            want, oupd = ref.cached_self_attention(
                q, k, v, oracle[0], current_start=c * Lq, frame_seqlen=T, sink_size=sink_f,
                local_attn_size=cap_f, attn_fn=attn,
            )
            torch.cuda.synchronize()
            rms_v = seen["v"].double().pow(2).mean(dim=1, keepdim=True).sqrt().clamp_min(1e-6)
            e = (x.cpu().double() - want.double()).abs() / rms_v
            _say(f"fp8 rollout c={c} {policy}: normalised max {float(e.max()):.3e} "
                 f"mean {float(e.mean()):.3e}")
            assert float(e.max()) <= FP8_NORM_MAX and float(e.mean()) <= FP8_NORM_MEAN, (
                c, policy, float(e.max()), float(e.mean()))
            if policy == "commit":
                apply_cache_updates([cache], [(0, upd)])
                ref.apply_cache_updates(oracle, [(0, oupd)])
        # committed cache: codes and scales equal the oracle quantisation of its bf16 cache
        live = cache.local_end // T
        for p in range(live):
            slot = cache.table[p]
            frame = oracle[0]["k"][:, p * T : (p + 1) * T].permute(0, 2, 1, 3)  # [B, H, T, D]
            codes, scale = ref.fp8_quantize(frame)
            got = cache.kpool[slot, :, :, :T].cpu().view(torch.uint8)
            assert torch.equal(got, codes.view(torch.uint8)), (c, p)
            assert torch.equal(cache.kscale[slot].cpu(), scale), (c, p)
