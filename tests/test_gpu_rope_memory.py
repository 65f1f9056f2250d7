"""GPU parity of memory-bank frames on pre-RoPE caches (bf16 and fp8) against the oracle.

Bank frames are written with their height/width-roped K copy (``write_bank``) and attended ahead
of the window at caller-given temporal positions (``attend_cached(memory_frames=...,
memory_positions=...)``), as the H3 memory path places bank rows ahead of the history at their
own positions (memory_kv_attention.py:97-137).  Oracle: ``cached_self_attention(rope=...,
memory_k=..., memory_positions=...)`` (pinned in tests/test_oracle.py).  bf16 caches: the bf16
bars of tests/helpers.py; fp8 caches (64-token frames: the fp8-MFMA kernel): the oracle attends
with that kernel's per-key-frame e4m3 query (``fp8_rope_attention`` at the positions the window
RoPE would use) over the decoded copies, and the error divided by each channel's V RMS stays
within the normalised fp8 bars of tests/helpers.py.
"""

import pytest
import torch

from oracle import wan_cache_ref as ref
from solarwm_amd import RopeConfig, apply_cache_updates, attend_cached, make_kv_cache_allocator

from .helpers import FP8_NORM_MAX, FP8_NORM_MEAN, assert_attn_close

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


@pytest.mark.parametrize("dtype,sink,echo,B", [(BF, 1, True, 1), (BF, 0, False, 2),
                                               (torch.float8_e4m3fn, 1, True, 2)])
def test_rope_cache_memory_frames_vs_oracle(gpu, dtype, sink, echo, B):
    gh, gw, H, nb, cap, n_bank = 8, 8, 2, 2, 5, 6
    T = gh * gw
    fp8 = dtype == torch.float8_e4m3fn
    print("rope memory", dtype, sink, echo, B, flush=True)
    cfg = RopeConfig(grid_hw=(gh, gw), use_echorope=echo)
    cache = make_kv_cache_allocator(
        num_layers=1, num_heads=H, head_dim=128, frame_sequence_length=T, local_attn_size=cap,
        sink_size=sink, num_frame_per_block=nb, bank_frames=n_bank, rope=cfg,
        cache_dtype=dtype if fp8 else None)(B, dtype=BF, device=gpu)[0]
    oc = ref.allocate_kv_cache(1, B, cap * T, H, 128, torch.float64 if fp8 else BF)[0]
    f = ref.wan_rope_freqs()
    orope = {"freqs": f, "grid_hw": (gh, gw), "use_echorope": echo, "rope_train_frames": None}
    g = torch.Generator().manual_seed(91)
    bank_k = torch.randn(B, n_bank * T, H, 128, generator=g).to(BF)
    bank_v = torch.randn(B, n_bank * T, H, 128, generator=g).to(BF)
    cache.write_bank(list(range(n_bank)), bank_k.to(gpu), bank_v.to(gpu))
    if fp8:
        bank_k_o = ref.fp8_rope_copy_effective(bank_k, (gh, gw), f, T)
        bank_v_o = ref.fp8_fake_quant_frames(bank_v.float(), T).double()
    else:
        bank_k_o, bank_v_o = bank_k, bank_v
    for c in range(4):  # the window fills at chunk 2; chunk 3 evicts
        for commit in (False, True):
            q, k, v = (torch.randn(B, nb * T, H, 128, generator=g).to(BF) for _ in range(3))
            idx, mpos = ([4, 1, 5], [9, 2, 6]) if c >= 2 else (None, None)
            x, info = attend_cached(q.to(gpu), k.to(gpu), v.to(gpu), cache, c * nb * T,
                                    memory_frames=idx, memory_positions=mpos)
            ko, vo = k, v
            if fp8:
                ko = ref.fp8_rope_copy_effective(k, (gh, gw), f, T)
                vo = ref.fp8_fake_quant_frames(v.float(), T).double()
            mem = {}
            if idx is not None:
                mem = dict(memory_k=ref.memory_gather(bank_k_o, idx, T),
                           memory_v=ref.memory_gather(bank_v_o, idx, T), memory_positions=mpos)
            rp = orope
            if fp8:
                def attend(qq, kk, vv, qp, kp):  # the copies: spatial pairs turned, temporal raw
                    kc = ref.rope_frames(kk, (gh, gw), [0] * (kk.shape[1] // T), f)
                    return ref.fp8_rope_attention(qq, kc, vv, (gh, gw), qp, kp, T)
                rp = dict(orope, attend=attend)
            want, oinfo = ref.cached_self_attention(
                q, ko, vo, oc, current_start=c * nb * T, frame_seqlen=T, sink_size=sink,
                local_attn_size=cap, rope=rp, **mem)
            torch.cuda.synchronize()
            if fp8:
                vw = torch.cat([mem["memory_v"], vo], 1) if idx is not None else vo
                rms_v = vw.double().pow(2).mean(dim=1, keepdim=True).sqrt()
                e = (x.cpu().double() - want.double()).abs() / rms_v
                assert float(e.max()) <= FP8_NORM_MAX and float(e.mean()) <= FP8_NORM_MEAN, (
                    c, commit, float(e.max()), float(e.mean()))
            else:
                assert_attn_close(x, want)
            if commit:
                apply_cache_updates([cache], [(0, info)])
                ref.apply_cache_updates([oc], [(0, oinfo)])
    with pytest.raises(ValueError, match="memory_positions"):
        attend_cached(q.to(gpu), k.to(gpu), v.to(gpu), cache, 4 * nb * T, memory_frames=[0])
