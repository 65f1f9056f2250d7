"""GPU parity of the PRoPE self-attention branch's cache (CausalPropeSelfAttention with a
kv_cache, causal_model.py:1296-1525) against the oracle's restatement
(oracle/prope_ref.py prope_branch_forward).

Bars as for fused PRoPE (tests/test_gpu_prope.py): against the float64 restatement our mean and
99.9th-percentile errors stay within 1.25x of the reference's own bf16 arithmetic and our
largest within 2.5x of its largest (or the plain bf16 bars); indices equal the oracle's after
every forward; the ``prope_k`` / ``prope_v`` view equals the oracle's cache of P⁻¹k / P⁻¹v within
one bf16 rounding of the float64 transform.
"""

import pytest
import torch

from oracle import prope_ref as pr
from oracle import wan_cache_ref as ref
from solarwm_amd import PropeConfig, make_kv_cache_allocator, prope_branch_attention

from .cameras import per_token, trajectory
from .helpers import MAX_ABS, MEAN_ABS

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _say(*a):
    print(*a, flush=True)


def _errors(got, want):
    d = (got.double() - want.double()).abs().flatten()
    return float(d.max()), float(d.kthvalue(max(1, int(d.numel() * 0.999))).values), float(d.mean())


@pytest.mark.parametrize("sink,cap,T,chunks,transform,B", [
    (1, 5, 64, 4, "linear", 1),
    (0, 4, 100, 4, "logd4", 2),
    (1, 21, 1560, 2, "linear", 1),
])
def test_branch_rollout_vs_oracle(gpu, sink, cap, T, chunks, transform, B):
    _say("prope branch rollout", sink, cap, T, chunks, transform, B)
    H, nb = 2, 2
    caches = make_kv_cache_allocator(
        num_layers=2, num_heads=H, head_dim=128, frame_sequence_length=T, local_attn_size=cap,
        sink_size=sink, num_frame_per_block=nb,
        prope_branch=PropeConfig(camera_translation_transform=transform))(B, dtype=BF, device=gpu)
    c1 = caches[1]
    assert "prope_k" in c1 and int(c1["prope_local_end_index"]) == 0
    oc = ref.allocate_kv_cache(1, B, cap * T, H, 128, BF)[0]
    vm, ks = trajectory(B, chunks * nb, seed=41, t_scale=0.6)
    vm_tok, ks_tok = per_token(vm, T), per_token(ks, T)
    g = torch.Generator().manual_seed(3)
    for c in range(chunks):
        for policy in ("none", "commit_detached"):
            q, k, v = (torch.randn(B, nb * T, H, 128, generator=g).to(BF) for _ in range(3))
            start = c * nb * T
            x = prope_branch_attention(q.to(gpu), k.to(gpu), v.to(gpu), c1, start,
                                       vm_tok.to(gpu), ks_tok.to(gpu), cache_update_policy=policy)
            cq, ck = (t[:, start : start + nb * T] for t in (vm_tok, ks_tok))
            args = dict(viewmats=cq, ks=ck, current_start=start, frame_seqlen=T, sink_size=sink,
                        local_attn_size=cap, transform=transform)
            shadow = {key: val.clone() for key, val in oc.items()}
            want_ref = pr.prope_branch_forward(q, k, v, shadow, cache_update_policy="none",
                                               emulate_bf16=True, **args)
            want = pr.prope_branch_forward(q, k, v, oc, cache_update_policy=policy, **args)
            torch.cuda.synchronize()
            assert torch.isfinite(x).all()
            e_ours, e_ref = _errors(x.cpu(), want), _errors(want_ref, want)
            _say(f"  chunk {c} {policy}: (max, p99.9, mean) ours "
                 f"{tuple(f'{e:.2e}' for e in e_ours)} reference {tuple(f'{e:.2e}' for e in e_ref)}")
            assert e_ours[0] <= max(MAX_ABS, 2.5 * e_ref[0]), "max"
            assert e_ours[1] <= max(MAX_ABS / 2, 1.25 * e_ref[1]), "p99.9"
            assert e_ours[2] <= max(MEAN_ABS, 1.25 * e_ref[2]), "mean"
            assert int(c1["prope_global_end_index"]) == int(oc["global_end_index"])
            assert int(c1["prope_local_end_index"]) == int(oc["local_end_index"])
    # the cache rows: P⁻¹k / P⁻¹v of each frame's camera (the oracle stored its bf16 rounding of
    # the float64 transform), live rows within two bf16 roundings
    live = c1.branch.local_end
    for name, key in (("prope_k", "k"), ("prope_v", "v")):
        got = c1[name].cpu()[:, :live].double()
        want = oc[key][:, :live].double()
        assert ((got - want).abs() <= want.abs() * 2.0**-7 + 1e-4).all(), name
    # the main cache of the layer is untouched by the branch
    assert c1.local_end == 0 and caches[0].branch.local_end == 0
