"""The product rollout driver over the slot cache on the GPU, against the oracle's rollout.

``driver.self_forcing_latents`` (the NFE4 sampler, stage2.py:627-771) drives a model whose
blocks attend through ``attend_cached`` and commit through ``driver.cached_forward``
(causal_model.py:2819-2844); the oracle's ``rollout`` (the same pass/commit pattern over the
reference's dense cache) receives the same per-(chunk, pass, layer) inputs.  Every pass's
attention output matches within the bf16 bars and the committed cache is bit-exact after the
rollout.  The dict surface hands out read-only ``k``/``v`` snapshots.
"""

from types import SimpleNamespace

import pytest
import torch

from oracle import wan_cache_ref as ref
from solarwm_amd import attend_cached, driver, make_kv_cache_allocator
from solarwm_amd._readonly import CacheWriteError

from .helpers import assert_attn_close

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _say(*a):
    print(*a, flush=True)


def test_sampler_over_slot_cache_matches_oracle_rollout(gpu):
    T, H, layers, cap, chunk, frames = 64, 2, 3, 6, 3, 12
    Lq = chunk * T
    _say("driver rollout", T, H, layers, cap, frames)

    def inputs(c, p, layer):
        g = torch.Generator().manual_seed(7000 + 100 * c + 10 * p + layer)
        return tuple(torch.randn(1, Lq, H, 128, generator=g).to(BF) for _ in range(3))

    ours, theirs = {}, {}

    class Model:
        scheduler = SimpleNamespace(add_noise=lambda clean, noise, t: clean)

        def __init__(self):
            self.passes = {}

        def __call__(self, latents, condition, camera, timestep, *, kv_cache, current_start,
                     cache_update_policy, **kw):
            c = current_start // Lq
            p = self.passes.get(c, 0)
            self.passes[c] = p + 1

            def block(i, cache):
                q, k, v = (t.to(gpu) for t in inputs(c, p, i))
                return attend_cached(q, k, v, cache, current_start)

            for i, x in enumerate(driver.cached_forward(kv_cache, block,
                                                        cache_update_policy=cache_update_policy)):
                ours[(c, p, i)] = x.cpu()
            return torch.zeros_like(latents)

        @staticmethod
        def flow_to_x0(noisy, flow, timestep):
            return noisy.float() - flow.float()

    kept = {}
    alloc = make_kv_cache_allocator(num_layers=layers, num_heads=H, head_dim=128,
                                    frame_sequence_length=T, local_attn_size=cap, sink_size=0,
                                    num_frame_per_block=chunk)

    def allocate(batch_size, *, dtype, device):
        kept["kv"] = alloc(batch_size, dtype=dtype, device=device)
        return kept["kv"]

    provider = SimpleNamespace(
        config={"model": {"num_frame_per_block": chunk, "latent_channels": 1,
                          "frame_sequence_length": T},
                "data": {"latent_shape": [frames, 1, 1, 1]}},
        device=gpu, diffusion=Model(), allocate_kv_cache=allocate,
        allocate_crossattn_cache=lambda b, *, dtype, device: [],
        denoising_steps=tuple(torch.tensor(float(s)) for s in (1000, 750, 500, 250)),
        _noise=lambda shape, g: torch.zeros(shape, device=gpu, dtype=BF))
    camera = {"viewmats": torch.eye(4).repeat(1, frames * T, 1, 1),
              "K": torch.eye(3).repeat(1, frames * T, 1, 1)}
    driver.self_forcing_latents(provider, SimpleNamespace(
        solver="self_forcing", num_inference_steps=4, rollout_latent_frames=frames),
        torch.zeros(1, 1, 1, 1, 1, dtype=BF), {}, camera, None)

    oracle = ref.allocate_kv_cache(layers, 1, cap * T, H, 128, BF)
    ref.rollout(frames // chunk, ["none"] * 4 + ["commit"], Lq, inputs, oracle, frame_seqlen=T,
                sink_size=0, local_attn_size=cap,
                attn_fn=lambda q, k, v: ref.attention(q, k, v, compute_dtype=torch.float32),
                on_output=lambda c, p, layer, x: theirs.__setitem__((c, p, layer), x))
    assert sorted(ours) == sorted(theirs) and len(ours) == 4 * 5 * layers
    for key in sorted(ours):
        assert_attn_close(ours[key], theirs[key])
    caches = kept["kv"]
    for layer in range(layers):
        k_view, v_view = caches[layer]["k"], caches[layer]["v"]
        torch.cuda.synchronize()
        assert torch.equal(k_view.cpu(), oracle[layer]["k"])
        assert torch.equal(v_view.cpu(), oracle[layer]["v"])
        assert int(caches[layer]["global_end_index"]) == int(oracle[layer]["global_end_index"])
        assert int(caches[layer]["local_end_index"]) == int(oracle[layer]["local_end_index"])
        with pytest.raises(CacheWriteError):
            k_view[:, :T] = 0  # the reference's slice write (causal_model.py:2894-2898)
