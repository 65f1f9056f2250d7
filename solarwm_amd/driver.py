"""Rollout driver of the cached path: the reference sampler's pass/commit pattern and the model's
block loop with its deferred commit.

* :func:`self_forcing_latents` — the NFE4 self-forcing sampler over one persistent KV cache
  (solar/backends/wan22/runtime/stage2.py:627-771), same arguments and provider protocol: per
  three-frame chunk, four ``cache_update_policy="none"`` forwards (the cache is read, never
  written) and one ``"commit_detached"`` forward of the clean chunk at t = 0 that commits it.
* :func:`rollout_passes` — that schedule as data (one :class:`CachePass` per forward), so a
  caller that drives the layers itself (``bench.py``, the parity tests) runs exactly the
  reference's order.
* :func:`cached_forward` — ``CausalWanModel.forward``'s block loop (causal_model.py:2819-2844):
  every block attends through its own cache, then, unless the policy is ``"none"``, all blocks
  commit together (``apply_cache_updates``) and the fused-PRoPE camera rows follow (committed
  with the pass, or dropped when a fused-PRoPE model committed without cameras).

The driver allocates through ``provider.allocate_kv_cache`` (the seam of stage2.py:1758-1764), so
``make_kv_cache_allocator`` plugs in unchanged.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable, Mapping, Sequence

import torch

from .attention import apply_cache_updates
from .prope import CameraPass, commit_camera_cache, drop_camera_cache

NONE = "none"
COMMIT = "commit_detached"


class BackendContractError(RuntimeError):
    """A rollout request outside the sampler's contract (the reference's BackendContractError,
    solar/errors.py:16)."""


@dataclass(frozen=True)
class CachePass:
    """One model forward of a rollout."""

    chunk: int  # chunk index
    start_frame: int  # first latent frame of the chunk
    current_start: int  # first token of the chunk (start_frame * frame tokens)
    step_index: int | None  # denoising step of a "none" pass; None for the commit pass
    policy: str  # "none" or "commit_detached"


def rollout_passes(latent_frames: int, chunk_frames: int, frame_tokens: int,
                   denoising_steps: int) -> list[CachePass]:
    """The forwards of one rollout in order (stage2.py:674-760): for every chunk, one ``none``
    pass per denoising step, then the commit pass, all at the chunk's ``current_start``."""
    if chunk_frames <= 0 or latent_frames % chunk_frames:
        raise BackendContractError("rollout horizon must divide into whole chunks")
    passes = []
    for c, f0 in enumerate(range(0, latent_frames, chunk_frames)):
        tok0 = f0 * frame_tokens
        passes.extend(CachePass(c, f0, tok0, s, NONE) for s in range(denoising_steps))
        passes.append(CachePass(c, f0, tok0, None, COMMIT))
    return passes


def cached_forward(
    kv_cache: Sequence[Any],
    block_fn: Callable[[int, Any], tuple[Any, tuple[int, int, Any]]],
    *,
    cache_update_policy: str = COMMIT,
    camera: CameraPass | None = None,
    fused_prope: bool = False,
) -> list[Any]:
    """Run every block and apply the deferred commit (causal_model.py:2819-2844).

    ``block_fn(block_index, block_cache)`` returns ``(x, (current_end, local_end_index,
    update))`` as ``attend_cached`` does.  Nothing is committed unless every block returned (a
    failing block leaves the cache untouched) and the policy is not ``"none"``.  ``camera`` is the
    pass's ``stage_camera_cache`` result; with ``fused_prope`` and no camera the commit drops the
    camera metadata, as the reference does for a camera-free commit of a fused-PRoPE model."""
    outs, infos = [], []
    for i, block_cache in enumerate(kv_cache):
        x, info = block_fn(i, block_cache)
        outs.append(x)
        infos.append((i, info))
    if infos and cache_update_policy != NONE:
        apply_cache_updates(kv_cache, infos)
        if fused_prope and camera is None:
            drop_camera_cache(kv_cache)
        else:
            commit_camera_cache(camera)
    return outs


# ---------------------------------------------------------------------------------------------
# the NFE4 sampler (stage2.py:627-771)
# ---------------------------------------------------------------------------------------------
def _warped_steps(raw_steps: Sequence[Any], table: torch.Tensor, num_train: int) -> tuple:
    """Public integer step labels mapped onto the shifted scheduler table (sgf.py:273-297): label
    r picks ``table[N - r]`` of the table extended by a final 0; a trailing 0 step is dropped."""
    table = torch.as_tensor(table).detach().to(torch.float32)
    if table.ndim != 1 or table.numel() != num_train:
        raise ValueError("scheduler_timesteps must contain the complete one-dimensional training table")
    ext = torch.cat([table, table.new_zeros(1)])
    out = []
    for raw in raw_steps:
        r = round(float(raw))
        if abs(float(raw) - r) > 1e-6 or not 0 <= r <= num_train:
            raise ValueError("SGF denoising labels must be integers in [0,N]")
        out.append(ext[num_train - r].reshape(()))
    if out and float(out[-1]) == 0.0:
        out.pop()
    if not out:
        raise ValueError("SGF denoising schedule has no non-zero step")
    return tuple(out)


def generation_steps(provider: Any) -> tuple:
    """The sampler's timesteps: ``provider.denoising_steps`` when set, else the configured labels
    warped onto the scheduler table (stage2.py:615-624)."""
    steps = getattr(provider, "denoising_steps", None)
    if steps is not None:
        return tuple(steps)
    train = provider.config["train"]
    return _warped_steps(train["denoising_step_list"],
                         provider.diffusion.scheduler.timesteps.to(provider.device),
                         int(train["num_train_timesteps"]))


def _tokens_timestep(timestep: torch.Tensor, frame_tokens: int) -> torch.Tensor:
    """[B, F] per-frame timesteps repeated over each frame's tokens (stage0p5.py:80-86)."""
    b, f = timestep.shape
    return timestep.unsqueeze(-1).expand(b, f, frame_tokens).reshape(b, f * frame_tokens)


def _chunk_camera(camera: Mapping[str, Any], f0: int, f1: int, frame_tokens: int) -> dict:
    return {name: camera[name][:, f0 * frame_tokens : f1 * frame_tokens] for name in ("viewmats", "K")}


def _with_first(x: torch.Tensor, first: torch.Tensor, start_frame: int) -> torch.Tensor:
    """The first chunk keeps the conditioning latent in frame 0 (stage2.py:373-378)."""
    if start_frame:
        return x
    x = x.clone()
    x[:, :1] = first
    return x


def self_forcing_latents(
    provider: Any,
    generation_pass: Any,
    first_latent: torch.Tensor,
    condition: Mapping[str, Any],
    camera: Mapping[str, Any],
    generator: Any,
) -> tuple[torch.Tensor, dict[str, Any]]:
    """Generate ``generation_pass.rollout_latent_frames`` latent frames chunk by chunk over one
    persistent KV cache (stage2.py:627-771).

    ``provider`` supplies ``config`` (model.num_frame_per_block, latent_channels,
    frame_sequence_length; data.latent_shape), ``device``, ``diffusion`` (called as
    ``diffusion(latents, condition, camera_chunk, timestep_tokens, sequence_length=...,
    kv_cache=..., crossattn_cache=..., current_start=..., cache_start=0,
    cache_update_policy=...)``, plus ``flow_to_x0`` and ``scheduler.add_noise``),
    ``allocate_kv_cache`` / ``allocate_crossattn_cache`` and ``_noise(shape, generator)``.
    Returns the latents and the schedule record."""
    if str(generation_pass.solver) != "self_forcing" or int(generation_pass.num_inference_steps) != 4:
        raise BackendContractError("Stage2 generation supports self_forcing NFE4 only")
    model_cfg = provider.config["model"]
    n_frames = int(generation_pass.rollout_latent_frames)
    chunk = int(model_cfg["num_frame_per_block"])
    if chunk != 3 or n_frames % chunk:
        raise BackendContractError("Stage2 generation horizon must divide into three-latent chunks")
    frame_tokens = int(model_cfg["frame_sequence_length"])
    lat_h, lat_w = (int(x) for x in provider.config["data"]["latent_shape"][-2:])
    dev = provider.device
    shape = (1, n_frames, int(model_cfg["latent_channels"]), lat_h, lat_w)
    output = torch.zeros(shape, device=dev, dtype=torch.bfloat16)
    output[:, 0] = first_latent[:, 0]
    noise = provider._noise(shape, generator)
    noise[:, 0] = first_latent[:, 0]
    steps = generation_steps(provider)
    if len(steps) != 4:
        raise BackendContractError("Stage2 shifted generation schedule must have four steps")

    kv_cache = provider.allocate_kv_cache(1, dtype=output.dtype, device=dev)
    cross_cache = provider.allocate_crossattn_cache(1, dtype=output.dtype, device=dev)
    if kv_cache and "_fused_prope_camera_metadata" not in kv_cache[0]:
        raise BackendContractError("Stage2 generation requires preallocated fused camera metadata")
    autocast = dict(device_type=dev.type, dtype=torch.bfloat16, enabled=dev.type == "cuda")

    def frame_timesteps(value: float, first_chunk: bool, dtype) -> torch.Tensor:
        t = torch.full((1, chunk), value, device=dev, dtype=dtype)
        if first_chunk:
            t[:, 0] = 0.0  # the conditioning frame is clean
        return t

    def forward(latents, cam, timestep, p: CachePass):
        return provider.diffusion(
            latents, condition, cam, _tokens_timestep(timestep, frame_tokens),
            sequence_length=chunk * frame_tokens, kv_cache=kv_cache, crossattn_cache=cross_cache,
            current_start=p.current_start, cache_start=0, cache_update_policy=p.policy)

    latents = None
    try:
        for p in rollout_passes(n_frames, chunk, frame_tokens, len(steps)):
            f0, first = p.start_frame, p.start_frame == 0
            cam = _chunk_camera(camera, f0, f0 + chunk, frame_tokens)
            if p.policy == COMMIT:
                if not bool(torch.isfinite(latents).all().item()):
                    raise BackendContractError(f"Stage2 generation chunk {p.chunk} is non-finite")
                output[:, f0 : f0 + chunk] = latents
                with torch.no_grad(), torch.autocast(**autocast):
                    forward(latents, cam, frame_timesteps(0.0, False, output.dtype), p)
                continue
            if p.step_index == 0:
                latents = noise[:, f0 : f0 + chunk].clone()
            t = frame_timesteps(float(steps[p.step_index].item()), first, output.dtype)
            with torch.autocast(**autocast):
                flow = forward(latents, cam, t, p)
                x0 = provider.diffusion.flow_to_x0(latents, flow, t)
            x0 = _with_first(x0, first_latent, f0)
            if p.step_index + 1 == len(steps):
                latents = x0
                continue
            t_next = frame_timesteps(float(steps[p.step_index + 1].item()), first, torch.float32)
            fresh = provider._noise(tuple(x0.shape), generator)
            latents = provider.diffusion.scheduler.add_noise(
                x0.flatten(0, 1).float(), fresh.flatten(0, 1).float(), t_next.flatten(0, 1),
            ).unflatten(0, (1, chunk)).to(output.dtype)
            latents = _with_first(latents, first_latent, f0)
    finally:
        del kv_cache, cross_cache
    return output, {
        "schema": "solarwm.wan22-stage2-self-forcing-schedule.v1",
        "solver": "self_forcing",
        "timesteps": [float(s.item()) for s in steps],
        "chunk_latent_frames": chunk,
        "persistent_kv_cache": True,
        "cache_update_policy": COMMIT,
        "camera_attention_mode": "fused_prope",
    }
