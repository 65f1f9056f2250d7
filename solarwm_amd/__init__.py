"""solarwm_amd — MI355X-native block-causal KV-cache inference path for SolarWM-style
chunked autoregressive video models.

Public surface (the reference's call signatures, solar/backends/wan22/runtime):
* :func:`make_kv_cache_allocator` → ``allocate_kv_cache(batch_size, *, dtype, device)``
* :class:`SlotKVCache` — one layer's cache (dict surface ``k``/``v``/``*_end_index``)
* :func:`attend_cached`, :func:`apply_cache_updates` — cached self-attention + deferred commit
* :func:`attention`, :func:`chunk_causal_attention` — dense drop-in attention ops
* :mod:`solarwm_amd.kernels` — thin wrappers of the C ABI in include/solarkv.h
* :class:`RopeConfig` — pre-RoPE caches with Wan RoPE applied on load (``rope=`` of the
  allocator)
* :class:`PropeConfig`, :func:`stage_camera_cache` — fused PRoPE camera transforms on the same
  caches (``prope=`` of the allocator; one camera pass per forward, ``camera=`` of
  :func:`attend_cached`)
* ``norm_q=`` / ``norm_k=`` of :func:`attend_cached` — q/k RMSNorm fused into the kernels
* :func:`make_crossattn_cache_allocator`, :func:`cross_attend` — the cross-attention K/V cache
* ``prope_branch=`` of the allocator, :func:`prope_branch_attention` — the cache of the PRoPE
  self-attention branch (camera_attention_mode "parallel")
* :mod:`solarwm_amd.driver` — the sampler's pass/commit driver and the block loop
"""

from .attention import (apply_cache_updates, attend_cached, attention, chunk_causal_attention,
                        prope_branch_attention)
from .crossattn import CrossAttnCache, cross_attend, make_crossattn_cache_allocator
from .cache import CacheGeometry, CachePlan, SlotKVCache, make_kv_cache_allocator, plan_cached_forward
from .prope import PropeConfig, commit_camera_cache, drop_camera_cache, stage_camera_cache
from .rope import RopeConfig

__all__ = [
    "CacheGeometry",
    "CachePlan",
    "CrossAttnCache",
    "PropeConfig",
    "RopeConfig",
    "SlotKVCache",
    "apply_cache_updates",
    "attend_cached",
    "attention",
    "chunk_causal_attention",
    "commit_camera_cache",
    "cross_attend",
    "drop_camera_cache",
    "make_crossattn_cache_allocator",
    "make_kv_cache_allocator",
    "plan_cached_forward",
    "prope_branch_attention",
    "stage_camera_cache",
]
