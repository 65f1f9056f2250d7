"""Cross-attention K/V cache of the Wan blocks, on the same kernels.

The reference computes the text context's K/V once per rollout into ``crossattn_cache`` (one
dict per block: ``k``, ``v`` ``[B, 512, H, D]`` and ``is_init``, stage2.py:1819-1854) and
reuses them in every later forward (WanCrossAttention.forward, model.py:152-184): q =
norm_q(q(x)), k = norm_k(k(context)), v = v(context), then attention over all context tokens
(``context_lens`` is None on the cached inference path, causal_model.py:2730).

Here each block's cache is one frame slot of ``context_tokens`` tokens in the self-attention
pool layout: the first call appends the context with K RMS-normalised inside the append, every
call runs the attention kernel with Q normalised at load.
"""

from __future__ import annotations

from collections.abc import Mapping
from typing import Any, Iterator

import torch

from . import kernels
from .attention import _row_norm


class CrossAttnCache(Mapping):
    """One block's cross-attention cache with the reference dict surface (``k``, ``v``,
    ``is_init``); ``k``/``v`` are materialised from the pool on access."""

    def __init__(self, batch: int, heads: int, context_tokens: int, *, dtype: torch.dtype, device):
        if dtype not in (torch.bfloat16, torch.float32):
            raise ValueError(f"cross-attention cache dtype {dtype} unsupported (bf16 or float32)")
        self.batch, self.heads, self.context_tokens = batch, heads, context_tokens
        self.dtype = dtype
        self.kpool, self.vpool, _, _ = kernels.new_pools(1, batch, heads, context_tokens, dtype, device)
        self.is_init = False

    def reset(self) -> None:
        self.is_init = False
        self.kpool.zero_()
        self.vpool.zero_()

    def fill(self, ctx_k: torch.Tensor, ctx_v: torch.Tensor, norm_k=None) -> None:
        """Store the context's K (normalised by ``norm_k``) and V; marks the cache initialised."""
        if ctx_k.shape != ctx_v.shape or tuple(ctx_k.shape) != (
                self.batch, self.context_tokens, self.heads, kernels.HEAD_DIM):
            raise ValueError(f"context K/V {tuple(ctx_k.shape)} do not match the cache "
                             f"[{self.batch}, {self.context_tokens}, {self.heads}, {kernels.HEAD_DIM}]")
        if ctx_k.dtype != self.dtype or ctx_v.dtype != self.dtype:
            raise ValueError(f"context K/V dtype must be {self.dtype}")
        kernels.append_frames(
            ctx_k, ctx_v, self.kpool, self.vpool, [0], frame_tokens=self.context_tokens,
            k_norm=_row_norm(ctx_k, norm_k, self.heads) if norm_k is not None else None)
        self.is_init = True

    def __getitem__(self, key: str) -> Any:
        if key == "is_init":
            return self.is_init
        if key in ("k", "v"):
            k, v = kernels.gather_frames(self.kpool, self.vpool, [0], frame_tokens=self.context_tokens)
            return k if key == "k" else v
        raise KeyError(key)

    def __iter__(self) -> Iterator[str]:
        return iter(("k", "v", "is_init"))

    def __len__(self) -> int:
        return 3


def make_crossattn_cache_allocator(*, num_layers: int, num_heads: int, head_dim: int,
                                   context_tokens: int = 512):
    """``allocate_crossattn_cache(batch_size, *, dtype, device) -> list[CrossAttnCache]``: the
    signature of ``Wan5BStage2Runtime.allocate_crossattn_cache`` (stage2.py:1819-1854), for its
    ``_crossattn_cache_allocator`` hook."""
    if head_dim != kernels.HEAD_DIM:
        raise ValueError(f"head_dim must be {kernels.HEAD_DIM}")

    def allocate_crossattn_cache(batch_size: int, *, dtype: torch.dtype, device: Any):
        return [CrossAttnCache(batch_size, num_heads, context_tokens, dtype=dtype, device=device)
                for _ in range(num_layers)]

    return allocate_crossattn_cache


def cross_attend(q: torch.Tensor, ctx_k: torch.Tensor | None, ctx_v: torch.Tensor | None,
                 cache: CrossAttnCache, *, norm_q=None, norm_k=None, context_lens=None,
                 softmax_scale: float | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """WanCrossAttention.forward after the projections (model.py:152-184): ``q`` = q(x), and on
    the first call ``ctx_k`` / ``ctx_v`` = k(context) / v(context) fill the cache (later calls
    ignore them, as the reference does once ``is_init`` is set).  Returns the attention output
    [B, L1, H, D] before ``flatten`` and ``self.o``."""
    if context_lens is not None:
        raise NotImplementedError("context_lens: the cached inference path attends every context "
                                  "token (causal_model.py:2730 passes None)")
    if not cache.is_init:
        if ctx_k is None or ctx_v is None:
            raise ValueError("the first cross-attention call needs the context K/V")
        cache.fill(ctx_k, ctx_v, norm_k)
    return kernels.attention_frames(
        q, cache.kpool, cache.vpool, [0], frame_tokens=cache.context_tokens,
        softmax_scale=softmax_scale, out=out,
        q_norm=_row_norm(q, norm_q, cache.heads) if norm_q is not None else None)
