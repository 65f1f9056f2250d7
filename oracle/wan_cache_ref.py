"""CPU restatement of SolarWM's KV-cache inference path — TEST INFRASTRUCTURE ONLY.

Written from reading the reference (not imported, not copied); citations are
``solar/backends/wan22/runtime/...`` relative to the reference repository.  The functions keep
the reference's op sequence — clone the cache, memmove the non-sink window, slice-assign the
chunk, ``cat`` sink and local windows, attention — on dense ``[B, tokens, H, D]`` CPU tensors.

Pinning (tests/test_oracle.py):
* ``cached_self_attention`` / ``apply_cache_updates`` index math and data movement — the
  published C1 known answer (visible key counts 1170..8190, evicted frames {1,2,3}, {4,5,6},
  {7,8,9}, final order [0, 10..29]); a token-labelled brute-force list model of "sink frames +
  the most recent window" on many geometries; recompute and ``none``-pass invariants.
* ``rollout`` — the C1 known answer reached through the driver with token-labelled K/V on two
  layers, plus the stage2 call pattern: layers in order within a pass, ``none`` passes leave the
  committed indices unchanged and see the same window as the chunk's commit pass.
* ``attention`` — explicit float64 loops of softmax(q kᵀ/√d) v; closed forms (identical keys →
  mean of V; one key → V; key-order invariance).
* ``sdpa_fallback_attention`` — the same float64 loops within the bf16 attention bars; values
  paired with the wrong keys fail them.
* ``inference_window_mask`` / ``block_classes`` — brute-force rule "chunk i sees chunks 0..i"
  and per-block full/partial/empty from the dense mask.
* ``fp8_quantize`` — every e4m3fn code decoded from sign/exponent/mantissa; each quantised value
  is the nearest code (ties to even) found by exhaustive search.
* ``memory_gather`` — index semantics checked against per-frame slicing.
* ``fp8_fake_quant_frames`` / ``fp8_fake_quant_rows`` — compositions of the pinned
  ``fp8_quantize``; checked for block independence and exact decoding of representable values.
* ``fp8_rope_query_frames`` / ``fp8_rope_attention`` — every logit of the quantised query
  against the RoPE copy stays within the e4m3 error bound of the float64 RoPE logits
  (rope_frames at p_q and p_k; a reversed angle, a wrong temporal/spatial split or a scale that
  lets a rotation clip fail it, planted rows included); identical keys give the mean of V; with
  every angle zero (one-token frames, equal positions) and zero temporal channels the query is
  ``fp8_fake_quant_rows``'s.
* ``cached_self_attention(rope={"attend": ...})`` — with an attend that rotates at the given
  positions it equals the built-in RoPE path exactly (sink and no-sink windows, memory frames).
* ``rope_params`` / ``wan_rope_freqs`` / ``rope_frames`` — angles against ``math.cos`` /
  ``math.sin`` of position × theta^(-2j/d) computed independently; the temporal/height/width
  channel split; rotation preserves each pair's norm; position 0 is the identity; scores depend
  only on position differences (shifting every position leaves q·k unchanged).
* ``window_relative_positions`` / ``rope_positions`` — hand-derived cases of the reference's
  allocation (sink frames at 0.., the query chunk pinned at the window tail, capping at the
  EchoRoPE horizon or ``rope_train_frames``, underflow errors).
* ``rms_norm_f64`` / ``wan_rms_norm`` — explicit loops; a constant row c maps to
  c / sqrt(c² + eps) · w; scale invariance; the reference's in-dtype bf16 sequence stays within
  a few bf16 roundings of the float64 form.
* ``cross_attention`` — the cache keeps the first context (a later context is ignored) and the
  result is attention over the normalised cached K.
"""

from __future__ import annotations

import math
from typing import Any, Callable, Sequence

import torch

E4M3_MAX = 448.0


# ---------------------------------------------------------------------------------------------
# attention (attention.py:141-188 — flash path semantics: cast non-half inputs to bf16,
# compute, return in q's dtype)
# ---------------------------------------------------------------------------------------------
def attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    softmax_scale: float | None = None,
    mask: torch.Tensor | None = None,
    compute_dtype: torch.dtype = torch.float64,
    round_inputs_to_bf16: bool = True,
) -> torch.Tensor:
    """softmax(q kᵀ · scale [masked]) v for [B, L, H, D]; ``mask`` [Lq, Lk] bool (True = keep).

    Inputs are first rounded to bf16 (attention.py:69-73 ``half()``), then the product is
    evaluated in ``compute_dtype`` with torch's SDPA math (the reference's own fallback op,
    attention.py:172-188) and returned in ``q.dtype`` (attention.py:138).
    """
    out_dtype = q.dtype
    if round_inputs_to_bf16:
        q, k, v = (x.to(torch.bfloat16) for x in (q, k, v))
    qt = q.transpose(1, 2).to(compute_dtype)
    kt = k.transpose(1, 2).to(compute_dtype)
    vt = v.transpose(1, 2).to(compute_dtype)
    scale = 1.0 / math.sqrt(q.shape[-1]) if softmax_scale is None else softmax_scale
    out = torch.nn.functional.scaled_dot_product_attention(
        qt, kt, vt, attn_mask=mask, scale=scale
    )
    return out.transpose(1, 2).contiguous().to(out_dtype)


def sdpa_fallback_attention(q, k, v):
    """The reference's SDPA fallback exactly (attention.py:172-188): bf16 SDPA, bf16 result.
    Used as the timed CPU baseline of the reference path."""
    qt = q.transpose(1, 2).to(torch.bfloat16)
    kt = k.transpose(1, 2).to(torch.bfloat16)
    vt = v.transpose(1, 2).to(torch.bfloat16)
    out = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt)
    return out.transpose(1, 2).contiguous()


# ---------------------------------------------------------------------------------------------
# cache allocation (stage2.py:1758-1817)
# ---------------------------------------------------------------------------------------------
def allocate_kv_cache(
    num_layers: int,
    batch_size: int,
    cache_tokens: int,
    num_heads: int,
    head_dim: int,
    dtype: torch.dtype,
) -> list[dict[str, Any]]:
    return [
        {
            "k": torch.zeros(batch_size, cache_tokens, num_heads, head_dim, dtype=dtype),
            "v": torch.zeros(batch_size, cache_tokens, num_heads, head_dim, dtype=dtype),
            "global_end_index": torch.zeros(1, dtype=torch.long),
            "local_end_index": torch.zeros(1, dtype=torch.long),
        }
        for _ in range(num_layers)
    ]


# ---------------------------------------------------------------------------------------------
# the cache branch of CausalWanSelfAttention.forward (causal_model.py:1028-1235), with q/k/v
# already projected and K already roped (RoPE is the identity here: inputs are post-RoPE)
# ---------------------------------------------------------------------------------------------
def cached_self_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    kv_cache: dict[str, Any],
    *,
    current_start: int,
    frame_seqlen: int,
    sink_size: int,
    local_attn_size: int,
    sink_recache_after_switch: bool = False,
    attn_fn: Callable[..., torch.Tensor] = attention,
    memory_k: torch.Tensor | None = None,
    memory_v: torch.Tensor | None = None,
    rope: dict[str, Any] | None = None,
    prope: dict[str, Any] | None = None,
    memory_positions: Sequence[int] | None = None,
):
    """Returns ``(x [B, Lq, H, D], (current_end, local_end_index, cache_update_info))``.

    ``memory_k``/``memory_v`` ([B, M, H, D], already gathered) are placed ahead of the window,
    as the H3 memory path orders ``[bank | history | current]`` (memory_kv_attention.py:97-137).
    With ``rope`` they are pre-RoPE too and frame f of the bank is rotated at temporal position
    ``memory_positions[f]`` (the H3 path rotates bank rows at their own positions,
    memory_kv_attention.py:112-114, :122-131; which positions is the caller's choice here).

    ``rope`` (``{"freqs", "grid_hw", "use_echorope", "rope_train_frames"}``) makes ``q``/``k``
    pre-RoPE, as the reference stores them: the cache keeps raw K and the query chunk, sink
    frames and local frames are rotated at the positions of ``rope_positions`` before attention
    (causal_model.py:1135-1199 with _rope_sink_local_and_query / _rope_q_and_window_k).  With
    ``rope["attend"]`` (a callable ``(q, k, v, q_positions, k_positions) -> x``) nothing is
    rotated here: the callable receives the raw query, the raw window (memory frames first) and
    the frame positions the rotation would use, and its result is the attention output.

    ``prope`` (``{"q_viewmats", "q_ks", "kv_viewmats", "kv_ks"}`` plus optional ``"transform"``
    and ``"emulate_bf16"``) applies fused PRoPE after RoPE (causal_model.py:1170-1199): query
    cameras are the chunk's [B, Lq, ...] tensors, key cameras the staged camera cache
    [B, cache_tokens, ...] of ``prope_ref.stage_fused_camera_cache``, cut to the window rows.
    """
    max_attention_size = 39600 if local_attn_size == -1 else local_attn_size * frame_seqlen
    current_end = current_start + q.shape[1]
    sink_tokens = sink_size * frame_seqlen
    kv_cache_size = kv_cache["k"].shape[1]
    num_new_tokens = q.shape[1]
    global_end = int(kv_cache["global_end_index"].item())
    local_end = int(kv_cache["local_end_index"].item())
    is_recompute = current_end <= global_end and current_start > 0

    if (
        local_attn_size != -1
        and current_end > global_end
        and num_new_tokens + local_end > kv_cache_size
    ):
        # rolling: evict the oldest non-sink tokens (causal_model.py:1036-1094)
        num_evicted = num_new_tokens + local_end - kv_cache_size
        num_rolled = local_end - num_evicted - sink_tokens
        local_end_index = local_end + current_end - global_end - num_evicted
        local_start_index = local_end_index - num_new_tokens
        temp_k = kv_cache["k"].detach().clone()
        temp_v = kv_cache["v"].detach().clone()
        src = slice(sink_tokens + num_evicted, sink_tokens + num_evicted + num_rolled)
        dst = slice(sink_tokens, sink_tokens + num_rolled)
        temp_k[:, dst] = temp_k[:, src].clone()
        temp_v[:, dst] = temp_v[:, src].clone()
        write_start = max(local_start_index, sink_tokens) if is_recompute else local_start_index
        roped_offset = max(0, write_start - local_start_index)
        write_len = max(0, local_end_index - write_start)
        if write_len > 0:
            temp_k[:, write_start:local_end_index] = k[:, roped_offset : roped_offset + write_len]
            temp_v[:, write_start:local_end_index] = v[:, roped_offset : roped_offset + write_len]
        info = {
            "action": "roll_and_insert",
            "sink_tokens": sink_tokens,
            "num_rolled_tokens": num_rolled,
            "num_evicted_tokens": num_evicted,
            "local_start_index": local_start_index,
            "local_end_index": local_end_index,
            "write_start_index": write_start,
            "write_end_index": local_end_index,
            "new_k": k[:, roped_offset : roped_offset + write_len],
            "new_v": v[:, roped_offset : roped_offset + write_len],
            "current_end": current_end,
            "is_recompute": is_recompute,
        }
    else:
        # direct insert (causal_model.py:1095-1133)
        local_end_index = local_end + current_end - global_end
        local_start_index = local_end_index - num_new_tokens
        temp_k = kv_cache["k"].detach().clone()
        temp_v = kv_cache["v"].detach().clone()
        write_start = max(local_start_index, sink_tokens) if is_recompute else local_start_index
        if sink_recache_after_switch:
            write_start = local_start_index
        roped_offset = max(0, write_start - local_start_index)
        write_len = max(0, local_end_index - write_start)
        if write_len > 0:
            temp_k[:, write_start:local_end_index] = k[:, roped_offset : roped_offset + write_len]
            temp_v[:, write_start:local_end_index] = v[:, roped_offset : roped_offset + write_len]
        info = {
            "action": "direct_insert",
            "local_start_index": local_start_index,
            "local_end_index": local_end_index,
            "write_start_index": write_start,
            "write_end_index": local_end_index,
            "new_k": k[:, roped_offset : roped_offset + write_len],
            "new_v": v[:, roped_offset : roped_offset + write_len],
            "current_end": current_end,
            "is_recompute": is_recompute,
        }

    # visible window (causal_model.py:1135-1199)
    nb = num_new_tokens // frame_seqlen
    if sink_tokens > 0:
        local_budget = max_attention_size - sink_tokens
        active_sink = min(sink_tokens, local_end_index)
        k_sink, v_sink = temp_k[:, :active_sink], temp_v[:, :active_sink]
        k_loc, v_loc = temp_k[:, :0], temp_v[:, :0]
        window = [(0, active_sink)]
        if local_budget > 0:
            local_start_for_window = max(sink_tokens, local_end_index - local_budget)
            k_loc = temp_k[:, local_start_for_window:local_end_index]
            v_loc = temp_v[:, local_start_for_window:local_end_index]
            window.append((local_start_for_window, local_end_index))
        if rope is not None:
            pos = rope_positions(
                num_sink_frames=active_sink // frame_seqlen, num_local_frames=k_loc.shape[1] // frame_seqlen,
                num_new_frames=nb, use_echorope=rope["use_echorope"],
                max_attention_size=max_attention_size, frame_seqlen=frame_seqlen,
                table_len=rope["freqs"].shape[0], rope_train_frames=rope.get("rope_train_frames"),
                current_start_frame=current_start // frame_seqlen, sink_branch=True)
            nl = k_loc.shape[1] // frame_seqlen
            q_pos = list(range(pos["q_start"], pos["q_start"] + nb))
            k_pos = list(range(k_sink.shape[1] // frame_seqlen)) + list(
                range(pos["local_start"], pos["local_start"] + nl))
            if "attend" not in rope:
                q = rope_frames(q, rope["grid_hw"], q_pos, rope["freqs"])
                k_sink = rope_frames(k_sink, rope["grid_hw"], range(k_sink.shape[1] // frame_seqlen),
                                     rope["freqs"])
                if nl > 0:
                    k_loc = rope_frames(k_loc, rope["grid_hw"], range(pos["local_start"], pos["local_start"] + nl),
                                        rope["freqs"])
        k_cat = torch.cat([k_sink, k_loc], dim=1)
        v_cat = torch.cat([v_sink, v_loc], dim=1)
    else:
        window_start = max(0, local_end_index - max_attention_size)
        window = [(window_start, local_end_index)]
        k_cat = temp_k[:, window_start:local_end_index]
        v_cat = temp_v[:, window_start:local_end_index]
        if rope is not None:
            nw = k_cat.shape[1] // frame_seqlen
            pos = rope_positions(
                num_sink_frames=0, num_local_frames=nw, num_new_frames=nb,
                use_echorope=rope["use_echorope"], max_attention_size=max_attention_size,
                frame_seqlen=frame_seqlen, table_len=rope["freqs"].shape[0], sink_branch=False)
            if nw == 0:
                raise RuntimeError("EchoRoPE attention got an empty K window")
            q_pos = list(range(pos["q_start"], pos["q_start"] + nb))
            k_pos = list(range(pos["local_start"], pos["local_start"] + nw))
            if "attend" not in rope:
                q = rope_frames(q, rope["grid_hw"], q_pos, rope["freqs"])
                k_cat = rope_frames(k_cat, rope["grid_hw"], k_pos, rope["freqs"])
    if memory_k is not None:
        mk = memory_k.to(k_cat.dtype)
        if rope is not None:
            nm = mk.shape[1] // frame_seqlen
            if memory_positions is None or len(memory_positions) != nm:
                raise ValueError("RoPE with memory-bank frames needs one position per bank frame")
            k_pos = list(memory_positions) + k_pos
            if "attend" not in rope:
                mk = rope_frames(mk, rope["grid_hw"], list(memory_positions), rope["freqs"])
        k_cat = torch.cat([mk, k_cat], dim=1)
        v_cat = torch.cat([memory_v.to(v_cat.dtype), v_cat], dim=1)
    if k_cat.shape[1] == 0:
        raise RuntimeError("KV-cache attention window is empty")
    if rope is not None and "attend" in rope:
        if prope is not None:
            raise NotImplementedError("rope['attend'] with PRoPE is outside this restatement")
        return rope["attend"](q, k_cat, v_cat, q_pos, k_pos), (current_end, local_end_index, info)
    if prope is not None:
        if memory_k is not None:
            raise NotImplementedError("PRoPE with memory-bank frames is outside this restatement")
        from . import prope_ref

        x = prope_ref.fused_prope_attention(
            q, k_cat, v_cat, q_viewmats=prope["q_viewmats"], q_ks=prope["q_ks"],
            kv_viewmats=prope_ref.visible_cameras(prope["kv_viewmats"], window),
            kv_ks=prope_ref.visible_cameras(prope["kv_ks"], window), attn_fn=attn_fn,
            transform=prope.get("transform", "linear"),
            emulate_bf16=prope.get("emulate_bf16", False))
        return x, (current_end, local_end_index, info)
    x = attn_fn(q, k_cat, v_cat)
    return x, (current_end, local_end_index, info)


def apply_cache_updates(kv_cache: list[dict[str, Any]], cache_update_infos) -> None:
    """CausalWanModel._apply_cache_updates (causal_model.py:2856-2921)."""
    with torch.no_grad():
        for block_index, (current_end, local_end_index, info) in cache_update_infos:
            if info is not None:
                cache = kv_cache[block_index]
                ws = info.get("write_start_index", info["local_start_index"])
                we = info.get("write_end_index", info["local_end_index"])
                new_k = info["new_k"].detach()
                new_v = info["new_v"].detach()
                if info["action"] == "roll_and_insert":
                    s = info["sink_tokens"]
                    r = info["num_rolled_tokens"]
                    e = info["num_evicted_tokens"]
                    cache["k"][:, s : s + r] = cache["k"][:, s + e : s + e + r].clone()
                    cache["v"][:, s : s + r] = cache["v"][:, s + e : s + e + r].clone()
                if we > ws and new_k.shape[1] == we - ws:
                    cache["k"][:, ws:we] = new_k
                    cache["v"][:, ws:we] = new_v
            is_recompute = False if info is None else info.get("is_recompute", False)
            if not is_recompute:
                kv_cache[block_index]["global_end_index"].fill_(current_end)
                kv_cache[block_index]["local_end_index"].fill_(local_end_index)


# ---------------------------------------------------------------------------------------------
# rollout driver: per chunk, N "none" passes then commit (stage2.py:674-760).  `passes` lists
# the policy of each forward of a chunk, e.g. ["none"] * 4 + ["commit"] (reference NFE4) or
# ["none", "commit"].
# ---------------------------------------------------------------------------------------------
def rollout(
    num_chunks: int,
    passes: Sequence[str],
    chunk_tokens: int,
    layer_inputs: Callable[[int, int, int], tuple[torch.Tensor, torch.Tensor, torch.Tensor]],
    kv_cache: list[dict[str, Any]],
    *,
    frame_seqlen: int,
    sink_size: int,
    local_attn_size: int,
    attn_fn: Callable[..., torch.Tensor] = attention,
    on_output: Callable[[int, int, int, torch.Tensor], None] | None = None,
) -> None:
    """Drive ``cached_self_attention`` over every layer; ``layer_inputs(chunk, pass, layer)``
    returns that layer's (q, k, v)."""
    for c in range(num_chunks):
        current_start = c * chunk_tokens
        for p, policy in enumerate(passes):
            infos = []
            for layer in range(len(kv_cache)):
                q, k, v = layer_inputs(c, p, layer)
                x, upd = cached_self_attention(
                    q, k, v, kv_cache[layer], current_start=current_start,
                    frame_seqlen=frame_seqlen, sink_size=sink_size,
                    local_attn_size=local_attn_size, attn_fn=attn_fn,
                )
                infos.append((layer, upd))
                if on_output is not None:
                    on_output(c, p, layer, x)
            if policy != "none":
                apply_cache_updates(kv_cache, infos)


# ---------------------------------------------------------------------------------------------
# chunk-causal mask (build_inference_window_block_mask, causal_model.py:474-534) and the block
# classification of _build_direct_block_mask (:245-302)
# ---------------------------------------------------------------------------------------------
def inference_window_mask(
    num_clean_frames: int, num_noisy_frames: int, frame_seqlen: int, num_frame_per_block: int
) -> tuple[torch.Tensor, int]:
    """Dense [P, P] mask over the right-padded sequence (P = total rounded up to 128) and the
    pad length, evaluating the reference's mask_mod for every (q, kv) pair."""
    total = (num_clean_frames + num_noisy_frames) * frame_seqlen
    padded = math.ceil(total / 128) * 128
    block = frame_seqlen * num_frame_per_block
    qi = torch.arange(padded)[:, None]
    ki = torch.arange(padded)[None, :]
    valid_q = qi < total
    chunk_index = qi // block
    causal = ki < torch.clamp((chunk_index + 1) * block, max=total)
    eye = qi == ki
    return eye | (valid_q & causal), padded - total


def block_classes(dense: torch.Tensor, block: int = 128) -> tuple[torch.Tensor, torch.Tensor]:
    """(full, partial) [nq, nk] block matrices of a dense mask: full = every entry visible,
    partial = some but not all."""
    n = dense.shape[0]
    nb = math.ceil(n / block)
    full = torch.zeros(nb, nb, dtype=torch.bool)
    partial = torch.zeros(nb, nb, dtype=torch.bool)
    for i in range(nb):
        for j in range(nb):
            tile = dense[i * block : (i + 1) * block, j * block : (j + 1) * block]
            full[i, j] = bool(tile.all())
            partial[i, j] = bool(tile.any()) and not bool(tile.all())
    return full, partial


# ---------------------------------------------------------------------------------------------
# memory bank gather (memory_retrieval.py:79-86): concatenate bank frames at arbitrary indices
# ---------------------------------------------------------------------------------------------
def memory_gather(bank: torch.Tensor, indices: Sequence[int], frame_seqlen: int) -> torch.Tensor:
    """``bank`` [B, n_frames*T, H, D] → cat of frames ``indices`` along tokens."""
    if not len(indices):
        return bank[:, :0]
    return torch.cat(
        [bank[:, int(i) * frame_seqlen : (int(i) + 1) * frame_seqlen] for i in indices], dim=1
    )


# ---------------------------------------------------------------------------------------------
# fp8 e4m3fn quantisation with one scale per (frame, head): scale = absmax / 448
# ---------------------------------------------------------------------------------------------
def fp8_quantize(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantise one frame of one head per leading index.

    ``x`` [..., T, D] (bf16 or fp32) → (codes float8_e4m3fn [..., T, D], scale float32 [...]).
    inv = 448 / absmax in fp32, y = clamp(x * inv, ±448) in fp32, code = RNE(y); absmax 0 → all
    codes 0 and scale 0.
    """
    xf = x.float()
    amax = xf.abs().amax(dim=(-2, -1))
    inv = torch.where(amax > 0, torch.tensor(E4M3_MAX, dtype=torch.float32) / amax,
                      torch.zeros_like(amax))
    y = (xf * inv[..., None, None]).clamp(-E4M3_MAX, E4M3_MAX)
    codes = y.to(torch.float8_e4m3fn)
    scale = amax / torch.tensor(E4M3_MAX, dtype=torch.float32)
    return codes, scale


def fp8_dequantize(codes: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    return codes.float() * scale[..., None, None]


def fp8_fake_quant_frames(x: torch.Tensor, frame_seqlen: int) -> torch.Tensor:
    """Token-major [B, n*T, H, D] -> the values an fp8 frame cache holds: each (frame, stream,
    head) block quantised with its own absmax/448 scale and decoded again (float32)."""
    B, L, H, D = x.shape
    n = L // frame_seqlen
    fr = x.reshape(B, n, frame_seqlen, H, D).permute(1, 0, 3, 2, 4)  # [n, B, H, T, D]
    codes, scale = fp8_quantize(fr)
    deq = fp8_dequantize(codes, scale)
    return deq.permute(1, 0, 3, 2, 4).reshape(B, L, H, D)


def fp8_fake_quant_rows(q: torch.Tensor) -> torch.Tensor:
    """Per-row (last dim) fp8 quantisation of bf16-rounded q with absmax/448 scales, decoded."""
    qf = q.to(torch.bfloat16).float()
    codes, scale = fp8_quantize(qf.unsqueeze(-2))
    return fp8_dequantize(codes, scale).squeeze(-2)


def fp8_rope_copy_effective(k: torch.Tensor, grid_hw: tuple[int, int], freqs: torch.Tensor,
                            frame_seqlen: int) -> torch.Tensor:
    """Raw K [B, n*T, H, D] -> the raw K a pre-RoPE fp8 cache effectively attends with (float64).

    The cache keeps a copy of K with its height/width pairs rotated (temporal pairs raw), the
    value a bf16 copy holds, quantised per (frame, stream, head) with its own absmax/448; the
    attention reads that copy.  Rotating the decoded copy back (the conjugate table at temporal
    position 0) gives the K whose window RoPE (``cached_self_attention(rope=...)``) reproduces
    the decoded copy exactly, so the oracle's own RoPE path runs on the quantised values.  Not
    a reference function: the reference has no fp8 cache (BASELINE config 5 defines the scales).
    """
    zero = [0] * (k.shape[1] // frame_seqlen)
    deq = fp8_rope_copy_decoded(k, grid_hw, freqs, frame_seqlen).double()
    return rope_frames(deq, grid_hw, zero, freqs.conj())


def fp8_rope_copy_decoded(k: torch.Tensor, grid_hw: tuple[int, int], freqs: torch.Tensor,
                          frame_seqlen: int) -> torch.Tensor:
    """Raw K [B, n*T, H, D] -> the decoded fp8 RoPE copy a pre-RoPE fp8 cache attends with
    (float32): height/width pairs rotated in float64 and rounded to bf16 (the bf16 copy, temporal
    pairs raw), then quantised per (frame, stream, head) with its own absmax/448 and decoded."""
    zero = [0] * (k.shape[1] // frame_seqlen)
    copy = rope_frames(k.double(), grid_hw, zero, freqs).to(torch.bfloat16)
    return fp8_fake_quant_frames(copy.float(), frame_seqlen)


def _inv_freq_f64(dim: int, theta: float) -> torch.Tensor:
    return 1.0 / torch.pow(torch.tensor(theta, dtype=torch.float64),
                           torch.arange(0, dim, 2, dtype=torch.float64) / dim)


def fp8_rope_query_frames(q: torch.Tensor, grid_hw: tuple[int, int], q_positions: Sequence[int],
                          k_positions: Sequence[int], frame_seqlen: int,
                          theta: float = 10000.0) -> torch.Tensor:
    """The e4m3 query the fp8 RoPE-on-load attention multiplies key frame j with, decoded:
    float32 [n_k, B, Lq, H, D] for q [B, n_q*T, H, D] whose frame f sits at ``q_positions[f]``.

    Not a reference function (the reference has no fp8 cache; BASELINE config 5 defines the
    scales): it states the quantisation contract of this repository's kernel so that a test can
    reproduce its codes exactly.  Every product and sum is an IEEE float32 operation rounded on
    its own; tables are float32 cos / sin of float64 angles:
    * q rounded to bf16; the height/width pairs (22..42, 43..63) turned by the token's own h / w
      (angle h·w_j, w·w_j with w_j = theta^(-2j/42)): u' = bf16(u c - v s), v' = bf16(u s + v c);
    * row bound = max(|u'|, |v'| over those pairs, sqrt(u u + v v) over the temporal pairs
      0..21), inv = 448 / bound (0 for an all-zero row), scale = bound / 448 — a bound no
      rotation of a temporal pair can exceed;
    * per key frame j: the temporal pairs turned by the angle (p_q - p_k[j])·w_i with w_i =
      theta^(-2i/44), rounded to bf16; code = RNE_e4m3(clamp(x · inv, ±448)); value = code · scale.
    """
    gh, gw = grid_hw
    B, L, H, D = q.shape
    T = frame_seqlen
    if L != len(q_positions) * T or T != gh * gw:
        raise ValueError("fp8_rope_query_frames: q needs len(q_positions) frames of gh*gw tokens")
    ct, ch, cw = rope_split(D)
    x = q.to(torch.bfloat16).float().reshape(B, L, H, D // 2, 2)
    u, v = x[..., 0], x[..., 1]
    tok = torch.arange(L) % T
    inv_s = _inv_freq_f64(2 * ch, theta)
    ang_s = torch.cat([(tok // gw).double()[:, None] * inv_s, (tok % gw).double()[:, None] * inv_s], 1)
    c, s = torch.cos(ang_s).float()[None, :, None, :], torch.sin(ang_s).float()[None, :, None, :]
    us, vs = u[..., ct:], v[..., ct:]
    u2 = (us * c - vs * s).to(torch.bfloat16).float()
    v2 = (us * s + vs * c).to(torch.bfloat16).float()
    ut, vt = u[..., :ct], v[..., :ct]
    bound = torch.maximum(torch.maximum(u2.abs(), v2.abs()).amax(-1),
                          torch.sqrt(ut * ut + vt * vt).amax(-1))
    e4 = torch.tensor(E4M3_MAX, dtype=torch.float32)
    inv = torch.where(bound > 0, e4 / bound, torch.zeros_like(bound))[..., None]
    scale = (bound / e4)[..., None]
    inv_t = _inv_freq_f64(2 * ct, theta)
    pq = torch.tensor(list(q_positions), dtype=torch.float64)[torch.arange(L) // T]
    out = []
    for pk in k_positions:
        ang = (pq - float(pk))[:, None] * inv_t
        c, s = torch.cos(ang).float()[None, :, None, :], torch.sin(ang).float()[None, :, None, :]
        u3 = (ut * c - vt * s).to(torch.bfloat16).float()
        v3 = (ut * s + vt * c).to(torch.bfloat16).float()
        y = torch.stack([torch.cat([u3, u2], -1), torch.cat([v3, v2], -1)], -1).reshape(B, L, H, D)
        codes = (y * inv).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
        out.append(codes.float() * scale)
    return torch.stack(out)


def fp8_rope_attention(q: torch.Tensor, k_copy: torch.Tensor, v: torch.Tensor,
                       grid_hw: tuple[int, int], q_positions: Sequence[int],
                       k_positions: Sequence[int], frame_seqlen: int, theta: float = 10000.0,
                       softmax_scale: float | None = None) -> torch.Tensor:
    """Attention of the fp8 RoPE-on-load path with its quantised queries, float64 softmax.

    ``k_copy`` [B, n_k*T, H, D]: the keys as the cache's RoPE copy holds them (height/width
    pairs rotated, temporal pairs raw; ``fp8_rope_copy_decoded``); key frame j sits at
    ``k_positions[j]``.  Logits of key frame j are ``fp8_rope_query_frames(...)[j] · k_copy_j``
    (the temporal turn by p_q - p_k on the query equals RoPE at p_q on q and p_k on k); softmax
    over every key in float64, times ``v``.  Returns float64 [B, Lq, H, D].
    """
    B, L, H, D = q.shape
    T, nk = frame_seqlen, len(k_positions)
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(D)
    qd = fp8_rope_query_frames(q, grid_hw, q_positions, k_positions, T, theta).double()
    kc = k_copy.double().reshape(B, nk, T, H, D)
    logits = torch.einsum("jblhd,bjthd->bhljt", qd, kc).reshape(B, H, L, nk * T) * scale
    p = torch.softmax(logits, dim=-1)
    return torch.einsum("bhlk,bkhd->blhd", p, v.double())


def e4m3_decode(code: int) -> float:
    """Value of an e4m3fn byte from its fields (bias 7; e=0 subnormal; 0x7f/0xff NaN)."""
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 0x7
    if e == 0xF and m == 0x7:
        return float("nan")
    if e == 0:
        return s * m * 2.0**-9
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)


# ---------------------------------------------------------------------------------------------
# RoPE for the cached path: table (model.py:28-35), Wan's temporal/height/width split
# (causal_model.py:1855-1866), the per-frame rotation of echorope_apply (causal_model.py:88-197;
# block_relativistic_rope :200-218 is the same transform), and the position allocation of the
# cache branch (_window_relative_positions :656-701, _echorope_pmax_frames :703-716,
# _rope_q_and_window_k :718-789, _rope_sink_local_and_query :791-876).
# ---------------------------------------------------------------------------------------------
def rope_params(max_seq_len: int, dim: int, theta: float = 10000.0) -> torch.Tensor:
    """complex128 [max_seq_len, dim/2]: exp(i * p * theta^(-2j/dim))."""
    assert dim % 2 == 0
    inv = 1.0 / torch.pow(torch.tensor(theta, dtype=torch.float64),
                          torch.arange(0, dim, 2, dtype=torch.float64) / dim)
    ang = torch.outer(torch.arange(max_seq_len, dtype=torch.float64), inv)
    return torch.polar(torch.ones_like(ang), ang)


def rope_split(head_dim: int) -> tuple[int, int, int]:
    """(temporal, height, width) complex pairs of a head: c - 2(c//3), c//3, c//3 with c = D/2."""
    c = head_dim // 2
    return c - 2 * (c // 3), c // 3, c // 3


def wan_rope_freqs(head_dim: int = 128, max_seq_len: int = 1024) -> torch.Tensor:
    """The model's table: [max_seq_len, D/2] complex, temporal | height | width parts."""
    d = head_dim
    return torch.cat([rope_params(max_seq_len, d - 4 * (d // 6)),
                      rope_params(max_seq_len, 2 * (d // 6)),
                      rope_params(max_seq_len, 2 * (d // 6))], dim=1)


def rope_frames(x: torch.Tensor, grid_hw: tuple[int, int], temporal_pos: Sequence[int],
                freqs: torch.Tensor) -> torch.Tensor:
    """Rotate ``x`` [B, F*H*W, heads, D] whose frame f sits at temporal position
    ``temporal_pos[f]`` and whose tokens are ordered (h, w) inside a frame; complex pairs
    (x[2i], x[2i+1]) are multiplied by the table entries in float64 and the result is cast back
    to x's dtype (echorope_apply with frame_indices)."""
    gh, gw = grid_hw
    B, L, n, D = x.shape
    F = len(temporal_pos)
    if L != F * gh * gw:
        raise ValueError(f"rope_frames: {L} tokens != {F} frames x {gh}x{gw}")
    ct, ch, cw = rope_split(D)
    ft, fh, fw = freqs.split([ct, ch, cw], dim=1)
    pos = torch.as_tensor(list(temporal_pos), dtype=torch.long)
    if F and (int(pos.min()) < 0 or int(pos.max()) >= ft.shape[0]):
        raise ValueError(f"temporal positions {list(temporal_pos)} outside the table")
    f_all = torch.cat([ft[pos].view(F, 1, 1, ct).expand(F, gh, gw, ct),
                       fh[:gh].view(1, gh, 1, ch).expand(F, gh, gw, ch),
                       fw[:gw].view(1, 1, gw, cw).expand(F, gh, gw, cw)], dim=-1).reshape(L, 1, -1)
    xc = torch.view_as_complex(x.to(torch.float64).reshape(B, L, n, D // 2, 2))
    return torch.view_as_real(xc * f_all).reshape(B, L, n, D).to(x.dtype)


def window_relative_positions(*, current_start_frame: int, num_new_frames: int,
                              num_context_frames: int, pmax: int) -> tuple[int, int]:
    """(q_start, local_start) of _window_relative_positions (query memory unused on this
    path): the query block ends at min(current_start + B - 1, pmax - 1) and the context ends
    with it."""
    q_last = min(current_start_frame + num_new_frames - 1, pmax - 1)
    q_start = q_last - num_new_frames + 1
    local_start = q_last - num_context_frames + 1 if num_context_frames > 0 else q_last
    return q_start, local_start


def echorope_pmax_frames(*, max_attention_size: int, frame_seqlen: int, table_len: int,
                         min_frames: int) -> int:
    return min(max(1, int(min_frames), int(max_attention_size // max(1, frame_seqlen))), table_len)


def rope_positions(*, num_sink_frames: int, num_local_frames: int, num_new_frames: int,
                   use_echorope: bool, max_attention_size: int, frame_seqlen: int,
                   table_len: int = 1024, rope_train_frames: int | None = None,
                   current_start_frame: int = 0, sink_branch: bool = True) -> dict[str, int]:
    """Temporal positions of the visible window and the query chunk.

    ``sink_branch`` selects _rope_sink_local_and_query (a sink is configured: sink frames at
    0..ns-1, then the local frames) or _rope_q_and_window_k (no sink: one window).  Returns
    ``{"q_start", "local_start", "num_sink"}``; the key positions of the window in ``cat``
    order are ``range(num_sink) + range(local_start, local_start + num_local)``.
    """
    nb, nl = num_new_frames, num_local_frames
    ns = num_sink_frames if sink_branch else 0
    pmax = echorope_pmax_frames(max_attention_size=max_attention_size, frame_seqlen=frame_seqlen,
                                table_len=table_len, min_frames=nb)
    if use_echorope:
        q_start, local_start = window_relative_positions(
            current_start_frame=max(0, ns + nl - nb), num_new_frames=nb,
            num_context_frames=nl, pmax=pmax)
    elif sink_branch:
        if rope_train_frames is None:
            q_last = ns + nl - 1
        else:
            q_last = min(current_start_frame + nb - 1, rope_train_frames - 1)
        q_start = q_last - nb + 1
        local_start = q_last - nl + 1 if nl > 0 else max(ns, q_start)
    else:
        q_start, local_start = nl - nb, 0
    if q_start < 0 or local_start < 0:
        if sink_branch:  # the reference's two checks word for word (causal_model.py:859, :766)
            raise ValueError(
                f"EchoRoPE underflow while assigning sink/local positions: B={nb}, R={nl}, "
                f"sink={ns}, q_start={q_start}, local_start={local_start}, pmax={pmax}")
        raise ValueError(
            f"EchoRoPE underflow while assigning window-relative positions: B={nb}, R={nl}, "
            f"q_start={q_start}, local_start={local_start}, pmax={pmax}")
    return {"q_start": q_start, "local_start": local_start, "num_sink": ns}


# ---------------------------------------------------------------------------------------------
# q/k RMSNorm before the cache (causal_model.py:908-910; WanRMSNorm model.py:69-84) and the
# cached cross-attention (WanCrossAttention.forward model.py:152-184)
# ---------------------------------------------------------------------------------------------
def wan_rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """WanRMSNorm as the reference evaluates it: ``x * rsqrt(mean(x²) + eps)`` in x's own dtype,
    then ``.type_as(x) * weight``, over the last dimension (the token's H*D channels)."""
    return (x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps)).type_as(x) * weight


def rms_norm_f64(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """The same normalisation evaluated in float64."""
    xd = x.to(torch.float64)
    return xd * torch.rsqrt(xd.pow(2).mean(dim=-1, keepdim=True) + eps) * weight.to(torch.float64)


def norm_heads(x: torch.Tensor, weight: torch.Tensor, eps: float, fn=rms_norm_f64) -> torch.Tensor:
    """Apply a row norm to [B, L, H, D] over the flattened H*D channels (the reference normalises
    the projection output [B, L, C] before ``.view(b, s, n, d)``)."""
    b, l, h, d = x.shape
    return fn(x.reshape(b, l, h * d), weight, eps).reshape(b, l, h, d)


def cross_attention(q_proj: torch.Tensor, ctx_k_proj: torch.Tensor, ctx_v_proj: torch.Tensor,
                    crossattn_cache: dict[str, Any] | None, *, norm_q: Callable, norm_k: Callable,
                    attn_fn: Callable[..., torch.Tensor] = attention) -> torch.Tensor:
    """WanCrossAttention.forward after the projections (model.py:152-184), context_lens None as
    on the cached inference path (causal_model.py:2730): q = norm_q(q(x)); K/V of the context
    are computed once into the cache (``is_init``) and reused; returns the attention output
    [B, L1, H, D] (before ``flatten`` and ``self.o``).  Inputs are [B, L, H, D]."""
    q = norm_q(q_proj)
    if crossattn_cache is not None:
        if not crossattn_cache["is_init"]:
            crossattn_cache["is_init"] = True
            crossattn_cache["k"] = norm_k(ctx_k_proj)
            crossattn_cache["v"] = ctx_v_proj
        k, v = crossattn_cache["k"], crossattn_cache["v"]
    else:
        k, v = norm_k(ctx_k_proj), ctx_v_proj
    return attn_fn(q, k, v)
