"""Host slot-table algebra (solarwm_amd.cache.SlotTable) against the oracle's dense cache.

A CPU dict stands in for the device pool (slot -> one frame of token labels), written exactly
where the append kernel would write.  After every pass the frames attention would read, and
after every commit the whole logical cache (all positions, stale ones included), must equal the
oracle's clone/memmove/slice-assign result bit for bit.
"""

import pytest
import torch

from oracle import wan_cache_ref as ref
from solarwm_amd.cache import CacheGeometry, SlotTable, plan_cached_forward


def _labels(start, n):
    return torch.arange(start, start + n, dtype=torch.float64).view(1, n, 1, 1)


class _Rec:
    def __call__(self, q, k, v):
        self.k = k.clone()
        return torch.zeros_like(q)


def _sim(geom, schedule, bank=None):
    """schedule: list of (current_start, n_tokens, policy, label_base).  Returns nothing;
    asserts equality at every step."""
    T = geom.frame_tokens
    cache = ref.allocate_kv_cache(1, 1, geom.cache_tokens, 1, 1, torch.float64)
    tab = SlotTable(geom)
    pool = {s: torch.zeros(T, dtype=torch.float64) for s in range(geom.n_slots)}
    if bank is not None:
        for i, frame in enumerate(bank):
            pool[geom.bank_slot0 + i] = frame.clone()
    for step, (start, n, policy, base, mem) in enumerate(schedule):
        newk = _labels(base, n)
        rec = _Rec()
        mem_k = None
        if mem:
            mem_k = torch.cat([bank[i] for i in mem]).view(1, -1, 1, 1)
        _, (cur_end, le, info) = ref.cached_self_attention(
            newk, newk, newk, cache[0], current_start=start, frame_seqlen=T,
            sink_size=geom.sink_frames,
            local_attn_size=geom.capacity_frames if geom.local_attn_size is None else geom.local_attn_size,
            attn_fn=rec, memory_k=mem_k, memory_v=mem_k,
        )
        plan, temp, staging, window = tab.plan(start, n)
        assert (plan.current_end, plan.local_end_index) == (cur_end, le)
        for key in ("action", "local_start_index", "local_end_index", "write_start_index",
                    "write_end_index", "is_recompute", "current_end"):
            assert info[key] == {
                "action": plan.action,
                "local_start_index": plan.local_start_index,
                "local_end_index": plan.local_end_index,
                "write_start_index": plan.write_start_index,
                "write_end_index": plan.local_end_index,
                "is_recompute": plan.is_recompute,
                "current_end": plan.current_end,
            }[key], key
        # append kernel: written frames go to staging slots
        ro = plan.roped_offset // T
        for i, s in enumerate(staging):
            pool[s] = newk[0, (ro + i) * T : (ro + i + 1) * T, 0, 0].clone()
        frames = (tab.bank_slots(mem) if mem else []) + window
        seen = torch.cat([pool[s] for s in frames]) if frames else torch.zeros(0)
        assert torch.equal(seen, rec.k[0, :, 0, 0]), f"step {step}: attention window differs"
        upd = tab.stage(plan, temp)
        if policy != "none":
            ref.apply_cache_updates(cache, [(0, (cur_end, le, info))])
            tab.commit(upd, cur_end, le)
        assert tab.global_end == int(cache[0]["global_end_index"].item())
        assert tab.local_end == int(cache[0]["local_end_index"].item())
        logical = torch.cat([pool[s] for s in tab.table])
        assert torch.equal(logical, cache[0]["k"][0, :, 0, 0]), f"step {step}: cache differs"
        # committed slots are never the staging target of a later pass
        assert len(set(tab.table) & set(tab.free_slots())) == 0


def _chunks(n_chunks, chunk_tokens, passes):
    out = []
    for c in range(n_chunks):
        for p, policy in enumerate(passes):
            out.append((c * chunk_tokens, chunk_tokens, policy, 100_000 * (1 + p) + c * chunk_tokens, None))
    return out


@pytest.mark.parametrize(
    "T,chunk_f,cap_f,sink_f",
    [(390, 3, 21, 1), (4, 3, 6, 0), (2, 1, 5, 2), (3, 2, 7, 1), (5, 4, 9, 3), (2, 3, 3, 0),
     (2, 1, 1, 0), (3, 2, 8, 0), (3, 3, 21, 1)],
)
def test_rollout_matches_oracle(T, chunk_f, cap_f, sink_f):
    geom = CacheGeometry(batch=1, heads=1, head_dim=128, frame_tokens=T, capacity_frames=cap_f,
                         sink_frames=sink_f, staging_frames=chunk_f)
    _sim(geom, _chunks(10, chunk_f * T, ["none", "none", "commit"]))


def test_reference_nfe4_pattern_and_recompute():
    T, chunk_f, cap_f, sink_f = 3, 3, 10, 1
    geom = CacheGeometry(batch=1, heads=1, head_dim=128, frame_tokens=T, capacity_frames=cap_f,
                         sink_frames=sink_f, staging_frames=chunk_f)
    Lq = chunk_f * T
    sched = _chunks(6, Lq, ["none"] * 4 + ["commit"])
    # recompute the last committed chunk twice (none, then commit), then continue
    sched += [(5 * Lq, Lq, "none", 900_000, None), (5 * Lq, Lq, "commit", 910_000, None)]
    sched += [(6 * Lq, Lq, "none", 920_000, None), (6 * Lq, Lq, "commit", 930_000, None)]
    _sim(geom, sched)


def test_memory_frames_ahead_of_window():
    T = 4
    geom = CacheGeometry(batch=1, heads=1, head_dim=128, frame_tokens=T, capacity_frames=7,
                         sink_frames=1, staging_frames=3, bank_frames=12)
    bank = [torch.full((T,), -1000.0 - i, dtype=torch.float64) for i in range(12)]
    g = torch.Generator().manual_seed(0)
    sched = []
    for c in range(6):
        mem = torch.randperm(12, generator=g)[:4].tolist()
        for p, pol in enumerate(["none", "commit"]):
            sched.append((c * 3 * T, 3 * T, pol, 50_000 * (p + 1) + c * 3 * T, mem))
    _sim(geom, sched, bank=bank)


def test_stale_update_and_bad_sizes_raise():
    geom = CacheGeometry(batch=1, heads=1, head_dim=128, frame_tokens=4, capacity_frames=6,
                         sink_frames=1, staging_frames=3)
    tab = SlotTable(geom)
    p1, t1, _, _ = tab.plan(0, 12)
    u1 = tab.stage(p1, t1)
    p2, t2, _, _ = tab.plan(0, 12)
    tab.stage(p2, t2)
    with pytest.raises(RuntimeError, match="stale"):
        tab.commit(u1, p1.current_end, p1.local_end_index)
    with pytest.raises(ValueError, match="whole number"):
        tab.plan(0, 10)
    with pytest.raises(ValueError, match="staging"):
        tab.plan(0, 16)
    with pytest.raises(IndexError):
        tab.bank_slots([0])


def test_plan_unbounded_window_is_direct_insert():
    geom = CacheGeometry(batch=1, heads=1, head_dim=128, frame_tokens=10, capacity_frames=50,
                         local_attn_size=-1, staging_frames=3)
    p = plan_cached_forward(geom, 0, 0, 0, 30)
    assert p.action == "direct_insert" and geom.max_attention_size == 39600


def test_bench_eviction_leg_counts_the_reference_bytes():
    """bench.py's eviction leg: the reference's clone + memmove per layer and pass at C2
    (causal_model.py:1054-1067) is 402.6 MB + 325.9 MB, and the slot table moves none."""
    import bench

    r = bench.eviction_latency(bench.CONFIGS["c2"], iters=50)
    # clone: K and V of the 21-frame cache, read + write; memmove: the 17 rolled frames
    assert r["reference_clone_bytes"] == 2 * 2 * 21 * 1560 * 12 * 128 * 2 == 402554880
    assert r["reference_memmove_bytes"] == 2 * 2 * 17 * 1560 * 12 * 128 * 2 == 325877760
    assert r["device_bytes"] == 0 and r["host_us_per_layer_pass"] > 0
