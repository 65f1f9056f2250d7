"""Host-side contract of the drop-in cache and the rollout driver (no GPU).

* The injected allocator passes the reference drivers' contract check right after allocation
  (stage2.py:466-469, :671-672 require ``"_fused_prope_camera_metadata"`` on layer 0, which the
  reference allocator preallocates, stage2.py:1799-1816).
* The NFE4 sampler (``driver.self_forcing_latents``) reproduces the call pattern the reference's
  own test pins for ``_stage2_self_forcing_latents``
  (tests/backends/wan22/test_stage2_runtime.py:141-221), with the slot-cache allocator injected.
* Writes through the dict surface (``.fill_`` of the indices, causal_model.py:2916-2921;
  ``cache[key] = ...``, :2011; ``pop``, :2841; ``.copy_`` of the camera rows, :2068-2075) raise
  instead of being lost.
* ``cached_forward`` commits all blocks only after every block ran and only for a committing
  policy (causal_model.py:2819-2844).
"""

from types import SimpleNamespace

import pytest
import torch

from solarwm_amd import driver, make_kv_cache_allocator
from solarwm_amd._readonly import CacheWriteError

META = "_fused_prope_camera_metadata"


def _alloc(layers=2, T=2, cap=6, sink=0, chunk=3, **kw):
    return make_kv_cache_allocator(num_layers=layers, num_heads=1, head_dim=128,
                                   frame_sequence_length=T, local_attn_size=cap, sink_size=sink,
                                   num_frame_per_block=chunk, **kw)


def test_allocator_preallocates_camera_metadata_on_layer0():
    caches = _alloc(layers=3, T=4, cap=5)(2, dtype=torch.bfloat16, device="cpu")
    assert META in caches[0] and all(META not in c for c in caches[1:])
    meta = caches[0][META]
    assert set(meta) == {"viewmats", "K"}
    assert tuple(meta["viewmats"].shape) == (2, 20, 4, 4) and meta["viewmats"].dtype == torch.float32
    assert tuple(meta["K"].shape) == (2, 20, 3, 3) and meta["K"].dtype == torch.float32
    assert not meta["viewmats"].any() and not meta["K"].any()
    assert len(caches[0]) == 5 and len(caches[1]) == 4
    assert list(caches[0]) == ["k", "v", "global_end_index", "local_end_index", META]


class _Scheduler:
    def add_noise(self, clean, noise, timestep):
        del noise, timestep
        return clean


class _Student:
    """Records every call like the reference test's fake student, and reads the cache the way
    the reference model does before attending (indices, camera metadata)."""

    def __init__(self):
        self.scheduler = _Scheduler()
        self.calls = []

    def __call__(self, noisy, condition, camera, timestep, **kwargs):
        del condition
        cache = kwargs["kv_cache"]
        ends = (int(cache[0]["global_end_index"]), int(cache[0]["local_end_index"]))
        self.calls.append({"grad": torch.is_grad_enabled(), "camera_tokens": camera["K"].shape[1],
                           "timestep": timestep.clone(), "ends": ends, **kwargs})
        return torch.full_like(noisy, 0.25)

    @staticmethod
    def flow_to_x0(noisy, flow, timestep):
        sigma = timestep.float()
        while sigma.ndim < noisy.ndim:
            sigma = sigma.unsqueeze(-1)
        return noisy.float() - sigma * flow.float() / 1000.0


def _generation_pass(frames=6):
    return SimpleNamespace(solver="self_forcing", num_inference_steps=4,
                           rollout_latent_frames=frames)


def _provider(student, kv_alloc, allocations, noise_shapes):
    def kv_cache(batch_size, *, dtype, device):
        allocations["kv"] += 1
        return kv_alloc(batch_size, dtype=dtype, device=device)

    def cross_cache(batch_size, *, dtype, device):
        allocations["cross"] += 1
        return [{"k": torch.zeros(batch_size, 1), "v": torch.zeros(batch_size, 1), "is_init": False}]

    def noise(shape, generator):
        del generator
        shape = tuple(int(s) for s in shape)
        noise_shapes.append(shape)
        return torch.ones(shape, dtype=torch.bfloat16)

    return SimpleNamespace(
        config={"model": {"num_frame_per_block": 3, "latent_channels": 1,
                          "frame_sequence_length": 2},
                "data": {"latent_shape": [6, 1, 1, 1]}, "train": {"num_train_timesteps": 1000}},
        device=torch.device("cpu"), diffusion=student,
        denoising_steps=tuple(torch.tensor(v, dtype=torch.float32) for v in (1000, 750, 500, 250)),
        allocate_kv_cache=kv_cache, allocate_crossattn_cache=cross_cache, _noise=noise)


def test_sampler_call_pattern_with_injected_slot_cache():
    """test_stage2_runtime.py:141-221 with the slot-cache allocator injected."""
    student = _Student()
    allocations = {"kv": 0, "cross": 0}
    noise_shapes = []
    provider = _provider(student, _alloc(), allocations, noise_shapes)
    first = torch.full((1, 1, 1, 1, 1), 9.0, dtype=torch.bfloat16)
    camera = {"viewmats": torch.eye(4).repeat(1, 12, 1, 1), "K": torch.eye(3).repeat(1, 12, 1, 1)}
    latents, schedule = driver.self_forcing_latents(
        provider, _generation_pass(), first, {"prompt_embeds": torch.zeros((1, 1, 1))}, camera,
        torch.Generator())

    assert latents.shape == (1, 6, 1, 1, 1)
    assert torch.equal(latents[:, :1], first)
    assert allocations == {"kv": 1, "cross": 1}
    policies = [c["cache_update_policy"] for c in student.calls]
    assert len(student.calls) == 10
    assert policies.count("none") == 8 and policies.count("commit_detached") == 2
    assert policies == (["none"] * 4 + ["commit_detached"]) * 2
    assert [c["current_start"] for c in student.calls] == [0] * 5 + [6] * 5
    assert all(c["cache_start"] == 0 and c["sequence_length"] == 6 for c in student.calls)
    assert all(c["timestep"].dtype == torch.bfloat16 for c in student.calls)
    assert torch.unique(student.calls[1]["timestep"]).tolist() == [0.0, 752.0]
    assert torch.unique(student.calls[6]["timestep"]).tolist() == [752.0]
    assert torch.unique(student.calls[4]["timestep"]).tolist() == [0.0]  # commit at t = 0
    assert all(c["camera_tokens"] == 6 for c in student.calls)
    assert [c["grad"] for c in student.calls] == [True] * 4 + [False] + [True] * 4 + [False]
    assert schedule["timesteps"] == [1000.0, 750.0, 500.0, 250.0]
    assert schedule["persistent_kv_cache"] is True
    assert noise_shapes == [(1, 6, 1, 1, 1)] + [(1, 3, 1, 1, 1)] * 6
    # one persistent cache object across all calls
    assert len({id(c["kv_cache"]) for c in student.calls}) == 1


def test_sampler_rejects_cache_without_camera_metadata():
    student = _Student()
    alloc = _alloc()

    def popped(batch_size, *, dtype, device):
        caches = alloc(batch_size, dtype=dtype, device=device)
        caches[0].pop(META)
        return caches

    provider = _provider(student, popped, {"kv": 0, "cross": 0}, [])
    camera = {"viewmats": torch.eye(4).repeat(1, 12, 1, 1), "K": torch.eye(3).repeat(1, 12, 1, 1)}
    with pytest.raises(driver.BackendContractError, match="preallocated fused camera metadata"):
        driver.self_forcing_latents(provider, _generation_pass(), torch.zeros(1, 1, 1, 1, 1),
                                    {}, camera, None)
    assert student.calls == []


def test_sampler_contract_errors():
    provider = _provider(_Student(), _alloc(), {"kv": 0, "cross": 0}, [])
    with pytest.raises(driver.BackendContractError, match="NFE4"):
        driver.self_forcing_latents(provider, SimpleNamespace(solver="euler", num_inference_steps=4,
                                                              rollout_latent_frames=6),
                                    torch.zeros(1, 1, 1, 1, 1), {}, {}, None)
    with pytest.raises(driver.BackendContractError, match="three-latent chunks"):
        driver.self_forcing_latents(provider, _generation_pass(7), torch.zeros(1, 1, 1, 1, 1),
                                    {}, {}, None)


def test_warped_steps_follow_the_scheduler_table():
    table = torch.linspace(999.0, 0.0, 1000)
    steps = driver._warped_steps([1000, 750, 500, 250, 0], table, 1000)
    assert [float(s) for s in steps] == [float(table[0]), float(table[250]), float(table[500]),
                                         float(table[750])]
    with pytest.raises(ValueError, match="integers"):
        driver._warped_steps([10.5], table, 1000)


def test_rollout_passes_order():
    passes = driver.rollout_passes(9, 3, 1560, 4)
    assert len(passes) == 15
    assert [p.policy for p in passes] == (["none"] * 4 + ["commit_detached"]) * 3
    assert [p.current_start for p in passes] == [0] * 5 + [4680] * 5 + [9360] * 5
    assert [p.step_index for p in passes[:5]] == [0, 1, 2, 3, None]
    with pytest.raises(driver.BackendContractError):
        driver.rollout_passes(8, 3, 10, 4)


# ---------------------------------------------------------------------------------------------
# writes through the dict surface
# ---------------------------------------------------------------------------------------------
def test_index_writes_through_the_dict_raise():
    caches = _alloc()(1, dtype=torch.bfloat16, device="cpu")
    c = caches[1]
    assert int(c["global_end_index"]) == 0 and c["local_end_index"].item() == 0
    with pytest.raises(CacheWriteError, match="attend_cached"):
        c["global_end_index"].fill_(6)  # causal_model.py:2916-2921
    with pytest.raises(CacheWriteError):
        c["local_end_index"][0] = 6
    with pytest.raises(CacheWriteError):
        c["local_end_index"].copy_(torch.tensor([6]))
    with pytest.raises(CacheWriteError):
        torch.add(c["local_end_index"], 1, out=c["local_end_index"])
    scratch = c["global_end_index"].clone()  # copies are ordinary tensors
    scratch.fill_(3)
    assert int(scratch) == 3 and int(c["global_end_index"]) == 0


def test_mapping_writes_raise():
    caches = _alloc()(1, dtype=torch.bfloat16, device="cpu")
    with pytest.raises(CacheWriteError):
        caches[0][META] = {"viewmats": torch.zeros(1)}  # causal_model.py:2011
    with pytest.raises(CacheWriteError):
        caches[1]["prope_k"] = torch.zeros(1)
    with pytest.raises(CacheWriteError):
        caches[0].pop("k")
    with pytest.raises(CacheWriteError):
        del caches[0]["global_end_index"]
    with pytest.raises(CacheWriteError):
        caches[0].update({"k": torch.zeros(1)})
    assert caches[1].pop("prope_k", None) is None
    with pytest.raises(KeyError):
        caches[1]["prope_k"]


def test_camera_metadata_is_read_only_and_droppable():
    caches = _alloc()(1, dtype=torch.bfloat16, device="cpu")
    meta = caches[0][META]
    with pytest.raises(CacheWriteError):
        meta["viewmats"].copy_(torch.ones_like(meta["viewmats"]))  # causal_model.py:2068-2075
    with pytest.raises(CacheWriteError):
        meta["K"][:, 0] = torch.eye(3)
    with pytest.raises(TypeError):
        meta["viewmats"] = torch.zeros(1)
    temp = meta["viewmats"].detach().clone()  # the reference's staging copy is writable
    temp[:, 0] = torch.eye(4)
    # the reference drops stale metadata after a camera-free commit (causal_model.py:2838-2842)
    dropped = caches[0].pop(META, None)
    assert dropped is not None and META not in caches[0]
    assert caches[0].pop(META, None) is None
    assert len(caches[0]) == 4
    caches[0].reset()
    assert META in caches[0]


# ---------------------------------------------------------------------------------------------
# block loop with the deferred commit
# ---------------------------------------------------------------------------------------------
def _plan_only_block(current_start, n_tokens, fail_at=None):
    """The host half of attend_cached (plan + stage, no kernels)."""

    def block_fn(i, cache):
        if i == fail_at:
            raise RuntimeError("block failed")
        plan, temp, staging, window = cache.plan(current_start, n_tokens)
        upd = cache.stage(plan, temp)
        return window, (plan.current_end, plan.local_end_index, upd)

    return block_fn


def test_cached_forward_commits_only_committing_policies():
    caches = _alloc(layers=3, T=2, cap=6, chunk=3)(1, dtype=torch.bfloat16, device="cpu")
    tables0 = [list(c.table) for c in caches]
    driver.cached_forward(caches, _plan_only_block(0, 6), cache_update_policy="none")
    assert [list(c.table) for c in caches] == tables0
    assert all(c.global_end == 0 for c in caches)
    with pytest.raises(RuntimeError, match="block failed"):
        driver.cached_forward(caches, _plan_only_block(0, 6, fail_at=2),
                              cache_update_policy="commit_detached")
    assert [list(c.table) for c in caches] == tables0 and all(c.global_end == 0 for c in caches)
    windows = driver.cached_forward(caches, _plan_only_block(0, 6),
                                    cache_update_policy="commit_detached")
    assert all(len(w) == 3 for w in windows)
    assert all((c.global_end, c.local_end) == (6, 6) for c in caches)
    assert all(c.table[:3] == w for c, w in zip(caches, windows))


def test_cached_forward_drops_camera_metadata_on_camera_free_commit():
    caches = _alloc(layers=2, T=2, cap=6, chunk=3)(1, dtype=torch.bfloat16, device="cpu")
    driver.cached_forward(caches, _plan_only_block(0, 6), cache_update_policy="commit_detached",
                          fused_prope=True)
    assert META not in caches[0]


def test_prope_branch_cache_keys_and_writes():
    from solarwm_amd import PropeConfig

    caches = _alloc(layers=2, T=64, cap=4, chunk=2, prope_branch=PropeConfig())(
        1, dtype=torch.bfloat16, device="cpu")
    assert caches[0].branch is not None and caches[1].branch is not caches[0].branch
    for c in caches:
        assert {"prope_k", "prope_v", "prope_global_end_index", "prope_local_end_index"} <= set(c)
        assert int(c["prope_global_end_index"]) == 0 and int(c["prope_local_end_index"]) == 0
    with pytest.raises(CacheWriteError):
        caches[1]["prope_local_end_index"].fill_(3)  # causal_model.py:1512-1514
    with pytest.raises(CacheWriteError):
        caches[1].pop("prope_k")
    plain = _alloc(layers=1, T=64, cap=4, chunk=2)(1, dtype=torch.bfloat16, device="cpu")[0]
    assert "prope_k" not in plain  # the reference block runs the branch cache-free then
