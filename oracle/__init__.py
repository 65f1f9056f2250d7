"""CPU oracle for the block-causal KV-cache path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference PyTorch algorithm the HIP kernels replace.
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and only as the checker / the timed CPU baseline — never as a product code path.

Pinning status of each function (how a plausible mistake would be caught) is listed in the
module docstring of :mod:`oracle.wan_cache_ref`.
"""
