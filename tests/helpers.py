"""Shared assertions for the GPU parity tests."""

import torch

# Bars for bf16 attention (fp32 accumulation) against the float64 oracle.
MAX_ABS, MEAN_ABS = 2e-2, 1e-3
# Bar for attention over an fp8-e4m3 cache against the bf16-cache oracle.
FP8_MAX_ABS, FP8_MEAN_ABS = 3e-2, 3e-3


def assert_attn_close(got, want, max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    got = got.detach().cpu()
    assert torch.isfinite(got).all(), "non-finite attention output"
    err = (got.double() - want.double()).abs()
    assert float(err.max()) <= max_abs, f"max-abs error {float(err.max()):.3e} > {max_abs}"
    assert float(err.mean()) <= mean_abs, f"mean-abs error {float(err.mean()):.3e} > {mean_abs}"
