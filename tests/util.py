"""Shared helpers for the parity tests: seeded inputs (torch CPU generator, fp32, then cast -- the same tensors the
benchmark uses) and the bf16 tolerance of the layer's contract."""
from __future__ import annotations

import numpy as np
import torch

# Tolerance for bf16 outputs and gradients (fp32 accumulation on the GPU), with b the float64 oracle rounded once to
# the output's dtype (bf16) -- the best value a bf16 result can hold:
#   max relative error  = max|a - b| / max|b|   <= 2e-2
#   mean relative error = mean|a - b| / mean|b| <= 2e-3
MAX_REL = 2e-2
MEAN_REL = 2e-3


def rel_errors(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    diff = np.abs(a - b)
    return diff.max() / max(np.abs(b).max(), 1e-30), diff.mean() / max(np.abs(b).mean(), 1e-30)


def assert_close_bf16(a, b, name="", max_rel=MAX_REL, mean_rel=MEAN_REL):
    mx, mn = rel_errors(a, b)
    assert mx <= max_rel and mn <= mean_rel, f"{name}: max rel {mx:.3e} (<= {max_rel}), mean rel {mn:.3e} (<= {mean_rel})"
    return mx, mn


def make_inputs(T, d, E, h, seed=0, dtype=torch.bfloat16, w_std=0.02):
    """x ~ N(0,1) (T, d); router (E, d), wgu (E, d, 2h), wd (E, h, d) ~ N(0, w_std); generated in fp32 on CPU."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, d, generator=g).to(dtype)
    wr = (torch.randn(E, d, generator=g) * w_std).to(dtype)
    wgu = (torch.randn(E, d, 2 * h, generator=g) * w_std).to(dtype)
    wd = (torch.randn(E, h, d, generator=g) * w_std).to(dtype)
    return x, wr, wgu, wd


def f32(t):
    return t.detach().float().cpu().numpy()


def bits(t):
    """bf16 tensor -> uint16 bit patterns (numpy)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
