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


def random_layer_configs(n=12, seed=2024):
    """The seeded random layer configurations (case, T, d, E, k, h, renorm, zipf) of the GPU layer test; a fixed
    generator, so case i is the same draw in every run and for every n > i."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        E = int(rng.integers(2, 41))
        k = int(rng.integers(1, min(E, 6) + 1))
        T = int(rng.integers(1, 701))
        d = 8 * int(rng.integers(1, 66))    # 8 .. 520
        h = 8 * int(rng.integers(1, 66))
        renorm = bool(rng.integers(0, 2))
        zipf = bool(rng.integers(0, 3) == 0) and E - 2 >= k  # the two never-routed experts leave k to pick from
        out.append((i, T, d, E, k, h, renorm, zipf))
    return out


def reference_path_errors(oracle, x, wr, wgu, wd, dout, ids, rw_ref, logits, bias=None, renorm=True, fwd=None):
    """Relative errors (max, mean) of the reference's own bf16 CPU path (oracle.cpu_path.training_step_routed: torch
    bf16 grouped GEMMs and autograd, routed onto the oracle's ids) against the float64 oracle, per tensor: out, dx,
    dwgu, dwd, dwr.  This is what the reference's arithmetic achieves on the inputs; the layer's backward contract is
    to meet the bf16 tolerance, or, where the reference's own path misses it too, to be no worse than that path."""
    from oracle import cpu_path
    xs, wrs, wgus, wds = (t.detach().cpu().clone().requires_grad_(True) for t in (x, wr, wgu, wd))
    b = None if bias is None else torch.as_tensor(bias).float()
    out = cpu_path.training_step_routed(xs, wrs, wgus, wds, torch.as_tensor(ids), dout.cpu(), bias=b, renorm=renorm)
    if fwd is None:
        fwd = oracle.moe_forward(f32(x), ids, rw_ref, f32(wgu), f32(wd))
    ref = oracle.layer_backward(f32(x), f32(wr), ids, rw_ref, logits, f32(wgu), f32(wd), f32(dout), renorm=renorm,
                                fwd=fwd)
    R = oracle.round_bf16
    return {"out": rel_errors(f32(out), fwd["out"]), "dx": rel_errors(f32(xs.grad), R(ref["dx"])),
            "dwgu": rel_errors(f32(wgus.grad), R(ref["dwgu"])), "dwd": rel_errors(f32(wds.grad), R(ref["dwd"])),
            "dwr": rel_errors(f32(wrs.grad), R(ref["dwr"]))}


def boundary_tokens(ids, E, block_rows=256, per_tile=16, tail_rows=1024, tail_step=8, seed=0):
    """Tokens that own sorted rows where the grouped GEMMs' tile edges lie, for full-size sampled parity checks.
    Rows are in the layer's sorted order (stable sort of the flat (token, slot) ids, as aurora/hf_compat.py:69-72):
      - each expert's last m-tile of block_rows rows (usually partial: the row masks and the partial-tile main loop):
        its first and last row, the rows either side of every 64-row fragment edge inside it, and up to per_tile more
        drawn at random;
      - every tail_step-th of the last tail_rows sorted rows, and the last row: the highest tile ids, which a
        persistent grid runs in its final round (split into half-row units when that round is at most half full).
    Returns the sorted unique token indices."""
    ids = np.asarray(ids)
    k = ids.shape[1]
    flat = ids.reshape(-1)
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=E)
    starts = np.concatenate([[0], np.cumsum(counts)])
    rng = np.random.default_rng(seed)
    rows = []
    for e in range(E):
        c = int(counts[e])
        if c == 0:
            continue
        t0 = (c - 1) // block_rows * block_rows  # first row of the expert's last m-tile
        sel = {t0, c - 1}
        for f in range(t0 + 64, c, 64):
            sel.update((f - 1, f))
        sel.update(rng.integers(t0, c, size=min(per_tile, c - t0)).tolist())
        rows.extend(starts[e] + r for r in sel)
    M = flat.size
    rows.extend(range(max(0, M - tail_rows), M, tail_step))
    rows.append(M - 1)
    rows = np.asarray([r for r in rows if 0 <= r < M], dtype=np.int64)
    return np.unique(order[rows] // k)


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
