"""Drop-in for the reference's aurora/moe_triton.py: the same names and call signatures (BLOCK_M, m_bucket,
make_schedule, grouped_mm), served by hand-written gfx950 HIP kernels through the hmoe C ABI (no Triton).

    y[rows of e] = a[rows of e] @ w[e]   (grouped over experts in one persistent launch)

with the reference's fused extras: gather of A rows (a_idx), per-row scale (routing weight), scatter of Y rows
(y_idx); fp32 accumulation and one rounding to a.dtype on store (aurora/moe_triton.py:22-56).
"""
from __future__ import annotations

import torch

from . import ops

BLOCK_M = 64  # aurora/moe_triton.py:13 -- the row granularity of make_schedule's blocks


def m_bucket(M: int, E: int) -> int:
    """aurora/moe_triton.py:59-62: rows per expert rounded up to a power of two, clamped to [16, 1024].  The HIP
    kernels do not autotune per call; the value is kept for callers that key caches on it."""
    v = max(1, M // E)
    p = 1 << (v - 1).bit_length()
    return min(1024, max(16, p))


def make_schedule(counts: torch.Tensor, M: int):
    """aurora/moe_triton.py:93-107: per BLOCK_M-row block of the ceil(M/BLOCK_M)+E upper-bound grid, (expert or -1,
    first row, end row of that expert) as int32 tensors on counts.device, computed on the device (no host sync)."""
    return ops.make_schedule(counts, M, BLOCK_M)


def grouped_mm(a: torch.Tensor, w: torch.Tensor, counts: torch.Tensor, sched=None, a_idx=None, y_idx=None,
               scale=None, w_scale=None) -> torch.Tensor:
    """aurora/moe_triton.py:65-90.  a (M, K) sorted by expert -- or the unsorted token matrix when a_idx (M,) int32
    names the row to read --, w (E, K, N) with contiguous rows, counts (E,) rows per expert (sum = M) -> (M, N) of
    a.dtype.  scale[r] multiplies output row r; y_idx[r] is where row r is written.  `sched` (make_schedule's
    output) is accepted for call compatibility; the kernel derives its own tile map from `counts` on the device.
    a is bf16 or fp16 (the products run on the matching MFMA, the output has a's type); w has a's type, or is int8
    with w_scale (E, N) (aurora/moe_triton.py:44-51): the integers enter the 16-bit products exactly and the
    per-column scale multiplies the fp32 sum, before `scale`.  K and N need not be multiples of the copy granule:
    such operands are zero-padded on the device first (pad_operands)."""
    M = a_idx.numel() if a_idx is not None else a.shape[0]
    assert w.stride(2) == 1, "w must be (E, K, N) with contiguous rows"
    if a.dtype not in (torch.bfloat16, torch.float16) or w.dtype not in (a.dtype, torch.int8):
        raise TypeError(f"hmoe grouped_mm supports bf16 or fp16 a with w of a's type or int8 (got {a.dtype}, "
                        f"{w.dtype})")
    if (w.dtype == torch.int8) != (w_scale is not None):
        raise ValueError("int8 weights need w_scale (E, N); 16-bit weights take none")
    a = a.contiguous()
    if a_idx is not None and a_idx.dtype != torch.int32:
        a_idx = a_idx.to(torch.int32)
    if y_idx is not None and y_idx.dtype != torch.int32:
        y_idx = y_idx.to(torch.int32)
    N = w.shape[2]
    a, w, w_scale = pad_operands(a, w, w_scale)
    y = ops.grouped_mm(a, w, counts, M, a_idx=a_idx.contiguous() if a_idx is not None else None,
                       y_idx=y_idx.contiguous() if y_idx is not None else None, scale=scale, w_scale=w_scale)
    return y if y.shape[1] == N else y[:, :N].contiguous()


def pad_operands(a, w, w_scale=None):
    """Zero-pad K and N up to the kernels' copy granule (aurora/moe_triton.py:43-44,56 masks any K and N; the direct
    global -> LDS copies here move 16-byte pieces): K to a multiple of 8, N to 8 (16-bit weights) or 16 (int8
    weights, whose padded scale columns are zero).  Zero k terms add exact zeros to the fp32 sums and padded output
    columns are dropped, so the N valid columns are what the unpadded product gives.  Shapes already aligned pass
    through untouched; the padding is a device copy of a and w on each call (fuse_moe pads its stacks once)."""
    K, N = w.shape[1], w.shape[2]
    Kp = -(-K // 8) * 8
    Np = -(-N // (16 if w.dtype == torch.int8 else 8)) * (16 if w.dtype == torch.int8 else 8)
    if Kp != K:
        a = torch.nn.functional.pad(a, (0, Kp - K))
    if (Kp, Np) != (K, N):
        w = torch.nn.functional.pad(w, (0, Np - N, 0, Kp - K))
        if w_scale is not None:
            w_scale = torch.nn.functional.pad(w_scale, (0, Np - N))
    return a, w, w_scale
