"""Tensor-level wrappers of the hmoe C entry points.  Each allocates its outputs with torch (caching allocator),
validates layouts, and launches on the current stream of the tensors' device.  GPU tensors only."""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib as L


def _dev_stream(t):
    L.require_gpu(t, "input")
    return L.stream(t.device)


_SIDE_STREAMS = {}  # device index -> side stream (kept off the modules, which may be copied or pickled)


def side_stream(device: torch.device):
    """One side stream per device for work that overlaps the main stream's, created with the default priority."""
    key = device.index if device.index is not None else torch.cuda.current_device()
    if key not in _SIDE_STREAMS:
        _SIDE_STREAMS[key] = torch.cuda.Stream(device=key)
    return _SIDE_STREAMS[key]


_SIDE_EVENTS = {}  # device index -> (fork, join) events, reused by every fork to and join from the side stream


def side_events(device: torch.device):
    """A (fork, join) pair of events per device for forking work onto the side stream and joining it back: recorded
    and waited on in stream order, so one pair serves every fork (wait_stream would make a new event each time)."""
    key = device.index if device.index is not None else torch.cuda.current_device()
    if key not in _SIDE_EVENTS:
        _SIDE_EVENTS[key] = (torch.cuda.Event(), torch.cuda.Event())
    return _SIDE_EVENTS[key]


# Optional event probe: when `probe` is set to {op name: list}, each listed op records a (start, end) pair of
# torch.cuda.Events on the stream its kernels are launched on (the current stream) around its C call.
probe = None


class _Probe:
    def __init__(self, name):
        self.name = name
        self.ev = None

    def __enter__(self):
        if probe is not None and self.name in probe:
            self.ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            self.ev[0].record()
        return self

    def __exit__(self, *exc):
        if self.ev is not None:
            self.ev[1].record()
            probe[self.name].append(self.ev)
        return False


def _contig(t, name):
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


def _need(t, name, shape=None, dtypes=None, contig=True, min_rows=None):
    """Validate a tensor handed to a C entry point: the kernels trust the sizes they are given, so a wrong shape,
    dtype or layout must stop here rather than become an out-of-range access on the device.  shape entries of None
    are not checked; min_rows: at least that many rows (a gathered operand); a row-strided 2-D tensor passes when
    contig=False as long as its rows are contiguous."""
    if t is None:
        raise ValueError(f"{name} is required")
    L.require_gpu(t, name)
    if dtypes is not None and t.dtype not in dtypes:
        raise TypeError(f"{name}: dtype {t.dtype} not in {dtypes}")
    if shape is not None:
        if t.dim() != len(shape) or any(want is not None and got != want for got, want in zip(t.shape, shape)):
            raise ValueError(f"{name}: shape {tuple(t.shape)} does not match {shape}")
    if min_rows is not None and t.shape[0] < min_rows:
        raise ValueError(f"{name}: {t.shape[0]} rows, at least {min_rows} needed")
    if contig and not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if not contig and t.dim() == 2 and t.stride(1) != 1:
        raise ValueError(f"{name} rows must be contiguous")
    return t


_BF16 = (torch.bfloat16,)
_H16 = (torch.bfloat16, torch.float16)  # the activation types of the forward kernels
_I32 = (torch.int32,)


def _act_dtype(t, name):
    """The 16-bit activation type of a forward call (bf16 or fp16), as the C code of the entry points' dtype."""
    if t.dtype not in _H16:
        raise TypeError(f"{name}: the hmoe forward kernels take bf16 or fp16 activations (got {t.dtype})")
    return L.dt(t)



def _rows_index(idx, name, M):
    return None if idx is None else _need(idx, name, (M,), _I32)


def _router_args(x, wr):
    if x.dim() != 2 or wr.dim() != 2 or x.dtype != torch.bfloat16 or wr.dtype != torch.bfloat16:
        raise TypeError("router expects a bf16 (T, d) x and a bf16 (E, d) weight")
    if wr.shape[1] != x.shape[1]:
        raise ValueError(f"router weight {tuple(wr.shape)} does not match x of width {x.shape[1]}")
    if x.stride(1) != 1:
        raise ValueError("x rows must be contiguous")
    L.require_gpu(wr, "router weight")


def route_topk(x: torch.Tensor, wr: torch.Tensor, k: int, bias=None, renorm=True, scaling=1.0, want_logits=True):
    """Softmax top-k router -> (logits (T, E) fp32 or None, topk_ids (T, k) int32, topk_w (T, k) fp32)."""
    T, d = x.shape
    E = wr.shape[0]
    _router_args(x, wr)
    wr = _contig(wr, "router weight")
    if bias is not None:
        if tuple(bias.shape) != (E,):
            raise ValueError(f"logit bias: shape {tuple(bias.shape)}, expected ({E},)")
        bias = _contig(bias.to(torch.float32), "bias")
    s = _dev_stream(x)
    # above 16 experts the logits buffer is passed even when not wanted: small token counts route through it
    logits = torch.empty(T, E, device=x.device, dtype=torch.float32) if want_logits or E > 16 else None
    ids = torch.empty(T, k, device=x.device, dtype=torch.int32)
    w = torch.empty(T, k, device=x.device, dtype=torch.float32)
    with _Probe("route_topk"):
        L.call("hmoe_route_topk", L.ptr(x), x.stride(0), L.ptr(wr), L.ptr(bias), T, d, E, k, int(bool(renorm)),
               float(scaling), L.ptr(logits), L.ptr(ids), L.ptr(w), s)
    return (logits if want_logits else None), ids, w


def moe_forward(x, wr, wgu, wd, k, bias=None, renorm=True, scaling=1.0, want_logits=False):
    """The routed forward of a layer in one C call (hmoe_moe_forward): route_topk, routed_gate_up, down_scatter and
    combine, with the same outputs and their intermediates in one workspace, for callers whose host time per layer
    matters (small batches).  x (T, d) bf16 with contiguous rows; wr (E, d), wgu (E, d, 2h), wd (E, h, d) bf16,
    contiguous; bias (E,) or None -> (out (T, d) bf16, topk_ids (T, k) int32, topk_w (T, k) fp32, logits (T, E)
    fp32 or None)."""
    T, d = x.shape
    E = wr.shape[0]
    _router_args(x, wr)
    _need(wr, "router weight", (E, d), _BF16)
    if wgu.dim() != 3 or wd.dim() != 3:
        raise ValueError("wgu (E, d, 2h) and wd (E, h, d) expected")
    h = wd.shape[1]
    _need(wgu, "wgu", (E, d, 2 * h), _BF16)
    _need(wd, "wd", (E, h, d), _BF16)
    if bias is not None:
        if tuple(bias.shape) != (E,):
            raise ValueError(f"logit bias: shape {tuple(bias.shape)}, expected ({E},)")
        bias = _contig(bias.to(torch.float32), "bias")
    if probe is not None and any(n in probe for n in _FWD_OPS):
        # event timing of single ops (bench.py's probe) needs the launches apart: the same entry points one by one
        logits, ids, w = route_topk(x, wr, k, bias=bias, renorm=renorm, scaling=scaling, want_logits=want_logits)
        disp, act, _ = routed_gate_up(x, ids, E, wgu, topk_w=w, want_inv=True)
        y, _ = down_scatter(act, wd, disp.counts, T * k, disp.w_sorted, disp.order)
        return combine(y, T, k, inv_pos=disp.inv_pos), ids, w, logits
    lib = L.lib()
    ws_bytes = lib.hmoe_moe_forward_workspace_size(T, d, E, k, h)
    if ws_bytes == 0:
        raise ValueError(f"moe_forward: unsupported sizes T={T} d={d} E={E} k={k} h={h}")
    dev = x.device
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    out = torch.empty(T, d, device=dev, dtype=torch.bfloat16)
    ids = torch.empty(T, k, device=dev, dtype=torch.int32)
    w = torch.empty(T, k, device=dev, dtype=torch.float32)
    logits = torch.empty(T, E, device=dev, dtype=torch.float32) if want_logits else None
    with _Probe("moe_forward"):
        L.call("hmoe_moe_forward", L.ptr(x), x.stride(0), L.ptr(wr), L.ptr(bias), L.ptr(wgu), L.ptr(wd), T, d, E, k,
               h, int(bool(renorm)), float(scaling), L.ptr(out), L.ptr(ids), L.ptr(w), L.ptr(logits), L.ptr(ws),
               ws_bytes, _dev_stream(x))
    return out, ids, w, logits


_FWD_OPS = ("route_topk", "dispatch", "gate_up_swiglu", "down_scatter", "combine")


def moe_experts(x, ids, tw, wgu, wd, wgu_s=None, wd_s=None):
    """The expert part of a forward whose routing the caller's gate decided, in one C call (hmoe_moe_experts):
    routed_gate_up (with inv_pos) and down_scatter with the same outputs.  x (T, d) bf16 or fp16 with contiguous rows;
    ids (T, k) int32 / int64; tw (T, k); wgu (E, d, 2h) and wd (E, h, d) of x's type, or int8 with scales wgu_s
    (E, 2h) and wd_s (E, d) -> (y (T*k, d) in (token, slot) order, inv_pos (T*k,) int32, n_invalid (1,) int32); the
    combine (with inv_pos) sums y over the slots."""
    T, k = ids.shape
    if probe is not None and any(n in probe for n in _FWD_OPS):
        # event timing of single ops (bench.py's probe): the same entry points one by one
        disp, act, _ = routed_gate_up(x, ids, wgu.shape[0], wgu, topk_w=tw, wgu_s=wgu_s, want_inv=True)
        y, _ = down_scatter(act, wd, disp.counts, T * k, disp.w_sorted, disp.order, wd_s=wd_s)
        return y, disp.inv_pos, disp.n_invalid
    if x.dim() != 2 or x.shape[0] != T or x.stride(1) != 1:
        raise ValueError(f"x must be a ({T}, d) matrix with contiguous rows (got {tuple(x.shape)})")
    dt = _act_dtype(x, "x")
    d = x.shape[1]
    if wgu.dim() != 3 or wd.dim() != 3 or wgu.dtype not in (x.dtype, torch.int8) or wd.dtype != wgu.dtype:
        raise TypeError(f"wgu (E, d, 2h) and wd (E, h, d) of x's type or int8 expected (got {wgu.dtype}, {wd.dtype})")
    E, h = wgu.shape[0], wd.shape[1]
    L.require_gpu(x, "x")
    _need(ids, "topk_ids", (T, k), (torch.int32, torch.int64))
    if tuple(tw.shape) != (T, k):
        raise ValueError(f"topk_weight: shape {tuple(tw.shape)}, expected {(T, k)}")
    tw = _contig(tw if tw.dtype in (torch.float32, torch.bfloat16, torch.float16) else tw.float(), "topk_weight")
    _need(wgu, "wgu", (E, d, 2 * h), (wgu.dtype,))
    _need(wd, "wd", (E, h, d), (wd.dtype,))
    wgu_s = _w_scale(wgu, wgu_s, 2 * h)
    wd_s = _w_scale(wd, wd_s, d)
    w_dt = L.dt(wgu)
    lib = L.lib()
    ws_bytes = lib.hmoe_moe_experts_workspace_size(T, d, E, k, h, w_dt, dt)
    if ws_bytes == 0:
        raise ValueError(f"moe_experts: unsupported sizes T={T} d={d} E={E} k={k} h={h}")
    dev = x.device
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    y = torch.empty(T * k, d, device=dev, dtype=x.dtype)
    inv = torch.empty(T * k, device=dev, dtype=torch.int32)
    n_invalid = torch.empty(1, device=dev, dtype=torch.int32)
    L.call("hmoe_moe_experts", L.ptr(x), x.stride(0), L.ptr(ids), L.dt(ids), L.ptr(tw), L.dt(tw), L.ptr(wgu),
           L.ptr(wgu_s), L.dt(wgu_s) if wgu_s is not None else 0, L.ptr(wd), L.ptr(wd_s),
           L.dt(wd_s) if wd_s is not None else 0, w_dt, T, d, E, k, h, L.ptr(y), L.ptr(inv), L.ptr(n_invalid),
           L.ptr(ws), ws_bytes, dt, _dev_stream(x))
    return y, inv, n_invalid


def route_sigmoid_group(x: torch.Tensor, wr: torch.Tensor, k: int, n_group: int, topk_group: int, expert_bias=None,
                        scaling=1.0, want_scores=False):
    """BailingMoeV2 sigmoid, group-limited router -> (scores (T, E) fp32 or None, topk_ids (T, k) int32,
    topk_w (T, k) fp32)."""
    T, d = x.shape
    E = wr.shape[0]
    _router_args(x, wr)
    wr = _contig(wr, "router weight")
    if expert_bias is not None:
        if tuple(expert_bias.shape) != (E,):
            raise ValueError(f"expert bias: shape {tuple(expert_bias.shape)}, expected ({E},)")
        expert_bias = _contig(expert_bias.to(torch.float32), "expert bias")
    s = _dev_stream(x)
    # the scores buffer is passed even when not wanted: small token counts route through it (two launches that
    # spread the work over the chip)
    scores = torch.empty(T, E, device=x.device, dtype=torch.float32)
    ids = torch.empty(T, k, device=x.device, dtype=torch.int32)
    w = torch.empty(T, k, device=x.device, dtype=torch.float32)
    with _Probe("route_topk"):
        L.call("hmoe_route_sigmoid_group", L.ptr(x), x.stride(0), L.ptr(wr), L.ptr(expert_bias), T, d, E, k, n_group,
               topk_group, float(scaling), L.ptr(scores), L.ptr(ids), L.ptr(w), s)
    return (scores if want_scores else None), ids, w


@dataclass
class Dispatch:
    counts: torch.Tensor  # (E,) int32
    counts64: torch.Tensor  # (E,) int64 or None
    starts: torch.Tensor  # (E+1,) int32
    order: torch.Tensor  # (M,) int32  (= y_idx)
    a_idx: torch.Tensor  # (M,) int32
    inv_pos: torch.Tensor  # (M,) int32
    w_sorted: torch.Tensor  # (M,) bf16 or None
    xs: torch.Tensor  # (M, d) bf16 or None
    xs_tiles: torch.Tensor = None  # the sorted rows as row-group tiles (bf16 storage) or None
    n_invalid: torch.Tensor = None  # (1,) int32 on the device: flat rows whose expert id lies outside [0, E)


def dispatch(topk_ids: torch.Tensor, E: int, topk_w=None, x=None, want_counts64=False, want_inv=True,
             want_xs=True, want_tiles=False, dtype=None) -> Dispatch:
    """Stable counting sort of the flat routed rows (aurora/hf_compat.py:69-72, 78, 80) and optionally, with x, the
    row permutation xs = x[a_idx] (want_xs) and the same rows as row-group tiles for gate_up_swiglu_tiles
    (want_tiles).  Expert ids outside [0, E) route nowhere (inv_pos -1, counted in no expert); their number is left
    on the device in n_invalid, read without a host sync only when the caller asks.  The sorted routing weights (and
    the copied rows) have x's type, bf16 or fp16 (dtype without x; bf16 by default)."""
    T, k = topk_ids.shape
    M = T * k
    dev = topk_ids.device
    s = _dev_stream(topk_ids)
    ids = _need(topk_ids, "topk_ids", (T, k), (torch.int32, torch.int64))
    if topk_w is not None:
        if tuple(topk_w.shape) != (T, k):
            raise ValueError(f"topk_weight: shape {tuple(topk_w.shape)}, expected {(T, k)}")
        topk_w = _contig(topk_w, "topk_weight")
        if topk_w.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            topk_w = topk_w.float()
    if x is not None:
        dtype = x.dtype
    dtype = torch.bfloat16 if dtype is None else dtype
    if dtype not in _H16:
        raise TypeError(f"dispatch: activations must be bf16 or fp16 (got {dtype})")
    counts = torch.empty(E, device=dev, dtype=torch.int32)
    counts64 = torch.empty(E, device=dev, dtype=torch.int64) if want_counts64 else None
    starts = torch.empty(E + 1, device=dev, dtype=torch.int32)
    order = torch.empty(M, device=dev, dtype=torch.int32)
    a_idx = torch.empty(M, device=dev, dtype=torch.int32)
    inv = torch.empty(M, device=dev, dtype=torch.int32) if want_inv else None
    w_sorted = torch.empty(M, device=dev, dtype=dtype) if topk_w is not None else None
    n_invalid = torch.empty(1, device=dev, dtype=torch.int32)
    xs = tiles = None
    d = 0
    ldx = 0
    if x is not None:
        _need(x, "x", (T, None), _H16, contig=False)  # xs = x[a_idx] reads rows a_idx < T
        d = x.shape[1]
        ldx = x.stride(0)
        if want_xs:
            xs = torch.empty(M, d, device=dev, dtype=dtype)
        if want_tiles:
            tiles = torch.empty(L.lib().hmoe_xs_tiles_bytes(M, E, d) // 2, device=dev, dtype=dtype)
    ws_bytes = L.lib().hmoe_dispatch_workspace_size(T, k, E)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    with _Probe("dispatch"):
        L.call("hmoe_dispatch_tiles", L.ptr(ids), L.dt(ids), L.ptr(topk_w), L.dt(topk_w) if topk_w is not None else 0,
               T, k, E, L.ptr(x), ldx, d, L.ptr(xs), L.ptr(tiles), L.ptr(counts), L.ptr(counts64), L.ptr(starts),
               L.ptr(order), L.ptr(a_idx), L.ptr(inv), L.ptr(w_sorted), L.ptr(n_invalid), L.ptr(ws), ws_bytes,
               L.dt(dtype), s)
    return Dispatch(counts, counts64, starts, order, a_idx, inv, w_sorted, xs, tiles, n_invalid)


def make_schedule(counts: torch.Tensor, M: int, block_m: int = 64):
    E = counts.numel()
    nb = -(-M // block_m) + E
    s = _dev_stream(counts)
    counts = _contig(counts, "counts")
    if counts.dtype not in (torch.int32, torch.int64):
        counts = counts.to(torch.int64)
    out = [torch.empty(nb, device=counts.device, dtype=torch.int32) for _ in range(3)]
    with _Probe("make_schedule"):
        L.call("hmoe_make_schedule", L.ptr(counts), L.dt(counts), E, M, block_m, *(L.ptr(o) for o in out), s)
    return tuple(out)


def _counts(counts, E):
    """Rows per expert, (E,) int32 or int64 on the GPU: the kernels read E entries."""
    if counts.dtype not in (torch.int32, torch.int64):
        counts = counts.to(torch.int64)
    return _need(counts, "counts", (E,), (torch.int32, torch.int64))


def grouped_mm(a, w, counts, M, a_idx=None, y_idx=None, scale=None, w_scale=None, out=None):
    """y[y_idx[r] or r] = (a[a_idx[r] or r] @ w[e(r)]) * w_scale[e(r)] * scale[r], y (M, N) bf16.  The index
    values are trusted (in range: a_idx < rows of a, y_idx < M); everything else is checked here."""
    if w.dim() != 3 or w.dtype not in (a.dtype, torch.int8):
        raise TypeError(f"w must be an (E, K, N) stack of a's type or int8 (got {tuple(w.shape)} {w.dtype})")
    E, K, N = w.shape
    s = _dev_stream(a)
    _act_dtype(a, "a")
    counts = _counts(counts, E)
    if a.stride(1) != 1:
        a = a.contiguous()
    if w.stride(2) != 1:
        w = w.contiguous()
    a_idx = _rows_index(a_idx, "a_idx", M)
    y_idx = _rows_index(y_idx, "y_idx", M)
    _need(a, "a", (None, K), _H16, contig=False, min_rows=min(1, M) if a_idx is not None else M)
    if a_idx is not None and a.shape[0] * a.stride(0) * 2 >= 2 ** 31:
        raise ValueError("a gathered through a_idx must span less than 2 GiB (32-bit row offsets)")
    if w_scale is not None:
        w_scale = _contig(w_scale, "w_scale")
        if w_scale.shape != (E, N):
            raise ValueError(f"w_scale must be (E, N) = {(E, N)}, got {tuple(w_scale.shape)}")
    if out is not None:
        _need(out, "out", (M, N), (a.dtype,), contig=False)
    y = out if out is not None else torch.empty(M, N, device=a.device, dtype=a.dtype)
    if scale is not None:
        scale = _contig(scale, "scale")
        if scale.dtype not in (a.dtype, torch.float32):
            scale = scale.float()
        _need(scale, "scale", (M,))
    with _Probe("grouped_mm"):
        L.call("hmoe_grouped_mm", L.ptr(a), a.stride(0), L.dt(a), L.ptr(w), L.dt(w), E, K, N, w.stride(0), w.stride(1),
               L.ptr(counts), L.dt(counts), M, L.ptr(a_idx), L.ptr(y_idx), L.ptr(scale),
               L.dt(scale) if scale is not None else 0, L.ptr(w_scale), L.dt(w_scale) if w_scale is not None else 0,
               L.ptr(y), y.stride(0), s)
    return y


def _w_scale(w, w_s, n):
    """int8 weights need their (E, n) per-column scales; bf16 weights take none."""
    if (w.dtype == torch.int8) != (w_s is not None):
        raise ValueError("int8 weights come with a scale (E, N); bf16 weights take none")
    if w_s is not None:
        w_s = _contig(w_s, "weight scale")
        if w_s.shape != (w.shape[0], n) or w_s.dtype not in (torch.bfloat16, torch.float32):
            raise ValueError(f"weight scale must be bf16 or fp32 of shape {(w.shape[0], n)}")
    return w_s


def gate_up_swiglu(x, wgu, counts, M, a_idx=None, keep_gu=False, wgu_s=None):
    """act = bf16(bf16(silu(g)) * u) for [g | u] = x[a_idx] @ wgu[e]; wgu bf16, or int8 with per-column scales
    wgu_s (E, 2h) (inference only: no gu)."""
    if wgu.dim() != 3 or wgu.dtype not in (x.dtype, torch.int8) or wgu.shape[2] % 2:
        raise TypeError(f"wgu must be an (E, d, 2h) stack of x's type or int8 (got {tuple(wgu.shape)} {wgu.dtype})")
    E, d, h2 = wgu.shape
    h = h2 // 2
    s = _dev_stream(x)
    dt = _act_dtype(x, "x")
    wgu = _contig(wgu, "wgu")
    counts = _counts(counts, E)
    wgu_s = _w_scale(wgu, wgu_s, h2)
    a_idx = _rows_index(a_idx, "a_idx", M)
    _need(x, "x", (None, d), _H16, contig=False, min_rows=min(1, M) if a_idx is not None else M)
    act = torch.empty(M, h, device=x.device, dtype=x.dtype)
    if wgu_s is not None:
        if keep_gu:
            raise ValueError("int8 weights are inference only (no gu kept)")
        with _Probe("gate_up_swiglu"):
            L.call("hmoe_gate_up_swiglu_i8", L.ptr(x), x.stride(0), L.ptr(a_idx), L.ptr(wgu), L.ptr(wgu_s),
                   L.dt(wgu_s), E, d, h, L.ptr(counts), L.dt(counts), M, L.ptr(act), dt, s)
        return act, None
    gu = torch.empty(M, h2, device=x.device, dtype=x.dtype) if keep_gu else None
    with _Probe("gate_up_swiglu"):
        L.call("hmoe_gate_up_swiglu", L.ptr(x), x.stride(0), L.ptr(a_idx), L.ptr(wgu), E, d, h, L.ptr(counts),
               L.dt(counts), M, L.ptr(act), L.ptr(gu), dt, s)
    return act, gu


def gate_up_swiglu_tiles(xs_tiles, wgu, counts, M, keep_gu=False):
    """gate_up_swiglu on the row-group tiles a dispatch(want_tiles=True) wrote (16-bit weights of the tiles' type):
    identical act / gu."""
    if wgu.dim() != 3 or wgu.dtype != xs_tiles.dtype or wgu.shape[2] % 2:
        raise TypeError(f"wgu must be an (E, d, 2h) stack of the tiles' type (got {tuple(wgu.shape)} {wgu.dtype})")
    E, d, h2 = wgu.shape
    h = h2 // 2
    s = _dev_stream(xs_tiles)
    dt = _act_dtype(xs_tiles, "xs_tiles")
    wgu = _contig(wgu, "wgu")
    counts = _counts(counts, E)
    _need(xs_tiles, "xs_tiles", (L.lib().hmoe_xs_tiles_bytes(M, E, d) // 2,), _H16)
    act = torch.empty(M, h, device=xs_tiles.device, dtype=xs_tiles.dtype)
    gu = torch.empty(M, h2, device=xs_tiles.device, dtype=xs_tiles.dtype) if keep_gu else None
    with _Probe("gate_up_swiglu"):
        L.call("hmoe_gate_up_swiglu_tiles", L.ptr(xs_tiles), L.ptr(wgu), E, d, h, L.ptr(counts), L.dt(counts), M,
               L.ptr(act), L.ptr(gu), dt, s)
    return act, gu


# The tiles save about 7% of the gate/up GEMM (2 M d 2h flops) for M d 2 more bytes written by the dispatch, so
# they pay for wide hidden layers only.  Whole forward passes, same process: h = 4096 (C3) 1290 against 1297 us,
# h = 2048 (C2, 2048 tokens) 143 against 128, h = 320 (BailingMoeV2-like, bf16) 807 against 747.  Below this the
# GEMM gathers the rows itself.
TILES_MIN_H = 4096


def routed_gate_up(x, ids, E, wgu, topk_w=None, wgu_s=None, keep_gu=False, want_xs=False, want_inv=True):
    """dispatch + gate/up GEMM of the routed rows: with bf16 weights and a wide hidden layer the dispatch writes the
    rows as row-group tiles and the GEMM reads them (1 KB copies); otherwise (int8 weights, h below TILES_MIN_H,
    tiles past the GEMM's 32-bit offsets) the GEMM gathers the rows of x itself.  want_xs: also the row-major
    permuted copy (the gate/up weight gradient reads it).  Returns (Dispatch, act, gu)."""
    T, k = ids.shape
    M = T * k
    d = x.shape[1]
    h = wgu.shape[2] // 2
    tiles = (wgu_s is None and wgu.dtype == x.dtype and h >= TILES_MIN_H
             and L.lib().hmoe_xs_tiles_bytes(M, E, d) < (1 << 31))
    disp = dispatch(ids, E, topk_w=topk_w, x=x if (tiles or want_xs) else None, want_inv=want_inv, want_xs=want_xs,
                    want_tiles=tiles, dtype=x.dtype)
    if tiles:
        act, gu = gate_up_swiglu_tiles(disp.xs_tiles, wgu, disp.counts, M, keep_gu=keep_gu)
        disp.xs_tiles = None  # read once: not kept alive with the dispatch
    elif want_xs:
        act, gu = gate_up_swiglu(disp.xs, wgu, disp.counts, M, keep_gu=keep_gu, wgu_s=wgu_s)
    else:
        act, gu = gate_up_swiglu(x, wgu, disp.counts, M, a_idx=disp.a_idx, keep_gu=keep_gu, wgu_s=wgu_s)
    return disp, act, gu


def down_scatter(act, wd, counts, M, w_sorted, y_idx, keep_yhat=False, wd_s=None):
    """y[y_idx[r]] = bf16(act[r] @ wd[e] * w_sorted[r]); wd bf16, or int8 with per-column scales wd_s (E, d)."""
    if wd.dim() != 3 or wd.dtype not in (act.dtype, torch.int8):
        raise TypeError(f"wd must be an (E, h, d) stack of act's type or int8 (got {tuple(wd.shape)} {wd.dtype})")
    E, h, d = wd.shape
    s = _dev_stream(act)
    dt = _act_dtype(act, "act")
    wd = _contig(wd, "wd")
    counts = _counts(counts, E)
    wd_s = _w_scale(wd, wd_s, d)
    _need(act, "act", (M, h), _H16)
    y_idx = _rows_index(y_idx, "y_idx", M)
    if w_sorted is not None:
        _need(w_sorted, "w_sorted", (M,), (act.dtype,))
    y = torch.empty(M, d, device=act.device, dtype=act.dtype)
    if wd_s is not None:
        if keep_yhat:
            raise ValueError("int8 weights are inference only (no yhat kept)")
        with _Probe("down_scatter"):
            L.call("hmoe_down_scatter_i8", L.ptr(act), L.ptr(wd), L.ptr(wd_s), L.dt(wd_s), E, h, d, L.ptr(counts),
                   L.dt(counts), M, L.ptr(w_sorted), L.ptr(y_idx), L.ptr(y), dt, s)
        return y, None
    yhat = torch.empty(M, d, device=act.device, dtype=act.dtype) if keep_yhat else None
    with _Probe("down_scatter"):
        L.call("hmoe_down_scatter", L.ptr(act), L.ptr(wd), E, h, d, L.ptr(counts), L.dt(counts), M, L.ptr(w_sorted),
               L.ptr(y_idx), L.ptr(y), L.ptr(yhat), dt, s)
    return y, yhat


def combine(y, T, k, add=None, inv_pos=None):
    """out[t] = bf16(sum_j y[t*k + j]) (+ add[t], rounded once more: bf16 + bf16).  inv_pos (T*k,) from the dispatch:
    slots routed nowhere (inv_pos < 0: an expert id outside [0, E)) add zeros instead of their unwritten rows."""
    d = y.shape[1]
    _need(y, "y", (T * k, d), _H16)
    dt = _act_dtype(y, "y")
    inv_pos = _rows_index(inv_pos, "inv_pos", T * k)
    out = torch.empty(T, d, device=y.device, dtype=y.dtype)
    with _Probe("combine"):
        if add is None:
            L.call("hmoe_combine", L.ptr(_contig(y, "y")), L.ptr(inv_pos), T, k, d, L.ptr(out), dt, _dev_stream(y))
        else:
            if add.shape != (T, d) or add.dtype != y.dtype:
                raise ValueError(f"add must be {y.dtype} of shape {(T, d)}")
            L.call("hmoe_combine_add", L.ptr(_contig(y, "y")), L.ptr(inv_pos), T, k, d, L.ptr(_contig(add, "add")),
                   L.ptr(out), dt, _dev_stream(y))
    return out


def combine_bwd(dout, yhat, disp: Dispatch, k):
    """(dys (M, d) bf16, dtopk_w (T, k) fp32): the routing-weighted upstream rows in sorted order and, with yhat
    (the unscaled down-projection rows, sorted), <dout[t], yhat[r]>; yhat None: (dys, None)."""
    T, d = dout.shape
    M = T * k
    dout = dout.contiguous()
    if yhat is not None:
        _need(yhat, "yhat", (M, d), _BF16)
    _need(dout, "dout", (T, d), _BF16)
    for t_, n_ in ((disp.order, "order"), (disp.a_idx, "a_idx")):
        _need(t_, n_, (M,), _I32)
    _need(disp.w_sorted, "w_sorted", (M,), _BF16)
    dys = torch.empty(M, d, device=dout.device, dtype=torch.bfloat16)
    dtw = torch.empty(T, k, device=dout.device, dtype=torch.float32) if yhat is not None else None
    with _Probe("combine_bwd"):
        L.call("hmoe_combine_bwd", L.ptr(dout), L.ptr(yhat), L.ptr(disp.order), L.ptr(disp.a_idx), L.ptr(disp.w_sorted),
               M, k, d, L.ptr(dys), L.ptr(dtw), _dev_stream(dout))
    return dys, dtw


def down_dgrad_swiglu(dy, wd, counts, M, gu, a_idx=None, w_sorted=None):
    """dgu (M, 2h) from the upstream gradient dy (T, d) gathered through a_idx (or sorted rows (M, d) when a_idx is
    None) and scaled by w_sorted in fp32."""
    _need(wd, "wd", (None, None, None), _BF16)
    E, h, d = wd.shape
    counts = _counts(counts, E)
    a_idx = _rows_index(a_idx, "a_idx", M)
    _need(dy, "dy", (None, d), _BF16, min_rows=min(1, M) if a_idx is not None else M)
    _need(gu, "gu", (M, 2 * h), _BF16)
    if w_sorted is not None:
        _need(w_sorted, "w_sorted", (M,), _BF16)
    dgu = torch.empty(M, 2 * h, device=dy.device, dtype=torch.bfloat16)
    with _Probe("down_dgrad_swiglu"):
        L.call("hmoe_down_dgrad_swiglu", L.ptr(dy), L.ptr(a_idx), L.ptr(w_sorted), L.ptr(wd), E, h, d, L.ptr(counts),
               L.dt(counts), M, L.ptr(gu), L.ptr(dgu), _dev_stream(dy))
    return dgu


def down_dgrad_swiglu_dw(dy, wd, counts, M, gu, order, k, a_idx=None, w_sorted=None):
    """(dgu, dtopk_w): down_dgrad_swiglu's dgu and, from the same product, the routing-weight gradient dtopk_w (T, k)
    fp32 = sum_n (dy[t] @ wd[e]^T)[n] * act[r][n], act recomputed from gu as the forward rounds it."""
    _need(wd, "wd", (None, None, None), _BF16)
    E, h, d = wd.shape
    counts = _counts(counts, E)
    a_idx = _rows_index(a_idx, "a_idx", M)
    _need(dy, "dy", (None, d), _BF16, min_rows=min(1, M) if a_idx is not None else M)
    _need(gu, "gu", (M, 2 * h), _BF16)
    order = _rows_index(order, "order", M)
    if order is None:
        raise ValueError("order is required")
    if w_sorted is not None:
        _need(w_sorted, "w_sorted", (M,), _BF16)
    if M % k:
        raise ValueError(f"M = {M} is not a multiple of k = {k}")
    dgu = torch.empty(M, 2 * h, device=dy.device, dtype=torch.bfloat16)
    dtw = torch.empty(M // k, k, device=dy.device, dtype=torch.float32)
    ws_bytes = L.lib().hmoe_down_dgrad_dw_workspace_size(M, h)
    ws = torch.empty(ws_bytes, device=dy.device, dtype=torch.uint8)
    with _Probe("down_dgrad_swiglu"):
        L.call("hmoe_down_dgrad_swiglu_dw", L.ptr(dy), L.ptr(a_idx), L.ptr(w_sorted), L.ptr(wd), E, h, d,
               L.ptr(counts), L.dt(counts), M, L.ptr(gu), L.ptr(dgu), L.ptr(order), L.ptr(dtw), L.ptr(ws), ws_bytes,
               _dev_stream(dy))
    return dgu, dtw


def gate_up_dgrad(dgu, wgu, counts, M, dtype=torch.float32):
    _need(wgu, "wgu", (None, None, None), _BF16)
    E, d, h2 = wgu.shape
    counts = _counts(counts, E)
    _need(dgu, "dgu", (M, h2), _BF16)
    dxs = torch.empty(M, d, device=dgu.device, dtype=dtype)
    with _Probe("gate_up_dgrad"):
        L.call("hmoe_gate_up_dgrad", L.ptr(dgu), L.ptr(wgu), E, d, h2 // 2, L.ptr(counts), L.dt(counts), M, L.ptr(dxs),
               L.dt(dxs), _dev_stream(dgu))
    return dxs


def grouped_wgrad(a, b, counts, E, dtype=torch.bfloat16):
    M, P = a.shape
    N = b.shape[1]
    counts = _counts(counts, E)
    _need(a, "a", (M, P), _BF16, contig=False)
    _need(b, "b", (M, N), _BF16, contig=False)
    dw = torch.empty(E, P, N, device=a.device, dtype=dtype)
    with _Probe("grouped_wgrad"):
        L.call("hmoe_grouped_wgrad", L.ptr(a), a.stride(0), L.ptr(b), b.stride(0), E, P, N, L.ptr(counts), L.dt(counts), M,
               L.ptr(dw), L.dt(dw), _dev_stream(a))
    return dw


def router_bwd(logits, ids, dtw, x, renorm=True, scaling=1.0, dwr_dtype=torch.float32, want_dwr=True):
    T, E = logits.shape
    k = ids.shape[1]
    d = x.shape[1]
    _need(logits, "logits", (T, E), (torch.float32,))
    _need(ids, "topk_ids", (T, k), _I32)
    _need(dtw, "dtopk_w", (T, k), (torch.float32,))
    _need(x, "x", (T, d), _BF16, contig=False)
    dl = torch.empty(T, E, device=logits.device, dtype=torch.float32)
    dwr = torch.empty(E, d, device=logits.device, dtype=dwr_dtype) if want_dwr else None
    ws_bytes = L.lib().hmoe_router_bwd_workspace_size(T, E, d) if want_dwr else 0
    ws = torch.empty(max(ws_bytes, 1), device=logits.device, dtype=torch.uint8)
    with _Probe("router_bwd"):
        L.call("hmoe_router_bwd", L.ptr(logits), L.ptr(ids), L.ptr(dtw), T, E, k, int(bool(renorm)), float(scaling),
               L.ptr(x), x.stride(0), d, L.ptr(dl), L.ptr(dwr), L.dt(dwr_dtype), L.ptr(ws) if want_dwr else None, ws_bytes,
               _dev_stream(logits))
    return dl, dwr


def unpermute_bwd(dxs, inv_pos, T, k, dlogits=None, wr=None):
    d = dxs.shape[1]
    E = wr.shape[0] if wr is not None else 0
    _need(dxs, "dxs", (T * k, d), (torch.float32, torch.bfloat16))
    _need(inv_pos, "inv_pos", (T * k,), _I32)
    if (dlogits is None) != (wr is None):
        raise ValueError("dlogits and wr come together")
    if wr is not None:
        _need(wr, "wr", (E, d), _BF16)
        _need(dlogits, "dlogits", (T, E), (torch.float32,))
    dx = torch.empty(T, d, device=dxs.device, dtype=torch.bfloat16)
    with _Probe("unpermute_bwd"):
        L.call("hmoe_unpermute_bwd", L.ptr(dxs), L.dt(dxs), L.ptr(inv_pos), L.ptr(dlogits), L.ptr(wr), T, k, d, E,
               L.ptr(dx), _dev_stream(dxs))
    return dx
