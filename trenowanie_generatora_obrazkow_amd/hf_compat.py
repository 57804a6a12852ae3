"""Drop-in for the MoE half of the reference's aurora/hf_compat.py (:62-169): `fuse_moe` stacks the experts of
DeepSeek/Bailing-style MoE blocks and installs `_fused_moe_infer` as their `moe_infer`; here the batched path is
mode "hip" (hmoe kernels), selected ahead of everything else.  There is no silent fallback: on a GPU device the
HIP self-test must pass or mode selection raises; CPU devices are rejected (the kernels have no CPU path).
"""
from __future__ import annotations

import types

import torch

from . import ops
from .moe_triton import grouped_mm


@torch.no_grad()
def _fused_moe_infer(self, x, topk_ids, topk_weight):
    """aurora/hf_compat.py:63-82 (the fused branch): stable sort of the flat routed rows by expert, gate/up GEMM
    over gathered token rows with the SwiGLU fused into its epilogue, down GEMM scaled by the bf16-rounded routing
    weight and scattered back to (token, slot) order, sum over the k slots.  Layers fused with quant="int8" run the
    int8-weight forms of the two GEMMs (per-column scales applied to the fp32 sums).  Blocks whose act_fn is not
    silu run the two grouped GEMMs with the module's act_fn applied to g, times u, in between (the reference's
    order of operations).  Widths fuse_moe padded are padded on x and cut from the output.  An expert id outside [0, E)
    in topk_ids routes its slot nowhere: the slot adds nothing to the output, and the count of such ids is kept on
    the device in self._n_invalid (read by invalid_expert_ids, which is the only place that synchronises)."""
    n, k = topk_ids.shape
    E, dp = self._wgu.shape[0], self._wgu.shape[1]
    if self._mode is None:  # decided on the device the weights ended up on
        self._mode = _pick_mode(x.device, x.dtype)
    d = x.shape[-1]
    x = x.contiguous() if dp == d else torch.nn.functional.pad(x, (0, dp - d))  # stacks padded by fuse_moe
    M = n * k
    if _is_silu(self._act):
        # dispatch, both fused projections, routing weight and scatter in one C call
        y, inv_pos, self._n_invalid = ops.moe_experts(x, topk_ids.contiguous(), topk_weight.contiguous(), self._wgu,
                                                      self._wd, wgu_s=self._wgu_s, wd_s=self._wd_s)
    else:
        # any other activation: the module's own act_fn between the two grouped GEMMs, as the reference's fused
        # branch applies it (aurora/hf_compat.py:79-81); gathered rows in, routing weight and scatter in the down GEMM
        disp = ops.dispatch(topk_ids.contiguous(), E, topk_w=topk_weight.contiguous(), want_xs=False, dtype=x.dtype)
        g, u = ops.grouped_mm(x, self._wgu, disp.counts, M, a_idx=disp.a_idx, w_scale=self._wgu_s).chunk(2, dim=-1)
        y = ops.grouped_mm((self._act(g) * u).contiguous(), self._wd, disp.counts, M, y_idx=disp.order,
                           scale=disp.w_sorted, w_scale=self._wd_s)
        self._n_invalid, inv_pos = disp.n_invalid, disp.inv_pos
    out = ops.combine(y, n, k, inv_pos=inv_pos)
    return out if dp == d else out[:, :d].contiguous()


def _is_silu(act):
    """The activations the fused SwiGLU epilogue computes: silu(g) * u (torch's functional silu or an nn.SiLU)."""
    return act is torch.nn.functional.silu or isinstance(act, torch.nn.SiLU)


def invalid_expert_ids(model) -> int:
    """Expert ids outside [0, E) seen by the last moe_infer call of every fused block of `model` (one host sync).
    The fused path gives such a slot no contribution instead of reading unwritten memory; this tells the caller that
    its gate produced them."""
    total = 0
    for mod in model.modules():
        n = getattr(mod, "_n_invalid", None)
        if isinstance(n, torch.Tensor):
            total += int(n.item())
    return total


def _pad_stacks(wgu, wd, granule):
    """Zero-pad the stacked (E, d, 2h) gate|up and (E, h, d) down weights so that d and h are multiples of `granule`
    (8 for 16-bit weights, 16 for int8: the GEMMs' copy granule; the reference's Triton kernel masks any width).
    Padded gate and up columns give g = u = 0, so the padded hidden columns are act(0) * 0 = 0, and the down
    weights' padded rows are zero as well: the first d output columns are those of the unpadded layer, exactly (the
    extra k terms add exact zeros to the fp32 sums).  int8 scales of the padded columns come out at the floor value
    and multiply zeros."""
    E, d, h2 = wgu.shape
    h = h2 // 2
    dp, hp = -(-d // granule) * granule, -(-h // granule) * granule
    if (dp, hp) == (d, h):
        return wgu, wd
    gu = wgu.new_zeros(E, dp, 2 * hp)
    gu[:, :d, :h] = wgu[:, :, :h]
    gu[:, :d, hp:hp + h] = wgu[:, :, h:]
    dn = wd.new_zeros(E, hp, dp)
    dn[:, :h, :d] = wd
    return gu, dn


def _dequant(w, scale, dtype):
    """aurora/hf_compat.py:102-103."""
    return w if scale is None else w.to(dtype) * scale.to(dtype).unsqueeze(1)


def _quant_int8(w):
    """aurora/hf_compat.py:106-110: (E, K, N) -> int8 weights and a per-(expert, output column) scale."""
    scale = w.float().abs().amax(dim=1).clamp(min=1e-8) / 127
    return (w.float() / scale.unsqueeze(1)).round().clamp(-127, 127).to(torch.int8), scale.to(torch.bfloat16)


def _self_test(fn, device, dtype, quant=False):
    """aurora/hf_compat.py:112-121: fn(a, w, w_scale, counts) against plain matmuls on 48x64 @ (3, 64, 32) with
    counts [16, 0, 32] (an empty expert in the middle), allclose(atol=0.1, rtol=0.05).  quant: fn gets int8 weights
    and their scales, the reference product their dequantised values."""
    g = torch.Generator(device="cpu").manual_seed(0)
    a = torch.randn(48, 64, generator=g).to(device=device, dtype=dtype)
    b = torch.randn(3, 64, 32, generator=g).to(device=device, dtype=dtype)
    counts = torch.tensor([16, 0, 32], device=device)
    w, ws = _quant_int8(b) if quant else (b, None)
    ref_w = _dequant(w, ws, dtype).float()
    ref = torch.cat([a[:16].float() @ ref_w[0], a[16:].float() @ ref_w[2]])
    return torch.allclose(fn(a, w, ws, counts).float(), ref, atol=1e-1, rtol=5e-2)


def _pick_mode(device, dtype):
    """aurora/hf_compat.py:124-139, with one mode: "hip" on a ROCm GPU once the known-answer tests pass in the
    activations' dtype (bf16 or fp16)."""
    if device.type != "cuda":
        raise RuntimeError("hmoe fused MoE needs a ROCm GPU device (the kernels have no CPU path)")
    if dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"hmoe fused MoE runs bf16 or fp16 activations (got {dtype})")
    fn = lambda a, w, s, c: grouped_mm(a, w, c, w_scale=s)
    if not (_self_test(fn, device, dtype) and _self_test(fn, device, dtype, quant=True)):
        raise RuntimeError("hmoe grouped_mm failed its known-answer self-test on this device")
    return "hip"


def fuse_moe(model, quant=""):
    """aurora/hf_compat.py:142-169: swap every MoE block's per-expert loop for the batched version; the per-expert
    modules are dropped (the stacked weights replace them).  Inference only.  quant="int8" (aurora/hf_compat.py:
    159-162): expert weights stored as int8 with a per-(expert, output column) bf16 scale, half the memory; the
    GEMMs read the int8 weights directly and still multiply in bf16."""
    assert quant in ("", "int8"), quant
    n = 0
    for mod in model.modules():
        experts = getattr(mod, "experts", None)
        if experts is None or not hasattr(mod, "moe_infer") or not isinstance(experts, torch.nn.ModuleList):
            continue
        # stacked per-expert weights, (E, in, out) and contiguous: wgu holds the gate then the up projection along
        # its last axis, wd the down projection; registered as non-persistent buffers so that moving the module to a
        # device or dtype carries them along
        wgu = torch.stack([torch.cat([e.gate_proj.weight, e.up_proj.weight]).t() for e in experts]).contiguous()
        wd = torch.stack([e.down_proj.weight.t() for e in experts]).contiguous()
        wgu, wd = _pad_stacks(wgu, wd, 16 if quant else 8)
        for name, w in (("_wgu", wgu), ("_wd", wd)):
            w, sc = _quant_int8(w) if quant else (w, None)
            mod.register_buffer(name, w, persistent=False)
            mod.register_buffer(name + "_s", sc, persistent=False)
        del wgu, wd
        mod._act = experts[0].act_fn
        mod._mode = None
        mod.moe_infer = types.MethodType(_fused_moe_infer, mod)
        del mod.experts
        mod.experts = list(range(mod._wgu.shape[0]))  # the expert count stays available as len(mod.experts)
        n += 1
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    return n
