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
    int8-weight forms of the two GEMMs (per-column scales applied to the fp32 sums).  An expert id outside [0, E)
    in topk_ids routes its slot nowhere: the slot adds nothing to the output, and the count of such ids is kept on
    the device in self._n_invalid (read by invalid_expert_ids, which is the only place that synchronises)."""
    n, k = topk_ids.shape
    E = self._wgu.shape[0]
    if self._mode is None:  # decided on the device the weights ended up on
        self._mode = _pick_mode(x.device, x.dtype)
    if self._act is not torch.nn.functional.silu and not isinstance(self._act, torch.nn.SiLU):
        raise NotImplementedError("the hmoe SwiGLU epilogue implements silu(g) * u only")
    x = x.contiguous()
    disp, act, _ = ops.routed_gate_up(x, topk_ids.contiguous(), E, self._wgu, topk_w=topk_weight.contiguous(),
                                      wgu_s=self._wgu_s, want_inv=True)
    M = n * k
    y, _ = ops.down_scatter(act, self._wd, disp.counts, M, disp.w_sorted, disp.order, wd_s=self._wd_s)
    self._n_invalid = disp.n_invalid
    return ops.combine(y, n, k, inv_pos=disp.inv_pos)


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
