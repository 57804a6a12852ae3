"""Drop-in for the reference's BailingMoeV2 MoE block (cpral/Poziomka-Baza), aurora/hf_pipeline.py:314-370:
`PoziomkaMLP`, `PoziomkaGate` and `PoziomkaMoE` with the same constructor arguments, module tree, parameter and buffer
names, shapes and dtypes, so a state dict written for the reference classes loads unchanged (export.py:62-72 stores
the experts as int8 with bf16 per-column scales, exactly these buffers).

Forward, inference only (the reference block is frozen), served by the hmoe kernels:

  1. router (`hmoe_route_sigmoid_group`): fp32 logits, sigmoid scores, expert bias for selection, group-limited top-k
     (best `topk_group` of `n_group` groups by the sum of their two largest routing values), weights = the selected
     scores renormalised and scaled (aurora/hf_pipeline.py:352-359);
  2. stable counting sort of the routed rows (`hmoe_dispatch`), the routing weight rounded to bf16 (:361);
  3. gate/up grouped GEMM over the int8 experts with the SwiGLU in its epilogue, scale after the fp32 sum, one
     rounding (:365-367); down grouped GEMM, per-column scale, routing weight, one rounding, rows scattered back to
     (token, slot) order (:368-369);
  4. the shared expert (a dense SwiGLU MLP, :342 / :322) as the same two GEMMs over one "expert" holding every token;
  5. combine: the k slots summed in fp32, rounded, plus the shared expert's output (:369-370).

`load_export` reads the exported text encoder (export.py:62-102) into these blocks, `export_state` writes them back
in that format, and `swap_moe` replaces the reference's blocks inside a loaded trunk.  Calls take any token count
(packed captions of varying total length, aurora/slayer.py:383-432) without a host synchronisation, so a forward of
a fixed token count can be captured in a HIP graph and replayed.

The reference adds the k slot outputs with `index_add_` in expert order; here they are summed in slot order (same
terms, fp32 accumulation; the bf16 results can differ in the last place).  There is no CPU path: tensors must live
on a ROCm GPU.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import ops


def _bf16_exact(w: torch.Tensor, name: str) -> torch.Tensor:
    """The hmoe kernels read bf16 weights; a wider weight must hold bf16 values (the reference's exports do)."""
    if w.dtype == torch.bfloat16:
        return w
    wb = w.to(torch.bfloat16)
    if not torch.equal(wb.to(w.dtype), w):
        raise TypeError(f"{name}: the hmoe kernels take bf16 weights; this {w.dtype} weight is not bf16-exact")
    return wb


class _StackedMLP:
    """A dense SwiGLU MLP run as a one-expert grouped GEMM pair: [gate | up] stacked (1, d, 2h), down (1, h, d) --
    the layout fuse_moe gives the routed experts (aurora/hf_compat.py:154-155).  Rebuilt when a weight changes."""

    def __init__(self):
        self.key = None
        self.wgu = self.wd = None

    def get(self, mlp: "PoziomkaMLP"):
        ws = (mlp.gate_proj.weight, mlp.up_proj.weight, mlp.down_proj.weight)
        key = tuple((w.data_ptr(), w._version, w.device, w.dtype) for w in ws)
        if key != self.key:
            g, u, dn = (_bf16_exact(w.detach(), n) for w, n in zip(ws, ("gate_proj", "up_proj", "down_proj")))
            self.wgu = torch.cat([g, u]).t().contiguous().unsqueeze(0)
            self.wd = dn.t().contiguous().unsqueeze(0)
            self.key = key
        return self.wgu, self.wd


_ROW_COUNTS = {}  # device index -> int32 arange, entry T = T
_OLD_ROW_COUNTS = []  # outgrown aranges, never freed: kernels on any stream may still read them


def _one_count(T: int, device: torch.device) -> torch.Tensor:
    """(1,) int32 on `device` holding T, the row count of a one-expert grouped GEMM: a view of a cached arange (no
    launch per call), grown by doubling; while a graph is being captured and the arange is too short, a fill kernel
    instead (allocations made under capture belong to the graph)."""
    key = device.index if device.index is not None else torch.cuda.current_device()
    ar = _ROW_COUNTS.get(key)
    if ar is None or ar.numel() <= T:
        if torch.cuda.is_current_stream_capturing():
            return torch.full((1,), T, dtype=torch.int32, device=device)
        if ar is not None:
            _OLD_ROW_COUNTS.append(ar)
        ar = torch.arange(max(1024, 1 << T.bit_length()), dtype=torch.int32, device=device)
        torch.cuda.current_stream(device).synchronize()  # complete before any stream reads it
        _ROW_COUNTS[key] = ar
    return ar[T:T + 1]


def _dense_swiglu(x2: torch.Tensor, wgu: torch.Tensor, wd: torch.Tensor) -> torch.Tensor:
    """bf16(bf16(silu(bf16(x Wg))) * bf16(x Wu)) Wd rounded to bf16 -- F.linear / F.silu in bf16 (aurora/
    hf_pipeline.py:322) -- for x2 (T, d) bf16."""
    T = x2.shape[0]
    one = _one_count(T, x2.device)
    act, _ = ops.gate_up_swiglu(x2, wgu, one, T)
    y, _ = ops.down_scatter(act, wd, one, T, None, None)
    return y


class PoziomkaMLP(nn.Module):
    """aurora/hf_pipeline.py:314-322: down(silu(gate(x)) * up(x)), bias-free, bf16."""

    def __init__(self, d, hidden):
        super().__init__()
        self.gate_proj = nn.Linear(d, hidden, bias=False)
        self.up_proj = nn.Linear(d, hidden, bias=False)
        self.down_proj = nn.Linear(hidden, d, bias=False)
        self._stack = _StackedMLP()

    @torch.no_grad()
    def forward(self, x):
        shape = x.shape
        x2 = x.reshape(-1, shape[-1]).contiguous()
        if x2.dtype != torch.bfloat16:
            raise TypeError(f"hmoe PoziomkaMLP runs bf16 activations (got {x2.dtype})")
        wgu, wd = self._stack.get(self)
        return _dense_swiglu(x2, wgu, wd).view(shape)


class PoziomkaGate(nn.Module):
    """aurora/hf_pipeline.py:325-329: router weight (E, d) and the selection-only expert bias (E,)."""

    def __init__(self, d, experts):
        super().__init__()
        self.weight = nn.Parameter(torch.zeros(experts, d))
        self.register_buffer("expert_bias", torch.zeros(experts))


class PoziomkaMoE(nn.Module):
    """aurora/hf_pipeline.py:332-370: BailingMoeV2 sparse MoE with int8 experts and one shared expert, inference
    only.  Buffers as the reference: _wgu (E, d, 2h) int8 = [gate | up], _wgu_s (E, 2h) bf16, _wd (E, h, d) int8,
    _wd_s (E, d) bf16 (bf16 expert stacks with the scales set to None are accepted too)."""

    def __init__(self, d, hidden, experts, top_k, n_group, topk_group, scaling, shared_hidden):
        super().__init__()
        self.top_k, self.n_group, self.topk_group, self.scaling = top_k, n_group, topk_group, scaling
        self.gate = PoziomkaGate(d, experts)
        self.shared_experts = PoziomkaMLP(d, shared_hidden)
        self.register_buffer("_wgu", torch.zeros(experts, d, 2 * hidden, dtype=torch.int8))
        self.register_buffer("_wgu_s", torch.zeros(experts, 2 * hidden, dtype=torch.bfloat16))
        self.register_buffer("_wd", torch.zeros(experts, hidden, d, dtype=torch.int8))
        self.register_buffer("_wd_s", torch.zeros(experts, d, dtype=torch.bfloat16))
        self._gate_key = None
        self._gate_w = None
        # The shared expert runs on a side stream of the same (default) priority, so its GEMMs can take the CUs the
        # routed GEMMs leave idle in their last rounds; False runs it after the routed path on the current stream.
        self.overlap_shared = True

    def _gate_tensors(self):
        """bf16 router weight and fp32 expert bias as the kernel takes them, converted once per weight version."""
        w, b = self.gate.weight, self.gate.expert_bias
        key = (w.data_ptr(), w._version, w.device, w.dtype, b.data_ptr(), b._version, b.dtype)
        if key != self._gate_key:
            self._gate_w = (_bf16_exact(w.detach(), "gate.weight").contiguous(),
                            b.detach().to(torch.float32).contiguous())
            self._gate_key = key
        return self._gate_w

    @torch.no_grad()
    def forward(self, x):
        shape = x.shape
        x2 = x.reshape(-1, shape[-1]).contiguous()
        if x2.dtype != torch.bfloat16:
            raise TypeError(f"hmoe PoziomkaMoE runs bf16 activations (got {x2.dtype})")
        T, k, E = x2.shape[0], self.top_k, self._wgu.shape[0]
        gw, gb = self._gate_tensors()
        wgu_sh, wd_sh = self.shared_experts._stack.get(self.shared_experts)
        side = ops.side_stream(x2.device) if self.overlap_shared and T > 0 else None
        if side is not None:  # fork: the shared expert needs only x
            main = torch.cuda.current_stream(x2.device)
            fork_ev, join_ev = ops.side_events(x2.device)
            fork_ev.record(main)
            side.wait_event(fork_ev)
            with torch.cuda.stream(side):
                shared = _dense_swiglu(x2, wgu_sh, wd_sh)
            x2.record_stream(side)
        _, ids, w = ops.route_sigmoid_group(x2, gw, k, self.n_group, self.topk_group, expert_bias=gb,
                                            scaling=self.scaling)
        # dispatch, both int8 projections, routing weight and scatter in one C call
        y, _, _ = ops.moe_experts(x2, ids, w, self._wgu, self._wd, wgu_s=self._wgu_s, wd_s=self._wd_s)
        if side is not None:  # join before the combine reads the shared output
            join_ev.record(side)
            main.wait_event(join_ev)
            shared.record_stream(main)
        else:
            shared = _dense_swiglu(x2, wgu_sh, wd_sh)
        return ops.combine(y, T, k, add=shared).view(shape)



# ---------------------------------------------------------------------------------------------------------------
# On-disk format: the exported text encoder (export.py:62-102) and swapping the reference's blocks
# ---------------------------------------------------------------------------------------------------------------
_MOE_KEYS = ("gate.weight", "gate.expert_bias", "shared_experts.gate_proj.weight", "shared_experts.up_proj.weight",
             "shared_experts.down_proj.weight", "_wgu", "_wgu_s", "_wd", "_wd_s")


def _export_paths(path):
    import os
    if os.path.isdir(path):
        d = os.path.join(path, "text_encoder") if os.path.isdir(os.path.join(path, "text_encoder")) else path
        return os.path.join(d, "config.json"), os.path.join(d, "diffusion_pytorch_model.safetensors")
    return os.path.join(os.path.dirname(path), "config.json"), path


def load_export(path, device=None, dtype=torch.bfloat16) -> dict:
    """The MoE blocks of an exported Poziomka text encoder, as export.py:62-102 writes it: `text_encoder/config.json`
    (lm_* fields) and `diffusion_pytorch_model.safetensors` holding the fused trunk under "lm." (layer i's block
    under "lm.layers.{i}.mlp.": gate.weight, gate.expert_bias, shared_experts.{gate,up,down}_proj.weight, and the
    int8 stacks _wgu / _wgu_s / _wd / _wd_s of aurora/hf_compat.py:154-162).  `path` is the export root, its
    text_encoder directory, or the safetensors file.  Returns {layer index: PoziomkaMoE} for the MoE layers
    (index >= lm_dense_layers), floating tensors in `dtype` (the trunk runs bf16), on `device`."""
    import json

    from safetensors import safe_open
    cfg_path, st_path = _export_paths(path)
    with open(cfg_path) as f:
        cfg = json.load(f)
    if cfg.get("lm_arch") != "poziomka":
        raise ValueError(f"{cfg_path}: not a Poziomka text encoder export (lm_arch={cfg.get('lm_arch')!r})")
    blocks = {}
    with safe_open(st_path, framework="pt", device="cpu") as f:
        keys = set(f.keys())
        for i in range(cfg["lm_dense_layers"], cfg["lm_blocks"]):
            pre = f"lm.layers.{i}.mlp."
            missing = [k for k in _MOE_KEYS if pre + k not in keys]
            if missing:
                raise KeyError(f"{st_path}: layer {i} lacks {missing}")
            m = PoziomkaMoE(cfg["lm_dim"], cfg["lm_moe_intermediate"], cfg["lm_experts"], cfg["lm_top_k"],
                            cfg["lm_n_group"], cfg["lm_topk_group"], cfg["lm_routed_scaling"],
                            cfg["lm_shared_intermediate"])
            sd = {k: f.get_tensor(pre + k) for k in _MOE_KEYS}
            m.gate.expert_bias = torch.empty_like(sd["gate.expert_bias"])  # loaded in the dtype it was stored in
            m.load_state_dict(sd, strict=True)
            blocks[i] = _place(m, dtype, device)
    return blocks


def _place(m: PoziomkaMoE, dtype, device) -> PoziomkaMoE:
    """m's floating tensors in `dtype` on `device`, except the expert bias: it only takes part in the selection,
    which the reference computes as scores + expert_bias.float() (aurora/hf_pipeline.py:353), so it keeps the
    precision it has (an fp32 bias rounded to bf16 could select other experts)."""
    bias = m.gate.expert_bias
    m = m.to(dtype=dtype)
    m.gate.expert_bias = bias
    return m.to(device=device) if device is not None else m


def export_state(blocks: dict) -> dict:
    """{layer index: PoziomkaMoE} -> the "lm.layers.{i}.mlp." tensors of the export format (load_export's keys)."""
    return {f"lm.layers.{i}.mlp.{k}": v.detach().cpu().contiguous()
            for i, m in blocks.items() for k, v in m.state_dict().items()}


def from_reference(mod) -> PoziomkaMoE:
    """A PoziomkaMoE with the configuration and tensors of the reference's block (aurora/hf_pipeline.py:332-346, or
    any module with the same attributes and state dict), on the same device and dtypes."""
    E, d, h2 = mod._wgu.shape
    sh = mod.shared_experts.gate_proj.weight.shape[0]
    m = PoziomkaMoE(d, h2 // 2, E, mod.top_k, mod.n_group, mod.topk_group, mod.scaling, sh)
    m.gate.expert_bias = torch.empty_like(mod.gate.expert_bias)  # the reference block's bias keeps its dtype
    m = _place(m, mod.gate.weight.dtype, mod._wgu.device)
    m.load_state_dict(mod.state_dict(), strict=True)
    return m


def swap_moe(model) -> int:
    """Replace every reference PoziomkaMoE block inside `model` (recognised by its attributes: _wgu, gate,
    shared_experts, top_k, n_group, topk_group, scaling) by this module's PoziomkaMoE with the same tensors.
    Returns the number of blocks replaced."""
    n = 0
    for parent in list(model.modules()):
        for name, child in list(parent.named_children()):
            if isinstance(child, PoziomkaMoE):
                continue
            if all(hasattr(child, a) for a in ("_wgu", "gate", "shared_experts", "top_k", "n_group", "topk_group",
                                                "scaling")):
                setattr(parent, name, from_reference(child))
                n += 1
    return n
