"""Host-side logic of the drop-in surfaces, without a GPU: the moe_triton facade's helpers and argument checks,
fuse_moe's weight stacking (aurora/hf_compat.py:142-169), mode selection refusing a CPU device, and the MoESwiGLU
module's parameters.  No kernel is launched."""
import math

import pytest
import torch
import torch.nn as nn

from trenowanie_generatora_obrazkow_amd import MoESwiGLU, moe_triton
from trenowanie_generatora_obrazkow_amd import hf_compat


def ref_m_bucket(M, E):
    """aurora/moe_triton.py:59-62 with triton.next_power_of_2 (smallest power of two >= n)."""
    n = max(1, M // E)
    p = 1
    while p < n:
        p *= 2
    return min(1024, max(16, p))


@pytest.mark.parametrize("M,E", [(0, 1), (1, 1), (48, 3), (32768, 16), (8192 * 8, 128), (100, 128), (5000, 7),
                                 (2 ** 20, 1)])
def test_m_bucket(M, E):
    assert moe_triton.m_bucket(M, E) == ref_m_bucket(M, E)
    assert moe_triton.BLOCK_M == 64


def test_facade_rejects_cpu_and_unsupported():
    a = torch.randn(48, 64).bfloat16()
    w = torch.randn(3, 64, 32).bfloat16()
    counts = torch.tensor([16, 0, 32])
    with pytest.raises(RuntimeError, match="GPU"):
        moe_triton.grouped_mm(a, w, counts)
    with pytest.raises(AssertionError):
        moe_triton.grouped_mm(a, w.transpose(1, 2).contiguous().transpose(1, 2), counts)
    with pytest.raises(ValueError):  # bf16 weights take no scale, int8 weights need one
        moe_triton.grouped_mm(a, w, counts, w_scale=torch.ones(3, 32))
    with pytest.raises(ValueError):
        moe_triton.grouped_mm(a, w.to(torch.int8), counts)
    with pytest.raises(RuntimeError, match="GPU"):
        moe_triton.grouped_mm(a, w.to(torch.int8), counts, w_scale=torch.ones(3, 32, dtype=torch.bfloat16))
    with pytest.raises(TypeError):
        moe_triton.grouped_mm(a.float(), w.float(), counts)
    with pytest.raises(RuntimeError, match="GPU"):
        moe_triton.make_schedule(counts, 48)


class _Expert(nn.Module):
    def __init__(self, d, h):
        super().__init__()
        self.gate_proj = nn.Linear(d, h, bias=False)
        self.up_proj = nn.Linear(d, h, bias=False)
        self.down_proj = nn.Linear(h, d, bias=False)
        self.act_fn = nn.functional.silu


class _Block(nn.Module):
    def __init__(self, d, h, E):
        super().__init__()
        self.experts = nn.ModuleList([_Expert(d, h) for _ in range(E)])

    def moe_infer(self, x, ids, w):
        raise AssertionError


def test_fuse_moe_stacks_reference_layout():
    torch.manual_seed(0)
    d, h, E = 32, 24, 5
    model = nn.Sequential(_Block(d, h, E), _Block(d, h, E))
    gates = [[e.gate_proj.weight.clone() for e in b.experts] for b in model]
    ups = [[e.up_proj.weight.clone() for e in b.experts] for b in model]
    downs = [[e.down_proj.weight.clone() for e in b.experts] for b in model]
    assert hf_compat.fuse_moe(model) == 2
    for bi, b in enumerate(model):
        assert b._wgu.shape == (E, d, 2 * h) and b._wd.shape == (E, h, d)
        for e in range(E):
            torch.testing.assert_close(b._wgu[e, :, :h], gates[bi][e].t())  # [gate | up], (in, out)
            torch.testing.assert_close(b._wgu[e, :, h:], ups[bi][e].t())
            torch.testing.assert_close(b._wd[e], downs[bi][e].t())
        assert b._wgu.is_contiguous() and b._wgu_s is None and b._mode is None
        assert b.experts == list(range(E))
        with pytest.raises(RuntimeError, match="GPU"):
            b.moe_infer(torch.randn(4, d), torch.zeros(4, 2, dtype=torch.long), torch.ones(4, 2))


def test_fuse_moe_int8_buffers():
    """quant="int8" (aurora/hf_compat.py:159-162): int8 stacked weights with (E, out) bf16 scales that dequantise
    to within half a step of the stacked bf16 weights."""
    torch.manual_seed(1)
    d, h, E = 32, 48, 5
    blk = _Block(d, h, E)
    wgu = torch.stack([torch.cat([e.gate_proj.weight, e.up_proj.weight]).t() for e in blk.experts]).detach()
    wd = torch.stack([e.down_proj.weight.t() for e in blk.experts]).detach()
    assert hf_compat.fuse_moe(nn.Sequential(blk), quant="int8") == 1
    assert blk._wgu.dtype == torch.int8 and blk._wgu.shape == (E, d, 2 * h)
    assert blk._wd.dtype == torch.int8 and blk._wd.shape == (E, h, d)
    assert blk._wgu_s.shape == (E, 2 * h) and blk._wd_s.shape == (E, d) and blk._wgu_s.dtype == torch.bfloat16
    for q, s, w in ((blk._wgu, blk._wgu_s, wgu), (blk._wd, blk._wd_s, wd)):
        deq = hf_compat._dequant(q, s, torch.float32)
        # half a step from rounding q, plus 127 x the bf16 rounding of the scale (<= 2^-8 relative)
        assert ((deq - w).abs() <= s.float().unsqueeze(1) * (0.5 + 127 * 2.0 ** -8) * 1.01).all()
    with pytest.raises(RuntimeError, match="GPU"):
        blk.moe_infer(torch.randn(4, d), torch.zeros(4, 2, dtype=torch.long), torch.ones(4, 2))


@pytest.mark.parametrize("quant,gr", [("", 8), ("int8", 16)])
def test_fuse_moe_pads_off_granule_widths(quant, gr):
    """Widths off the kernels' copy granule: the stacks are zero-padded to it once, the real block sits in place
    ([gate | pad | up | pad] along the output axis), int8 values and scales of the real columns are those of the
    unpadded stack bit for bit, and the padded layer computed in float64 equals the unpadded one on the d columns
    (padded hidden columns are silu(0) * 0 and meet zero down rows)."""
    torch.manual_seed(3)
    d, h, E = 36, 20, 3
    blk = _Block(d, h, E)
    wgu = torch.stack([torch.cat([e.gate_proj.weight, e.up_proj.weight]).t() for e in blk.experts]).detach()
    wd = torch.stack([e.down_proj.weight.t() for e in blk.experts]).detach()
    assert hf_compat.fuse_moe(nn.Sequential(blk), quant=quant) == 1
    dp, hp = -(-d // gr) * gr, -(-h // gr) * gr
    assert blk._wgu.shape == (E, dp, 2 * hp) and blk._wd.shape == (E, hp, dp)
    cols = list(range(h)) + list(range(hp, hp + h))
    if quant:
        q_gu, s_gu = hf_compat._quant_int8(wgu)
        q_d, s_d = hf_compat._quant_int8(wd)
        assert torch.equal(blk._wgu[:, :d, cols], q_gu) and torch.equal(blk._wgu_s[:, cols], s_gu)
        assert torch.equal(blk._wd[:, :h, :d], q_d) and torch.equal(blk._wd_s[:, :d], s_d)
        gu_p, d_p = hf_compat._dequant(blk._wgu, blk._wgu_s, torch.float64), hf_compat._dequant(blk._wd, blk._wd_s,
                                                                                                  torch.float64)
        gu_r, d_r = hf_compat._dequant(q_gu, s_gu, torch.float64), hf_compat._dequant(q_d, s_d, torch.float64)
    else:
        assert torch.equal(blk._wgu[:, :d, cols], wgu) and torch.equal(blk._wd[:, :h, :d], wd)
        gu_p, d_p, gu_r, d_r = blk._wgu.double(), blk._wd.double(), wgu.double(), wd.double()
    pad_mask = torch.ones(E, dp, 2 * hp, dtype=torch.bool)
    pad_mask[:, :d, cols] = False
    assert (gu_p[pad_mask] == 0).all() and d_p[:, h:].abs().sum() == 0 and d_p[:, :, d:].abs().sum() == 0
    x = torch.randn(7, d, dtype=torch.float64)
    xp = torch.nn.functional.pad(x, (0, dp - d))
    for e in range(E):
        gp = xp @ gu_p[e]
        yp = (torch.nn.functional.silu(gp[:, :hp]) * gp[:, hp:]) @ d_p[e]
        g = x @ gu_r[e]
        y = (torch.nn.functional.silu(g[:, :h]) * g[:, h:]) @ d_r[e]
        torch.testing.assert_close(yp[:, :d], y, rtol=1e-12, atol=1e-12)


def test_pad_operands_for_grouped_mm():
    """moe_triton.pad_operands: K to a multiple of 8, N to 8 (16-bit weights) or 16 (int8), zeros in the padding,
    aligned shapes passed through as the same tensors."""
    a, w = torch.randn(10, 13).bfloat16(), torch.randn(3, 13, 7).bfloat16()
    ap, wp, sp = moe_triton.pad_operands(a, w)
    assert ap.shape == (10, 16) and wp.shape == (3, 16, 8) and sp is None
    assert torch.equal(ap[:, :13], a) and (ap[:, 13:] == 0).all()
    assert torch.equal(wp[:, :13, :7], w) and wp[:, 13:].abs().sum() == 0 and wp[:, :, 7:].abs().sum() == 0
    q, s = torch.randint(-127, 128, (3, 16, 20), dtype=torch.int8), torch.rand(3, 20).bfloat16()
    a16 = torch.randn(4, 16).bfloat16()
    ap, qp, sp = moe_triton.pad_operands(a16, q, s)
    assert ap is a16 and qp.shape == (3, 16, 32) and sp.shape == (3, 32)
    assert torch.equal(qp[:, :, :20], q) and (qp[:, :, 20:] == 0).all() and torch.equal(sp[:, :20], s)
    w8 = torch.randn(2, 16, 8).bfloat16()
    assert moe_triton.pad_operands(a16, w8)[1] is w8


def test_quant_int8_matches_reference_rule():
    w = torch.randn(3, 64, 16)
    q, s = hf_compat._quant_int8(w)
    assert q.dtype == torch.int8 and s.dtype == torch.bfloat16
    deq = hf_compat._dequant(q, s, torch.float32)
    assert (deq - w).abs().max() <= (w.abs().amax(1).max() / 127) * 0.51 + 1e-2


def test_moe_swiglu_module_shapes():
    torch.manual_seed(0)
    m = MoESwiGLU(64, 96, 8, top_k=2)
    assert m.router_weight.shape == (8, 64) and m.w_gu.shape == (8, 64, 192) and m.w_d.shape == (8, 96, 64)
    assert m.w_gu.dtype == torch.bfloat16
    # the reference's initialisation convention: N(0, in_features ** -0.5) (aurora/model.py:393-396)
    for p, fan_in in ((m.router_weight, 64), (m.w_gu, 64), (m.w_d, 96)):
        assert abs(p.float().std().item() / fan_in ** -0.5 - 1) < 0.1
    m2 = MoESwiGLU(64, 96, 8, top_k=2, init_std=0.02)
    assert abs(m2.w_gu.float().std().item() - 0.02) < 2e-3
    assert m.logit_bias.dtype == torch.float32 and (m.logit_bias == 0).all()
    with pytest.raises(RuntimeError, match="GPU"):
        m(torch.randn(2, 5, 64))


def test_reference_init_code_runs_on_moe_block():
    """The reference initialises a block's FFN through nn.Linear attributes: Denoiser.init_block (aurora/model.py:
    393-396: normal_(lin.weight, std=lin.in_features ** -0.5) for mlp.in_proj and mlp.out_proj), the text encoder's
    init_weights (:308-312: in_proj the same way, out_proj zeroed) and train_pp --init (train_pp.py:1420-1421:
    out_proj zeroed in new blocks).  Those loops, restated here on a stand-in block whose mlp is a MoESwiGLU, reach
    the stacked expert parameters: every expert gets the fan-in std, out_proj zeroes every expert, the state dict
    keeps only the stacked names."""
    torch.manual_seed(1)
    dim, hidden, E = 256, 512, 8
    block = nn.Module()
    block.mlp = MoESwiGLU(dim, hidden, E, init_std=0.5)
    with torch.no_grad():
        for lin in (block.mlp.in_proj, block.mlp.out_proj):        # init_block
            nn.init.normal_(lin.weight, std=lin.in_features ** -0.5)
    assert block.mlp.in_proj.in_features == dim and block.mlp.out_proj.in_features == hidden
    assert block.mlp.in_proj.out_features == 2 * hidden and block.mlp.out_proj.out_features == dim
    for w, fan_in in ((block.mlp.w_gu, dim), (block.mlp.w_d, hidden)):
        per_expert = w.detach().float().reshape(E, -1).std(dim=1)
        assert torch.allclose(per_expert, torch.full((E,), fan_in ** -0.5), rtol=0.03), per_expert
    with torch.no_grad():
        nn.init.normal_(block.mlp.in_proj.weight, std=block.mlp.in_proj.in_features ** -0.5)   # text init_weights
        nn.init.zeros_(block.mlp.out_proj.weight)
    assert not block.mlp.w_d.detach().float().abs().any()
    assert block.mlp.in_proj.weight is block.mlp.w_gu and block.mlp.out_proj.weight is block.mlp.w_d
    assert set(block.state_dict()) == {"mlp.router_weight", "mlp.w_gu", "mlp.w_d", "mlp.logit_bias"}


def test_moe_swiglu_rejects_mismatched_shapes_before_launch():
    """The functional layer cross-checks router, expert stacks, bias and k on the host, before any kernel call
    (here on CPU tensors: the shape errors come first)."""
    from trenowanie_generatora_obrazkow_amd import moe_swiglu
    E, d, h, T = 4, 64, 32, 10
    x = torch.zeros(T, d, dtype=torch.bfloat16)
    wr, wgu, wd = (torch.zeros(s, dtype=torch.bfloat16) for s in ((E, d), (E, d, 2 * h), (E, h, d)))
    for args, err in (((x, torch.zeros(E + 1, d, dtype=torch.bfloat16), wgu, wd, 2), ValueError),
                      ((x, wr, torch.zeros(E, d, 2 * h + 2, dtype=torch.bfloat16), wd, 2), ValueError),
                      ((x, wr, wgu, torch.zeros(E, h, d, dtype=torch.int8), 2), TypeError),
                      ((x.float(), wr, wgu, wd, 2), TypeError),
                      ((x, wr, wgu, wd, 0), ValueError)):
        with pytest.raises(err):
            moe_swiglu(*args)
    with pytest.raises(ValueError):
        moe_swiglu(x, wr, wgu, wd, 2, logit_bias=torch.zeros(E - 1))


def test_poziomka_module_layout():
    """PoziomkaMoE keeps the reference's module tree, names, shapes and dtypes (aurora/hf_pipeline.py:314-346), so the
    reference's state dicts load unchanged; its forward refuses CPU tensors (no CPU path)."""
    from trenowanie_generatora_obrazkow_amd.poziomka import PoziomkaMLP, PoziomkaMoE
    d, h, E, sh = 64, 32, 16, 48
    m = PoziomkaMoE(d, h, E, 4, 4, 2, 2.5, sh)
    sd = m.state_dict()
    expect = {"gate.weight": ((E, d), torch.float32), "gate.expert_bias": ((E,), torch.float32),
              "shared_experts.gate_proj.weight": ((sh, d), torch.float32),
              "shared_experts.up_proj.weight": ((sh, d), torch.float32),
              "shared_experts.down_proj.weight": ((d, sh), torch.float32),
              "_wgu": ((E, d, 2 * h), torch.int8), "_wgu_s": ((E, 2 * h), torch.bfloat16),
              "_wd": ((E, h, d), torch.int8), "_wd_s": ((E, d), torch.bfloat16)}
    assert set(sd) == set(expect)
    for key, (shape, dt) in expect.items():
        assert tuple(sd[key].shape) == shape and sd[key].dtype == dt, key
    assert (m.top_k, m.n_group, m.topk_group, m.scaling) == (4, 4, 2, 2.5)
    m2 = PoziomkaMoE(d, h, E, 4, 4, 2, 2.5, sh)
    m2.load_state_dict(sd)
    mb = m.to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        mb(torch.zeros(3, d, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="GPU"):
        PoziomkaMLP(d, sh).bfloat16()(torch.zeros(2, d, dtype=torch.bfloat16))


def _rand_block(d, h, E, sh, seed):
    from trenowanie_generatora_obrazkow_amd.poziomka import PoziomkaMoE
    g = torch.Generator().manual_seed(seed)
    m = PoziomkaMoE(d, h, E, 4, 4, 2, 2.5, sh)
    with torch.no_grad():
        for name, t in list(m.named_parameters()) + list(m.named_buffers()):
            if t.dtype == torch.int8:
                t.copy_(torch.randint(-127, 128, t.shape, generator=g, dtype=torch.int8))
            else:
                t.copy_(torch.randn(t.shape, generator=g) * 0.02)
    return m.to(torch.bfloat16)


def test_poziomka_export_round_trip(tmp_path):
    """load_export reads the layout export.py:62-102 writes (config.json lm_* fields; the fused trunk under "lm.",
    layer i's block under "lm.layers.{i}.mlp."), skips dense layers and other tensors, and export_state writes the same
    keys back."""
    import json

    from safetensors.torch import save_file

    from trenowanie_generatora_obrazkow_amd.poziomka import export_state, load_export
    d, h, E, sh = 64, 32, 16, 48
    blocks = {i: _rand_block(d, h, E, sh, seed=i) for i in (1, 2)}
    sd = export_state(blocks)
    assert "lm.layers.1.mlp._wgu" in sd and "lm.layers.2.mlp.shared_experts.down_proj.weight" in sd
    sd["lm.layers.0.mlp.gate_proj.weight"] = torch.zeros(128, d, dtype=torch.bfloat16)  # the dense first layer
    sd["lm.word_embeddings.weight"] = torch.zeros(10, d, dtype=torch.bfloat16)
    sd["blocks.0.attn.qkv.weight"] = torch.zeros(8, 8)  # refiner tensors
    te = tmp_path / "text_encoder"
    te.mkdir()
    save_file(sd, str(te / "diffusion_pytorch_model.safetensors"))
    cfg = {"lm_arch": "poziomka", "lm_blocks": 3, "lm_dense_layers": 1, "lm_dim": d, "lm_moe_intermediate": h,
           "lm_experts": E, "lm_top_k": 4, "lm_n_group": 4, "lm_topk_group": 2, "lm_routed_scaling": 2.5,
           "lm_shared_intermediate": sh}
    (te / "config.json").write_text(json.dumps(cfg))
    for p in (tmp_path, te, te / "diffusion_pytorch_model.safetensors"):
        got = load_export(str(p))
        assert sorted(got) == [1, 2]
        for i, m in got.items():
            ref = blocks[i].state_dict()
            for k, v in m.state_dict().items():
                assert v.dtype == ref[k].dtype and torch.equal(v, ref[k]), (i, k)
            assert (m.top_k, m.n_group, m.topk_group, m.scaling) == (4, 4, 2, 2.5)
    cfg["lm_arch"] = "gollem"
    (te / "config.json").write_text(json.dumps(cfg))
    with pytest.raises(ValueError):
        load_export(str(tmp_path))


def test_swap_moe_replaces_reference_blocks():
    """swap_moe finds blocks with the reference PoziomkaMoE's attributes (a stand-in class here) and replaces them by
    this package's PoziomkaMoE with identical tensors."""
    from trenowanie_generatora_obrazkow_amd.poziomka import PoziomkaMoE, swap_moe
    d, h, E, sh = 64, 32, 16, 48
    src = _rand_block(d, h, E, sh, seed=7)

    class RefBlock(nn.Module):  # same attributes and state layout as aurora/hf_pipeline.py:332-346
        def __init__(self):
            super().__init__()
            self.top_k, self.n_group, self.topk_group, self.scaling = 4, 4, 2, 2.5
            self.gate = nn.Module()
            self.gate.weight = nn.Parameter(src.gate.weight.detach().clone())
            self.gate.register_buffer("expert_bias", src.gate.expert_bias.clone())
            self.shared_experts = nn.Module()
            for n in ("gate_proj", "up_proj", "down_proj"):
                lin = nn.Linear(1, 1, bias=False)
                lin.weight = nn.Parameter(getattr(src.shared_experts, n).weight.detach().clone())
                setattr(self.shared_experts, n, lin)
            for n in ("_wgu", "_wgu_s", "_wd", "_wd_s"):
                self.register_buffer(n, getattr(src, n).clone())

    class Layer(nn.Module):
        def __init__(self):
            super().__init__()
            self.mlp = RefBlock()

    model = nn.Sequential(Layer(), Layer())
    assert swap_moe(model) == 2
    for layer in model:
        assert isinstance(layer.mlp, PoziomkaMoE)
        for k, v in layer.mlp.state_dict().items():
            assert torch.equal(v, src.state_dict()[k]), k
    assert swap_moe(model) == 0


def test_poziomka_expert_bias_keeps_its_precision(tmp_path):
    """The reference selects experts on scores + expert_bias.float() (aurora/hf_pipeline.py:353), so an fp32 bias
    must survive from_reference / swap_moe and load_export unrounded even when the block's weights are bf16: a bias
    that is not bf16-exact comes back bit for bit, in fp32."""
    import json

    from safetensors.torch import save_file

    from trenowanie_generatora_obrazkow_amd.poziomka import export_state, from_reference, load_export
    d, h, E, sh = 64, 32, 16, 48
    src = _rand_block(d, h, E, sh, seed=3)
    bias = (torch.randn(E, generator=torch.Generator().manual_seed(4)) * 0.01 + 1e-3).float()
    assert not torch.equal(bias.bfloat16().float(), bias)  # not representable in bf16
    src.gate.expert_bias = bias.clone()
    m = from_reference(src)
    assert m.gate.expert_bias.dtype == torch.float32 and torch.equal(m.gate.expert_bias, bias)
    assert m.gate.weight.dtype == torch.bfloat16
    te = tmp_path / "text_encoder"
    te.mkdir()
    save_file(export_state({1: src}), str(te / "diffusion_pytorch_model.safetensors"))
    cfg = {"lm_arch": "poziomka", "lm_blocks": 2, "lm_dense_layers": 1, "lm_dim": d, "lm_moe_intermediate": h,
           "lm_experts": E, "lm_top_k": 4, "lm_n_group": 4, "lm_topk_group": 2, "lm_routed_scaling": 2.5,
           "lm_shared_intermediate": sh}
    (te / "config.json").write_text(json.dumps(cfg))
    got = load_export(str(tmp_path))[1]
    assert got.gate.expert_bias.dtype == torch.float32 and torch.equal(got.gate.expert_bias, bias)
    assert got.gate.weight.dtype == torch.bfloat16 and got._wgu_s.dtype == torch.bfloat16


def _reference_rule(prefix, name, p):
    """The group the reference's param_groups gives a parameter (train.py:314-325): the token embedding, 2-D matrices
    under `.blocks.` of the text encoder or the denoiser ("hidden": Muon), other 2-D matrices ("proj": AdamW with
    weight decay), everything else ("other": AdamW without)."""
    full = f"{prefix}.{name}"
    if full == "te.token_embedding.weight":
        return "emb"
    if prefix in ("te", "den") and ".blocks." in f".{name}" and p.ndim == 2 and not name.endswith("mod_table"):
        return "hidden"
    if p.ndim == 2 and not name.endswith("mod_table"):
        return "proj"
    return "other"


def test_moe_param_groups_against_the_reference_rule():
    """A denoiser-like module whose block MLP is a MoESwiGLU: under the reference's grouping rule alone the router
    would go to Muon ("hidden") and the expert stacks to AdamW's "other" group (no weight decay); with
    moe_param_groups the stacks get the hidden learning rate and weight decay, the router its own AdamW group, and
    filtering the returned ids leaves no MoE parameter for the rule (so none is in two groups), while the block's
    other matrices still go to Muon."""
    from trenowanie_generatora_obrazkow_amd import moe_param_groups

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.attn = nn.Linear(64, 64, bias=False)
            self.norm = nn.LayerNorm(64)
            self.mlp = MoESwiGLU(64, 96, experts=4, top_k=2, device="cpu")

    class Den(nn.Module):
        def __init__(self):
            super().__init__()
            self.patch_in = nn.Linear(16, 64)
            self.blocks = nn.ModuleList([Block(), Block()])

    den = Den()
    named = [("den", n, p) for n, p in den.named_parameters()]
    before = {n: _reference_rule(pre, n, p) for pre, n, p in named}
    assert before["blocks.0.mlp.router_weight"] == "hidden"
    assert before["blocks.0.mlp.w_gu"] == "other" and before["blocks.1.mlp.w_d"] == "other"

    groups, ids = moe_param_groups(den, lr=0.02, weight_decay=0.1, router_lr=1e-3)
    by_name = {g["name"]: g for g in groups}
    ex, rt = by_name["moe_experts"], by_name["moe_router"]
    mlps = [b.mlp for b in den.blocks]
    assert [id(p) for p in ex["params"]] == [id(p) for m in mlps for p in (m.w_gu, m.w_d)]
    assert [id(p) for p in rt["params"]] == [id(m.router_weight) for m in mlps]
    assert ex["lr"] == ex["base_lr"] == 0.02 and ex["weight_decay"] == 0.1
    assert rt["lr"] == 1e-3 and rt["weight_decay"] == 0.0
    rest = [(pre, n, p) for pre, n, p in named if id(p) not in ids]
    after = {n: _reference_rule(pre, n, p) for pre, n, p in rest}
    assert not any(".mlp." in n for n in after)
    assert after["blocks.0.attn.weight"] == "hidden" and after["patch_in.weight"] == "proj"
    assert len(rest) + len(ids) == len(named)
    # the groups build an optimizer as they are
    torch.optim.AdamW(groups, betas=(0.9, 0.95))
