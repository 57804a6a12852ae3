"""The BailingMoeV2 block (aurora/hf_pipeline.py:314-370) on the GPU against the oracle: the sigmoid, group-limited
router bit for bit (ids, weights, scores), the combine with the shared expert's addend, and PoziomkaMoE's forward
(int8 experts + shared expert) at small shapes and at the real one (E=128, top-8, d=2048, h=320)."""
import numpy as np
import pytest
import torch

from tests.util import assert_close_bf16, bits, f32

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,d,E,k,n_group,topk_group", [(1000, 2048, 128, 8, 8, 2), (333, 1536, 256, 8, 8, 4),
                                                        (200, 520, 64, 6, 4, 2), (100, 256, 32, 4, 4, 4),
                                                        (77, 1024, 16, 2, 1, 1)])
def test_route_sigmoid_group(oracle, T, d, E, k, n_group, topk_group):
    from trenowanie_generatora_obrazkow_amd import ops
    print(f"sigmoid group router T={T} d={d} E={E} k={k} groups {topk_group}/{n_group}", flush=True)
    g = torch.Generator().manual_seed(T + E)
    x = torch.randn(T, d, generator=g).bfloat16()
    wr = (torch.randn(E, d, generator=g) * 0.02).bfloat16()
    bias = torch.randn(E, generator=g) * 0.05
    dev = torch.device("cuda")
    for b in (None, bias):
        sc, ids, w = ops.route_sigmoid_group(x.to(dev), wr.to(dev), k, n_group, topk_group,
                                             expert_bias=None if b is None else b.to(dev), scaling=2.5,
                                             want_scores=True)
        _, rids, rw, rsc = oracle.route_sigmoid_group(bits(x), bits(wr), k, n_group, topk_group,
                                                      None if b is None else b.numpy(), 2.5)
        np.testing.assert_array_equal(ids.cpu().numpy(), rids)
        np.testing.assert_array_equal(w.cpu().numpy(), rw)
        np.testing.assert_array_equal(sc.cpu().numpy(), rsc)


def test_combine_add(oracle):
    from trenowanie_generatora_obrazkow_amd import ops
    T, k, d = 300, 8, 2048
    g = torch.Generator().manual_seed(9)
    y = torch.randn(T * k, d, generator=g).bfloat16()
    add = torch.randn(T, d, generator=g).bfloat16()
    out = ops.combine(y.cuda(), T, k, add=add.cuda())
    s = f32(y).reshape(T, k, d)
    acc = s[:, 0].copy()
    for j in range(1, k):
        acc = (acc + s[:, j]).astype(np.float32)  # fp32 sum in slot order
    ref = oracle.round_bf16(oracle.round_bf16(acc).astype(np.float32) + f32(add))
    np.testing.assert_array_equal(f32(out), ref)


def _make_block(oracle, d, h, E, k, n_group, topk_group, shared_h, seed):
    from trenowanie_generatora_obrazkow_amd.poziomka import PoziomkaMoE
    g = torch.Generator().manual_seed(seed)
    m = PoziomkaMoE(d, h, E, k, n_group, topk_group, 2.5, shared_h)
    with torch.no_grad():
        m.gate.weight.copy_(torch.randn(E, d, generator=g) * 0.02)
        m.gate.expert_bias.copy_(torch.randn(E, generator=g) * 0.05)
        for lin in (m.shared_experts.gate_proj, m.shared_experts.up_proj, m.shared_experts.down_proj):
            lin.weight.copy_(torch.randn(lin.weight.shape, generator=g) * 0.02)
        for name, shape in (("_wgu", (E, d, 2 * h)), ("_wd", (E, h, d))):
            q, s = oracle.quant_int8((torch.randn(shape, generator=g) * 0.02).numpy())
            getattr(m, name).copy_(torch.from_numpy(q))
            getattr(m, name + "_s").copy_(torch.from_numpy(s).bfloat16())
    return m.to(torch.bfloat16)  # the trunk runs in bf16: floating parameters and buffers become bf16


def _oracle_forward(oracle, m, x, k, n_group, topk_group):
    """Router, int8 experts and the shared expert from the module's own (bf16) tensors."""
    sh = m.shared_experts
    _, ids, w, _ = oracle.route_sigmoid_group(bits(x), bits(m.gate.weight), k, n_group, topk_group,
                                              f32(m.gate.expert_bias), m.scaling)
    xf = f32(x)
    moe = oracle.moe_forward(xf, ids, w, m._wgu.cpu().numpy().astype(np.float32),
                             m._wd.cpu().numpy().astype(np.float32), wgu_s=f32(m._wgu_s).astype(np.float64),
                             wd_s=f32(m._wd_s).astype(np.float64))
    wgu_sh = np.concatenate([f32(sh.gate_proj.weight), f32(sh.up_proj.weight)]).T[None]
    wd_sh = f32(sh.down_proj.weight).T[None]
    T = x.shape[0]
    shared = oracle.moe_forward(xf, np.zeros((T, 1), np.int64), np.ones((T, 1), np.float32), wgu_sh, wd_sh)
    return ids, oracle.round_bf16(moe["out"].astype(np.float64) + shared["out"].astype(np.float64)), shared["out"]


@pytest.mark.parametrize("T,d,h,E,k,n_group,topk_group", [(300, 512, 320, 32, 4, 4, 2),
                                                          (512, 2048, 320, 128, 8, 8, 2)])
def test_poziomka_moe_forward(oracle, T, d, h, E, k, n_group, topk_group):
    from trenowanie_generatora_obrazkow_amd import ops
    print(f"PoziomkaMoE T={T} d={d} h={h} E={E} k={k} groups {topk_group}/{n_group}", flush=True)
    m = _make_block(oracle, d, h, E, k, n_group, topk_group, h, seed=T + E)
    g = torch.Generator().manual_seed(T)
    x = torch.randn(2, T // 2, d, generator=g).bfloat16()
    mc = m.cuda()
    y = mc(x.cuda())
    assert y.shape == x.shape and y.dtype == torch.bfloat16
    x2 = x.reshape(T, d)
    ids, ref, shared_ref = _oracle_forward(oracle, m, x2, k, n_group, topk_group)
    _, gids, _ = ops.route_sigmoid_group(x2.cuda(), mc.gate.weight, k, n_group, topk_group,
                                         expert_bias=mc.gate.expert_bias, scaling=2.5)
    np.testing.assert_array_equal(gids.cpu().numpy(), ids)
    assert_close_bf16(f32(y).reshape(T, d), ref, "PoziomkaMoE")
    assert_close_bf16(f32(mc.shared_experts(x.cuda())).reshape(T, d), shared_ref, "shared expert")


def test_poziomka_varying_tokens(oracle):
    """Packed-caption calls (aurora/slayer.py:383-432): one block called with token counts that change call by call,
    no host synchronisation, each checked against the oracle; at 8192 tokens (the LM server's max_tokens) a sample
    of tokens is checked."""
    m = _make_block(oracle, 512, 320, 32, 4, 4, 2, 320, seed=11).cuda()
    g = torch.Generator().manual_seed(12)
    y0 = m(torch.empty(0, 512, dtype=torch.bfloat16, device="cuda"))  # an empty call returns an empty batch
    assert y0.shape == (0, 512)
    for T in (1, 17, 300, 2049):
        print(f"PoziomkaMoE T={T}", flush=True)
        x = torch.randn(T, 512, generator=g).bfloat16()
        y = m(x.cuda())
        _, ref, _ = _oracle_forward(oracle, m, x, 4, 4, 2)
        assert_close_bf16(f32(y), ref, f"T={T}")
    big = _make_block(oracle, 2048, 320, 128, 8, 8, 2, 320, seed=13).cuda()
    x = torch.randn(8192, 2048, generator=g).bfloat16()
    y = f32(big(x.cuda()))
    sample = np.array([0, 1, 2, 777, 4095, 4096, 6000, 8190, 8191] + list(range(100, 8192, 97)))
    _, ref, _ = _oracle_forward(oracle, big, x[sample], 8, 8, 2)
    assert_close_bf16(y[sample], ref, "T=8192 sample")


def test_poziomka_shared_overlap_bit_exact(oracle):
    """The shared expert on its side stream (overlap_shared, the default) gives the serial block's output bit for bit,
    for empty, single-token and larger calls, with other work queued on the current stream before each call."""
    m = _make_block(oracle, 512, 320, 32, 4, 4, 2, 320, seed=21).cuda()
    g = torch.Generator().manual_seed(22)
    for T in (0, 1, 300, 4096):
        print(f"PoziomkaMoE overlap T={T}", flush=True)
        x = torch.randn(T, 512, generator=g).bfloat16().cuda()
        m.overlap_shared = False
        ref = m(x).clone()
        m.overlap_shared = True
        torch.ones(1 << 20, device="cuda").mul_(2.0)  # unrelated work on the current stream ahead of the call
        got = m(x)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"T={T}"


def test_poziomka_graph_replay(oracle):
    """The forward at a fixed token count captured in a HIP graph (no host synchronisation, no allocation outside the
    graph's pool) and replayed on new inputs: every replay equals the eager forward bit for bit."""
    m = _make_block(oracle, 512, 320, 32, 4, 4, 2, 320, seed=21).cuda()
    g = torch.Generator().manual_seed(22)
    T = 1024
    xs = [torch.randn(T, 512, generator=g).bfloat16().cuda() for _ in range(4)]
    static_x = xs[0].clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        m(static_x)  # warm-up on the capture stream's device (first-use attributes set outside the capture)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_y = m(static_x)
    for i, x in enumerate(xs):
        eager = m(x)
        torch.cuda.synchronize()
        static_x.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_y, eager), f"replay {i}"


def test_poziomka_export_loaded_on_gpu(oracle, tmp_path):
    """The exported text encoder format (export.py:62-102): a safetensors file holding the fused trunk under "lm."
    (layer i's MoE block under "lm.layers.{i}.mlp.", a dense first layer and other tensors beside it) and
    text_encoder/config.json with the lm_* fields export.py writes.  load_export(..., device="cuda") builds the MoE
    blocks; each one's forward on the GPU matches the oracle run on the tensors as stored (fp32 expert bias kept
    unrounded, int8 experts with bf16 scales, bf16 router and shared expert)."""
    import json

    from safetensors.torch import save_file

    from trenowanie_generatora_obrazkow_amd.poziomka import export_state, load_export
    d, h, E, k, n_group, topk_group, sh = 512, 320, 32, 4, 4, 2, 320
    blocks = {}
    for i in (1, 2):
        m = _make_block(oracle, d, h, E, k, n_group, topk_group, sh, seed=40 + i)
        m.gate.expert_bias = torch.randn(E, generator=torch.Generator().manual_seed(50 + i)) * 0.05  # fp32
        blocks[i] = m
    sd = export_state(blocks)
    sd["lm.layers.0.mlp.gate_proj.weight"] = torch.zeros(1024, d, dtype=torch.bfloat16)  # the dense first layer
    sd["lm.layers.1.attention.query_key_value.weight"] = torch.zeros(64, d, dtype=torch.bfloat16)
    sd["lm.word_embeddings.weight"] = torch.zeros(100, d, dtype=torch.bfloat16)
    sd["blocks.0.attn.qkv.weight"] = torch.zeros(8, 8)  # the trained refiner's tensors
    te = tmp_path / "text_encoder"
    te.mkdir()
    save_file(sd, str(te / "diffusion_pytorch_model.safetensors"))
    cfg = {"_class_name": "AuroraLMTextEncoder", "kind": "lm", "lm_arch": "poziomka", "vocab_size": 100,
           "lm_blocks": 3, "lm_dim": d, "lm_heads": 8, "lm_kv_heads": 2, "lm_head_dim": 64, "lm_rotary_dim": 32,
           "lm_rope_theta": 10000.0, "lm_norm_eps": 1e-6, "lm_dense_layers": 1, "lm_intermediate": 1024,
           "lm_moe_intermediate": h, "lm_experts": E, "lm_top_k": k, "lm_n_group": n_group,
           "lm_topk_group": topk_group, "lm_routed_scaling": 2.5, "lm_shared_intermediate": sh}
    (te / "config.json").write_text(json.dumps(cfg))
    loaded = load_export(str(tmp_path), device="cuda")
    assert sorted(loaded) == [1, 2]
    g = torch.Generator().manual_seed(60)
    for i, m in loaded.items():
        print(f"export layer {i}", flush=True)
        assert m._wgu.is_cuda and m.gate.expert_bias.dtype == torch.float32
        x = torch.randn(2, 150, d, generator=g).bfloat16()
        y = m(x.cuda())
        ids, ref, _ = _oracle_forward(oracle, blocks[i], x.reshape(-1, d), k, n_group, topk_group)
        _, gids, _ = ops_route(m, x.reshape(-1, d), k, n_group, topk_group)
        np.testing.assert_array_equal(gids, ids)
        assert_close_bf16(f32(y).reshape(-1, d), ref, f"exported layer {i}")


def ops_route(m, x2, k, n_group, topk_group):
    from trenowanie_generatora_obrazkow_amd import ops
    sc, ids, w = ops.route_sigmoid_group(x2.cuda(), m.gate.weight, k, n_group, topk_group,
                                        expert_bias=m.gate.expert_bias, scaling=m.scaling)
    return sc, ids.cpu().numpy(), w
