"""The C-ABI library (libhmoe.so) loads without a GPU and exports exactly the entry points include/hmoe.h declares,
with the argument counts the Python binding uses; argument validation returns the documented error codes before
any device work (no kernel is launched here).  CPU only."""
import ctypes
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hmoe.h")


def header_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    protos = re.findall(r"^(?:int|size_t|const char\*)\s+(hmoe_\w+)\(([^;]*?)\);", src, flags=re.M | re.S)
    return {name: (0 if args.strip() == "void" else args.count(",") + 1) for name, args in protos}


@pytest.fixture(scope="module")
def lib():
    from trenowanie_generatora_obrazkow_amd import _lib
    return _lib


def test_every_declared_symbol_is_exported(lib):
    decl = header_functions()
    assert len(decl) >= 17
    so = ctypes.CDLL(lib.LIB_PATH)
    for name in decl:
        assert hasattr(so, name), f"{name} declared in include/hmoe.h but not exported"


def test_binding_matches_header(lib):
    decl = header_functions()
    assert set(decl) == set(lib.SIGNATURES), set(decl) ^ set(lib.SIGNATURES)
    for name, nargs in decl.items():
        assert len(lib.SIGNATURES[name][1]) == nargs, name


def test_exports_nothing_undeclared(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\sT\s(hmoe_\w+)", out))
    assert exported == set(header_functions())


def test_version_and_errors(lib):
    L = lib.lib()
    assert L.hmoe_abi_version() == 2
    for code, word in ((0, "ok"), (-1, "argument"), (-2, "shape"), (-3, "type"), (-4, "launch"), (-5, "workspace"),
                       (-7, "scratch")):
        assert word in L.hmoe_error_string(code).decode()


def test_argument_validation_codes(lib):
    L = lib.lib()
    P = 4096  # a non-null stand-in address: never dereferenced, no kernel is launched on these paths
    # router: negative T, bad alignment, too many experts
    assert L.hmoe_route_topk(P, 8, P, None, -1, 8, 4, 2, 1, 1.0, None, P, P, None) == -1
    assert L.hmoe_route_topk(P, 8, P, None, 0, 8, 4, 2, 1, 1.0, None, P, P, None) == 0  # empty input
    assert L.hmoe_route_topk(P, 8, P, None, 4, 8, 300, 2, 1, 1.0, None, P, P, None) == -2
    assert L.hmoe_route_topk(P + 2, 8, P, None, 4, 8, 4, 2, 1, 1.0, None, P, P, None) == -1
    assert L.hmoe_route_topk(P, 8, P, None, 4, 12, 4, 2, 1, 1.0, None, P, P, None) == -1  # d % 8
    # sigmoid group router: E % n_group, group size a power of two in [2, 64], enough experts in the kept groups
    assert L.hmoe_route_sigmoid_group(P, 8, P, None, 4, 8, 128, 8, 6, 2, 2.5, None, P, P, None) == -2
    assert L.hmoe_route_sigmoid_group(P, 8, P, None, 4, 8, 96, 8, 8, 2, 2.5, None, P, P, None) == -2  # 12 per group
    assert L.hmoe_route_sigmoid_group(P, 8, P, None, 4, 8, 128, 8, 8, 9, 2.5, None, P, P, None) == -2
    assert L.hmoe_route_sigmoid_group(P, 8, P, None, 4, 8, 16, 5, 8, 2, 2.5, None, P, P, None) == -2  # 5 > 2 * 2
    assert L.hmoe_route_sigmoid_group(P, 8, P, None, 0, 8, 128, 8, 8, 2, 2.5, None, P, P, None) == 0
    # dispatch: dtype, workspace, E bounds
    ws = L.hmoe_dispatch_workspace_size(16, 2, 4)
    assert L.hmoe_dispatch(P, 2, None, 0, 16, 2, 4, None, 0, 0, None, P, None, P, P, P, P, None, None, P, ws, 0,
                           None) == -3
    assert L.hmoe_dispatch(P, 4, None, 0, 16, 2, 4, None, 0, 0, None, P, None, P, P, P, P, None, None, P, ws - 1, 0,
                           None) == -5
    assert L.hmoe_dispatch(P, 4, None, 0, 16, 2, 2000, None, 0, 0, None, P, None, P, P, P, P, None, None, P, ws, 0,
                           None) == -2
    # a missing order or topk_ids is refused before the first launch (counts / starts stay untouched)
    assert L.hmoe_dispatch(P, 4, None, 0, 16, 2, 4, None, 0, 0, None, P, None, P, None, P, P, None, None, P, ws, 0,
                           None) == -1
    assert L.hmoe_dispatch(None, 4, None, 0, 16, 2, 4, None, 0, 0, None, P, None, P, P, P, P, None, None, P, ws, 0,
                           None) == -1
    # the activation type: bf16 (0) or fp16 (1)
    assert L.hmoe_dispatch(P, 4, None, 0, 16, 2, 4, None, 0, 0, None, P, None, P, P, P, P, None, None, P, ws, 2,
                           None) == -3
    # grouped_mm: K % 8, fp32 input, int8 weights
    assert L.hmoe_grouped_mm(P, 64, 0, P, 0, 3, 60, 32, 60 * 32, 32, P, 4, 48, None, None, None, 0, None, 0, P, 32,
                             None) == -2
    assert L.hmoe_grouped_mm(P, 64, 2, P, 2, 3, 64, 32, 64 * 32, 32, P, 4, 48, None, None, None, 0, None, 0, P, 32,
                             None) == -3  # fp32 activations
    assert L.hmoe_grouped_mm(P, 64, 1, P, 0, 3, 64, 32, 64 * 32, 32, P, 4, 48, None, None, None, 0, None, 0, P, 32,
                             None) == -3  # fp16 a with bf16 w
    assert L.hmoe_grouped_mm(P, 64, 1, P, 1, 3, 64, 32, 64 * 32, 32, P, 4, 48, None, None, P, 0, None, 0, P, 32,
                             None) == -3  # fp16 a with a bf16 row scale
    assert L.hmoe_grouped_mm(P, 64, 0, P, 0, 3, 64, 32, 64 * 32, 32, P, 4, 48, None, None, None, 0, P, 0, P, 32,
                             None) == -3
    assert L.hmoe_grouped_mm(P, 64, 0, P, 0, 3, 64, 32, 64 * 32, 32, P, 4, 0, None, None, None, 0, None, 0, P, 32,
                             None) == 0  # M == 0: nothing to do
    assert L.hmoe_grouped_mm(P, 64, 0, P, 0, 3, 64, 32, 64 * 32, 32, None, 4, 48, None, None, None, 0, None, 0, P,
                             32, None) == -1
    # int8 weights: scales required, N % 16, scale dtype
    assert L.hmoe_grouped_mm(P, 64, 0, P, 5, 3, 64, 32, 64 * 32, 32, P, 4, 48, None, None, None, 0, None, 0, P, 32,
                             None) == -1
    assert L.hmoe_grouped_mm(P, 64, 0, P, 5, 3, 64, 40, 64 * 48, 48, P, 4, 48, None, None, None, 0, P, 0, P, 40,
                             None) == -2
    assert L.hmoe_grouped_mm(P, 64, 0, P, 5, 3, 64, 32, 64 * 32, 32, P, 4, 48, None, None, None, 0, P, 3, P, 32,
                             None) == -3
    assert L.hmoe_gate_up_swiglu_i8(P, 64, None, P, P, 0, 3, 64, 24, P, 4, 48, P, 0, None) == -2  # h % 16
    assert L.hmoe_gate_up_swiglu_i8(P, 64, None, P, P, 0, 3, 64, 32, P, 4, 0, P, 0, None) == 0
    assert L.hmoe_gate_up_swiglu_i8(P, 64, None, None, P, 0, 3, 64, 32, P, 4, 48, P, 0, None) == -1
    assert L.hmoe_gate_up_swiglu_i8(P, 64, None, P, P, 0, 3, 64, 32, P, 4, 48, P, 2, None) == -3  # fp32 activations
    assert L.hmoe_down_scatter_i8(P, P, P, 4, 3, 32, 64, P, 4, 48, P, P, P, 0, None) == -3  # scale dtype
    assert L.hmoe_down_scatter_i8(P, P, P, 0, 3, 32, 72, P, 4, 48, P, P, P, 1, None) == -2  # d % 16
    # direct-load offsets beyond 2^31 bytes
    assert L.hmoe_gate_up_swiglu(P, 4096, P, P, 3, 4096, 65536, P, 4, 1 << 20, P, None, 0, None) == -2
    assert L.hmoe_down_scatter(P, P, 3, 64, 64, P, 4, 48, P, P, P, None, 4, None) == -3  # int64 activations
    # 2^31 routed rows or more (the GEMMs keep row starts in 32 bits)
    assert L.hmoe_down_scatter(P, P, 3, 64, 64, P, 4, 1 << 31, P, P, P, None, 0, None) == -2
    assert L.hmoe_grouped_wgrad(P, 64, P, 64, 3, 64, 64, P, 4, 1 << 31, P, 2, None) == -2
    # wgrad: output dtype, shapes
    assert L.hmoe_grouped_wgrad(P, 64, P, 64, 3, 64, 64, P, 4, 48, P, 3, None) == -3
    assert L.hmoe_grouped_wgrad(P, 64, P, 64, 3, 60, 64, P, 4, 48, P, 2, None) == -2
    # combine / backward elementwise
    assert L.hmoe_combine(P, None, 4, 2, 12, P, 0, None) == -1
    assert L.hmoe_combine(P, None, 4, 2, 16, P, 2, None) == -3
    assert L.hmoe_unpermute_bwd(P, 5, P, None, None, 4, 2, 64, 0, P, None) == -3
    assert L.hmoe_router_bwd(P, P, P, 16, 300, 2, 1, 1.0, P, 64, 64, P, None, 2, None, 0, None) == -2
    assert L.hmoe_router_bwd(P, P, P, 16, 8, 2, 1, 1.0, P, 64, 64, P, P, 2, None, 0, None) == -5
    # one-call forward: workspace missing / short, misaligned operands, widths off the granule, k > E, empty input
    ws = L.hmoe_moe_forward_workspace_size(4, 64, 8, 2, 64)
    fwd = lambda x, T, d, E, k, h, ws_ptr, ws_b: L.hmoe_moe_forward(x, d, P, None, P, P, T, d, E, k, h, 1, 1.0, P, P, P,
                                                                    None, ws_ptr, ws_b, None)
    assert fwd(P, 4, 64, 8, 2, 64, None, 0) == -5
    assert fwd(P, 4, 64, 8, 2, 64, P, ws - 1) == -5
    assert fwd(P + 8, 4, 64, 8, 2, 64, P, ws) == -1
    assert fwd(P, 4, 64, 8, 2, 64, P + 16, ws) == -1  # workspace not 256-byte aligned
    assert fwd(P, 4, 64, 8, 2, 60, P, L.hmoe_moe_forward_workspace_size(4, 64, 8, 2, 60)) == -2
    assert fwd(P, 4, 64, 8, 9, 64, P, ws) == -1
    assert fwd(P, 0, 64, 8, 2, 64, None, 0) == 0
    # one-call experts: workspace, int8 weights without scales, a 16-bit weight type other than the activations',
    # widths off the int8 granule, misaligned workspace
    BF, F16, I8, I32_, F32 = 0, 1, 5, 3, 2
    wse = L.hmoe_moe_experts_workspace_size(4, 64, 8, 2, 64, BF, BF)
    exp = lambda wdt, h, wgu_s, wd_s, ws_ptr, ws_b, dt=BF: L.hmoe_moe_experts(
        P, 64, P, I32_, P, F32, P, wgu_s, BF, P, wd_s, BF, wdt, 4, 64, 8, 2, h, P, P, P, ws_ptr, ws_b, dt, None)
    assert exp(BF, 64, None, None, P, wse - 1) == -5
    assert exp(I8, 64, None, None, P, L.hmoe_moe_experts_workspace_size(4, 64, 8, 2, 64, I8, BF)) == -1
    assert exp(F16, 64, None, None, P, wse) == -3
    assert exp(I8, 40, P, P, P, L.hmoe_moe_experts_workspace_size(4, 64, 8, 2, 40, I8, BF)) == -2
    assert exp(BF, 64, None, None, P + 64, wse) == -1
    assert exp(BF, 64, None, None, P, wse, dt=F32) == -3
    assert L.hmoe_moe_experts_workspace_size(-1, 64, 8, 2, 64, BF, BF) == 0


def test_workspace_queries(lib):
    L = lib.lib()
    a = L.hmoe_dispatch_workspace_size(16384, 2, 16)
    b = L.hmoe_dispatch_workspace_size(16384, 2, 128)
    assert 0 < a < b and a % 256 == 0
    # one fp32 (E, d) partial per 128-token chunk
    assert L.hmoe_router_bwd_workspace_size(16384, 16, 1536) == 128 * 16 * 1536 * 4
    assert L.hmoe_router_bwd_workspace_size(129, 16, 1536) == 2 * 16 * 1536 * 4
    # one-call forward: at least the router logits (T E), act (M h), y (M d), the sort arrays and the dispatch
    # workspace; the row-group tiles only from h = 4096 on; 0 for sizes no entry point takes
    T, d, E, k = 2048, 1024, 8, 2
    M = T * k
    base = T * E * 4 + M * 2048 * 2 + M * d * 2 + 3 * M * 4 + M * 2 + L.hmoe_dispatch_workspace_size(T, k, E)
    small = L.hmoe_moe_forward_workspace_size(T, d, E, k, 2048)
    assert base <= small < base + 16 * 256 and small % 256 == 0
    wide = L.hmoe_moe_forward_workspace_size(T, d, E, k, 4096)
    assert wide - small >= M * 2048 * 2 + L.hmoe_xs_tiles_bytes(M, E, d)
    assert L.hmoe_moe_forward_workspace_size(T, d, E, 9, 2048) == 0 and L.hmoe_moe_forward_workspace_size(-1, d, E, k, 64) == 0


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 2 and "one GPU" in r.stderr
