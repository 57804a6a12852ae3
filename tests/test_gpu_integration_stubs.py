"""The ctypes bindings INTEGRATION.md shows a maintainer (grouped_mm, the one-call forward) run as written and give
the package's own results bit for bit, so the documented argument lists match the C ABI."""
import os
import re

import pytest
import torch

from tests.util import make_inputs

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _stubs():
    src = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```python\n(.*?)```", src, flags=re.S)
    code = "\n".join(b for b in blocks if "_L.hmoe_grouped_mm.argtypes" in b or "_L.hmoe_moe_forward.argtypes" in b)
    lib = os.path.join(ROOT, "trenowanie_generatora_obrazkow_amd", "_lib", "libhmoe.so")
    code = code.replace('"trenowanie_generatora_obrazkow_amd/_lib/libhmoe.so"', repr(lib))
    ns = {}
    exec(code, ns)
    return ns


def test_documented_bindings_match_the_package():
    from trenowanie_generatora_obrazkow_amd import moe_triton, ops
    ns = _stubs()
    assert "grouped_mm" in ns and "moe_forward" in ns
    dev = torch.device("cuda")
    x, wr, wgu, wd = (t.to(dev) for t in make_inputs(300, 512, 8, 256, seed=3))
    out, ids, w = ns["moe_forward"](x, wr, wgu, wd, 2)
    ref = ops.moe_forward(x, wr, wgu, wd, 2)
    assert torch.equal(out.view(torch.int16), ref[0].view(torch.int16))
    assert torch.equal(ids, ref[1]) and torch.equal(w, ref[2])
    counts = torch.tensor([100, 0, 200], dtype=torch.int32, device=dev)
    g = torch.Generator().manual_seed(0)
    a = torch.randn(300, 64, generator=g).bfloat16().to(dev)
    wg = (torch.randn(3, 64, 128, generator=g) * 0.1).bfloat16().to(dev)
    y = ns["grouped_mm"](a, wg, counts)
    assert torch.equal(y.view(torch.int16), moe_triton.grouped_mm(a, wg, counts).view(torch.int16))
