"""Writes the small golden fixtures under tests/golden/ from the CPU oracle (oracle/), on seeded inputs.

The oracle functions used here are pinned in tests/test_oracle.py against closed forms, brute force, torch's own
routines (softmax/topk, argsort/bincount, _grouped_mm, autograd) and hand-derived known answers; the fixtures
freeze their outputs so that any later change to the oracle or to the HIP path is caught against fixed data.

Run from the repository root:  python tests/golden/gen_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import build as ob  # noqa: E402

if not os.path.exists(ob.OUT):
    ob.build()
from oracle import moe_oracle as O  # noqa: E402


def bf16_values(rng, shape, std=1.0):
    return O.round_bf16(rng.standard_normal(shape).astype(np.float32) * np.float32(std))


def router_cases():
    rng = np.random.default_rng(11)
    out = {}
    for name, (T, d, E, k, renorm, scaling, zipf) in {
        "a": (64, 256, 8, 2, True, 1.0, False),
        "b": (33, 520, 5, 3, False, 2.5, False),
        "c": (128, 1536, 16, 2, True, 1.0, True),
    }.items():
        x = bf16_values(rng, (T, d))
        wr = bf16_values(rng, (E, d), 0.02)
        bias = O.zipf_bias(E, seed=3) if zipf else None
        logits, ids, w = O.route(O.f32_to_bf16_bits(x), O.f32_to_bf16_bits(wr), k, bias=bias, renorm=renorm,
                                 scaling=scaling)
        out.update({f"{name}_x": O.f32_to_bf16_bits(x), f"{name}_wr": O.f32_to_bf16_bits(wr),
                    f"{name}_bias": bias if bias is not None else np.zeros(0, np.float32),
                    f"{name}_params": np.array([T, d, E, k, int(renorm)], np.int64),
                    f"{name}_scaling": np.float32(scaling), f"{name}_logits": logits, f"{name}_ids": ids,
                    f"{name}_w": w})
    np.savez_compressed(os.path.join(HERE, "router.npz"), **out)


def dispatch_cases():
    rng = np.random.default_rng(12)
    out = {}
    for name, (T, k, E) in {"a": (100, 3, 7), "b": (257, 2, 16), "c": (40, 8, 128)}.items():
        p = np.array([0.0 if e % 5 == 1 else 1.0 / (e + 1) for e in range(E)])
        ids = rng.choice(E, size=(T, k), p=p / p.sum()).astype(np.int64)
        r = O.dispatch(ids, E)
        out.update({f"{name}_ids": ids, f"{name}_E": np.int64(E), f"{name}_counts": r["counts"],
                    f"{name}_order": r["order"], f"{name}_a_idx": r["a_idx"], f"{name}_inv_pos": r["inv_pos"]})
    np.savez_compressed(os.path.join(HERE, "dispatch.npz"), **out)


def schedule_cases():
    out = {}
    for i, counts in enumerate([[16, 0, 32], [0, 0, 5], [64, 64, 1, 0, 200], [0] * 7 + [1000], [130] * 16]):
        c = np.array(counts, np.int64)
        be, br, re_ = O.make_schedule(c, int(c.sum()))
        out.update({f"s{i}_counts": c, f"s{i}_block_e": be, f"s{i}_block_row": br, f"s{i}_row_end": re_})
    np.savez_compressed(os.path.join(HERE, "schedule.npz"), **out)


def selftest_case():
    """The reference's known-answer construction (aurora/hf_compat.py:112-121): 48x64 @ (3, 64, 32), counts
    [16, 0, 32]; expected = per-expert float64 matmul, rounded once to bf16."""
    rng = np.random.default_rng(13)
    a = bf16_values(rng, (48, 64))
    b = bf16_values(rng, (3, 64, 32))
    counts = np.array([16, 0, 32], np.int64)
    y = O.grouped_mm(a, b, counts)
    np.savez_compressed(os.path.join(HERE, "selftest.npz"), a=O.f32_to_bf16_bits(a), b=O.f32_to_bf16_bits(b),
                        counts=counts, y=O.f32_to_bf16_bits(y))


def layer_case():
    rng = np.random.default_rng(14)
    T, d, E, k, h = 48, 64, 4, 2, 32
    x = bf16_values(rng, (T, d))
    wr = bf16_values(rng, (E, d), 0.05)
    wgu = bf16_values(rng, (E, d, 2 * h), 0.05)
    wd = bf16_values(rng, (E, h, d), 0.05)
    dout = bf16_values(rng, (T, d))
    logits, ids, w = O.route(O.f32_to_bf16_bits(x), O.f32_to_bf16_bits(wr), k)
    fwd = O.moe_forward(x, ids, w, wgu, wd)
    bwd = O.layer_backward(x, wr, ids, w, logits, wgu, wd, dout, fwd=fwd)
    np.savez_compressed(os.path.join(HERE, "layer.npz"), x=O.f32_to_bf16_bits(x), wr=O.f32_to_bf16_bits(wr),
                        wgu=O.f32_to_bf16_bits(wgu), wd=O.f32_to_bf16_bits(wd), dout=O.f32_to_bf16_bits(dout),
                        params=np.array([T, d, E, k, h], np.int64), logits=logits, ids=ids, w=w,
                        out=O.f32_to_bf16_bits(fwd["out"]), dx=bwd["dx"], dwr=bwd["dwr"], dwgu=bwd["dwgu"],
                        dwd=bwd["dwd"], dtopk_w=bwd["dtopk_w"], dlogits=bwd["dlogits"])


if __name__ == "__main__":
    router_cases()
    dispatch_cases()
    schedule_cases()
    selftest_case()
    layer_case()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
