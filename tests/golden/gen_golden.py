"""Writes the golden fixtures under tests/golden/ from the CPU oracle.

The reference (Josephur/fni8-serve) commits no vectors for this path, and its
arithmetic lives in the closed `fni8` wheel, which is absent, so these are
regression vectors of the oracle after it has been pinned by tests/test_oracle.py.
They freeze the oracle's exact outputs so that a later change to the oracle or to
the kernels shows up as a fixture mismatch.

    python tests/golden/gen_golden.py
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402
from oracle import oracle  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def quant_cases():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((12, 512)) * rng.uniform(0.01, 50, (12, 1))).astype(np.float16)
    x[rng.random(x.shape) < 0.01] *= 20
    x[0] = 0
    x[1, :] = np.float16(1e-7)
    x[2, ::2] = 2.5
    x[2, 1::2] = -127
    x[3, 11] = np.inf
    x[4, 100] = np.nan
    x[5] = np.float16(65504)
    q, s = oracle.quant_rowwise_f16(x)
    np.savez_compressed(os.path.join(HERE, "quant_rows.npz"), x=x, q=q, s=s)


def linear_small():
    rng = np.random.default_rng(11)
    M, N, K = 8, 64, 256
    x = rng.standard_normal((M, K)).astype(np.float16)
    x[rng.random(x.shape) < 0.01] *= 20
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws = rng.uniform(0.001, 0.02, N).astype(np.float16).astype(np.float32)
    bias = (rng.standard_normal(N) * 0.5).astype(np.float16)
    y, xq, xs, acc = oracle.linear_w8a8_f16(x, w, ws, bias)
    np.savez_compressed(os.path.join(HERE, "linear_small.npz"), x=x, w=w, ws=ws, bias=bias,
                        y=y, xq=xq, xs=xs, acc=acc)


def linear_cpu_case():
    """Qwen3-0.6B gate_up at M=8 (N=6144, K=1024): inputs come from the seeded
    workload generators; the fixture stores their digests and the outputs'."""
    pkg = __graft_entry__.load_package()
    from importlib import import_module
    wl = import_module(pkg.__name__ + ".workloads")
    c = wl.CPU_CASE
    x = wl.activations(c["M"], c["K"], seed=7).numpy()
    q, s = wl.weight_i8(c["N"], c["K"], seed=8)
    q, s = q.numpy(), s.numpy()
    y, xq, xs, acc = oracle.linear_w8a8_f16(x, q, s)
    out = {"M": c["M"], "N": c["N"], "K": c["K"], "x_seed": 7, "w_seed": 8,
           "sha256": {"x": sha(x), "w": sha(q), "ws": sha(s), "xq": sha(xq), "xs": sha(xs),
                      "acc": sha(acc), "y": sha(y.view(np.uint16))},
           "acc_row0_first8": acc[0, :8].tolist(),
           "y_row7_last4_bits": y[7, -4:].view(np.uint16).tolist()}
    with open(os.path.join(HERE, "linear_qwen3_0p6b_gate_up_m8.json"), "w") as f:
        json.dump(out, f, indent=1)


def moe_small():
    rng = np.random.default_rng(13)
    T, E, k, H, I = 24, 8, 2, 128, 64
    logits = rng.standard_normal((T, E)).astype(np.float32) - np.log1p(rng.permutation(E))
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    topi = np.argsort(-p, axis=1, kind="stable")[:, :k].astype(np.int32)
    topw = np.take_along_axis(p, topi, axis=1)
    topw = (topw / topw.sum(axis=1, keepdims=True)).astype(np.float16)
    x = rng.standard_normal((T, H)).astype(np.float16)
    wg = rng.integers(-127, 128, (E, 2 * I, H), dtype=np.int8)
    sg = rng.uniform(0.001, 0.02, (E, 2 * I)).astype(np.float32)
    seg, rt, rs, pos = oracle.moe_sort(topi, E)
    xq, xs = oracle.quant_rowwise_f16(x)
    h, hacc = oracle.grouped_w8a8_f16(xq, xs, wg, sg, seg, row_index=rt, want_acc=True)
    out = oracle.moe_combine_f16(h[:, :H], topi, topw, pos)
    np.savez_compressed(os.path.join(HERE, "moe_small.npz"), topi=topi, topw=topw, x=x, wg=wg,
                        sg=sg, seg=seg, row_token=rt, row_slot=rs, pos=pos, h=h, hacc=hacc,
                        combined=out)


if __name__ == "__main__":
    quant_cases()
    linear_small()
    linear_cpu_case()
    moe_small()
    print("fixtures written to", HERE)
