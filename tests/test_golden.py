"""The oracle reproduces the committed golden fixtures bit for bit (CPU), and the
HIP path reproduces them too (GPU).  Fixtures: tests/golden/gen_golden.py."""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

from oracle import oracle

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    with np.load(os.path.join(G, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _same_f32(a, b):
    return np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(a[~np.isnan(a)], b[~np.isnan(b)])


def test_oracle_quant_rows_fixture():
    f = _load("quant_rows.npz")
    q, s = oracle.quant_rowwise_f16(f["x"])
    assert np.array_equal(q, f["q"]) and _same_f32(s, f["s"])


def test_oracle_linear_small_fixture():
    f = _load("linear_small.npz")
    y, xq, xs, acc = oracle.linear_w8a8_f16(f["x"], f["w"], f["ws"], f["bias"])
    assert np.array_equal(xq, f["xq"]) and np.array_equal(xs, f["xs"])
    assert np.array_equal(acc, f["acc"])
    assert np.array_equal(y.view(np.uint16), f["y"].view(np.uint16))


def test_oracle_cpu_case_digest(pkg, wl):
    with open(os.path.join(G, "linear_qwen3_0p6b_gate_up_m8.json")) as fh:
        d = json.load(fh)
    x = wl.activations(d["M"], d["K"], seed=d["x_seed"]).numpy()
    q, s = wl.weight_i8(d["N"], d["K"], seed=d["w_seed"])
    q, s = q.numpy(), s.numpy()
    assert _sha(x) == d["sha256"]["x"] and _sha(q) == d["sha256"]["w"]
    y, xq, xs, acc = oracle.linear_w8a8_f16(x, q, s)
    assert _sha(xq) == d["sha256"]["xq"] and _sha(acc) == d["sha256"]["acc"]
    assert _sha(y.view(np.uint16)) == d["sha256"]["y"]
    assert acc[0, :8].tolist() == d["acc_row0_first8"]


def test_oracle_moe_fixture():
    f = _load("moe_small.npz")
    seg, rt, rs, pos = oracle.moe_sort(f["topi"], f["wg"].shape[0])
    assert np.array_equal(seg, f["seg"]) and np.array_equal(rt, f["row_token"])
    assert np.array_equal(pos, f["pos"])
    xq, xs = oracle.quant_rowwise_f16(f["x"])
    h, hacc = oracle.grouped_w8a8_f16(xq, xs, f["wg"], f["sg"], seg, row_index=rt, want_acc=True)
    assert np.array_equal(hacc, f["hacc"]) and np.array_equal(h.view(np.uint16), f["h"].view(np.uint16))
    H = f["x"].shape[1]
    out = oracle.moe_combine_f16(h[:, :H], f["topi"], f["topw"], pos)
    assert np.array_equal(out.view(np.uint16), f["combined"].view(np.uint16))


@pytest.mark.gpu
def test_gpu_matches_fixtures(pkg, wl, cuda):
    f = _load("quant_rows.npz")
    q, s = pkg.quantize_rowwise(torch.from_numpy(f["x"]).cuda())
    assert np.array_equal(q.cpu().numpy(), f["q"]) and _same_f32(s.cpu().numpy(), f["s"])

    f = _load("linear_small.npz")
    qt = pkg.QTensor(torch.from_numpy(f["w"]).cuda(), torch.from_numpy(f["ws"]).cuda(),
                     scheme="per_row_i8")
    y, xq, xs, acc = pkg.linear_with_intermediates(torch.from_numpy(f["x"]).cuda(), qt,
                                                   torch.from_numpy(f["bias"]).cuda(), want_acc=True)
    assert np.array_equal(acc.cpu().numpy(), f["acc"])
    assert np.array_equal(y.cpu().numpy().view(np.uint16), f["y"].view(np.uint16))

    with open(os.path.join(G, "linear_qwen3_0p6b_gate_up_m8.json")) as fh:
        d = json.load(fh)
    x = wl.activations(d["M"], d["K"], seed=d["x_seed"])
    qw, sw = wl.weight_i8(d["N"], d["K"], seed=d["w_seed"])
    y, xq, xs, acc = pkg.linear_with_intermediates(
        x.cuda(), pkg.QTensor(qw.cuda(), sw.cuda(), scheme="per_row_i8"), want_acc=True)
    assert _sha(xq.cpu().numpy()) == d["sha256"]["xq"]
    assert _sha(acc.cpu().numpy()) == d["sha256"]["acc"]
    assert _sha(y.cpu().numpy().view(np.uint16)) == d["sha256"]["y"]

    f = _load("moe_small.npz")
    E = f["wg"].shape[0]
    topi = torch.from_numpy(f["topi"]).cuda()
    seg, rt, pos = pkg.moe_sort(topi, E)
    assert np.array_equal(seg.cpu().numpy(), f["seg"]) and np.array_equal(pos.cpu().numpy(), f["pos"])
    xq, xs = pkg.quantize_rowwise(torch.from_numpy(f["x"]).cuda())
    R = f["topi"].size
    h, hacc = pkg.gemm_w8a8_grouped(xq, xs, torch.from_numpy(f["wg"]).cuda(),
                                    torch.from_numpy(f["sg"]).cuda(), seg, R, row_index=rt,
                                    want_acc=True)
    assert np.array_equal(hacc.cpu().numpy(), f["hacc"])
    H = f["x"].shape[1]
    out = pkg.moe_combine(h[:, :H].contiguous(), topi, torch.from_numpy(f["topw"]).cuda(), pos)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), f["combined"].view(np.uint16))
