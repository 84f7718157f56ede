"""GPU parity of the grouped (MoE) path: routing sort, grouped W8A8 GEMMs and the
weighted combine, against the oracle and against the per-expert loop it replaces
(fni8serve/models/moe.py:97-105)."""
import numpy as np
import pytest
import torch

from oracle import oracle
from oracle.reference_cpu import reference_moe_loop

pytestmark = pytest.mark.gpu


def _routing(wl, T, E, k, seed):
    logits = wl.router_logits(T, E, seed=seed)
    topw, topi = wl.route(logits, k)
    return topw, topi


@pytest.mark.parametrize("T", [1, 16, 256, 4096])
def test_moe_sort_matches_oracle(pkg, wl, cuda, T):
    E, k = wl.MOE["experts"], wl.MOE["top_k"]
    _, topi = _routing(wl, T, E, k, seed=T)
    seg, rt, pos = pkg.moe_sort(topi.cuda(), E)
    torch.cuda.synchronize()
    seg_r, rt_r, _, pos_r = oracle.moe_sort(topi.numpy(), E)
    assert np.array_equal(seg.cpu().numpy(), seg_r)
    assert np.array_equal(rt.cpu().numpy(), rt_r)
    assert np.array_equal(pos.cpu().numpy(), pos_r)


def test_moe_sort_skewed_and_empty_experts(pkg, cuda):
    E, T, k = 64, 300, 4
    g = torch.Generator().manual_seed(5)
    # most tokens on experts 0-3, many experts empty, every row's ids distinct
    topi = torch.stack([torch.randperm(6, generator=g)[:k] for _ in range(T)])
    topi[::7] = torch.tensor([60, 61, 62, 63])
    seg, rt, pos = pkg.moe_sort(topi.cuda(), E)
    seg_r, rt_r, _, pos_r = oracle.moe_sort(topi.numpy(), E)
    assert np.array_equal(seg.cpu().numpy(), seg_r)
    assert np.array_equal(rt.cpu().numpy(), rt_r)
    assert np.array_equal(pos.cpu().numpy(), pos_r)


@pytest.mark.parametrize("T", [16, 256, 4096])
@pytest.mark.parametrize("proj", ["gate_up", "down"])
def test_grouped_gemm_bitexact(pkg, wl, cuda, T, proj):
    E, k, H, I = (wl.MOE[n] for n in ("experts", "top_k", "hidden", "inter"))
    N, K = (2 * I, H) if proj == "gate_up" else (H, I)
    _, topi = _routing(wl, T, E, k, seed=T + 1)
    w, ws = wl.expert_weights(E, N, K, seed=3 if proj == "gate_up" else 4)
    seg, rt, _ = pkg.moe_sort(topi.cuda(), E)
    R = T * k
    if proj == "gate_up":  # token rows, gathered by row_token
        x = wl.activations(T, K, seed=T + 2)
        aq, as_ = pkg.quantize_rowwise(x.cuda())
        y, acc = pkg.gemm_w8a8_grouped(aq, as_, w.cuda(), ws.cuda(), seg, R, row_index=rt,
                                       want_acc=True)
    else:                  # already-sorted rows
        x = wl.activations(R, K, seed=T + 2)
        aq, as_ = pkg.quantize_rowwise(x.cuda())
        y, acc = pkg.gemm_w8a8_grouped(aq, as_, w.cuda(), ws.cuda(), seg, R, want_acc=True)
    torch.cuda.synchronize()
    seg_r, rt_r, _, _ = oracle.moe_sort(topi.numpy(), E)
    aq_r, as_r = oracle.quant_rowwise_f16(x.numpy())
    assert np.array_equal(aq.cpu().numpy(), aq_r)
    ri = rt_r if proj == "gate_up" else None
    if R <= 2048:
        yr, accr = oracle.grouped_w8a8_f16(aq_r, as_r, w.numpy(), ws.numpy(), seg_r,
                                           row_index=ri, want_acc=True)
        assert np.array_equal(acc.cpu().numpy(), accr)
        assert np.array_equal(y.cpu().numpy().view(np.uint16), yr.view(np.uint16))
    else:  # sample rows: each sorted row r is expert e's GEMM of its own activation row
        rng = np.random.default_rng(T)
        rows = np.unique(np.concatenate([[0, R - 1], rng.choice(R, 64, replace=False)]))
        expert = np.searchsorted(seg_r, rows, side="right") - 1
        src = ri[rows] if ri is not None else rows
        accs = np.stack([oracle.gemm_i8(aq_r[s_:s_ + 1], w.numpy()[e])[0]
                         for s_, e in zip(src, expert)])
        assert np.array_equal(acc.cpu().numpy()[rows], accs)
        ys = np.stack([oracle.dequant_f16(a[None], as_r[s_:s_ + 1], ws.numpy()[e])[0]
                       for a, s_, e in zip(accs, src, expert)])
        assert np.array_equal(y.cpu().numpy()[rows].view(np.uint16), ys.view(np.uint16))


@pytest.mark.parametrize("T", [256, 4096])
@pytest.mark.parametrize("proj", ["gate_up", "down"])
def test_grouped_gemm_shipped_kernel_rows(pkg, wl, cuda, T, proj):
    """The grouped GEMM as SparseMoE runs it (no accumulator output), sampled
    sorted rows against the oracle's per-expert GEMM, bit for bit."""
    E, k, H, I = (wl.MOE[n] for n in ("experts", "top_k", "hidden", "inter"))
    N, K = (2 * I, H) if proj == "gate_up" else (H, I)
    _, topi = _routing(wl, T, E, k, seed=T + 5)
    w, ws = wl.expert_weights(E, N, K, seed=13 if proj == "gate_up" else 14)
    seg, rt, _ = pkg.moe_sort(topi.cuda(), E)
    R = T * k
    A = T if proj == "gate_up" else R
    x = wl.activations(A, K, seed=T + 6)
    aq, as_ = pkg.quantize_rowwise(x.cuda())
    y = pkg.gemm_w8a8_grouped(aq, as_, w.cuda(), ws.cuda(), seg, R,
                              row_index=rt if proj == "gate_up" else None)
    torch.cuda.synchronize()
    seg_r, rt_r, _, _ = oracle.moe_sort(topi.numpy(), E)
    aq_r, as_r = oracle.quant_rowwise_f16(x.numpy())
    rng = np.random.default_rng(T + 77)
    rows = np.unique(np.concatenate([[0, R - 1], rng.choice(R, 64, replace=False)]))
    expert = np.searchsorted(seg_r, rows, side="right") - 1
    src = rt_r[rows] if proj == "gate_up" else rows
    ys = np.stack([oracle.dequant_f16(oracle.gemm_i8(aq_r[s_:s_ + 1], w.numpy()[e]),
                                      as_r[s_:s_ + 1], ws.numpy()[e])[0]
                   for s_, e in zip(src, expert)])
    assert np.array_equal(y.cpu().numpy()[rows].view(np.uint16), ys.view(np.uint16))


_SPARSE = [0, 1, 0, 0, 33, 0, 2, 0, 0, 0, 0, 17, 0, 0, 0, 0, 0, 1, 0, 0, 0, 0, 0, 0]


@pytest.mark.parametrize("sizes,N,K", [
    # <= 4 rows/expert: the grouped MFMA decode kernel over 16-row tiles
    ([0, 1, 5, 0, 3, 2, 0, 1], 200, 768),        # ~1.5 rows/expert, one wave (short K)
    (_SPARSE, 200, 1024),                        # 2.25 rows/expert, a 3-tile segment
    (_SPARSE, 136, 2048),                        # the same with 2-wave workgroups
    # <= 40 rows/expert: the tile kernel over 64-row segment tiles
    ([0, 70, 1, 17, 33, 0, 2, 4], 1536, 2048),   # ~16 rows/expert, a 2-tile segment
    ([40, 0, 64, 65, 1, 30, 48, 63], 104, 1024),  # ~39 rows/expert, N % 128 != 0
    # > 40 rows/expert: the tile kernel over 128-row tiles, partial last tiles,
    # work items in XCD order (segments of 0 to 1000 rows, 1 to 12 n-tiles)
    ([0, 1, 63, 64, 65, 127, 128, 129, 191, 192, 255, 256, 300, 700], 264, 768),
    ([129, 0, 383, 64, 2, 256], 512, 2048),
    ([256, 0, 255, 257, 512, 513, 1000, 1], 1536, 512),
    ([600, 3, 300], 384, 256),
    ([0, 1, 63, 64, 65, 127, 128, 129, 300], 200, 640),  # K % 256 != 0: 64-byte K steps
])
@pytest.mark.parametrize("gather", [False, True])
def test_grouped_mfma_segments_bitexact(pkg, wl, cuda, sizes, N, K, gather):
    """Skewed expert segments (empty, single-row, multi-tile) through the grouped
    MFMA kernel, with bias and, optionally, a token gather by row index."""
    E = len(sizes)
    seg_r = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    R = int(seg_r[-1])
    rng = np.random.default_rng(R + N + K)
    w, ws = wl.expert_weights(E, N, K, seed=R + 7)
    bias = torch.from_numpy((rng.standard_normal((E, N)) * 3).astype(np.float16))
    A = R + 11 if gather else R
    x = wl.activations(A, K, seed=R + 3)
    aq, as_ = pkg.quantize_rowwise(x.cuda())
    ri = rng.integers(0, A, R).astype(np.int32) if gather else None
    y, acc = pkg.gemm_w8a8_grouped(aq, as_, w.cuda(), ws.cuda(), torch.from_numpy(seg_r).cuda(), R,
                                   row_index=None if ri is None else torch.from_numpy(ri).cuda(),
                                   bias=bias.cuda(), want_acc=True)
    torch.cuda.synchronize()
    aq_r, as_r = oracle.quant_rowwise_f16(x.numpy())
    yr, accr = oracle.grouped_w8a8_f16(aq_r, as_r, w.numpy(), ws.numpy(), seg_r, row_index=ri,
                                       bias=bias.numpy(), want_acc=True)
    assert np.array_equal(acc.cpu().numpy(), accr)
    assert np.array_equal(y.cpu().numpy().view(np.uint16), yr.view(np.uint16))


@pytest.mark.parametrize("E,mean_rows,N,K", [(300, 60, 256, 512), (260, 12, 200, 1024)])
def test_grouped_many_experts_bitexact(pkg, wl, cuda, E, mean_rows, N, K):
    """More than 256 experts: the work-item lookup keeps the first 256 experts'
    offsets in registers and scans the rest in a second loop; items in both parts
    (128-row tiles at ~60 rows per expert, 64-row tiles at ~12), with empty
    experts, against the oracle bit for bit."""
    rng = np.random.default_rng(E + K)
    sizes = rng.integers(0, 2 * mean_rows, E)
    sizes[rng.choice(E, E // 5, replace=False)] = 0
    sizes[-1] = 2 * mean_rows + 3   # the last expert (second loop) is never empty
    seg_r = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    R = int(seg_r[-1])
    w, ws = wl.expert_weights(E, N, K, seed=E + 5)
    A = R // 2 + 7
    x = wl.activations(A, K, seed=E + 6)
    aq, as_ = pkg.quantize_rowwise(x.cuda())
    ri = rng.integers(0, A, R).astype(np.int32)
    y, acc = pkg.gemm_w8a8_grouped(aq, as_, w.cuda(), ws.cuda(), torch.from_numpy(seg_r).cuda(), R,
                                   row_index=torch.from_numpy(ri).cuda(), want_acc=True)
    torch.cuda.synchronize()
    aq_r, as_r = oracle.quant_rowwise_f16(x.numpy())
    yr, accr = oracle.grouped_w8a8_f16(aq_r, as_r, w.numpy(), ws.numpy(), seg_r, row_index=ri,
                                       want_acc=True)
    assert np.array_equal(acc.cpu().numpy(), accr)
    assert np.array_equal(y.cpu().numpy().view(np.uint16), yr.view(np.uint16))


@pytest.mark.parametrize("T", [16, 256])
def test_combine_bitexact(pkg, wl, cuda, T):
    E, k, H = wl.MOE["experts"], wl.MOE["top_k"], wl.MOE["hidden"]
    topw, topi = _routing(wl, T, E, k, seed=T + 9)
    _, _, pos = pkg.moe_sort(topi.cuda(), E)
    y = wl.activations(T * k, H, seed=T + 10)
    out = pkg.moe_combine(y.cuda(), topi.cuda(), topw.cuda(), pos)
    _, _, _, pos_r = oracle.moe_sort(topi.numpy(), E)
    out_r = oracle.moe_combine_f16(y.numpy(), topi.numpy(), topw.numpy(), pos_r)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), out_r.view(np.uint16))


def _small_moe(pkg, wl, E=16, H=256, I=128, k=4, seed=0):
    """Experts quantized from N(0, 0.05^2) fp16 weights, as the reference's MoE
    tests build them (tests/test_deepseek.py:219-227)."""
    g = torch.Generator().manual_seed(seed)
    experts = []
    for e in range(E):
        gu = (torch.randn(2 * I, H, generator=g) * 0.05).half()
        dn = (torch.randn(H, I, generator=g) * 0.05).half()
        experts.append((pkg.to_qtensor(gu.cuda()), pkg.to_qtensor(dn.cuda())))
    gate = (torch.randn(E, H, generator=g) * 0.05).half().cuda()
    return pkg.SparseMoE(gate=gate, experts=experts, top_k=k, norm_topk_prob=True)


@pytest.mark.parametrize("T", [1, 7, 64, 600])
def test_sparse_moe_equals_expert_loop(pkg, wl, cuda, T):
    """The grouped module output equals the reference's loop run over the same
    W8A8 linears (`_experts_loop` drives ops.linear per expert), bit for bit."""
    moe = _small_moe(pkg, wl)
    x = (wl.activations(T, 256, seed=T) * 0.5).cuda().reshape(1, T, 256)
    xf = x.reshape(-1, 256)
    with torch.inference_mode():
        topw, topi = moe.route(xf)
        grouped = moe.experts_grouped(xf, topw, topi)
        looped = moe._experts_loop(xf, topw, topi)
        torch.cuda.synchronize()
        assert torch.equal(grouped, looped)
        y = moe(x)
    assert y.shape == x.shape and torch.isfinite(y).all()


def test_sparse_moe_close_to_cpu_reference(pkg, wl, cuda):
    """Against the CPU restatement of the loop with oracle linears: the routed
    int8 GEMMs match exactly; silu runs on different devices, so the end result is
    compared with a tolerance."""
    moe = _small_moe(pkg, wl, seed=3)
    T = 40
    x = (wl.activations(T, 256, seed=99) * 0.5)
    xf = x.cuda()
    with torch.inference_mode():
        topw, topi = moe.route(xf)
        out = moe.experts_grouped(xf, topw, topi).cpu().float().numpy()
    ref = reference_moe_loop(x.numpy(), topi.cpu().numpy(), topw.cpu().numpy(),
                             moe.w_gate_up.cpu().numpy(), moe.s_gate_up.cpu().numpy(),
                             moe.w_down.cpu().numpy(), moe.s_down.cpu().numpy()).astype(np.float32)
    cos = (out * ref).sum() / np.sqrt((out * out).sum() * (ref * ref).sum())
    rel = np.linalg.norm(out - ref) / np.linalg.norm(ref)
    print(f"grouped MoE vs CPU loop: cos {cos:.6f}, relative error {rel:.2e}", flush=True)
    assert cos > 0.999 and rel < 2e-2


@pytest.mark.parametrize("k", [1, 3, 8, 12])
@pytest.mark.parametrize("H", [2048, 204])
def test_combine_topk_widths(pkg, cuda, k, H):
    """The top-8 combine (k <= 8 and H % 8 == 0: slots ordered by a sorting
    network, every row of the token loaded before the sum) and the generic one
    (k > 8, or H not a multiple of 8) against the oracle, bit for bit."""
    E, T = 64, 37
    rng = np.random.default_rng(k * 1000 + H)
    topi = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    topw = rng.random((T, k)).astype(np.float16)
    y = rng.standard_normal((T * k, H)).astype(np.float16)
    _, _, pos = pkg.moe_sort(torch.from_numpy(topi).cuda(), E)
    out = pkg.moe_combine(torch.from_numpy(y).cuda(), torch.from_numpy(topi).cuda(),
                          torch.from_numpy(topw).cuda(), pos)
    _, _, _, pos_r = oracle.moe_sort(topi, E)
    out_r = oracle.moe_combine_f16(y, topi, topw, pos_r)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), out_r.view(np.uint16))


@pytest.mark.parametrize("k", [4, 8])
def test_combine_skips_out_of_range_experts(pkg, cuda, k):
    """A slot whose expert id is out of range has no row (the sort marks it -1):
    the combine leaves it out of the sum.  The oracle gets the same slots with
    weight 0 on row 0, which adds +0 to a finite sum."""
    E, T, H = 16, 9, 512
    rng = np.random.default_rng(k)
    topi = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    topi[0, 0], topi[3, k - 1], topi[5, 1] = E + 3, -1, E
    topw = (rng.random((T, k)) + 0.1).astype(np.float16)
    y = rng.standard_normal((T * k, H)).astype(np.float16)
    _, _, pos = pkg.moe_sort(torch.from_numpy(topi).cuda(), E)
    out = pkg.moe_combine(torch.from_numpy(y).cuda(), torch.from_numpy(topi).cuda(),
                          torch.from_numpy(topw).cuda(), pos)
    pos_h = pos.cpu().numpy()
    bad = (topi < 0) | (topi >= E)
    assert (pos_h[bad] == -1).all() and (pos_h[~bad] >= 0).all()
    out_r = oracle.moe_combine_f16(y, topi, np.where(bad, np.float16(0), topw),
                                   np.where(bad, 0, pos_h).astype(np.int32))
    assert np.array_equal(out.cpu().numpy().view(np.uint16), out_r.view(np.uint16))


@pytest.mark.parametrize("T", [16, 256])
def test_sparse_moe_int8_layer_against_oracle_qwen3_30b_shape(pkg, wl, cuda, T):
    """The whole SparseMoE layer over per_row_i8 experts at the Qwen3-30B-A3B
    expert shape (128 experts, top-8, hidden 2048, intermediate 768), bit for
    bit against the oracle's restatement of the reference's expert loop
    (fni8serve/models/moe.py:97-105) on the module's own routing: the stable
    sort, per expert linear_w8a8_f16 (gate_up) -> act_and_mul_f16 (silu) ->
    linear_w8a8_f16 (down), and the fp16 index_add combine in expert order."""
    print(f"int8 moe layer T={T}", flush=True)
    E, k, H, I = wl.MOE["experts"], wl.MOE["top_k"], 2048, 768
    g = torch.Generator().manual_seed(T)

    def qt(n, kk, seed):
        q, _ = wl.weight_i8(n, kk, seed=seed)
        s = (torch.rand(n, generator=g) * 0.0015 + 0.0005).float()
        return pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
    experts = [(qt(2 * I, H, 2000 + e), qt(H, I, 3000 + e)) for e in range(E)]
    gate = (torch.randn(E, H, generator=g) * 0.05).half().cuda()
    moe = pkg.SparseMoE(gate=gate, experts=experts, top_k=k, norm_topk_prob=True)
    x = (wl.activations(T, H, seed=T + 11) * 0.5).cuda().reshape(1, T, H)
    with torch.inference_mode():
        out = moe(x)
        topw, topi = moe.route(x.reshape(-1, H))
    torch.cuda.synchronize()
    seg, rt, _, pos = oracle.moe_sort(topi.cpu().numpy(), E)
    xf = x.reshape(-1, H).cpu().numpy()
    ys = np.zeros((T * k, H), np.float16)
    for e in range(E):
        lo, hi = int(seg[e]), int(seg[e + 1])
        if hi == lo:
            continue
        gu, dn = experts[e]
        h, _, _, _ = oracle.linear_w8a8_f16(xf[rt[lo:hi]], gu.data.cpu().numpy(),
                                            gu.scale.cpu().numpy(), None)
        a = oracle.act_and_mul_f16(h, "silu")
        yd, _, _, _ = oracle.linear_w8a8_f16(a, dn.data.cpu().numpy(), dn.scale.cpu().numpy(), None)
        ys[lo:hi] = yd
    want = oracle.moe_combine_f16(ys, topi.cpu().numpy(), topw.cpu().numpy(), pos)
    got = out.reshape(T, H).cpu().numpy()
    assert np.isfinite(want.astype(np.float32)).all()
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
