"""GPU parity of the W4A8 linear (per_group_i4 int4 weights) against the oracle
(oracle/w4a8_oracle.c): int8 activations, fp32 scales and fp16 outputs bit for
bit, on the decode GEMVs (1-4 tokens), the MFMA decode kernel (5-64 tokens)
and the MFMA tile kernel (more tokens), every supported group size, Qwen3-8B's
shapes and ragged ones.  Each output
element depends only on its own activation row and weight row, so at full size
the oracle checks sampled rows and columns.  Also the reference's own W4 seam
test (tests/test_smoke.py:83-94: cosine against the fp16 dequantized weight)
and the fused MLP on W4 weights.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as o

pytestmark = pytest.mark.gpu


def _w4(pkg, N, K, G, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    codes = torch.randint(-8, 8, (N, K), device="cuda", generator=g)
    packed = ((codes[:, 0::2] & 0xF) | ((codes[:, 1::2] & 0xF) << 4)).to(torch.uint8)
    scale = torch.rand(N, K // G, device="cuda", generator=g) * 0.02 + 1e-3
    return pkg.QTensor(packed.contiguous(), scale.contiguous(), scheme="per_group_i4",
                       group_size=G, codebook="int4")


def _x(M, K, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(M, K, device="cuda", generator=g).half()
    if M * K >= 64:
        flat = x.view(-1)
        idx = torch.randint(0, flat.numel(), (max(1, flat.numel() // 100),), device="cuda",
                            generator=g)
        flat[idx] *= 20  # 1% outliers x20, as the benchmark activations
    return x


def _check(pkg, x, qt, bias, rows=None, cols=None):
    y, xq, xs, _ = pkg.ops.linear_with_intermediates(x, qt, bias)
    xn = x.cpu().numpy()
    q_ref, s_ref = o.quant_rowwise_f16(xn)
    assert np.array_equal(xq.cpu().numpy(), q_ref) and np.array_equal(xs.cpu().numpy(), s_ref)
    r = np.arange(x.shape[0]) if rows is None else rows
    c = np.arange(qt.data.shape[0]) if cols is None else cols
    w = qt.data.cpu().numpy()[c]
    ws = qt.scale.cpu().numpy()[c]
    b = None if bias is None else bias.cpu().numpy()[c]
    want = o.gemm_w4a8(q_ref[r], s_ref[r], w, ws, qt.group_size, bias=b)
    got = y.cpu().numpy()[np.ix_(r, c)]
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("G", [32, 64, 128, 256])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 16, 64, 130])
def test_w4a8_small_shapes_bitexact(pkg, M, G):
    """Every output element against the oracle; N ragged (not a multiple of the
    tile or of the GEMV's 16 rows per workgroup)."""
    print(f"w4a8 M={M} G={G}", flush=True)
    N, K = 200, 1024
    qt = _w4(pkg, N, K, G, seed=M * 7 + G)
    bias = torch.randn(N, device="cuda").half() if M % 2 else None
    _check(pkg, _x(M, K, seed=M + G), qt, bias)


@pytest.mark.parametrize("M", [1, 4, 16, 512])
@pytest.mark.parametrize("shape", [(6144, 4096), (4096, 12288)], ids=["qkv", "down"])
def test_w4a8_qwen3_8b_shapes_sampled(pkg, M, shape):
    """Qwen3-8B's QKV and down shapes at group size 128 (the converter's
    default, fni8serve/convert.py:89), 8 sampled rows x 256 sampled columns
    against the oracle, the rest covered by the row/column independence."""
    print(f"w4a8 qwen3 M={M} shape={shape}", flush=True)
    N, K = shape
    qt = _w4(pkg, N, K, 128, seed=M + N)
    rng = np.random.default_rng(M)
    rows = np.sort(rng.choice(M, min(M, 8), replace=False))
    cols = np.sort(rng.choice(N, 256, replace=False))
    _check(pkg, _x(M, K, seed=M), qt, None, rows, cols)


@pytest.mark.parametrize("G", [32, 64, 128, 256])
@pytest.mark.parametrize("shape", [(4096, 4096), (3072, 2048), (4096, 12288)],
                         ids=["o", "n3072_k2048", "down"])
def test_w4a8_one_token_launch_table_bitexact(pkg, shape, G):
    """One token at the launch table's stream shapes (O-like K <= 4096, N <= 4096
    with 8 | K/256, and the down shape): the fused launch (fp16 x) and the
    prequantized GEMM, with bias, against the oracle on the first and last 64
    columns and 128 sampled ones (each output column depends only on its own
    weight row)."""
    print(f"w4a8 one-token table shape={shape} G={G}", flush=True)
    N, K = shape
    qt = _w4(pkg, N, K, G, seed=N + K + G)
    bias = torch.randn(N, device="cuda").half()
    rng = np.random.default_rng(N + G)
    cols = np.unique(np.concatenate([np.arange(64), np.arange(N - 64, N),
                                     rng.choice(N, 128, replace=False)]))
    x = _x(1, K, seed=K + G)
    _check(pkg, x, qt, bias, None, cols)
    xq, xs = pkg.quantize_rowwise(x)
    y = pkg.gemm_w4a8(xq, xs, qt, bias)
    want = o.gemm_w4a8(xq.cpu().numpy(), xs.cpu().numpy(), qt.data.cpu().numpy()[cols],
                       qt.scale.cpu().numpy()[cols], G, bias=bias.cpu().numpy()[cols])
    assert np.array_equal(y.cpu().numpy()[:, cols].view(np.uint16), want.view(np.uint16))


def test_w4a8_matches_the_reference_seam_test(pkg):
    """tests/test_smoke.py:83-94: W4A8 against F.linear with the fp16
    dequantized weight, cosine >= 0.985 in the reference; printed here."""
    from importlib import import_module
    _dequant_weight = import_module("fni8serve_amd.layers.linear")._dequant_weight
    g = torch.Generator().manual_seed(0)
    w = torch.randn(128, 256, generator=g)
    wg = w.reshape(128, 256 // 32, 32)
    s = wg.abs().amax(-1, keepdim=True) / 7
    c = torch.round(wg / s).clamp_(-7, 7).reshape(128, 256).to(torch.int64)
    packed = ((c[:, 0::2] & 0xF) | ((c[:, 1::2] & 0xF) << 4)).to(torch.uint8)
    qt = pkg.QTensor(packed.cuda(), s.squeeze(-1).float().cuda(), scheme="per_group_i4",
                     group_size=32, codebook="int4")
    lin = pkg.LinearW8A8(qt)
    x = torch.randn(8, 256, device="cuda", dtype=torch.float16)
    y = lin(x)
    ref = torch.nn.functional.linear(x.float(), _dequant_weight(qt).float())
    cos = torch.nn.functional.cosine_similarity(y.flatten().float(), ref.flatten(), dim=0).item()
    print(f"W4A8 vs fp16 dequant reference: cosine {cos:.6f}")
    assert cos >= 0.999 and torch.isfinite(y).all()


@pytest.mark.parametrize("M", [1, 16, 256])
def test_gated_mlp_w4_fused_equals_unfused(pkg, M):
    N_gu, K, I = 2 * 1536, 2048, 1536
    gu = _w4(pkg, N_gu, K, 128, seed=1)
    dn = _w4(pkg, K, I, 128, seed=2)
    mlp = pkg.GatedMLP(gu, dn, act="silu")
    x = _x(M, K, seed=3) * 0.1
    fused = mlp(x)
    unfused = mlp.down_proj(mlp.act_fn(mlp.gate_up_proj(x)))
    assert torch.isfinite(fused).all() and torch.equal(fused, unfused)


def test_w4a8_argument_errors(pkg):
    qt = _w4(pkg, 64, 256, 32, seed=0)
    x = torch.randn(2, 256, device="cuda").half()
    nf4 = pkg.QTensor(qt.data, qt.scale, scheme="per_group_i4", group_size=32, codebook="nf4")
    with pytest.raises(ValueError, match="int4 codebook"):
        pkg.linear(x, nf4)
    bad = pkg.QTensor(qt.data, qt.scale, scheme="per_group_i4", group_size=48, codebook="int4")
    with pytest.raises(ValueError, match="group size"):
        pkg.linear(x, bad)
    with pytest.raises(ValueError, match="in_features"):
        pkg.linear(torch.randn(2, 128, device="cuda").half(), qt)


@pytest.mark.parametrize("G", [32, 128, 256])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 8])
def test_w4a8_prequantized_gemm_bitexact(pkg, M, G):
    """gemm_w4a8 on int8 activations (the path after act_and_mul_quant) against
    the oracle, and against the one-launch linear on the same activations."""
    print(f"w4a8 prequantized M={M} G={G}", flush=True)
    N, K = 300, 3072
    qt = _w4(pkg, N, K, G, seed=M * 3 + G)
    x = _x(M, K, seed=M * 5 + G)
    xq, xs = pkg.quantize_rowwise(x)
    bias = torch.randn(N, device="cuda").half()
    y = pkg.gemm_w4a8(xq, xs, qt, bias)
    want = o.gemm_w4a8(xq.cpu().numpy(), xs.cpu().numpy(), qt.data.cpu().numpy(),
                       qt.scale.cpu().numpy(), G, bias=bias.cpu().numpy())
    assert np.array_equal(y.cpu().numpy().view(np.uint16), want.view(np.uint16))
    assert torch.equal(y, pkg.linear(x, qt, bias))


@pytest.mark.parametrize("G", [64, 128, 256])
@pytest.mark.parametrize("M", [5, 8, 16, 17, 31, 32, 33, 48, 63, 64])
@pytest.mark.parametrize("K", [256, 512, 1536, 4096])
def test_w4a8_mfma_decode_bitexact(pkg, M, K, G):
    """5..64 tokens, group sizes 64..256: the MFMA decode kernel (waves split K
    in rounds of slabs, exact group sums folded in order).  K = 256, 512 and
    1536 take the one- and two-wave shapes, 4096 the four-wave ones; N is
    ragged (not a multiple of 16 or 32 rows); every output element against
    the oracle, bias on odd M."""
    print(f"w4a8 mfma M={M} K={K} G={G}", flush=True)
    N = 200 if K <= 1536 else 72
    qt = _w4(pkg, N, K, G, seed=M * 11 + K + G)
    bias = torch.randn(N, device="cuda").half() if M % 2 else None
    _check(pkg, _x(M, K, seed=M * 13 + G), qt, bias)


def test_w4a8_mfma_strided_rows(pkg):
    """Activation rows with a stride (a view of a wider buffer)."""
    M, K, N, G = 24, 2048, 96, 128
    qt = _w4(pkg, N, K, G, seed=5)
    big = _x(M, K + 256, seed=6)
    x = big[:, 128:128 + K]
    _check(pkg, x, qt, None)


@pytest.mark.parametrize("G", [64, 128, 256])
@pytest.mark.parametrize("K", [1024, 2048, 3072, 4096, 6144, 8192, 10240, 12288, 16384])
@pytest.mark.parametrize("M", [2, 3, 4])
def test_w4a8_fused_mfma_bitexact(pkg, M, K, G):
    """2..4 tokens: the MFMA decode kernel with the quantization fused in (one
    launch).  Up to K = 4096 every M runs it, on four waves (K = 2048, 4096)
    or two (K = 1024, 3072); above, 2 tokens run it at every chunk count of
    the four-wave shape (K = 2048 * chunks: 3, 4, 6, 8) and 3-4 tokens, like
    K = 10240, take the quantize launch plus the MFMA kernel.  xq, xs and
    every output element against the oracle, ragged N, bias on odd M."""
    print(f"w4a8 fused mfma M={M} K={K} G={G}", flush=True)
    N = 72
    qt = _w4(pkg, N, K, G, seed=M * 17 + K + G)
    bias = torch.randn(N, device="cuda").half() if M % 2 else None
    _check(pkg, _x(M, K, seed=M * 19 + K + G), qt, bias)


@pytest.mark.parametrize("G", [64, 256])
@pytest.mark.parametrize("N,K", [(4100, 4096), (4127, 2048)])
def test_w4a8_fused_mfma_32_row_blocks(pkg, N, K, G):
    """4 tokens with N above 4096: 32 weight rows per workgroup (two MFMA
    blocks), N ragged so the last workgroup holds a partial block; sampled
    columns (the last ones included) against the oracle, with bias."""
    print(f"w4a8 fused mfma 32-row N={N} K={K} G={G}", flush=True)
    M = 4
    qt = _w4(pkg, N, K, G, seed=N + K + G)
    cols = np.concatenate([np.sort(np.random.default_rng(N).choice(N - 64, 448, replace=False)),
                           np.arange(N - 64, N)])
    _check(pkg, _x(M, K, seed=G), qt, torch.randn(N, device="cuda").half(), cols=cols)


@pytest.mark.parametrize("ld_pad", [64, 3])
@pytest.mark.parametrize("M", [2, 3, 4])
def test_w4a8_fused_mfma_wide_and_strided(pkg, M, ld_pad):
    """The wide-N shape (N >= 16384: 32 rows, two waves, one slab per round;
    2-3 tokens, 4 take the quantize launch) on a row view of a wider buffer.
    A row stride that is a multiple of 8 elements stays on the fused kernel;
    an odd one falls back to the quantize launch.  Sampled columns against the
    oracle (rows and columns are independent)."""
    print(f"w4a8 fused mfma wide M={M} ld_pad={ld_pad}", flush=True)
    K, N, G = 4096, 16400, 128
    qt = _w4(pkg, N, K, G, seed=ld_pad)
    big = _x(M, K + ld_pad + 8, seed=ld_pad + 1)
    x = big[:, 8:8 + K]
    cols = np.sort(np.random.default_rng(ld_pad).choice(N, 512, replace=False))
    cols[-1] = N - 1
    _check(pkg, x, qt, torch.randn(N, device="cuda").half(), cols=cols)


def test_w4a8_fused_mfma_special_rows(pkg):
    """Zero, subnormal-only, inf, -65504 and NaN rows through the fused
    quantization: xq and the output against the oracle (NaN where the oracle
    has NaN, equal bits elsewhere)."""
    K, N, G = 4096, 200, 128
    rows = np.zeros((4, K), np.float16)
    rows[1, 7] = 6e-8                    # subnormal only
    rows[2, :] = np.linspace(-3, 3, K)
    rows[2, 99] = np.inf                 # inf row: inf scale, q = 0
    rows[3, :] = np.float16(-65504)
    rows[3, ::3] = 2.5
    nan_rows = np.ones((2, K), np.float16)
    nan_rows[1, 1000] = np.nan
    qt = _w4(pkg, N, K, G, seed=23)
    w, ws = qt.data.cpu().numpy(), qt.scale.cpu().numpy()
    for arr in (rows, nan_rows):
        y, xq, xs, _ = pkg.ops.linear_with_intermediates(torch.from_numpy(arr).cuda(), qt, None)
        q_ref, s_ref = o.quant_rowwise_f16(arr)
        assert np.array_equal(xq.cpu().numpy(), q_ref)
        got_s = xs.cpu().numpy()
        assert np.array_equal(np.isnan(got_s), np.isnan(s_ref))
        assert np.array_equal(got_s[~np.isnan(s_ref)].view(np.uint32),
                              s_ref[~np.isnan(s_ref)].view(np.uint32))
        want = o.gemm_w4a8(q_ref, s_ref, w, ws, G)
        a = y.cpu().numpy()
        assert np.array_equal(np.isnan(a), np.isnan(want))
        assert np.array_equal(a[~np.isnan(a)].view(np.uint16), want[~np.isnan(want)].view(np.uint16))


@pytest.mark.parametrize("G", [64, 128, 256])
@pytest.mark.parametrize("K", [512, 1536, 4096])
@pytest.mark.parametrize("M,N", [(9, 16400), (16, 16391), (17, 16400), (33, 16391),
                                 (48, 16400), (64, 16391)])
def test_w4a8_rowblock_bitexact(pkg, M, N, K, G):
    """9..64 tokens on wide N: the row-block kernel (waves split the weight
    rows, one shared activation tile, folds in registers).  N leaves the last
    workgroup with waves wholly past N (16400) or a partial 16-row block
    (16391); K = 512 is one batch, 1536 an odd number of them.  All rows,
    sampled columns (the last 64 included) against the oracle, with bias."""
    print(f"w4a8 rowblock M={M} N={N} K={K} G={G}", flush=True)
    qt = _w4(pkg, N, K, G, seed=M + K + G)
    cols = np.concatenate([np.sort(np.random.default_rng(M + K).choice(N - 64, 384, replace=False)),
                           np.arange(N - 64, N)])
    _check(pkg, _x(M, K, seed=M * 3 + K + G), qt, torch.randn(N, device="cuda").half(), cols=cols)


@pytest.mark.parametrize("N", [1, 8, 17])
@pytest.mark.parametrize("M", [2, 9, 40])
def test_w4a8_mfma_decode_narrow_n(pkg, M, N):
    """Fewer weight rows than one 16-row block (rows past N repeat row N-1 and
    are never stored), and one row past a block."""
    print(f"w4a8 mfma narrow M={M} N={N}", flush=True)
    K, G = 512, 64
    qt = _w4(pkg, N, K, G, seed=M + N)
    bias = torch.randn(N, device="cuda").half()
    _check(pkg, _x(M, K, seed=M * 3 + N), qt, bias)


@pytest.mark.parametrize("M,N,K", [(65, 264, 1024), (300, 520, 2048), (512, 1000, 4096)])
def test_w4a8_tile8_group256_bitexact(pkg, M, N, K):
    """Group size 256 above 64 tokens: the 8-wave two-stage tile kernel (two
    workgroup rows, ragged M and N, bias), every element against the oracle."""
    print(f"w4a8 tile8 M={M} N={N} K={K}", flush=True)
    qt = _w4(pkg, N, K, 256, seed=M + N)
    bias = torch.randn(N, device="cuda").half()
    _check(pkg, _x(M, K, seed=M * 7 + K), qt, bias)


@pytest.mark.parametrize("T,G,H,I", [(3, 64, 512, 256), (40, 64, 512, 256),
                                     (200, 128, 1024, 768), (512, 256, 1024, 768),
                                     (24, 32, 512, 256)])
def test_sparse_moe_w4_experts_against_oracle(pkg, T, G, H, I):
    """SparseMoE over per_group_i4 int4 experts (the reference builds experts
    from any QTensor scheme, fni8serve/models/moe.py:56; its converter writes
    per_group_i4 for weight_bits=4, convert.py:130-131): the layer output bit for
    bit against the oracle's sort, per-expert W4A8 chain (gate_up, silu-and-mul,
    down) and combine, on the same routing.  G = 64..256 run the grouped
    W4A8 GEMM (16-row segment tiles at T = 3 and 40, 64-row ones at T = 200,
    where down's K = 768 is an odd number of slabs, the tile kernel's 128-row
    ones at T = 512); G = 32 keeps the per-expert modules."""
    print(f"w4 moe T={T} G={G}", flush=True)
    E, k = 16, 4
    experts = [(_w4(pkg, 2 * I, H, G, seed=e), _w4(pkg, H, I, G, seed=100 + e)) for e in range(E)]
    g = torch.Generator(device="cuda").manual_seed(T)
    gate = (torch.randn(E, H, device="cuda", generator=g) * 0.05).half()
    moe = pkg.SparseMoE(gate=gate, experts=experts, top_k=k, norm_topk_prob=True)
    assert moe.grouped_w4 == (G >= 64)
    x = _x(T, H, seed=T + 7).reshape(1, T, H)
    out = moe(x)
    topw, topi = moe.route(x.reshape(-1, H))
    torch.cuda.synchronize()
    seg, rt, _, pos = o.moe_sort(topi.cpu().numpy(), E)
    xf = x.reshape(-1, H).cpu().numpy()
    ys = np.zeros((T * k, H), np.float16)
    for e in range(E):
        lo, hi = int(seg[e]), int(seg[e + 1])
        if hi == lo:
            continue
        gu, dn = experts[e]
        h, _, _ = o.linear_w4a8_f16(xf[rt[lo:hi]], gu.data.cpu().numpy(), gu.scale.cpu().numpy(), G)
        a = o.act_and_mul_f16(h, "silu")
        yd, _, _ = o.linear_w4a8_f16(a, dn.data.cpu().numpy(), dn.scale.cpu().numpy(), G)
        ys[lo:hi] = yd
    want = o.moe_combine_f16(ys, topi.cpu().numpy(), topw.cpu().numpy(), pos)
    assert np.array_equal(out.reshape(T, H).cpu().numpy().view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("T", [16, 256])
def test_sparse_moe_w4_layer_qwen3_30b_shape(pkg, T):
    """The int4-expert SparseMoE layer at the Qwen3-30B-A3B expert shape the
    benchmark times (128 experts, top-8, hidden 2048, intermediate 768, group
    128) on the grouped W4A8 GEMM, bit for bit against the oracle chain: sort,
    per expert linear_w4a8_f16 (gate_up) -> silu-and-mul -> linear_w4a8_f16
    (down), combine (fni8serve/models/moe.py:97-105)."""
    print(f"w4 moe layer qwen3-30b T={T}", flush=True)
    E, k, H, I, G = 128, 8, 2048, 768, 128
    experts = [(_w4(pkg, 2 * I, H, G, seed=4000 + e), _w4(pkg, H, I, G, seed=5000 + e))
               for e in range(E)]
    for gu, dn in experts:  # smaller scales keep every fp16 partial finite
        gu.scale.mul_(0.1)
        dn.scale.mul_(0.1)
    g = torch.Generator(device="cuda").manual_seed(T)
    gate = (torch.randn(E, H, device="cuda", generator=g) * 0.05).half()
    moe = pkg.SparseMoE(gate=gate, experts=experts, top_k=k, norm_topk_prob=True)
    assert moe.grouped_w4
    x = (_x(T, H, seed=T + 17) * 0.5).reshape(1, T, H)
    with torch.inference_mode():
        out = moe(x)
        topw, topi = moe.route(x.reshape(-1, H))
    torch.cuda.synchronize()
    seg, rt, _, pos = o.moe_sort(topi.cpu().numpy(), E)
    xf = x.reshape(-1, H).cpu().numpy()
    ys = np.zeros((T * k, H), np.float16)
    for e in range(E):
        lo, hi = int(seg[e]), int(seg[e + 1])
        if hi == lo:
            continue
        gu, dn = experts[e]
        h, _, _ = o.linear_w4a8_f16(xf[rt[lo:hi]], gu.data.cpu().numpy(), gu.scale.cpu().numpy(), G)
        a = o.act_and_mul_f16(h, "silu")
        yd, _, _ = o.linear_w4a8_f16(a, dn.data.cpu().numpy(), dn.scale.cpu().numpy(), G)
        ys[lo:hi] = yd
    want = o.moe_combine_f16(ys, topi.cpu().numpy(), topw.cpu().numpy(), pos)
    assert np.isfinite(want.astype(np.float32)).all()
    assert np.array_equal(out.reshape(T, H).cpu().numpy().view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("G", [64, 128, 256])
@pytest.mark.parametrize("K", [768, 1024])
@pytest.mark.parametrize("per_expert,E,N", [(1, 8, 200), (4, 64, 2000), (20, 8, 200),
                                            (60, 8, 200), (150, 8, 200)])
def test_w4a8_grouped_gemm_bitexact(pkg, per_expert, E, N, K, G):
    """The grouped W4A8 GEMM against the oracle expert by expert: ragged
    segments (one expert empty), the row-block kernel's 16-row segment tiles
    on two waves (mean 1 row per expert, a small grid) and on four (mean 4, 64
    experts), its 32- and 64-row tiles (20, 60) and the tile kernel's 128-row
    ones (150), K = 768 (odd slab count) and 1024, activation rows gathered
    through a row map, bias, and `rows` beyond the sorted rows (those are not
    written)."""
    print(f"w4a8 grouped per_expert={per_expert} E={E} K={K} G={G}", flush=True)
    rng = np.random.default_rng(per_expert + K + G)
    lens = rng.integers(0, 2 * per_expert + 1, E)
    lens[1] = 0
    lens[0] = max(lens[0], 1)
    R = int(lens.sum())
    seg = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    A = R + 5
    rmap = rng.integers(0, A, R + 7).astype(np.int32)
    xq = rng.integers(-127, 128, (A, K)).astype(np.int8)
    xs = rng.uniform(0.001, 0.05, A).astype(np.float32)
    qts = [_w4(pkg, N, K, G, seed=e * 13 + K + G) for e in range(E)]
    w = torch.stack([q.data for q in qts]).contiguous()
    ws = torch.stack([q.scale for q in qts]).contiguous()
    bias = torch.randn(E, N, device="cuda").half()
    y = pkg.ops.gemm_w4a8_grouped(torch.from_numpy(xq).cuda(), torch.from_numpy(xs).cuda(), w, ws,
                                  G, torch.from_numpy(seg).cuda(), R + 7,
                                  row_index=torch.from_numpy(rmap).cuda(), bias=bias)
    got = y.cpu().numpy()
    wn, wsn, bn = w.cpu().numpy(), ws.cpu().numpy(), bias.cpu().numpy()
    for e in range(E):
        lo, hi = int(seg[e]), int(seg[e + 1])
        if hi == lo:
            continue
        rows = rmap[lo:hi]
        want = o.gemm_w4a8(xq[rows], xs[rows], wn[e], wsn[e], G, bias=bn[e])
        assert np.array_equal(got[lo:hi].view(np.uint16), want.view(np.uint16)), f"expert {e}"


@pytest.mark.parametrize("T", [4, 40])
def test_sparse_moe_w4_graph_capture(pkg, T):
    """The int4 expert layer on the grouped W4A8 GEMM has no host sync, so it
    is captured in one HIP graph; each replay on new inputs equals the eager
    forward bit for bit (the reference declines MoE layers for capture,
    fni8serve/engine/cuda_graph.py:190-191)."""
    print(f"w4 moe graph T={T}", flush=True)
    E, H, I, k, G = 16, 512, 256, 4, 64
    experts = [(_w4(pkg, 2 * I, H, G, seed=e), _w4(pkg, H, I, G, seed=100 + e)) for e in range(E)]
    g = torch.Generator(device="cuda").manual_seed(T)
    gate = (torch.randn(E, H, device="cuda", generator=g) * 0.05).half()
    moe = pkg.SparseMoE(gate=gate, experts=experts, top_k=k, norm_topk_prob=True)
    assert moe.grouped_w4
    x_static = _x(T, H, seed=T + 3).reshape(1, T, H)
    with torch.inference_mode():
        eager0 = moe(x_static).clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                moe(x_static)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            y_static = moe(x_static)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_static, eager0)
        for rep in range(3):
            x_new = _x(T, H, seed=T * 10 + rep).reshape(1, T, H)
            x_static.copy_(x_new)
            y_static.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            want = moe(x_new)
            torch.cuda.synchronize()
            assert torch.isfinite(want).all()
            assert torch.equal(y_static, want), rep
