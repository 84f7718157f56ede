"""The C-ABI library loads without a GPU, exports every entry point declared in
include/fni8amd.h, and rejects bad arguments before touching a device."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fni8amd.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|void|const char\*)\s+(fni8_\w+)\s*\(",
                                 text, re.M)))


@pytest.fixture(scope="module")
def lib(pkg):
    from importlib import import_module
    return import_module("fni8serve_amd._lib").load()


def test_header_declares_the_entry_points():
    names = _declared()
    for n in ("fni8_quantize_rowwise_f16", "fni8_gemm_w8a8", "fni8_linear_w8a8_f16",
              "fni8_moe_sort", "fni8_gemm_w8a8_grouped", "fni8_moe_combine_f16",
              "fni8_strerror", "fni8_last_error", "fni8_version"):
        assert n in names


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), f"{name} declared in fni8amd.h but not exported"


def test_binding_covers_every_declared_compute_entry(pkg):
    from importlib import import_module
    b = import_module("fni8serve_amd._lib")
    assert set(_declared()) == (set(b.SIGNATURES) | set(b.STRING_FUNCS) | set(b.INT64_FUNCS)
                                | set(b.VOID_FUNCS))


def test_version_and_error_strings(lib):
    assert lib.fni8_version().decode().startswith("fni8amd")
    assert lib.fni8_strerror(0) == b"ok"
    assert b"NULL" in lib.fni8_strerror(-1)
    assert lib.fni8_strerror(-99) == b"unknown error"


def test_argument_errors_return_before_any_launch(lib):
    P = ctypes.c_void_p
    fake = P(0x1000)  # never dereferenced: every call below fails its argument checks
    # NULL required pointer
    rc = lib.fni8_linear_w8a8_f16(None, 64, 1, 64, fake, fake, 8, None, fake, 8, fake, fake, None, None)
    assert rc == -1 and b"required" in lib.fni8_last_error()
    # the entry point that allocates nothing: beyond its scratch (M * K > 48 MiB)
    rc = lib.fni8_linear_w8a8_f16_noalloc(fake, 12288, 4097, 12288, fake, fake, 8, None, fake, 8, None)
    assert rc == -2 and b"no-allocation scratch" in lib.fni8_last_error()
    # K not a multiple of 4 (the reference's quantizable rule, convert.py:128)
    rc = lib.fni8_linear_w8a8_f16(fake, 66, 1, 66, fake, fake, 8, None, fake, 8, fake, fake, None, None)
    assert rc == -2 and b"multiple of 4" in lib.fni8_last_error()
    # leading dimension shorter than the row
    rc = lib.fni8_linear_w8a8_f16(fake, 32, 1, 64, fake, fake, 8, None, fake, 8, fake, fake, None, None)
    assert rc == -4
    # misaligned int8 operand
    rc = lib.fni8_gemm_w8a8(P(0x1001), 64, fake, 1, 64, fake, fake, 8, None, fake, 8, None, None)
    assert rc == -3
    # grouped: bad expert count; sort: top-k beyond the combine limit
    rc = lib.fni8_gemm_w8a8_grouped(fake, fake, None, 8, 64, fake, fake, 0, 8, fake, None, fake, None, None)
    assert rc == -2
    rc = lib.fni8_moe_sort(fake, 4, 33, 8, fake, fake, fake, None)
    assert rc == -2
    rc = lib.fni8_quantize_rowwise_f16(fake, -1, 64, 64, fake, 64, fake, None)
    assert rc == -2


def test_grouped_w4a8_argument_errors(lib):
    P = ctypes.c_void_p
    fake = P(0x1000)  # never dereferenced: every call fails its argument checks
    args = lambda aq=fake, K=512, E=4, G=128: (aq, fake, None, 8, K, fake, fake, E, 64, G, fake,
                                               None, fake, None)
    rc = lib.fni8_gemm_w4a8_grouped(*args(G=32))   # group 32: the dense kernels only
    assert rc == -2 and b"grouped W4A8" in lib.fni8_last_error()
    rc = lib.fni8_gemm_w4a8_grouped(*args(K=384))  # K not a multiple of 256
    assert rc == -2 and b"multiple of 256" in lib.fni8_last_error()
    assert lib.fni8_gemm_w4a8_grouped(*args(E=0)) == -2
    assert lib.fni8_gemm_w4a8_grouped(*args(aq=P(0x1008))) == -3  # aq 16-byte alignment
    assert lib.fni8_gemm_w4a8_grouped(*args(K=200)) == -2          # K % G
    rc = lib.fni8_gemm_w4a8_grouped(None, fake, None, 8, 512, fake, fake, 4, 64, 128, fake, None,
                                    fake, None)
    assert rc == -1


def test_act_and_norm_argument_errors(lib):
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: every call fails its checks
    F = ctypes.c_float
    # unknown activation code
    assert lib.fni8_act_and_mul_f16(fake, 16, 1, 8, 7, fake, 8, None) == -2
    assert b"activation" in lib.fni8_last_error()
    # row stride shorter than gate | up
    assert lib.fni8_act_and_mul_f16(fake, 15, 1, 8, 0, fake, 8, None) == -4
    # the fused quantization needs I % 4 == 0 (the consuming GEMM's K rule)
    assert lib.fni8_act_and_mul_quant_f16(fake, 20, 1, 10, 0, fake, 10, fake, None) == -2
    assert lib.fni8_act_and_mul_quant_f16(None, 16, 1, 8, 0, fake, 8, fake, None) == -1
    # rmsnorm: NaN / negative eps, short strides, missing weight, misaligned x
    assert lib.fni8_rmsnorm_f16(fake, 8, None, 0, fake, F(float("nan")), 0, 1, 8, fake, 8,
                                None, 0, None) == -2
    assert lib.fni8_rmsnorm_f16(fake, 8, None, 0, fake, F(-1.0), 0, 1, 8, fake, 8, None, 0,
                                None) == -2
    assert lib.fni8_rmsnorm_f16(fake, 8, fake, 4, fake, F(1e-6), 0, 1, 8, fake, 8, fake, 8,
                                None) == -4
    assert lib.fni8_rmsnorm_f16(fake, 8, None, 0, None, F(1e-6), 0, 1, 8, fake, 8, None, 0,
                                None) == -1
    assert lib.fni8_rmsnorm_f16(ctypes.c_void_p(0x1001), 8, None, 0, fake, F(1e-6), 0, 1, 8,
                                fake, 8, None, 0, None) == -3
    assert lib.fni8_rmsnorm_quant_f16(fake, 10, None, 0, fake, F(1e-6), 0, 1, 10, fake, 10,
                                      fake, None, 0, None) == -2
    assert lib.fni8_rmsnorm_quant_f16(fake, 8, None, 0, fake, F(1e-6), 0, 1, 8, None, 8, fake,
                                      None, 0, None) == -1


def test_moe_route_argument_errors(lib):
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: every call fails its checks
    F = ctypes.c_float
    # E above 1024, k above 32 or E, unknown scoring
    assert lib.fni8_moe_route(fake, 1, 2048, 2048, 0, None, 0, 0, 8, 1, F(1.0), fake, fake, None) == -2
    assert lib.fni8_moe_route(fake, 1, 128, 128, 0, None, 0, 0, 33, 1, F(1.0), fake, fake, None) == -2
    assert lib.fni8_moe_route(fake, 1, 4, 4, 0, None, 0, 0, 5, 1, F(1.0), fake, fake, None) == -2
    assert lib.fni8_moe_route(fake, 1, 128, 128, 2, None, 0, 0, 8, 1, F(1.0), fake, fake, None) == -2
    # groups must divide E, be <= 64, and topk_group within [1, groups]
    assert lib.fni8_moe_route(fake, 1, 100, 100, 1, None, 8, 4, 8, 1, F(1.0), fake, fake, None) == -2
    assert lib.fni8_moe_route(fake, 1, 256, 256, 1, None, 128, 4, 8, 1, F(1.0), fake, fake, None) == -2
    assert lib.fni8_moe_route(fake, 1, 256, 256, 1, None, 8, 9, 8, 1, F(1.0), fake, fake, None) == -2
    # non-finite scale, short stride, NULL output
    assert lib.fni8_moe_route(fake, 1, 128, 128, 0, None, 0, 0, 8, 1, F(float("inf")), fake, fake,
                              None) == -2
    assert lib.fni8_moe_route(fake, 2, 128, 100, 0, None, 0, 0, 8, 1, F(1.0), fake, fake, None) == -4
    assert lib.fni8_moe_route(fake, 1, 128, 128, 0, None, 0, 0, 8, 1, F(1.0), None, fake, None) == -1


def test_split_k_workspace_size_and_argument_checks(lib):
    """The prefill GEMM's split-K workspace: 8 XCD regions of one 128-byte flag
    line per output tile and split (rounded up to 256 bytes), then `split` - 1
    int32 partial tiles per output tile, for the plan the test hook forces; none
    where the plan cannot split
    (tile count not a multiple of 8, K / 128 not a multiple of the split) or at
    decode sizes; a misaligned workspace is an argument error raised before any
    launch."""
    def need(M, N, K, bm, bn, split):
        tiles = -(-M // bm) * -(-N // bn)
        return ((8 * tiles * split * 128 + 255) // 256) * 256 + tiles * (split - 1) * bm * bn * 4
    try:
        for (M, N, K, bm, bn, split) in ((2048, 4096, 12288, 256, 256, 2),
                                         (512, 4096, 12288, 128, 256, 4),
                                         (500, 1000, 1024, 256, 128, 4),
                                         (500, 1000, 1024, 256, 256, 2)):
            lib.fni8_debug_gemm_plan(bm, bn, split)
            assert lib.fni8_linear_workspace_bytes(M, N, K) == need(M, N, K, bm, bn, split)
        # 3 x 4 = 12 tiles; 1152 / 128 = 9 k-tiles: the forced plan is not taken
        lib.fni8_debug_gemm_plan(128, 256, 2)
        assert lib.fni8_linear_workspace_bytes(300, 1000, 1024) != need(300, 1000, 1024, 128, 256, 2)
        lib.fni8_debug_gemm_plan(256, 256, 2)
        assert lib.fni8_linear_workspace_bytes(512, 2048, 1152) == 0
        lib.fni8_debug_gemm_plan(256, 128, 1)
        assert lib.fni8_linear_workspace_bytes(2048, 4096, 12288) == 0
    finally:
        lib.fni8_debug_gemm_plan(0, 0, 0)
    for M in (17, 33, 64):
        assert lib.fni8_linear_workspace_bytes(M, 4096, 12288) == 0
    assert lib.fni8_linear_workspace_bytes(2048, 4096, 12288) > 0  # down at M = 2048 splits K
    P = ctypes.c_void_p
    fake = P(0x1000)
    rc = lib.fni8_gemm_w8a8_ws(fake, 4096, fake, 512, 4096, fake, fake, 64, None, fake, 64, None,
                               P(0x1080), 1 << 20, None)
    assert rc == -3 and b"workspace" in lib.fni8_last_error()
    rc = lib.fni8_gemm_w8a8_ws(fake, 4096, fake, 512, 4096, fake, fake, 64, None, fake, 64, None,
                               fake, -5, None)
    assert rc == -3
    rc = lib.fni8_gemm_w8a8_ws(None, 4096, fake, 512, 4096, fake, fake, 64, None, fake, 64, None,
                               fake, 1 << 20, None)
    assert rc == -1


def test_act_quant_workspace_size_and_argument_checks(lib):
    """fni8_act_and_mul_quant_f16_ws: 8 XCD regions of (M rounded up to 8) * G
    128-byte lines for G = ceil(I / 2048) parts per row, 2 <= G <= 8 and
    M <= 128; none otherwise (one workgroup per row).  A misaligned workspace
    is an argument error raised before any launch."""
    for M, I in ((1, 12288), (64, 12288), (128, 12288), (33, 4112), (9, 3072), (5, 16384)):
        G = -(-I // 2048)
        assert lib.fni8_act_and_mul_quant_workspace_bytes(M, I) == 8 * (-(-M // 8) * 8) * G * 128
    assert lib.fni8_act_and_mul_quant_workspace_bytes(64, 12288) == 393216
    for M, I in ((0, 12288), (129, 12288), (4096, 12288), (16, 768), (16, 2048), (4, 1004),
                 (2, 16392), (2, 40000)):
        assert lib.fni8_act_and_mul_quant_workspace_bytes(M, I) == 0, (M, I)
    P = ctypes.c_void_p
    fake = P(0x1000)
    rc = lib.fni8_act_and_mul_quant_f16_ws(fake, 24576, 4, 12288, 0, fake, 12288, fake,
                                           P(0x1080), 1 << 20, None)
    assert rc == -3 and b"workspace" in lib.fni8_last_error()
    rc = lib.fni8_act_and_mul_quant_f16_ws(fake, 24576, 4, 12288, 7, fake, 12288, fake, fake,
                                           1 << 20, None)
    assert rc == -2


def test_workspace_size_and_argument_checks(lib):
    """The one-launch path's workspace: 8 regions of (2304 + M*K rounded up to
    256) bytes for the shapes it takes (5..16 tokens on QKV- and down-shaped
    weights, 5..8 on O-shaped ones), none otherwise; a misaligned workspace is
    an argument error raised before any launch."""
    for M, N, K in ((5, 4096, 4096), (8, 4096, 4096), (16, 6144, 4096), (7, 4096, 12288),
                    (8, 100, 4096), (16, 4096, 12288)):
        assert lib.fni8_linear_workspace_bytes(M, N, K) == 8 * (2304 + ((M * K + 255) // 256) * 256)
    assert lib.fni8_linear_workspace_bytes(16, 4096, 12288) == 1591296
    for M, N, K in ((0, 4096, 4096), (1, 4096, 4096), (4, 4096, 4096), (9, 4096, 4096),
                    (17, 6144, 4096), (64, 4096, 12288), (16, 24576, 4096), (16, 6144, 12288),
                    (16, 4096, 1024), (16, 4096, 8192)):
        assert lib.fni8_linear_workspace_bytes(M, N, K) == 0, (M, N, K)
    P = ctypes.c_void_p
    fake = P(0x1000)
    rc = lib.fni8_linear_w8a8_f16_ws(fake, 4096, 16, 4096, fake, fake, 64, None, fake, 64, fake,
                                     fake, None, P(0x1080), 1 << 20, None)
    assert rc == -3 and b"workspace" in lib.fni8_last_error()
    rc = lib.fni8_linear_w8a8_f16_ws(None, 4096, 16, 4096, fake, fake, 64, None, fake, 64, fake,
                                     fake, None, fake, 1 << 20, None)
    assert rc == -1
    rc = lib.fni8_linear_w8a8_f16_ws(fake, 4096, 16, 4096, fake, fake, 64, None, fake, 64, fake,
                                     fake, None, fake, -1, None)
    assert rc == -3
