"""Pins the oracle's act_and_mul and RMSNorm (oracle/act_norm_oracle.c).

The reference's fused kernels for these (`fni8.act_and_mul`, `fni8.rmsnorm`)
live in a closed wheel; its eager fallbacks are F.silu(g) * u,
F.gelu(g, approximate="tanh") * u (fni8serve/layers/activation.py:20-42) and
RMSNorm._norm (fni8serve/layers/norm.py:37-58).  The oracle's own convention
is checked against what the mathematics fixes (float64 closed forms, exact
known answers, error bounds) and against those torch fallbacks, with the
tolerances written in each test.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as o

ALL_F16 = np.arange(65536, dtype=np.uint16).view(np.float16)
FINITE_F16 = ALL_F16[np.isfinite(ALL_F16)]


def _ulp32(x):
    return np.spacing(np.abs(x).astype(np.float32)).astype(np.float64)


def _f16_ulp(x):
    return np.spacing(np.abs(x).astype(np.float16)).astype(np.float64)


# ---- exp --------------------------------------------------------------------

def test_exp_within_one_ulp_on_a_dense_sweep():
    """Every 97th fp32 bit pattern in [-86, 88] (23 M points): within 1 ulp of
    float64 exp.  A wrong split constant of ln2 or a dropped Horner term breaks
    this bound."""
    pos = np.arange(0, 0x42B00000 + 1, 97, dtype=np.uint32).view(np.float32)
    neg = -np.arange(0, 0x42AC0000 + 1, 97, dtype=np.uint32).view(np.float32)
    x = np.concatenate([pos, neg])
    x = x[(x >= -86) & (x <= 88)]
    y = o.exp_cw(x).astype(np.float64)
    ex = np.exp(x.astype(np.float64))
    err = np.abs(y - ex) / _ulp32(ex)
    assert err.max() <= 1.0, err.max()
    assert (err > 0.5).mean() < 0.01  # correctly rounded almost everywhere


def test_exp_known_answers():
    assert o.exp_cw(np.float32([0.0]))[0] == 1.0
    # exp(k ln2) = 2^k up to the rounding of the argument
    for k in (-120, -1, 1, 60, 126):
        x = np.float32(k * math.log(2))
        assert abs(float(o.exp_cw(np.float32([x]))[0]) / math.exp(float(x)) - 1) < 2 ** -23
    # the ends of the domain stay normal numbers
    lo, hi = o.exp_cw(np.float32([-86.0, 88.0]))
    assert lo > np.finfo(np.float32).tiny and np.isfinite(hi)


# ---- activations ------------------------------------------------------------

def _silu64(g):
    with np.errstate(over="ignore"):
        return g / (1 + np.exp(-g))


def _gelu64(g):
    # g * sigmoid(2y) == 0.5 g (1 + tanh(y)) without the cancellation near tanh = -1
    y = math.sqrt(2 / math.pi) * (g + 0.044715 * g ** 3)
    with np.errstate(over="ignore"):
        return g / (1 + np.exp(-2 * y))


@pytest.mark.parametrize("act", ["silu", "gelu_tanh"])
def test_act_f32_over_every_fp16_gate(act):
    """act(g) for every finite fp16 g against the float64 closed form.  The
    error is bounded by (4 + c |t|) ulp, t the argument of exp: a relative
    error e in t becomes |t| e in exp(t).  For silu t = -g is exact (c = 1 for
    the rounding inside exp); for gelu t carries about six roundings (g^3,
    0.044715, the sum, the scale: c = 6).  Where the exact value underflows
    below 1e-30 the result is as small."""
    g = FINITE_F16.astype(np.float32)
    gd = g.astype(np.float64)
    a = o.act_f32(g, act).astype(np.float64)
    ex = _silu64(gd) if act == "silu" else _gelu64(gd)
    t = -gd if act == "silu" else -2 * math.sqrt(2 / math.pi) * (gd + 0.044715 * gd ** 3)
    c = 1 if act == "silu" else 6
    big = np.abs(ex) > 1e-30
    err = np.abs(a[big] - ex[big]) / _ulp32(ex[big])
    bound = 4 + c * np.abs(np.clip(t[big], -86, 88))
    assert (err <= bound).all(), (err / bound).max()
    assert np.abs(a[~big]).max() < 1e-29
    assert (np.sign(a[big]) == np.sign(ex[big])).all()


@pytest.mark.parametrize("act", ["silu", "gelu_tanh"])
def test_act_and_mul_fp16_within_one_ulp_of_exact(act):
    """out = fp16(act(g) * u): over every fp16 gate with u = 1 and random (g, u)
    pairs, within one fp16 ulp of the exact value and equal to its
    round-to-nearest almost everywhere."""
    rng = np.random.default_rng(0)
    g = np.concatenate([FINITE_F16, (rng.standard_normal(200_000) * 4).astype(np.float16)])
    u = np.concatenate([np.ones(FINITE_F16.size, np.float16),
                        (rng.standard_normal(200_000) * 2).astype(np.float16)])
    x = np.stack([g, u], 1)  # rows of I = 1: [gate | up]
    out = o.act_and_mul_f16(x, act)[:, 0].astype(np.float64)
    gd, ud = g.astype(np.float64), u.astype(np.float64)
    ex = (_silu64(gd) if act == "silu" else _gelu64(gd)) * ud
    fin = np.isfinite(ex) & (np.abs(ex) < 65504)
    err = np.abs(out[fin] - ex[fin])
    tol = _f16_ulp(ex[fin])
    assert (err <= tol).all()
    rne = ex[fin].astype(np.float16).astype(np.float64)
    assert (out[fin] != rne).mean() < 1e-3


@pytest.mark.parametrize("act", ["silu", "gelu_tanh"])
def test_act_and_mul_against_torch_fallbacks(act):
    """The reference's CPU path rounds twice (fp16 act, then the fp16 product);
    the oracle rounds once.  Against that eager fallback: within 2 fp16 ulp;
    against torch's fp32 forms rounded once to fp16: within 1 ulp and equal
    except at near-ties (< 0.1 %).  torch evaluates gelu as
    0.5 g (1 + tanh y), which cancels in fp32 when tanh y is near -1 (g < -5:
    absolute error up to |g| 2^-24 before the product with u), so its gelu
    comparisons allow |g u| 2^-23 more."""
    rng = np.random.default_rng(1)
    M, I = 64, 1024
    x = (rng.standard_normal((M, 2 * I)) * 3).astype(np.float16)
    out = o.act_and_mul_f16(x, act).astype(np.float64)
    xt = torch.from_numpy(x)
    gate, up = xt.chunk(2, dim=-1)
    if act == "silu":
        eager = (F.silu(gate) * up)
        f32 = (F.silu(gate.float()) * up.float()).half()
    else:
        eager = (F.gelu(gate, approximate="tanh") * up)
        f32 = (F.gelu(gate.float(), approximate="tanh") * up.float()).half()
    eager = eager.double().numpy()
    f32 = f32.double().numpy()
    ulp = _f16_ulp(np.maximum(np.abs(out), 2 ** -14))
    g64, u64 = x[:, :I].astype(np.float64), x[:, I:].astype(np.float64)
    cancel = 0.0 if act == "silu" else np.abs(g64 * u64) * 2.0 ** -23
    assert (np.abs(out - eager) <= 2 * ulp + cancel).all()
    assert (np.abs(out - f32) <= ulp + cancel).all()
    clean = g64 > -2  # outside torch's cancelling tail
    assert (out[clean] != f32[clean]).mean() < 1e-3


def test_act_known_answers():
    x = np.float16([[0.0, 1.0, 2.0, 3.0], [-0.0, 5.0, -1.0, 7.0]])  # I = 2
    s = o.act_and_mul_f16(x, "silu")
    assert s[0, 0] == 0 and s[1, 0] == 0                    # silu(0) * u = 0
    assert s[0, 1] == np.float16(1 / (1 + math.exp(-1)) * 3)  # silu(1) * 3
    big = np.float16([[60000.0, 0.5], ])  # silu(g) = g for large g; up = 0.5
    assert o.act_and_mul_f16(big, "silu")[0, 0] == np.float16(30000.0)
    neg = np.float16([[-60000.0, 2.0]])  # silu of a large negative gate: 0 (negative side)
    r = o.act_and_mul_f16(neg, "silu")[0, 0]
    assert r == 0 and np.signbit(r)
    ge = o.act_and_mul_f16(np.float16([[0.0, 1.0]]), "gelu_tanh")[0, 0]
    assert ge == 0
    nan = o.act_and_mul_f16(np.float16([[np.nan, 1.0]]), "silu")[0, 0]
    assert np.isnan(nan)


def test_act_quant_is_quant_of_act():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((8, 2 * 520)) * 2).astype(np.float16)
    for act in ("silu", "gelu_tanh"):
        q, s = o.act_and_mul_quant_f16(x, act)
        q2, s2 = o.quant_rowwise_f16(o.act_and_mul_f16(x, act))
        assert np.array_equal(q, q2) and np.array_equal(s, s2)


# ---- RMSNorm ----------------------------------------------------------------

def test_sumsq_fixed_error_bound_and_exact_cases():
    rng = np.random.default_rng(3)
    for K in (1, 7, 8, 100, 2048, 4096, 5000, 65536):
        h = (rng.standard_normal(K) * rng.choice([1e-3, 1.0, 30.0])).astype(np.float16)
        got = float(o.sumsq_fixed(h))
        exact = math.fsum(float(v) ** 2 for v in h.astype(np.float64))
        # recursive summation of n non-negative terms: relative error <= (n-1) u
        assert abs(got - exact) <= (K + 300) * 2 ** -24 * exact
    # exact when every partial sum is representable
    assert float(o.sumsq_fixed(np.ones(4096, np.float16))) == 4096.0
    h = np.zeros(3000, np.float16)
    h[[0, 1234, 2999]] = [3.0, 4.0, 12.0]
    assert float(o.sumsq_fixed(h)) == 169.0


def test_sumsq_fixed_follows_the_stated_order():
    """A row where the order shows: 8192 (square 2^26, fp32 ulp 8) first, ones
    elsewhere.  Summed left to right, every 1 after the first element is
    rounded away; in the fixed order only the ones sharing the big element's
    accumulator are, the rest gather in their own accumulators and survive.  So
    the two results differ, the fixed order's is the one the stated order gives
    (restated here in Python floats rounded to fp32) and far closer to the
    exact sum."""
    K = 8 * 256 * 3
    h = np.ones(K, np.float16)
    h[0] = 8192.0
    f32 = np.float32

    seq = f32(0)
    for v in h:
        seq = f32(seq + f32(v) * f32(v))
    lanes = [f32(0)] * 256
    for c in range(K // 8):
        for k in range(8 * c, 8 * c + 8):
            lanes[c % 256] = f32(lanes[c % 256] + f32(h[k]) * f32(h[k]))
    waves = []
    for w in range(4):
        p = lanes[64 * w:64 * w + 64]
        for d in (32, 16, 8, 4, 2, 1):
            p = [f32(p[i] + p[i ^ d]) for i in range(64)]
        waves.append(p[0])
    want = f32(f32(waves[0] + waves[1]) + f32(waves[2] + waves[3]))
    got = o.sumsq_fixed(h)
    assert got == want and got != seq
    exact = 2 ** 26 + K - 1
    assert abs(float(got) - exact) < abs(float(seq) - exact) / 100


def _rms64(x, w, eps, unit):
    xd = x.astype(np.float64)
    wd = w.astype(np.float64) + (1.0 if unit else 0.0)
    r = 1 / np.sqrt((xd ** 2).mean(-1, keepdims=True) + eps)
    return xd * r * wd


@pytest.mark.parametrize("unit", [False, True])
def test_rmsnorm_within_one_ulp_of_exact(unit):
    rng = np.random.default_rng(4)
    M, K = 48, 4096
    x = (rng.standard_normal((M, K)) * rng.uniform(0.01, 20, (M, 1))).astype(np.float16)
    w = (rng.uniform(0.5, 1.5, K) - (1.0 if unit else 0.0)).astype(np.float16)
    out, _ = o.rmsnorm_f16(x, w, 1e-6, unit_offset=unit)
    ex = _rms64(x, w, 1e-6, unit)
    err = np.abs(out.astype(np.float64) - ex)
    assert (err <= _f16_ulp(np.maximum(np.abs(ex), 2 ** -14))).all()
    assert (out.astype(np.float64) != ex.astype(np.float16).astype(np.float64)).mean() < 0.01


def test_rmsnorm_against_torch_eager_norm():
    """fni8serve/layers/norm.py:37-58 eager, on the CPU in torch: the residual
    add is torch's fp16 add bit for bit, the normed output within 1 fp16 ulp."""
    rng = np.random.default_rng(5)
    M, K = 32, 2048
    x = rng.standard_normal((M, K)).astype(np.float16)
    res = (rng.standard_normal((M, K)) * 4).astype(np.float16)
    w = rng.uniform(0.2, 2.0, K).astype(np.float16)
    eps = 1e-6
    out, h = o.rmsnorm_f16(x, w, eps, residual=res)
    xt = torch.from_numpy(x) + torch.from_numpy(res)  # fp16 add, as norm.py:56
    assert np.array_equal(h.view(np.uint16), xt.numpy().view(np.uint16))
    xf = xt.float()
    ref = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * torch.from_numpy(w).float()).half()
    ref = ref.double().numpy()
    got = out.astype(np.float64)
    assert (np.abs(got - ref) <= _f16_ulp(np.maximum(np.abs(ref), 2 ** -14))).all()
    assert (got != ref).mean() < 0.02


def test_rmsnorm_known_answers_and_identities():
    w1 = np.ones(16, np.float16)
    out, _ = o.rmsnorm_f16(np.full((1, 16), 3.0, np.float16), w1, 0.0)
    assert (out == 1.0).all()                                # c / sqrt(c^2) = 1
    out, _ = o.rmsnorm_f16(np.zeros((1, 16), np.float16), w1, 1e-6)
    assert (out == 0).all()                                  # zero row stays zero
    rng = np.random.default_rng(6)
    x = rng.standard_normal((4, 1000)).astype(np.float16)
    a, _ = o.rmsnorm_f16(x, np.zeros(1000, np.float16), 1e-5, unit_offset=True)
    b, _ = o.rmsnorm_f16(x, np.ones(1000, np.float16), 1e-5, unit_offset=False)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))  # Gemma's (1 + 0) == 1
    y, _ = o.rmsnorm_f16(-x, np.ones(1000, np.float16), 1e-5)
    z, _ = o.rmsnorm_f16(x, np.ones(1000, np.float16), 1e-5)
    assert np.array_equal(y, -z)                             # odd in x
    q, s, h = o.rmsnorm_quant_f16(x, np.ones(1000, np.float16), 1e-5, residual=x)
    n, h2 = o.rmsnorm_f16(x, np.ones(1000, np.float16), 1e-5, residual=x)
    q2, s2 = o.quant_rowwise_f16(n)
    assert np.array_equal(q, q2) and np.array_equal(s, s2) and np.array_equal(h, h2)
