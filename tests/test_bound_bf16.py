"""The sparse variant's error bound, checked by emulating its bf16 sweep on the CPU.

The default kernel (sparse) sweeps every (point, component) pair on bf16
matrix cores.  Each fp32 operand is split into bf16 hi + lo, three products
per term are issued (lo*hi, hi*lo, hi*hi), and the sums accumulate in fp32.
A pair is evaluated exactly only if its upper bound ll + E reaches the
point's window, so the bound E must hold for every pair.  If it did not, a
dominant pair could be skipped and nothing downstream would notice.

This test restates the sweep's arithmetic in numpy, following the kernel
step by step:
  * the coefficients as ``write_coeffs`` forms them (fgmm_common.hip);
  * the point operands as ``pass1_x32_kernel`` splits them (fgmm_x32.hip):
    x^2 rounded to fp32, then each value split into bf16 hi + lo with
    round-to-nearest-even;
  * per 32-feature step, the three products in the kernel's order
    (lo*hi, hi*lo, hi*hi), into two fp32 accumulators (the x^2 half a0, and
    the bias + x half a1);
  * ll = fl(a0 + a1), E = fma(2c, -a0, Z) in fp32.
It then asserts |ll - ll_exact| <= E on adversarial rows.  ll_exact is the
fp64 direct form log2(e) (log_coeff - sum (x - mu)^2 / (2 var)), and c is
the library's own constant (fgmm_error_model).

Hardware assumption.  The order in which one v_mfma_f32_16x16x32_bf16 adds
its 32 exact products to the fp32 accumulator is not documented.  The bound
assumes the result is no worse than some association of fp32 additions,
each rounding a partial sum by at most 2^-24 relative.  The test therefore
checks three accumulation models of the instruction:
  * sequential fp32 adds in feature order;
  * sequential fp32 adds in reverse order;
  * the exact sum of the 32 products, rounded once into the accumulator.
The bound must hold under each of them.
"""
import ctypes
import math

import numpy as np
import pytest

LOG2E = 1.4426950408889634
LOG2PI = 1.8378770664093454


def bf16(a):
    """fp32 -> bf16 (round to nearest even), returned as fp32 values."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def split(a):
    a = np.asarray(a, np.float32)
    h = bf16(a)
    return h, bf16((a - h).astype(np.float32))


def mfma_acc(acc, prods, model):
    """acc (fp32 [M]) plus the 32 products of one instruction (fp32 [M, 32],
    each exact) under accumulation model `model`."""
    if model == "exact_once":
        return (acc.astype(np.float64) + prods.astype(np.float64).sum(axis=1)).astype(np.float32)
    order = range(prods.shape[1]) if model == "seq" else range(prods.shape[1] - 1, -1, -1)
    for i in order:
        acc = (acc + prods[:, i]).astype(np.float32)
    return acc


def sweep(x, mu, var, lp, c_bf, model):
    """Emulated kernel output for M pairs (row m of x against row m of the
    component parameters).  Returns (ll, E, ll_exact, base) where base =
    |bias| + D + 2|a0| is the bound's scale."""
    M, d = x.shape
    dpb = (((d + 15) // 16 * 16) + 31) // 32 * 32
    pad = dpb - d
    x = np.pad(x.astype(np.float32), ((0, 0), (0, pad)))
    iv = 1.0 / var.astype(np.float64)
    fa = np.pad((-0.5 * LOG2E * iv).astype(np.float32), ((0, 0), (0, pad)))
    fb = np.pad((LOG2E * mu.astype(np.float64) * iv).astype(np.float32), ((0, 0), (0, pad)))
    lc = lp.astype(np.float64) - 0.5 * (d * LOG2PI + np.log(var.astype(np.float64)).sum(1))
    q = (mu.astype(np.float64) ** 2 * iv).sum(1)
    be = LOG2E * (lc - 0.5 * q)
    bias32 = be.astype(np.float32)
    Z = (c_bf * (np.abs(be) + 0.5 * LOG2E * q) * (1.0 + 1e-6)).astype(np.float32)
    slope = np.float32(2.0 * c_bf)

    x2h, x2l = split((x * x).astype(np.float32))
    x1h, x1l = split(x)
    ah, al = split(fa)
    bh, bl = split(fb)
    a0 = np.zeros(M, np.float32)
    a1 = bias32.copy()
    for u in range(dpb // 32):
        s = slice(32 * u, 32 * u + 32)
        for A, B in ((al, x2h), (ah, x2l), (ah, x2h)):
            a0 = mfma_acc(a0, (A[:, s] * B[:, s]).astype(np.float32), model)
    for u in range(dpb // 32):
        s = slice(32 * u, 32 * u + 32)
        for A, B in ((bl, x1h), (bh, x1l), (bh, x1h)):
            a1 = mfma_acc(a1, (A[:, s] * B[:, s]).astype(np.float32), model)
    ll = (a0 + a1).astype(np.float32)
    E = (slope.astype(np.float64) * -a0.astype(np.float64) + Z).astype(np.float32)  # fmaf
    diff = x[:, :d].astype(np.float64) - mu.astype(np.float64)
    ll_exact = LOG2E * (lc - 0.5 * (diff * diff * iv).sum(1))
    base = np.abs(be) + 0.5 * LOG2E * q + 2.0 * np.abs(a0.astype(np.float64))
    return ll.astype(np.float64), E.astype(np.float64), ll_exact, base


def worst_split(rng, size, lo, hi):
    """Values in [lo, hi] whose bf16 hi/lo split leaves the largest residue:
    mantissas just below a bf16 rounding midpoint, and the lo part again just
    below a midpoint."""
    v = rng.uniform(lo, hi, size * 8).astype(np.float32)
    h, l_ = split(v)
    resid = np.abs(v.astype(np.float64) - h - l_) / np.maximum(np.abs(v), 1e-30)
    drop = np.abs(l_.astype(np.float64)) / np.maximum(np.abs(v), 1e-30)
    score = resid * 2**16 + drop * 2**8
    return v[np.argsort(-score)[:size]]


def adversarial_rows(rng, M, d):
    """Rows in the style of C5's outliers: x in [-20, 20], var down to 1/16,
    |mu| up to 20, split-residue-heavy values, and sign patterns that make
    every dropped or rounded term add up."""
    cases = []
    # outliers far from a narrow component
    x = rng.uniform(-20, 20, (M, d))
    mu = rng.uniform(-20, 20, (M, d))
    var = np.full((M, d), 1.0 / 16)
    cases.append((x, mu, var))
    # x = mu: the two halves cancel, the error scale is all |a0| and D
    mu = rng.uniform(-20, 20, (M, d))
    cases.append((mu + rng.normal(0, 1e-3, (M, d)), mu, np.exp(rng.uniform(np.log(1 / 16), np.log(4), (M, d)))))
    # x = -mu: |P2 x| = |P1| (mu^2 + x^2), the bound's base is tight
    mu = rng.uniform(5, 20, (M, d)) * rng.choice([-1, 1], (M, d))
    cases.append((-mu, mu, np.full((M, d), 1.0 / 16)))
    # worst split residues, all of one sign, mu = 0 (D = 0: the 2|a0| term alone)
    xs = worst_split(rng, M * d, 1.0, 20.0).reshape(M, d)
    vs = 1.0 / worst_split(rng, M * d, 1.0, 16.0).reshape(M, d)
    cases.append((xs, np.zeros((M, d)), vs))
    # worst split residues in x, mu and var, same signs
    ms = worst_split(rng, M * d, 1.0, 20.0).reshape(M, d)
    cases.append((xs, ms, vs))
    return [(a.astype(np.float32), b.astype(np.float32), c.astype(np.float32)) for a, b, c in cases]


@pytest.fixture(scope="module")
def consts():
    from flashgmm_amd import _lib
    lib = _lib.load()

    def get(d):
        c32, cbf = ctypes.c_double(), ctypes.c_double()
        _lib.check(lib.fgmm_error_model(d, ctypes.byref(c32), ctypes.byref(cbf)))
        return c32.value, cbf.value
    return get


def test_error_model_constants(consts):
    """The constants follow the derivation in fgmm_internal.h: per term 3 x
    2^-16 (two split residues and the dropped lo*lo product) + (3 dpb + 8)
    2^-24 (chained fp32 additions and input roundings), doubled."""
    for d, dpb in ((1, 32), (32, 32), (33, 64), (64, 64), (100, 128), (128, 128)):
        _, cbf = consts(d)
        assert cbf == 2.0 * (3 * 2.0**-16 + (3 * dpb + 8) * 2.0**-24)
        assert 1.3e-4 < consts(128)[1] < 1.4e-4


@pytest.mark.parametrize("d", [128, 64, 33])
@pytest.mark.parametrize("model", ["seq", "rev", "exact_once"])
def test_bf16_split_sweep_stays_within_bound(consts, d, model):
    rng = np.random.default_rng(1000 + d)
    c_bf = consts(d)[1]
    worst = 0.0
    for x, mu, var in adversarial_rows(rng, 256, d):
        lp = np.full(x.shape[0], -math.log(512), np.float32)
        ll, E, ll_exact, base = sweep(x, mu, var, lp, c_bf, model)
        err = np.abs(ll - ll_exact)
        assert np.all(err <= E), (f"d={d} {model}: |ll_bf - ll_exact| {err.max():.4g} > "
                                  f"E {E[err.argmax()]:.4g}")
        worst = max(worst, float((err / base).max()))
    # the measured error, relative to the bound's scale, against the constant
    print(f"[bound] d={d} {model}: max |err| / (|bias|+D+2|a0|) = {worst:.3e}, c_bf = {c_bf:.3e}")
    assert worst < c_bf


def test_bound_without_a0_term_fails(consts):
    """Teeth: the same emulation rejects a bound that leaves out the 2|a0|
    term (the rounding of the x^2 half).  With mu = 0 the bound's other terms
    are tiny, so the x^2 half's error must be covered by 2c|a0| alone."""
    rng = np.random.default_rng(7)
    c_bf = consts(128)[1]
    x, mu, var = adversarial_rows(rng, 256, 128)[3]
    lp = np.full(x.shape[0], -math.log(512), np.float32)
    ll, E, ll_exact, base = sweep(x, mu, var, lp, c_bf, "seq")
    a0_abs = (base - 0.0) / 2.0   # base = |bias| + D + 2|a0|, here D = 0
    E_no_a0 = E - 2.0 * c_bf * a0_abs
    assert np.any(np.abs(ll - ll_exact) > np.maximum(E_no_a0, 0.0))
