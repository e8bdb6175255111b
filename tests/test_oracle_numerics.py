"""Pins the oracle's scalar numerics: fp16 conversions, exp/log/rsqrt."""
import numpy as np


def test_h2f_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = oracle.h2f(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f2h_rne_matches_ieee_cast(oracle):
    rng = np.random.default_rng(1)
    # random bit patterns over the whole float range, plus all halfway points
    x = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    halves = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    h32 = halves.astype(np.float64)
    fin = np.isfinite(h32)
    mids = ((h32[fin][:-1] + h32[fin][1:]) / 2).astype(np.float32)
    x = np.concatenate([x, mids, np.array([65504, 65519.99, 65520, 1e-8, 2**-25, 2**-24, -0.0],
                                          dtype=np.float32)])
    ours = oracle.f2h(x)
    ref = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.all((ours[nan] & 0x7C00) == 0x7C00) and np.all((ours[nan] & 0x3FF) != 0)


def test_f2h_trunc_rules(oracle):
    lib = oracle.lib()
    # vk_session.cpp:69-89: truncation, fp32 subnormals and fp16-subnormal results flush
    assert lib.orc_f2h_trunc(1.0) == 0x3C00
    assert lib.orc_f2h_trunc(1.0009765) == 0x3C00          # below 1+2^-10: truncated
    assert lib.orc_f2h_trunc(-2.5) == 0xC100
    assert lib.orc_f2h_trunc(1e-5) == 0x0000               # fp16 subnormal range -> +0
    assert lib.orc_f2h_trunc(-1e-5) == 0x8000
    assert lib.orc_f2h_trunc(1e-40) == 0x0000              # fp32 subnormal -> 0
    assert lib.orc_f2h_trunc(70000.0) == 0x7C00
    assert lib.orc_f2h_trunc(float("inf")) == 0x7C00
    assert lib.orc_f2h_trunc(float("nan")) == 0x7E00
    assert lib.orc_f2h_trunc(65519.0) == 0x7BFF            # truncation never rounds up


def _ulps32(a, b):
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


def test_expf_accuracy(oracle):
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.uniform(-87, 88, 1 << 20), rng.uniform(-1, 1, 1 << 16),
                        np.linspace(-0.5, 0.5, 4097)]).astype(np.float32)
    ours = oracle.expf(x)
    ref = np.exp(x.astype(np.float64)).astype(np.float32)
    assert _ulps32(ours, ref).max() <= 2
    # special values and the subnormal / overflow edges
    sp = np.array([0.0, -0.0, 88.72, 88.73, -103.9, -104.0, -np.inf, np.inf], dtype=np.float32)
    o = oracle.expf(sp)
    assert o[0] == 1.0 and o[1] == 1.0 and np.isfinite(o[2]) and np.isinf(o[3])
    assert o[4] > 0 and o[5] == 0 and o[6] == 0 and np.isinf(o[7])
    assert np.isnan(oracle.expf(np.array([np.nan], dtype=np.float32)))[0]


def test_logf_accuracy(oracle):
    rng = np.random.default_rng(3)
    x = np.concatenate([np.exp(rng.uniform(-80, 80, 1 << 20)), rng.uniform(0.5, 2, 1 << 16),
                        1 + rng.uniform(0, 1e-3, 4096)]).astype(np.float32)
    ours = oracle.logf(x).astype(np.float64)
    ref = np.log(x.astype(np.float64))
    # relative 2 ulp, or an absolute error of 2^-24 near log(1) = 0
    err = np.abs(ours - ref)
    assert np.all(err <= np.maximum(2.5 * np.spacing(np.abs(ref).astype(np.float32)), 2 ** -24))
    o = oracle.logf(np.array([1.0, 0.0, -1.0, np.inf], dtype=np.float32))
    assert o[0] == 0.0 and np.isneginf(o[1]) and np.isnan(o[2]) and np.isposinf(o[3])
