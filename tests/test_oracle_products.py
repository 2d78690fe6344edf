"""Pins the oracle's products: the C restatement (the CPU baseline) is bit-identical to the
reference's compiled mxfp4_gemm / mxfp4_gemm_t wherever the reference can run (K <= 4096 for
the forward), and both agree with the textbook float64 product, including at the BASELINE
shapes the reference's fixed tile cannot hold."""
import numpy as np
import pytest

import oracle


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


SHAPES = [(1, 256, 128), (16, 256, 128), (9, 128, 256), (5, 4096, 61), (33, 1024, 200), (3, 96, 17)]


@pytest.mark.parametrize("M,K,R", SHAPES)
def test_gemm_bit_identical_to_reference(reflib, clib, rng, M, K, R):
    x = rng.standard_normal((M, K)).astype(np.float32)
    p, s = oracle.random_mx(rng, (R, K), 110, 130)
    assert np.array_equal(bits(clib.gemm(x, p, s)), bits(reflib.gemm(x, p, s)))


@pytest.mark.parametrize("M,K,R", SHAPES)
def test_gemm_t_bit_identical_to_reference(reflib, clib, rng, M, K, R):
    dy = rng.standard_normal((M, R)).astype(np.float32)
    p, s = oracle.random_mx(rng, (R, K), 110, 130)
    assert np.array_equal(bits(clib.gemm_t(dy, p, s)), bits(reflib.gemm_t(dy, p, s)))


@pytest.mark.parametrize("M,K,R", SHAPES + [(4, 7168, 64), (2, 2048, 300)])
def test_products_match_float64(clib, rng, M, K, R):
    x = rng.standard_normal((M, K)).astype(np.float32)
    dy = rng.standard_normal((M, R)).astype(np.float32)
    p, s = oracle.random_mx(rng, (R, K), 117, 121)
    assert oracle.rel_l2(clib.gemm(x, p, s), oracle.gemm(x, p, s)) < 1e-6
    assert oracle.rel_l2(clib.gemm_t(dy, p, s), oracle.gemm_t(dy, p, s)) < 1e-6


def test_special_cases(clib, rng):
    K, R = 256, 24
    x = rng.standard_normal((3, K)).astype(np.float32)
    # all scales damaged -> exact zeros (mxfp4_gemm.c:16-18)
    p, _ = oracle.random_mx(rng, (R, K), 0, 0)
    s = np.full((R, K // 32), 255, np.uint8)
    assert np.all(clib.gemm(x, p, s) == 0)
    # one nonzero code per row -> the product picks one x column, scaled exactly
    p = np.zeros((R, K // 2), np.uint8)
    s = np.full((R, K // 32), 127, np.uint8)
    cols = rng.integers(0, K, size=R)
    for r, c in enumerate(cols):
        p[r, c // 2] = (0x2 if c % 2 == 0 else 0x20)  # code 2 = 1.0
    y = clib.gemm(x, p, s)
    assert np.array_equal(y, x[:, cols])
    # M = 1 (GEMV) against the float64 product
    p, s = oracle.random_mx(rng, (R, K), 120, 125)
    assert oracle.rel_l2(clib.gemm(x[:1], p, s), oracle.gemm(x[:1], p, s)) < 1e-6


def test_dequant_then_matmul_equals_product(clib, rng):
    """The >48-row path of the reference (C dequant then sgemm, lazy_trainer.py:756-759) and the
    fused path compute the same product."""
    p, s = oracle.random_mx(rng, (64, 512), 117, 121)
    x = rng.standard_normal((50, 512)).astype(np.float32)
    w = clib.dequant(p, s)
    assert oracle.rel_l2(x.astype(np.float64) @ w.astype(np.float64).T, clib.gemm(x, p, s)) < 1e-6
