"""The reference trainer's CPU composition (oracle/reference_path.py: fused C products up to 48
rows per expert, C dequantisation + torch sgemm above, lazy_trainer.py:746-880) against the
float64 oracle, with buckets on both sides of the 48-row switch. This is the path bench.py
times as the CPU baseline."""
import numpy as np
import pytest

import oracle
from oracle import reference_path
from tests.conftest import assert_close


@pytest.mark.parametrize("act", ["swiglu", "situ"])
def test_reference_path_both_branches(clib, act):
    rng = np.random.default_rng(71)
    E, D, F = 6, 256, 128
    ex = oracle.random_experts(rng, E, D, F, 119, 123)
    sizes = [120, 49, 48, 10, 1, 0]        # 120 and 49 rows take dequant + sgemm, the rest the fused kernels
    first = np.concatenate([np.full(c, e) for e, c in enumerate(sizes)]).astype(np.int64)
    rng.shuffle(first)
    N = first.size
    second = (first + 1 + rng.integers(0, E - 1, N)) % E
    idx = np.stack([first, second], 1).astype(np.int64)
    w = rng.dirichlet([1, 1], N).astype(np.float32)
    h = rng.standard_normal((N, D)).astype(np.float32)
    g = rng.standard_normal((N, D)).astype(np.float32)
    counts = np.bincount(idx.ravel(), minlength=E)
    assert (counts > 48).any() and (counts <= 48).any()
    out = reference_path.routed_forward(clib, h, idx, w, ex, act)
    assert_close(out, oracle.routed_forward(h, idx, w, ex, act), f"reference path fwd {act}", rel=1e-5, cos=0.99999999)
    gh, gw = reference_path.routed_backward(clib, h, idx, w, ex, g, act)
    gh64, gw64 = oracle.routed_backward(h, idx, w, ex, g, act)
    assert_close(gh, gh64, f"reference path grad_h {act}", rel=1e-5, cos=0.99999999)
    assert_close(gw, gw64, f"reference path grad_w {act}", rel=1e-5, cos=0.99999999)


def test_fused_branch_equals_c_composition(clib):
    """With every bucket at or below 48 rows the composition is the fused C path, which the C
    oracle's own composition also runs: the same products, so results agree to fp32 rounding of
    the GLU and the index_add order."""
    rng = np.random.default_rng(72)
    E, D, F, N = 16, 512, 256, 64
    ex = oracle.random_experts(rng, E, D, F, 118, 122)
    idx, w = oracle.softmax_topk(rng.standard_normal((N, E)).astype(np.float32), 4)
    assert np.bincount(idx.ravel(), minlength=E).max() <= 48
    h = rng.standard_normal((N, D)).astype(np.float32)
    out = reference_path.routed_forward(clib, h, idx, w, ex)
    assert_close(out, clib.moe_forward(h, idx, w, ex), "fused branch vs C composition", rel=1e-6, cos=0.9999999999)
