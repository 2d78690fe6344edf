"""mxfp4_gemm_noalloc, the allocation-free variant of mxfp4_gemm, through the C ABI.

It stages x's activation tiles in the library's static device scratch instead of a caller
workspace; the kernels are the same, so its output must equal mxfp4_gemm's bit for bit. Two calls
in a row (the second smaller) check that the scratch left behind by one call does not leak into
the next; a size beyond the scratch must be rejected without a launch."""
import ctypes

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    from lazylora_amd import native
    return native._load_library()


def case(msg):
    print(f"\n[case] {msg}", flush=True)


def gemm_ws(lib, x, p, s):
    M, K = x.shape
    R = p.shape[0]
    y = torch.empty((M, R), dtype=torch.float32, device="cuda")
    nws = lib.mxfp4_gemm_workspace_size(M, K, R)
    ws = torch.empty(nws, dtype=torch.uint8, device="cuda")
    rc = lib.mxfp4_gemm(y.data_ptr(), x.data_ptr(), p.data_ptr(), s.data_ptr(), M, K, R, ws.data_ptr(), nws,
                        torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.mxfp4_last_error()
    return y


def gemm_noalloc(lib, x, p, s):
    M, K = x.shape
    R = p.shape[0]
    y = torch.full((M, R), float("nan"), dtype=torch.float32, device="cuda")
    rc = lib.mxfp4_gemm_noalloc(y.data_ptr(), x.data_ptr(), p.data_ptr(), s.data_ptr(), M, K, R,
                                torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.mxfp4_last_error()
    return y


@pytest.mark.parametrize("K,R,M1,M2", [(7168, 2048, 256, 7), (2048, 7168, 40, 16), (4128, 96, 33, 1)])
def test_noalloc_equals_workspace_entry(lib, K, R, M1, M2):
    """Two calls in a row, the second with a smaller input (fewer rows, so the first call's
    tiles are still in the scratch), each bit-identical to mxfp4_gemm with its own workspace;
    K = 4128 exercises the zero padding of a partial 512-wide chunk."""
    rng = np.random.default_rng(K + R)
    pk, sc = oracle.random_mx(rng, (R, K), 117, 121)
    P, S = torch.from_numpy(pk).cuda(), torch.from_numpy(sc).cuda()
    for M in (M1, M2):
        case(f"gemm_noalloc M={M} K={K} R={R}")
        x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda()
        got = gemm_noalloc(lib, x, P, S)
        want = gemm_ws(lib, x, P, S)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"M={M}: differs from mxfp4_gemm"
        if M <= 16:
            ref = oracle.gemm(x.cpu().numpy(), pk, sc)
            assert oracle.rel_l2(got.cpu().numpy(), ref) <= 5e-3


def test_noalloc_rejects_sizes_beyond_scratch(lib):
    case("gemm_noalloc beyond its 16 MiB scratch")
    K, R = 7168, 64
    M = 16 * 71  # 71 tiles of 14 chunks x 16896 B > 16 MiB
    x = torch.zeros((M, K), dtype=torch.float32, device="cuda")
    p = torch.zeros((R, K // 2), dtype=torch.uint8, device="cuda")
    s = torch.zeros((R, K // 32), dtype=torch.uint8, device="cuda")
    y = torch.zeros((M, R), dtype=torch.float32, device="cuda")
    rc = lib.mxfp4_gemm_noalloc(y.data_ptr(), x.data_ptr(), p.data_ptr(), s.data_ptr(), M, K, R,
                                torch.cuda.current_stream().cuda_stream)
    assert rc == -2 and b"16 MiB" in lib.mxfp4_last_error()
    ok = gemm_noalloc(lib, x[: 16 * 70], p, s)  # 70 tiles fit
    torch.cuda.synchronize()
    assert torch.equal(ok, torch.zeros_like(ok))
