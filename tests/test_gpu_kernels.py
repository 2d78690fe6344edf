"""Single-expert kernels on the GPU against the oracle, through the C ABI (via lazylora_amd.native).

Bar: dequant bit-exact; products within rel-L2 5e-3 and cosine 0.9999 of the reference's
fp32 C path (this repo's C restatement, bit-identical to it where the reference runs)."""
import numpy as np
import pytest
import torch

import oracle
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def k():
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    from lazylora_amd.native import kernel
    return kernel()


def cuda(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def case(msg):
    print(f"\n[case] {msg}", flush=True)


def test_dequant_all_pairs_bit_exact(k):
    case("dequant: all 65536 (byte, scale) pairs")
    packed = np.repeat(np.arange(256, dtype=np.uint8), 16)[None, :].repeat(256, axis=0)
    scales = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 256, axis=1)
    got = k.dequant(cuda(packed), cuda(scales)).cpu().numpy()
    want = oracle.dequant(packed, scales)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequant_expert_matrix_bit_exact(k, rng):
    case("dequant: [2048, 7168] random codes and scales")
    p, s = oracle.random_mx(rng, (2048, 7168), 0, 255)
    got = k.dequant(cuda(p), cuda(s)).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), oracle.dequant(p, s).view(np.uint32))


def test_dequant_bf16_all_pairs_bit_exact(k):
    case("dequant bf16: all 65536 (byte, scale) pairs")
    packed = np.repeat(np.arange(256, dtype=np.uint8), 16)[None, :].repeat(256, axis=0)
    scales = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 256, axis=1)
    got = k.dequant(cuda(packed), cuda(scales), out_dtype=torch.bfloat16)
    assert got.dtype == torch.bfloat16 and got.shape == (256, 8192)
    want32 = oracle.dequant(packed, scales)
    assert not (want32.view(np.uint32) & 0xFFFF).any()  # every decoded value is exact in bf16
    want = torch.from_numpy(want32).to(torch.bfloat16)  # the reference's .to(bfloat16)
    assert torch.equal(got.cpu().view(torch.int16), want.view(torch.int16))


def test_dequantize_mxfp4_mirror(k, rng):
    """lazylora_amd.streaming.dequantize_mxfp4 against the reference's _dequantize_mxfp4 contract
    (expert_streamer.py:104-154): bf16 by default, fp32 / fp16 on request, one scale per row,
    NumPy and CPU inputs."""
    case("dequantize_mxfp4: dtypes, per-row scales, NumPy and CPU inputs")
    from lazylora_amd.streaming import _dequantize_mxfp4, dequantize_mxfp4
    p, s = oracle.random_mx(rng, (96, 320), 0, 255)
    want32 = oracle.dequant(p, s)
    w = dequantize_mxfp4(cuda(p), cuda(s))
    assert w.dtype == torch.bfloat16 and w.is_cuda
    assert torch.equal(w.cpu().view(torch.int16), torch.from_numpy(want32).to(torch.bfloat16).view(torch.int16))
    w32 = _dequantize_mxfp4(cuda(p), cuda(s), out_dtype=torch.float32)
    assert np.array_equal(w32.cpu().numpy().view(np.uint32), want32.view(np.uint32))
    w16 = dequantize_mxfp4(cuda(p), cuda(s), out_dtype=torch.float16)
    assert w16.dtype == torch.float16 and torch.equal(w16.cpu(), torch.from_numpy(want32).to(torch.float16))
    s1 = rng.integers(0, 256, 96).astype(np.uint8)  # one scale byte per row
    want1 = oracle.dequant(p, np.repeat(s1[:, None], 320 // 32, axis=1))
    w1 = dequantize_mxfp4(cuda(p), cuda(s1), out_dtype=torch.float32)
    assert np.array_equal(w1.cpu().numpy().view(np.uint32), want1.view(np.uint32))
    wn = dequantize_mxfp4(p, s)
    assert isinstance(wn, np.ndarray) and wn.dtype == np.float32
    assert np.array_equal(wn.view(np.uint32), want32.view(np.uint32))
    wc = dequantize_mxfp4(torch.from_numpy(p), torch.from_numpy(s))
    assert wc.device.type == "cpu" and wc.dtype == torch.bfloat16
    with pytest.raises(ValueError):
        dequantize_mxfp4(cuda(p), cuda(s), group_size=16)


GEMM_SHAPES = [
    (1, 256, 128), (16, 256, 128), (64, 128, 256),                 # config-1 expert shapes
    (1, 7168, 2048), (4, 7168, 2048), (16, 7168, 2048),             # config-2 gate/up, M sweep
    (64, 7168, 2048), (256, 7168, 2048), (16, 2048, 7168),          # ... and down
    (5, 96, 17), (33, 160, 100), (17, 640, 65),                     # ragged: K % 128 != 0, R % 64 != 0
    (20, 1024, 100), (7, 512, 200), (3, 1536, 300), (40, 4608, 72), # K % 512 == 0 with ragged R,
]                                                                   # odd and > 8 super-chunk counts


@pytest.mark.parametrize("M,K,R", GEMM_SHAPES)
def test_gemm_matches_reference_path(k, clib, rng, M, K, R):
    case(f"gemm M={M} K={K} R={R}")
    x = rng.standard_normal((M, K)).astype(np.float32)
    p, s = oracle.random_mx(rng, (R, K), 117, 121)
    got = k.gemm(cuda(x), cuda(p), cuda(s)).cpu().numpy()
    assert got.shape == (M, R)
    assert_close(got, clib.gemm(x, p, s), f"gemm {M}x{K}x{R}")


@pytest.mark.parametrize("M,K,R", GEMM_SHAPES)
def test_gemm_t_matches_reference_path(k, clib, rng, M, K, R):
    case(f"gemm_t M={M} K={K} R={R}")
    dy = rng.standard_normal((M, R)).astype(np.float32)
    p, s = oracle.random_mx(rng, (R, K), 117, 121)
    got = k.gemm_t(cuda(dy), cuda(p), cuda(s)).cpu().numpy()
    assert got.shape == (M, K)
    assert_close(got, clib.gemm_t(dy, p, s), f"gemm_t {M}x{K}x{R}", rel=2e-5, cos=0.99999999)


def test_damaged_scales_contribute_zero(k, clib, rng):
    case("gemm / gemm_t / dequant with scale bytes 253, 254, 255 sprinkled in")
    M, K, R = 8, 1024, 96
    p, s = oracle.random_mx(rng, (R, K), 117, 121)
    hit = rng.random(s.shape) < 0.1
    s[hit] = rng.integers(253, 256, size=int(hit.sum()))
    x = rng.standard_normal((M, K)).astype(np.float32)
    y = k.gemm(cuda(x), cuda(p), cuda(s)).cpu().numpy()
    assert np.all(np.isfinite(y))
    assert_close(y, clib.gemm(x, p, s), "gemm damaged")
    dy = rng.standard_normal((M, R)).astype(np.float32)
    t = k.gemm_t(cuda(dy), cuda(p), cuda(s)).cpu().numpy()
    assert np.all(np.isfinite(t))
    assert_close(t, clib.gemm_t(dy, p, s), "gemm_t damaged", rel=2e-5)
    w = k.dequant(cuda(p), cuda(s)).cpu().numpy()
    assert np.array_equal(w.view(np.uint32), oracle.dequant(p, s).view(np.uint32))


def test_all_scales_damaged_gives_zeros(k, rng):
    case("gemm with every scale byte = 255")
    p, _ = oracle.random_mx(rng, (64, 512), 0, 0)
    s = np.full((64, 16), 255, np.uint8)
    y = k.gemm(cuda(rng.standard_normal((4, 512)).astype(np.float32)), cuda(p), cuda(s)).cpu().numpy()
    assert np.all(y == 0)


def test_gemm_power_of_two_scaling_is_exact(k, rng):
    """Scaling x by 2^j moves only the activation block scales: the product scales exactly."""
    case("gemm power-of-two scaling")
    p, s = oracle.random_mx(rng, (256, 2048), 117, 121)
    x = rng.standard_normal((16, 2048)).astype(np.float32)
    a = k.gemm(cuda(x), cuda(p), cuda(s)).cpu().numpy()
    b = k.gemm(cuda(x * 32.0), cuda(p), cuda(s)).cpu().numpy()
    c = k.gemm(cuda(x / 1024.0), cuda(p), cuda(s)).cpu().numpy()
    assert np.array_equal(b, a * 32.0) and np.array_equal(c, a / 1024.0)


def test_products_are_deterministic(k, rng):
    case("gemm / gemm_t repeatability")
    p, s = oracle.random_mx(rng, (2048, 7168), 117, 121)
    P, S = cuda(p), cuda(s)
    x = cuda(rng.standard_normal((16, 7168)).astype(np.float32))
    dy = cuda(rng.standard_normal((16, 2048)).astype(np.float32))
    assert torch.equal(k.gemm(x, P, S), k.gemm(x, P, S))
    assert torch.equal(k.gemm_t(dy, P, S), k.gemm_t(dy, P, S))


def test_cpu_tensors_round_trip(k, clib, rng):
    """The unmodified CPU trainer passes CPU tensors: results come back on the CPU."""
    case("gemm with CPU tensors")
    p, s = oracle.random_mx(rng, (128, 256), 117, 121)
    x = rng.standard_normal((3, 256)).astype(np.float32)
    y = k.gemm(torch.from_numpy(x), torch.from_numpy(p), torch.from_numpy(s))
    assert y.device.type == "cpu"
    assert_close(y.numpy(), clib.gemm(x, p, s), "gemm cpu tensors")
