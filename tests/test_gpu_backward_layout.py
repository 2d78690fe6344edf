"""The backward layout (mxfp4_backward_layout, ExpertLayer.prepare_backward_layout): its bytes
against a NumPy construction from the definition in include/lazylora_mxfp4.h, and the routed
backward with it against the same layer without it. The transposed work-groups (one-tile and
large-bucket) read the same code and scale bytes from either layout and apply them in the same
order, so every result is bit-identical: uniform routing, large buckets with LoRA, only W1|W3 or
only W2 laid out, with and without the forward layout, and at the BASELINE config-4 size under
uniform and Zipf routing."""
import numpy as np
import pytest
import torch

import oracle
from test_gpu_forward_layout import adapters, inputs, layer_of

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def k():
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    from lazylora_amd.native import kernel
    return kernel()


def case(msg):
    print(f"\n[case] {msg}", flush=True)


def layout_numpy(packed: np.ndarray, scales: np.ndarray, R: int, K: int) -> np.ndarray:
    """Per expert: per block (32-row step st, 256-column stripe c), in order st * (K / 256) + c,
    the codes: load u, lane l = 16 g + n, bytes 8n .. 8n + 7 of the stripe in rows 32 st + 8g + 2u
    and 32 st + 8g + 2u + 1; then, after all codes, per block the scales: entry m = 8 g + j, byte
    q = the scale of row 32 st + 8g + q for MX block 8c + j."""
    E = packed.shape[0]
    nst, nstr = R // 32, K // 256
    # rows 32 st + 8 g + 2 u + parity, code bytes 128 c + 8 n + b
    p = packed.reshape(E, nst, 4, 4, 2, nstr, 16, 8)
    codes = p.transpose(0, 1, 5, 3, 2, 6, 4, 7)  # [E, st, c, u, g, n, parity, b]
    # rows 32 st + 8 g + q, scale columns 8 c + j
    s = scales.reshape(E, nst, 4, 8, nstr, 8)
    sc = s.transpose(0, 1, 4, 2, 5, 3)  # [E, st, c, g, j, q]
    return np.concatenate([codes.reshape(E, -1), sc.reshape(E, -1)], axis=1).reshape(-1)


@pytest.mark.parametrize("E,R,K", [(3, 64, 512), (2, 96, 768), (1, 2048, 7168), (2, 7168, 2048)])
def test_layout_bytes(k, E, R, K):
    case(f"backward layout bytes E={E} R={R} K={K}")
    rng = np.random.default_rng(E * 1000 + R + K)
    packed = rng.integers(0, 256, (E, R, K // 2), dtype=np.uint8)
    scales = rng.integers(0, 256, (E, R, K // 32), dtype=np.uint8)
    got = k.backward_layout(torch.from_numpy(packed).cuda(), torch.from_numpy(scales).cuda()).cpu().numpy()
    want = layout_numpy(packed, scales, R, K)
    assert got.size == want.size == k.lib.mxfp4_backward_layout_bytes(E, R, K)
    assert np.array_equal(got, want)


def test_layout_shape_limits(k):
    case("backward layout rejects R % 32 and K % 256")
    z = lambda *sh: torch.zeros(sh, dtype=torch.uint8, device="cuda")
    with pytest.raises(ValueError):
        k.backward_layout(z(1, 40, 256), z(1, 40, 16))  # R = 40
    with pytest.raises(ValueError):
        k.backward_layout(z(1, 64, 192), z(1, 64, 12))  # K = 384


def both_ways(k, L, H, I, W, G, act="swiglu", lora=None, forward_layout=True):
    """Forward, backward recomputing the forward and backward reusing it, without and with the
    backward layout (and with or without the forward layout on both sides): bit-identical."""
    if forward_layout:
        L.prepare_forward_layout()
    else:
        L.drop_forward_layout()
    res = []
    for use in (False, True):
        if use:
            assert L.prepare_backward_layout() > 0
        else:
            L.drop_backward_layout()
        ws = torch.empty(k.moe_workspace_bytes(H.shape[0], I.shape[1], L.E, L.D, L.F), dtype=torch.uint8,
                         device="cuda")
        out = k.routed_forward(H, I, W, L, act=act, save_for_backward=True, workspace=ws, lora=lora)
        reuse = k.routed_backward(H, I, W, L, G, act=act, reuse_forward=True, workspace=ws, lora=lora)
        recompute = k.routed_backward(H, I, W, L, G, act=act, lora=lora)
        res.append([out] + [t for r in (reuse, recompute) for t in (r[:2] + tuple(r[2]) if lora else r)])
    L.drop_backward_layout()
    L.drop_forward_layout()
    for i, (a, b) in enumerate(zip(*res)):
        assert torch.equal(a, b), f"result {i} differs with the backward layout"


@pytest.mark.parametrize("act", ["swiglu", "situ"])
def test_routed_layer_small_buckets(k, act):
    case(f"routed layer with/without backward layout, uniform top-2, {act}")
    rng = np.random.default_rng(71)
    L = layer_of(oracle.random_experts(rng, 8, 1024, 512, 119, 123))
    both_ways(k, L, *inputs(rng, 96, 1024, 8, 2), act=act)


def test_without_forward_layout(k):
    case("routed layer with/without backward layout, no forward layout")
    rng = np.random.default_rng(72)
    L = layer_of(oracle.random_experts(rng, 8, 1024, 512, 119, 123))
    both_ways(k, L, *inputs(rng, 80, 1024, 8, 2), forward_layout=False)


def test_routed_layer_large_buckets_and_lora(k):
    """Buckets of 150, 70, 30 and 6 rows: the large ones take the grouped transposed work-groups,
    the small ones the one-tile work-groups, both reading the backward layout (each its own way);
    LoRA terms join the W2 epilogue."""
    case("routed layer with/without backward layout, large buckets + LoRA r=8")
    rng = np.random.default_rng(73)
    L = layer_of(oracle.random_experts(rng, 4, 1024, 512, 118, 122))
    lora = adapters(oracle.random_lora(rng, 1024, 512, 8))
    both_ways(k, L, *inputs(rng, 0, 1024, 4, 1, sizes=[150, 70, 30, 6]), lora=lora)


def test_reference_expert_shape_with_lora(k):
    case("8 experts 2048x7168, 40 tokens top-2, LoRA r=16, with/without backward layout")
    rng = np.random.default_rng(74)
    L = layer_of(oracle.random_experts(rng, 8, 7168, 2048, 117, 121))
    lora = adapters(oracle.random_lora(rng, 7168, 2048, 16))
    both_ways(k, L, *inputs(rng, 40, 7168, 8, 2), act="situ", lora=lora)


def test_only_gate_up_laid_out(k):
    """F = 544 is not a multiple of 256: W2 has no backward layout (its transposed product reads
    the checkpoint layout), W1|W3 (K = D = 1024) read theirs."""
    case("routed layer, backward layout for W1|W3 only (F = 544)")
    rng = np.random.default_rng(75)
    L = layer_of(oracle.random_experts(rng, 6, 1024, 544, 119, 123))
    L.prepare_backward_layout()
    assert L._bl[0] is not None and L._bl[1] is not None and L._bl[2] is None
    both_ways(k, L, *inputs(rng, 64, 1024, 6, 2))


def test_only_down_laid_out(k):
    """D = 544 is not a multiple of 256: W1|W3 have no backward layout, W2 (K = F = 1024) has one."""
    case("routed layer, backward layout for W2 only (D = 544)")
    rng = np.random.default_rng(76)
    L = layer_of(oracle.random_experts(rng, 6, 544, 1024, 119, 123))
    L.prepare_backward_layout()
    assert L._bl[0] is None and L._bl[1] is None and L._bl[2] is not None
    both_ways(k, L, *inputs(rng, 64, 544, 6, 2))


def test_upload_drops_a_stale_layout(k):
    from lazylora_amd.loader import upload
    from lazylora_amd.streaming import host_layer_from
    case("loader.upload and in-place writes drop the backward layout")
    rng = np.random.default_rng(77)
    L = layer_of(oracle.random_experts(rng, 4, 512, 512, 119, 123))
    other = layer_of(oracle.random_experts(rng, 4, 512, 512, 119, 123))
    H, I, W, G = inputs(rng, 32, 512, 4, 2)
    L.prepare_backward_layout()
    upload(host_layer_from(other), L)
    torch.cuda.synchronize()
    assert L.layout_pointers() == (None, 0)
    want = k.routed_backward(H, I, W, other, G)
    got = k.routed_backward(H, I, W, L, G)
    assert all(torch.equal(a, b) for a, b in zip(got, want))
    L.prepare_backward_layout()
    L.w2s.copy_(layer_of(oracle.random_experts(rng, 4, 512, 512, 119, 123)).w2s)
    with pytest.warns(RuntimeWarning):
        got = k.routed_backward(H, I, W, L, G)
    L.drop_backward_layout()
    want = k.routed_backward(H, I, W, L, G)
    assert all(torch.equal(a, b) for a, b in zip(got, want))


@pytest.mark.parametrize("zipf", [False, True])
def test_baseline_size(k, zipf):
    """896 experts of 2048 x 7168, 1024 tokens, top-8 (random codes and scales
    2^-10..2^-6 in HBM), the backward with and without the backward layout."""
    case(f"config 4 with/without backward layout, {'zipf' if zipf else 'uniform'} routing")
    from lazylora_amd.experts import ExpertLayer
    E, D, F, N = 896, 7168, 2048, 1024
    gen = torch.Generator(device="cuda")
    gen.manual_seed(78)
    codes = lambda *sh: torch.randint(0, 256, sh, dtype=torch.uint8, device="cuda", generator=gen)
    scales = lambda *sh: torch.randint(117, 122, sh, dtype=torch.uint8, device="cuda", generator=gen)
    L = ExpertLayer(codes(E, F, D // 2), scales(E, F, D // 32), codes(E, F, D // 2), scales(E, F, D // 32),
                    codes(E, D, F // 2), scales(E, D, F // 32))
    rng = np.random.default_rng(79)
    logits = rng.standard_normal((N, E)).astype(np.float32)
    if zipf:
        logits = logits + oracle.zipf_offsets(rng, E)[None, :]
    idx, w = oracle.softmax_topk(logits, 8)
    H, I, W, G = (torch.from_numpy(a).cuda() for a in (rng.standard_normal((N, D)).astype(np.float32), idx, w,
                                                       rng.standard_normal((N, D)).astype(np.float32)))
    both_ways(k, L, H, I, W, G)
    del L
    torch.cuda.empty_cache()
