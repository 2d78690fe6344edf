"""The forward layout (mxfp4_forward_layout, ExpertLayer.prepare_forward_layout): its bytes
against a NumPy construction from the definition in include/lazylora_mxfp4.h, and the routed
layer with it against the same layer without it. The one-tile forward work-groups read the same
code bytes from either layout, in the same order, so every result is bit-identical, at small
shapes (uniform routing, large buckets, LoRA, only W1|W3 laid out) and at the BASELINE config-4
size."""
import numpy as np
import pytest
import torch

import oracle

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
    """Per expert: codes, per row group rg, super-chunk c, operand block q and lane l the 16 bytes
    of MX block 4 (l // 16) + q of super-chunk c of row 16 rg + l % 16; then scales, per rg, c and
    lane l the 4 scale bytes of blocks 4 (l // 16) .. + 3 of that super-chunk of that row. Rows past
    R repeat R - 1."""
    E = packed.shape[0]
    nsc, G = K // 512, (R + 15) // 16
    codes = np.empty((E, G, nsc, 4, 64, 16), np.uint8)
    sc = np.empty((E, G, nsc, 64, 4), np.uint8)
    for l in range(64):
        rows = np.minimum(np.arange(G) * 16 + l % 16, R - 1)
        chunks = packed[:, rows, :].reshape(E, G, nsc, 256)
        schunks = scales[:, rows, :].reshape(E, G, nsc, 16)
        for q in range(4):
            blk = 4 * (l // 16) + q
            codes[:, :, :, q, l, :] = chunks[:, :, :, blk * 16:(blk + 1) * 16]
        sc[:, :, :, l, :] = schunks[:, :, :, 4 * (l // 16):4 * (l // 16) + 4]
    return np.concatenate([codes.reshape(E, -1), sc.reshape(E, -1)], axis=1).reshape(-1)


@pytest.mark.parametrize("E,R,K", [(3, 40, 1024), (2, 64, 512), (1, 16, 7168)])
def test_layout_bytes(k, E, R, K):
    case(f"forward layout bytes E={E} R={R} K={K}")
    rng = np.random.default_rng(E * 1000 + R + K)
    packed = rng.integers(0, 256, (E, R, K // 2), dtype=np.uint8)
    scales = rng.integers(0, 256, (E, R, K // 32), dtype=np.uint8)
    got = k.forward_layout(torch.from_numpy(packed).cuda(), torch.from_numpy(scales).cuda()).cpu().numpy()
    want = layout_numpy(packed, scales, R, K)
    assert got.size == want.size == k.lib.mxfp4_forward_layout_bytes(E, R, K)
    assert np.array_equal(got, want)


def layer_of(ex):
    from lazylora_amd.experts import ExpertLayer
    t = [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (ex.w1p, ex.w1s, ex.w3p, ex.w3s, ex.w2p, ex.w2s)]
    return ExpertLayer(*t)


def adapters(lo):
    """(gate, up, down) objects shaped like the reference's LazyLoRALinear."""
    from types import SimpleNamespace as NS
    return tuple(NS(lora_A=torch.from_numpy(np.asarray(A, np.float32)).cuda(),
                    lora_B=torch.from_numpy(np.asarray(B, np.float32)).cuda(), scaling=s, dropout_rate=0.0)
                 for A, B, s in lo.adapters())


def both_ways(k, L, H, I, W, G, act="swiglu", lora=None, large=False):
    """Forward, backward recomputing the forward, and backward reusing it: without and with the
    forward layout. Without large buckets (experts of four or more 16-row tiles) the results are
    bit-identical: every product reads the same bytes in the same order either way. With them
    (large=True) the large-bucket forward takes its MX blocks in the one-tile kernels' grouping
    with the forward layout and four consecutive blocks per MFMA without it, so the fp32 sums
    differ in rounding only (a sum that lands on the other side of an e4m3 rounding boundary of the act
    requantisation moves one term of the down product): the two must agree to rel-L2 1e-4 (well
    below the 5e-3 parity bar,
    which each meets against the oracle in the routed-layer tests)."""
    res = []
    for use in (False, True):
        if use:
            assert L.prepare_forward_layout() > 0
        else:
            L.drop_forward_layout()
        ws = torch.empty(k.moe_workspace_bytes(H.shape[0], I.shape[1], L.E, L.D, L.F), dtype=torch.uint8,
                         device="cuda")
        out = k.routed_forward(H, I, W, L, act=act, save_for_backward=True, workspace=ws, lora=lora)
        reuse = k.routed_backward(H, I, W, L, G, act=act, reuse_forward=True, workspace=ws, lora=lora)
        recompute = k.routed_backward(H, I, W, L, G, act=act, lora=lora)
        flat = [out] + [t for r in (reuse, recompute) for t in (r[:2] + tuple(r[2]) if lora else r)]
        res.append(flat)
    L.drop_forward_layout()
    for i, (a, b) in enumerate(zip(*res)):
        if large:
            r = oracle.rel_l2(b.cpu().numpy(), a.cpu().numpy())
            print(f"result {i}: rel-L2 {r:.2e} between the layouts")
            assert r <= 1e-4, f"result {i} differs with the forward layout: rel-L2 {r:.2e}"
        else:
            assert torch.equal(a, b), f"result {i} differs with the forward layout"


def inputs(rng, N, D, E, topk, sizes=None):
    if sizes is not None:
        first = np.concatenate([np.full(c, e) for e, c in enumerate(sizes)]).astype(np.int64)
        rng.shuffle(first)
        N = first.size
        idx, w = first[:, None], rng.uniform(0.5, 1.5, (N, 1)).astype(np.float32)
    else:
        idx, w = oracle.softmax_topk(rng.standard_normal((N, E)).astype(np.float32), topk)
    h = rng.standard_normal((N, D)).astype(np.float32)
    g = rng.standard_normal((N, D)).astype(np.float32)
    return [torch.from_numpy(a).cuda() for a in (h, idx, w, g)]


@pytest.mark.parametrize("act", ["swiglu", "situ"])
def test_routed_layer_small_buckets(k, act):
    case(f"routed layer with/without forward layout, uniform top-2, {act}")
    rng = np.random.default_rng(61)
    L = layer_of(oracle.random_experts(rng, 8, 1024, 512, 119, 123))
    both_ways(k, L, *inputs(rng, 96, 1024, 8, 2), act=act)


def test_routed_layer_large_buckets_and_lora(k):
    """Buckets of 150, 70, 30 and 6 rows: the large ones take the GEMM-shaped work-groups, the
    small ones the one-tile work-groups, both reading the forward layout (each its own way); LoRA
    deltas join both epilogues."""
    case("routed layer with/without forward layout, large buckets + LoRA r=8")
    rng = np.random.default_rng(62)
    L = layer_of(oracle.random_experts(rng, 4, 1024, 512, 118, 122))
    lora = adapters(oracle.random_lora(rng, 1024, 512, 8))
    both_ways(k, L, *inputs(rng, 0, 1024, 4, 1, sizes=[150, 70, 30, 6]), lora=lora, large=True)


def test_reference_expert_shape_with_lora(k):
    """Experts of the BASELINE shape (W1/W3 2048 x 7168, W2 7168 x 2048: 14 and 4 super-chunks
    per row) with rank-16 adapters, with and without the forward layout."""
    case("8 experts 2048x7168, 40 tokens top-2, LoRA r=16, with/without forward layout")
    rng = np.random.default_rng(68)
    L = layer_of(oracle.random_experts(rng, 8, 7168, 2048, 117, 121))
    lora = adapters(oracle.random_lora(rng, 7168, 2048, 16))
    both_ways(k, L, *inputs(rng, 40, 7168, 8, 2), act="situ", lora=lora)


def test_only_gate_up_laid_out(k):
    """F = 544 is not a multiple of 512: W2 has no forward layout and the down product reads the
    checkpoint layout, W1|W3 (K = D = 1024) read theirs."""
    case("routed layer, forward layout for W1|W3 only (F = 544)")
    rng = np.random.default_rng(63)
    L = layer_of(oracle.random_experts(rng, 6, 1024, 544, 119, 123))
    L.prepare_forward_layout()
    assert L._fl[0] is not None and L._fl[1] is not None and L._fl[2] is None
    both_ways(k, L, *inputs(rng, 64, 1024, 6, 2))


def test_only_down_laid_out(k):
    """D = 544 is not a multiple of 512: W1|W3 have no forward layout, W2 (K = F = 1024) has one."""
    case("routed layer, forward layout for W2 only (D = 544)")
    rng = np.random.default_rng(67)
    L = layer_of(oracle.random_experts(rng, 6, 544, 1024, 119, 123))
    L.prepare_forward_layout()
    assert L._fl[0] is None and L._fl[1] is None and L._fl[2] is not None
    both_ways(k, L, *inputs(rng, 64, 544, 6, 2))


def test_upload_drops_a_stale_layout(k):
    from lazylora_amd.loader import upload
    from lazylora_amd.streaming import host_layer_from
    case("loader.upload drops the forward layout it would make stale")
    rng = np.random.default_rng(64)
    L = layer_of(oracle.random_experts(rng, 4, 512, 512, 119, 123))
    other = layer_of(oracle.random_experts(rng, 4, 512, 512, 119, 123))
    H, I, W, _ = inputs(rng, 32, 512, 4, 2)
    L.prepare_forward_layout()
    upload(host_layer_from(other), L)
    torch.cuda.synchronize()
    assert L.forward_layout_pointers() is None
    assert torch.equal(k.routed_forward(H, I, W, L), k.routed_forward(H, I, W, other))
    # an in-place write by any other route: the stale copy is dropped before the call reads it
    L.prepare_forward_layout()
    L.w1p.copy_(layer_of(oracle.random_experts(rng, 4, 512, 512, 119, 123)).w1p)
    with pytest.warns(RuntimeWarning):
        out = k.routed_forward(H, I, W, L)
    L.drop_forward_layout()
    assert torch.equal(out, k.routed_forward(H, I, W, L))


@pytest.mark.parametrize("zipf", [False, True])
def test_baseline_size(k, zipf):
    """896 experts of 2048 x 7168, 1024 tokens, top-8 (random codes and scales
    2^-10..2^-6 in HBM), forward and backward with and without the forward layout."""
    case(f"config 4 with/without forward layout, {'zipf' if zipf else 'uniform'} routing")
    from lazylora_amd.experts import ExpertLayer
    E, D, F, N = 896, 7168, 2048, 1024
    gen = torch.Generator(device="cuda")
    gen.manual_seed(65)
    codes = lambda *sh: torch.randint(0, 256, sh, dtype=torch.uint8, device="cuda", generator=gen)
    scales = lambda *sh: torch.randint(117, 122, sh, dtype=torch.uint8, device="cuda", generator=gen)
    L = ExpertLayer(codes(E, F, D // 2), scales(E, F, D // 32), codes(E, F, D // 2), scales(E, F, D // 32),
                    codes(E, D, F // 2), scales(E, D, F // 32))
    rng = np.random.default_rng(66)
    logits = rng.standard_normal((N, E)).astype(np.float32)
    if zipf:
        logits = logits + oracle.zipf_offsets(rng, E)[None, :]
    idx, w = oracle.softmax_topk(logits, 8)
    H, I, W, G = (torch.from_numpy(a).cuda() for a in (rng.standard_normal((N, D)).astype(np.float32), idx, w,
                                                       rng.standard_normal((N, D)).astype(np.float32)))
    both_ways(k, L, H, I, W, G, large=zipf)
    del L
    torch.cuda.empty_cache()
