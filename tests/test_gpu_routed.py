"""Routed-expert layer forward and backward on the GPU against the oracle.

Small configurations are compared in full with the float64 oracle; the BASELINE config-3/4
layer (896 experts of 2048x7168, 1024 tokens, top-8) is compared on sampled tokens against the
C restatement of the reference path, plus size-independent properties (token permutation,
expert relabelling, determinism, linearity in the combine weights)."""
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


def case(msg):
    print(f"\n[case] {msg}", flush=True)


def layer_of(ex: oracle.ExpertSet):
    from lazylora_amd.experts import ExpertLayer
    t = [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (ex.w1p, ex.w1s, ex.w3p, ex.w3s, ex.w2p, ex.w2s)]
    return ExpertLayer(*t)


def routing(rng, N, E, topk, zipf=False):
    logits = rng.standard_normal((N, E)).astype(np.float32)
    if zipf:
        logits = logits + oracle.zipf_offsets(rng, E)[None, :]
    return oracle.softmax_topk(logits, topk)


@pytest.mark.parametrize("act", ["swiglu", "situ"])
def test_config1_forward_backward(k, act):
    """D 256, 8 experts, top-2, FFN 128, 64 tokens, scales 2^-8..2^-4."""
    case(f"config 1 fwd+bwd {act}")
    rng = np.random.default_rng(11)
    ex = oracle.random_experts(rng, 8, 256, 128, 119, 123)
    h = rng.standard_normal((64, 256)).astype(np.float32)
    idx, w = routing(rng, 64, 8, 2)
    g = rng.standard_normal((64, 256)).astype(np.float32)
    L = layer_of(ex)
    H, I, W, G = (torch.from_numpy(a).cuda() for a in (h, idx, w, g))
    out = k.routed_forward(H, I, W, L, act=act).cpu().numpy()
    assert_close(out, oracle.routed_forward(h, idx, w, ex, act), f"config1 fwd {act}")
    gh, gw = k.routed_backward(H, I, W, L, G, act=act)
    gh64, gw64 = oracle.routed_backward(h, idx, w, ex, g, act)
    assert_close(gh.cpu().numpy(), gh64, f"config1 grad_h {act}")
    assert_close(gw.cpu().numpy(), gw64, f"config1 grad_w {act}")


def test_backward_reuse_equals_recompute(k):
    case("backward with reused forward state == backward with recompute")
    rng = np.random.default_rng(12)
    ex = oracle.random_experts(rng, 16, 512, 256, 117, 121)
    h = rng.standard_normal((96, 512)).astype(np.float32)
    idx, w = routing(rng, 96, 16, 4)
    g = rng.standard_normal((96, 512)).astype(np.float32)
    L = layer_of(ex)
    H, I, W, G = (torch.from_numpy(a).cuda() for a in (h, idx, w, g))
    ws = torch.empty(k.moe_workspace_bytes(96, 4, 16, 512, 256), dtype=torch.uint8, device="cuda")
    out = k.routed_forward(H, I, W, L, save_for_backward=True, workspace=ws)
    a = k.routed_backward(H, I, W, L, G, reuse_forward=True, workspace=ws)
    b = k.routed_backward(H, I, W, L, G, reuse_forward=False)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    assert torch.equal(out, k.routed_forward(H, I, W, L))


def test_medium_layer_full_compare(k, clib):
    """64 experts of the BASELINE expert shape (2048 x 7168), 128 tokens, top-8: every output
    compared against the C restatement of the reference path."""
    case("medium layer: E=64, D=7168, F=2048, N=128, top-8")
    rng = np.random.default_rng(13)
    ex = oracle.random_experts(rng, 64, 7168, 2048, 117, 121)
    h = rng.standard_normal((128, 7168)).astype(np.float32)
    idx, w = routing(rng, 128, 64, 8)
    g = rng.standard_normal((128, 7168)).astype(np.float32)
    L = layer_of(ex)
    H, I, W, G = (torch.from_numpy(a).cuda() for a in (h, idx, w, g))
    out = k.routed_forward(H, I, W, L, save_for_backward=False).cpu().numpy()
    assert_close(out, clib.moe_forward(h, idx, w, ex), "medium fwd")
    gh, gw = k.routed_backward(H, I, W, L, G)
    gh_c, gw_c = clib.moe_backward(h, idx, w, ex, g)
    assert_close(gh.cpu().numpy(), gh_c, "medium grad_h")
    assert_close(gw.cpu().numpy(), gw_c, "medium grad_w")


def test_skewed_routing_large_buckets(k):
    """Zipf-skewed routing puts hundreds of tokens on a few experts (many 16-row tiles)."""
    case("skewed routing: E=32, D=512, F=256, N=512, top-4")
    rng = np.random.default_rng(14)
    ex = oracle.random_experts(rng, 32, 512, 256, 117, 121)
    h = rng.standard_normal((512, 512)).astype(np.float32)
    logits = rng.standard_normal((512, 32)).astype(np.float32) + 3 * oracle.zipf_offsets(rng, 32)[None, :]
    idx, w = oracle.softmax_topk(logits, 4)
    counts = np.bincount(idx.ravel(), minlength=32)
    assert counts.max() > 100  # several 16-row tiles for one expert
    g = rng.standard_normal((512, 512)).astype(np.float32)
    L = layer_of(ex)
    H, I, W, G = (torch.from_numpy(a).cuda() for a in (h, idx, w, g))
    assert_close(k.routed_forward(H, I, W, L).cpu().numpy(), oracle.routed_forward(h, idx, w, ex), "skew fwd")
    gh, gw = k.routed_backward(H, I, W, L, G)
    gh64, gw64 = oracle.routed_backward(h, idx, w, ex, g)
    assert_close(gh.cpu().numpy(), gh64, "skew grad_h")
    assert_close(gw.cpu().numpy(), gw64, "skew grad_w")


@pytest.mark.parametrize("topk", [1, 2])
def test_large_bucket_groups(k, topk):
    """Buckets of 200, 65, 64, 49, 48, 17 and 1 rows: the experts with four or more 16-row tiles
    take the grouped work-groups (groups of 4 tiles, ragged last group and last tile), the rest the
    one-tile work-groups; K = 1024 and 512 keep both products on the path that splits them."""
    case(f"large-bucket groups: E=8, D=1024, F=512, top-{topk}")
    rng = np.random.default_rng(18 + topk)
    E, D, F = 8, 1024, 512
    ex = oracle.random_experts(rng, E, D, F, 118, 122)
    sizes = [200, 65, 64, 49, 48, 17, 1, 0]
    first = np.concatenate([np.full(c, e) for e, c in enumerate(sizes)]).astype(np.int64)
    rng.shuffle(first)
    N = first.size
    if topk == 1:
        idx = first[:, None]
        w = rng.uniform(0.5, 1.5, (N, 1)).astype(np.float32)
    else:
        second = (first + 1 + rng.integers(0, E - 1, N)) % E
        idx = np.stack([first, second], 1).astype(np.int64)
        w = rng.dirichlet([1, 1], N).astype(np.float32)
    h = rng.standard_normal((N, D)).astype(np.float32)
    g = rng.standard_normal((N, D)).astype(np.float32)
    L = layer_of(ex)
    H, I, W, G = (torch.from_numpy(a).cuda() for a in (h, idx, w, g))
    for act in ("swiglu", "situ"):
        assert_close(k.routed_forward(H, I, W, L, act=act).cpu().numpy(), oracle.routed_forward(h, idx, w, ex, act),
                     f"groups fwd {act}")
    gh, gw = k.routed_backward(H, I, W, L, G)
    gh64, gw64 = oracle.routed_backward(h, idx, w, ex, g)
    assert_close(gh.cpu().numpy(), gh64, "groups grad_h")
    assert_close(gw.cpu().numpy(), gw64, "groups grad_w")


def test_input_dtypes(k):
    """bf16 h gives the fp32 result of the same (bf16-representable) values; int32 ids = int64."""
    case("bf16 h, int32 topk ids")
    rng = np.random.default_rng(15)
    ex = oracle.random_experts(rng, 8, 256, 128, 119, 123)
    L = layer_of(ex)
    H = torch.from_numpy(rng.standard_normal((64, 256)).astype(np.float32)).cuda().bfloat16()
    idx, w = routing(rng, 64, 8, 2)
    I, W = torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda()
    a = k.routed_forward(H, I, W, L)
    b = k.routed_forward(H.float(), I.int(), W, L)
    assert torch.equal(a, b)


def test_invalid_ids(k):
    case("expert ids outside [0, E)")
    rng = np.random.default_rng(16)
    ex = oracle.random_experts(rng, 8, 256, 128, 119, 123)
    L = layer_of(ex)
    h = torch.from_numpy(rng.standard_normal((4, 256)).astype(np.float32)).cuda()
    idx = torch.tensor([[0, 9], [1, 2], [3, -1], [4, 5]], dtype=torch.int64)
    w = torch.full((4, 2), 0.5)
    with pytest.raises(ValueError):
        k.routed_forward(h, idx, w, L)  # host ids are checked before launch
    ws = torch.empty(k.moe_workspace_bytes(4, 2, 8, 256, 128), dtype=torch.uint8, device="cuda")
    out = k.routed_forward(h, idx.cuda(), w.cuda(), L, workspace=ws)  # device ids: skipped, flagged
    assert k.route_status(ws) & 1
    keep = torch.tensor([[0, 0], [1, 2], [3, 3], [4, 5]])
    wk = w.clone()
    wk[0, 1] = 0
    wk[2, 1] = 0
    ref = k.routed_forward(h, keep.cuda(), wk.cuda(), L)
    assert torch.allclose(out, ref, rtol=1e-6, atol=1e-6)


def test_autograd_node(k):
    case("RoutedExpertsFunction through torch.autograd")
    from lazylora_amd.routed import RoutedExpertsFunction
    rng = np.random.default_rng(17)
    ex = oracle.random_experts(rng, 8, 256, 128, 119, 123)
    L = layer_of(ex)
    h = torch.from_numpy(rng.standard_normal((32, 256)).astype(np.float32)).cuda().requires_grad_()
    idx, w = routing(rng, 32, 8, 2)
    I = torch.from_numpy(idx).cuda()
    W = torch.from_numpy(w).cuda().requires_grad_()
    out = RoutedExpertsFunction.apply(h, W, I, L, "situ")
    g = torch.randn_like(out)
    out.backward(g)
    gh, gw = k.routed_backward(h.detach(), I, W.detach(), L, g, act="situ")
    assert torch.equal(h.grad, gh) and torch.equal(W.grad, gw)


@pytest.fixture(scope="module")
def full_layer():
    """BASELINE config 3/4: 896 experts of (2048 x 7168) x 3, MXFP4, 20.96 GB in HBM."""
    E, D, F = 896, 7168, 2048
    gen = torch.Generator(device="cuda")
    gen.manual_seed(20)
    from lazylora_amd.experts import ExpertLayer
    def codes(*shape):
        return torch.randint(0, 256, shape, dtype=torch.uint8, device="cuda", generator=gen)
    def scales(*shape):
        return torch.randint(117, 122, shape, dtype=torch.uint8, device="cuda", generator=gen)
    L = ExpertLayer(codes(E, F, D // 2), scales(E, F, D // 32), codes(E, F, D // 2), scales(E, F, D // 32),
                    codes(E, D, F // 2), scales(E, D, F // 32))
    yield L
    del L
    torch.cuda.empty_cache()


def subset_experts(L, ids):
    t = [x[ids].cpu().numpy() for x in L.tensors()]
    return oracle.ExpertSet(*t)


@pytest.mark.parametrize("zipf", [False, True])
def test_baseline_layer_sampled_tokens(k, clib, full_layer, zipf):
    case(f"config 3/4 layer, zipf={zipf}: fwd+bwd, 6 sampled tokens vs C oracle")
    rng = np.random.default_rng(21 + zipf)
    N, E, topk = 1024, 896, 8
    h = rng.standard_normal((N, 7168)).astype(np.float32)
    idx, w = routing(rng, N, E, topk, zipf=zipf)
    g = rng.standard_normal((N, 7168)).astype(np.float32)
    H, I, W, G = (torch.from_numpy(a).cuda() for a in (h, idx, w, g))
    ws = torch.empty(k.moe_workspace_bytes(N, topk, E, 7168, 2048), dtype=torch.uint8, device="cuda")
    out = k.routed_forward(H, I, W, full_layer, save_for_backward=True, workspace=ws).cpu().numpy()
    gh, gw = k.routed_backward(H, I, W, full_layer, G, reuse_forward=True, workspace=ws)
    gh, gw = gh.cpu().numpy(), gw.cpu().numpy()
    toks = rng.choice(N, size=6, replace=False)
    used = np.unique(idx[toks])
    sub = subset_experts(full_layer, torch.from_numpy(used).cuda())
    remap = {int(e): i for i, e in enumerate(used)}
    sidx = np.vectorize(remap.get)(idx[toks])
    assert_close(out[toks], clib.moe_forward(h[toks], sidx, w[toks], sub), f"layer fwd zipf={zipf}")
    gh_c, gw_c = clib.moe_backward(h[toks], sidx, w[toks], sub, g[toks])
    assert_close(gh[toks], gh_c, f"layer grad_h zipf={zipf}")
    assert_close(gw[toks], gw_c, f"layer grad_w zipf={zipf}")


def test_baseline_layer_properties(k, full_layer):
    """Size-independent checks at the full shape: permuting tokens permutes every output
    bit-exactly; scaling all combine weights by 2 doubles the output; reruns are identical."""
    case("config 3 layer: permutation / linearity / determinism")
    rng = np.random.default_rng(23)
    N, E, topk = 1024, 896, 8
    H = torch.from_numpy(rng.standard_normal((N, 7168)).astype(np.float32)).cuda()
    idx, w = routing(rng, N, E, topk)
    I, W = torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda()
    out = k.routed_forward(H, I, W, full_layer)
    assert torch.equal(out, k.routed_forward(H, I, W, full_layer))
    perm = torch.from_numpy(rng.permutation(N)).cuda()
    assert torch.equal(k.routed_forward(H[perm], I[perm], W[perm], full_layer), out[perm])
    assert torch.equal(k.routed_forward(H, I, 2 * W, full_layer), 2 * out)
    G = torch.from_numpy(rng.standard_normal((N, 7168)).astype(np.float32)).cuda()
    gh, gw = k.routed_backward(H, I, W, full_layer, G)
    gh2, gw2 = k.routed_backward(H[perm], I[perm], W[perm], full_layer, G[perm])
    assert torch.equal(gh2, gh[perm]) and torch.equal(gw2, gw[perm])
