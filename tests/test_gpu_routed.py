"""Routed-expert layer forward and backward on the GPU against the oracle.

Small configurations are compared in full with the float64 oracle; the BASELINE config-3/4
layer (896 experts of 2048x7168, 1024 tokens, top-8) is compared on every token against the
C restatement of the reference path (uniform and Zipf routing, fp32 and bf16 activations), plus
size-independent properties (token permutation, determinism, linearity in the combine weights).
Activations with outlier channels (a few channels 10^1..10^4 times the rest, as in a residual
stream) are checked through the single-expert product and a routed layer."""
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


@pytest.mark.parametrize("topk,fl", [(1, False), (2, False), (1, True), (2, True)])
def test_large_bucket_groups(k, topk, fl):
    """Buckets of 200, 129, 65, 64, 49, 48, 17 and 1 rows: the experts with four or more 16-row
    tiles take the grouped work-groups (groups of 4 tiles, ragged last groups down to one tile,
    ragged last tile; with a forward layout (fl) wide groups of 8 tiles: 13 = 8 + 5, 9 = 8 + 1,
    5, 4), the rest the one-tile work-groups; K = 1024 and 512 keep both products on the path
    that splits them."""
    case(f"large-bucket groups: E=9, D=1024, F=512, top-{topk}, forward layout={fl}")
    rng = np.random.default_rng(18 + topk)
    E, D, F = 9, 1024, 512
    ex = oracle.random_experts(rng, E, D, F, 118, 122)
    sizes = [200, 129, 65, 64, 49, 48, 17, 1, 0]
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
    if fl:
        L.prepare_forward_layout()
    H, I, W, G = (torch.from_numpy(a).cuda() for a in (h, idx, w, g))
    for act in ("swiglu", "situ"):
        assert_close(k.routed_forward(H, I, W, L, act=act).cpu().numpy(), oracle.routed_forward(h, idx, w, ex, act),
                     f"groups fwd {act}")
    gh, gw = k.routed_backward(H, I, W, L, G)
    gh64, gw64 = oracle.routed_backward(h, idx, w, ex, g)
    assert_close(gh.cpu().numpy(), gh64, "groups grad_h")
    assert_close(gw.cpu().numpy(), gw64, "groups grad_w")


@pytest.mark.parametrize("h_bf16", [False, True])
def test_large_bucket_tiles_copied_from_token_rows(k, h_bf16):
    """With some small buckets the token-major rows of x are written, and the large buckets'
    activation tiles are copied from them; with only large buckets the tiles are quantised from x.
    Both must hold the same bytes: the tokens of two large experts, routed top-1 together with
    small buckets and then alone, get bit-identical outputs (each depends only on its own row)."""
    case(f"large-bucket tiles from token rows vs from x, bf16 h={h_bf16}")
    rng = np.random.default_rng(71)
    ex = oracle.random_experts(rng, 4, 1024, 512, 118, 122)
    L = layer_of(ex)
    first = np.concatenate([np.full(c, e) for e, c in enumerate([150, 70, 30, 6])]).astype(np.int64)
    rng.shuffle(first)
    N = first.size
    h = torch.from_numpy(rng.standard_normal((N, 1024)).astype(np.float32)).cuda()
    if h_bf16:
        h = h.bfloat16()
    w = torch.from_numpy(rng.uniform(0.5, 1.5, (N, 1)).astype(np.float32)).cuda()
    idx = torch.from_numpy(first[:, None]).cuda()
    out_mixed = k.routed_forward(h, idx, w, L)
    large = torch.from_numpy(np.nonzero(first < 2)[0]).cuda()
    out_large = k.routed_forward(h[large].contiguous(), idx[large].contiguous(), w[large].contiguous(), L)
    assert torch.equal(out_mixed[large], out_large)


@pytest.mark.parametrize("D,F", [(640, 384), (1024, 352)])
def test_large_bucket_ragged_columns(k, D, F):
    """Large buckets with output widths that leave the grouped transposed products partial
    column blocks (640 and 384: a 512-column item whose last stripes lie past the end) or send
    them to the one-tile work-groups (352, not a multiple of 128)."""
    case(f"large buckets, ragged widths: E=4, D={D}, F={F}, top-1")
    rng = np.random.default_rng(D + F)
    E = 4
    ex = oracle.random_experts(rng, E, D, F, 118, 122)
    sizes = [150, 70, 20, 3]
    idx = np.concatenate([np.full(c, e) for e, c in enumerate(sizes)]).astype(np.int64)
    rng.shuffle(idx)
    N = idx.size
    idx = idx[:, None]
    w = rng.uniform(0.5, 1.5, (N, 1)).astype(np.float32)
    h = rng.standard_normal((N, D)).astype(np.float32)
    g = rng.standard_normal((N, D)).astype(np.float32)
    L = layer_of(ex)
    H, I, W, G = (torch.from_numpy(a).cuda() for a in (h, idx, w, g))
    assert_close(k.routed_forward(H, I, W, L).cpu().numpy(), oracle.routed_forward(h, idx, w, ex), "ragged fwd")
    gh, gw = k.routed_backward(H, I, W, L, G)
    gh64, gw64 = oracle.routed_backward(h, idx, w, ex, g)
    assert_close(gh.cpu().numpy(), gh64, "ragged grad_h")
    assert_close(gw.cpu().numpy(), gw64, "ragged grad_w")


@pytest.mark.parametrize("D,F", [(640, 512), (1024, 352)])
def test_only_large_buckets_unsplit_product(k, D, F):
    """Every bucket large (at least 49 rows) while a product cannot split its buckets (its K is
    not a multiple of 512: D = 640 for gate/up, F = 352 for down): every tile then takes the
    one-tile work-groups, so x's token-major rows must still be written. Run twice on one reused
    workspace, the second time on other tokens, so stale rows of the first call would show."""
    case(f"only large buckets, unsplit product: E=4, D={D}, F={F}, top-1, reused workspace")
    rng = np.random.default_rng(D * 7 + F)
    E = 4
    ex = oracle.random_experts(rng, E, D, F, 118, 122)
    L = layer_of(ex)
    ws = None
    for call, sizes in enumerate(([150, 70, 64, 49], [64, 49, 130, 52])):
        idx = np.concatenate([np.full(c, e) for e, c in enumerate(sizes)]).astype(np.int64)
        rng.shuffle(idx)
        N = idx.size
        idx = idx[:, None]
        w = rng.uniform(0.5, 1.5, (N, 1)).astype(np.float32)
        h = rng.standard_normal((N, D)).astype(np.float32)
        g = rng.standard_normal((N, D)).astype(np.float32)
        if ws is None:
            ws = torch.empty(k.moe_workspace_bytes(340, 1, E, D, F), dtype=torch.uint8, device="cuda")
        H, I, W, G = (torch.from_numpy(a).cuda() for a in (h, idx, w, g))
        assert_close(k.routed_forward(H, I, W, L, workspace=ws).cpu().numpy(), oracle.routed_forward(h, idx, w, ex),
                     f"large-only fwd call {call}")
        gh, gw = k.routed_backward(H, I, W, L, G, workspace=ws)
        gh64, gw64 = oracle.routed_backward(h, idx, w, ex, g)
        assert_close(gh.cpu().numpy(), gh64, f"large-only grad_h call {call}")
        assert_close(gw.cpu().numpy(), gw64, f"large-only grad_w call {call}")


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


def test_top1_rows_written_directly(k):
    """Top-1 routing without LoRA: the down product writes each token's row into out itself (no
    combine), and tokens whose id is outside [0, E) get zero rows (out starts as garbage)."""
    case("top-1 routing: rows written by the down product, unrouted tokens zeroed")
    rng = np.random.default_rng(18)
    ex = oracle.random_experts(rng, 8, 512, 256, 119, 123)
    L = layer_of(ex)
    N = 70
    hn = rng.standard_normal((N, 512)).astype(np.float32)
    h = torch.from_numpy(hn).cuda()
    idx = rng.integers(0, 8, (N, 1)).astype(np.int64)
    idx[:20, 0] = 5  # one bucket of more than 16 rows
    idx[3, 0], idx[41, 0] = -1, 8
    w = rng.uniform(0.5, 1.5, (N, 1)).astype(np.float32)
    ws = torch.empty(k.moe_workspace_bytes(N, 1, 8, 512, 256), dtype=torch.uint8, device="cuda")
    ws.fill_(0x7F)
    out = k.routed_forward(h, torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda(), L, workspace=ws)
    assert k.route_status(ws) & 1
    assert torch.count_nonzero(out[3]) == 0 and torch.count_nonzero(out[41]) == 0
    keep = idx.copy()
    keep[3, 0] = keep[41, 0] = 0
    wk = w.copy()
    wk[3, 0] = wk[41, 0] = 0
    want = oracle.routed_forward(hn, keep, wk, ex, "swiglu")
    got = out.cpu().numpy()
    ok = np.ones(N, bool)
    ok[[3, 41]] = False
    assert_close(got[ok], want[ok], "top-1 direct rows")
    # against the same layer through top-2 with a zero-weight second slot (combined by the combine)
    idx2 = np.concatenate([keep, keep], axis=1)
    w2 = np.concatenate([wk, np.zeros_like(wk)], axis=1)
    two = k.routed_forward(h, torch.from_numpy(idx2).cuda(), torch.from_numpy(w2).cuda(), L).cpu().numpy()
    assert np.array_equal(got[ok], two[ok])


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


def test_autograd_node_cached_and_second_backward(k):
    """The reference node's `cached` replay (lazy_trainer.py:60-66): the forward returns the
    cached sum untouched and the backward recomputes; a second backward through a retained graph
    recomputes too and gives the same gradients."""
    case("RoutedExpertsFunction: cached replay, retain_graph second backward")
    from lazylora_amd.routed import RoutedExpertsFunction
    rng = np.random.default_rng(25)
    ex = oracle.random_experts(rng, 8, 256, 128, 119, 123)
    L = layer_of(ex)
    h0 = torch.from_numpy(rng.standard_normal((40, 256)).astype(np.float32)).cuda()
    idx, w = routing(rng, 40, 8, 2)
    I = torch.from_numpy(idx).cuda()
    W0 = torch.from_numpy(w).cuda()
    g = torch.from_numpy(rng.standard_normal((40, 256)).astype(np.float32)).cuda()
    want_gh, want_gw = oracle.routed_backward(h0.cpu().numpy(), idx, w, ex, g.cpu().numpy(), "situ")
    # cached replay: a sentinel cache must come back as is
    cached = torch.full((40, 256), 7.0, device="cuda")
    h = h0.clone().requires_grad_()
    W = W0.clone().requires_grad_()
    out = RoutedExpertsFunction.apply(h, W, I, L, "situ", cached)
    assert torch.equal(out, cached)
    out.backward(g)
    assert_close(h.grad.cpu().numpy(), want_gh, "cached grad_h")
    assert_close(W.grad.cpu().numpy(), want_gw, "cached grad_w")
    # retain_graph: the second backward recomputes (the forward's workspace is released after the first)
    h = h0.clone().requires_grad_()
    W = W0.clone().requires_grad_()
    out = RoutedExpertsFunction.apply(h, W, I, L, "situ")
    assert_close(out.detach().cpu().numpy(), oracle.routed_forward(h0.cpu().numpy(), idx, w, ex, "situ"), "node fwd")
    out.backward(g, retain_graph=True)
    gh1, gw1 = h.grad.clone(), W.grad.clone()
    h.grad = None
    W.grad = None
    out.backward(g)
    assert torch.equal(h.grad, gh1) and torch.equal(W.grad, gw1)
    with pytest.raises(ValueError):
        k.routed_backward(h0, I, W0, L, g, reuse_forward=True, workspace=None)


class _Streamer:
    """Stands in for DynamicExpertStreamer: yields (expert_id, ExpertWeightBundle-shaped object)
    for the active experts in a fixed scrambled ('disk') order (expert_streamer.py:315-369)."""

    def __init__(self, ex, order):
        from types import SimpleNamespace
        self.order, self.calls = order, 0
        self.bundles = {e: SimpleNamespace(expert_idx=e, packed=True,
                                           gate_packed=torch.from_numpy(ex.w1p[e]), gate_scale=torch.from_numpy(ex.w1s[e]),
                                           up_packed=torch.from_numpy(ex.w3p[e]), up_scale=torch.from_numpy(ex.w3s[e]),
                                           down_packed=torch.from_numpy(ex.w2p[e]), down_scale=torch.from_numpy(ex.w2s[e]))
                        for e in range(ex.w1p.shape[0])}

    def stream_experts(self, layer_idx, active):
        self.calls += 1
        for e in sorted(active, key=self.order.index):
            yield e, self.bundles[e]


def test_streamed_node_with_reference_signature(k):
    """StreamedRoutedExpertsFunction.apply(h_latent, topk_weights, topk_indices, trainer, layer_idx,
    bundle, active_experts, cached) streams packed bundles (CPU tensors, as the reference's
    streamer hands them over) once in forward and once in backward, against the oracle with
    SiTU-GLU and the layer's LoRA adapters; CPU h_latent as the reference trainer passes it."""
    case("StreamedRoutedExpertsFunction: bundles from a streamer, LoRA, CPU inputs")
    from types import SimpleNamespace
    from lazylora_amd.routed import StreamedRoutedExpertsFunction
    rng = np.random.default_rng(26)
    E, D, F, N, topk, r = 12, 256, 128, 48, 3, 4
    ex = oracle.random_experts(rng, E, D, F, 119, 123)
    idx, w = routing(rng, N, E, topk)
    active = sorted(set(idx.ravel().tolist()))
    streamer = _Streamer(ex, list(rng.permutation(E)))
    trainer = SimpleNamespace(expert_streamer=streamer,
                              config=SimpleNamespace(model=SimpleNamespace(num_experts=E)))

    def adapter(n_in, n_out):
        A = torch.from_numpy((0.05 * rng.standard_normal((r, n_in))).astype(np.float32))
        B = torch.from_numpy((0.05 * rng.standard_normal((n_out, r))).astype(np.float32))
        mod = SimpleNamespace(lora_A=A, lora_B=B, scaling=2.0, r=r, dropout_rate=0.0, grads=[])
        mod.accumulate_grad = lambda gA, gB, m=mod: m.grads.append((gA.cpu(), gB.cpu()))
        return mod

    bundle = SimpleNamespace(gate_lora=adapter(D, F), up_lora=adapter(D, F), down_lora=adapter(F, D))
    f64 = [t.numpy().astype(np.float64) for m in (bundle.gate_lora, bundle.up_lora, bundle.down_lora)
           for t in (m.lora_A, m.lora_B)]
    lo = oracle.LoRA(*f64, gate_s=2.0, up_s=2.0, down_s=2.0)
    h_np = rng.standard_normal((N, D)).astype(np.float32)
    g_np = rng.standard_normal((N, D)).astype(np.float32)
    h = torch.from_numpy(h_np).requires_grad_()
    W = torch.from_numpy(w).requires_grad_()
    out = StreamedRoutedExpertsFunction.apply(h, W, torch.from_numpy(idx), trainer, 3, bundle, active, None)
    assert out.device.type == "cpu" and streamer.calls == 1
    assert_close(out.detach().numpy(), oracle.routed_forward(h_np, idx, w, ex, "situ", lora=lo), "streamed node fwd")
    out.backward(torch.from_numpy(g_np))
    assert streamer.calls == 2
    want = oracle.routed_backward(h_np, idx, w, ex, g_np, "situ", lora=lo)
    assert_close(h.grad.numpy(), want[0], "streamed node grad_h")
    assert_close(W.grad.numpy(), want[1], "streamed node grad_w")
    got = [t for m in (bundle.gate_lora, bundle.up_lora, bundle.down_lora) for t in m.grads[0]]
    for n, (a, b) in enumerate(zip(got, want[2])):
        assert_close(a.numpy(), b, f"streamed node LoRA grad {n}")


@pytest.mark.parametrize("pinned", [False, True])
def test_streamed_node_ids_outside_active_set(k, pinned):
    """Routed ids that the active set leaves out get nothing, as in the reference's sweep over the
    streamed experts (lazy_trainer.py:806-880): no expert term and no adapter term in the output
    (equal to the oracle with those slots' weights zeroed), zero grad_w on those slots, and the
    adapter gradients of the streamed experts only. Bundles in pageable or pinned host memory;
    more bundles than staging buffers, so the buffers are reused within a pass."""
    case(f"streamed node, ids outside the active set, pinned bundles={pinned}")
    from types import SimpleNamespace
    from lazylora_amd.routed import StreamedRoutedExpertsFunction
    rng = np.random.default_rng(28)
    E, D, F, N, topk, r = 16, 512, 256, 64, 2, 4
    ex = oracle.random_experts(rng, E, D, F, 119, 123)
    idx, w = routing(rng, N, E, topk)
    routed = sorted(set(idx.ravel().tolist()))
    dropped = routed[::3]
    active = [e for e in routed if e not in dropped]
    streamer = _Streamer(ex, list(rng.permutation(E)))
    if pinned:
        for b in streamer.bundles.values():
            for a in ("gate_packed", "gate_scale", "up_packed", "up_scale", "down_packed", "down_scale"):
                setattr(b, a, getattr(b, a).pin_memory())
    trainer = SimpleNamespace(expert_streamer=streamer)

    def adapter(n_in, n_out):
        A = torch.from_numpy((0.05 * rng.standard_normal((r, n_in))).astype(np.float32))
        B = torch.from_numpy((0.05 * rng.standard_normal((n_out, r))).astype(np.float32))
        mod = SimpleNamespace(lora_A=A, lora_B=B, scaling=2.0, r=r, dropout_rate=0.0, grads=[])
        mod.accumulate_grad = lambda gA, gB, m=mod: m.grads.append((gA.cpu(), gB.cpu()))
        return mod

    bundle = SimpleNamespace(gate_lora=adapter(D, F), up_lora=adapter(D, F), down_lora=adapter(F, D))
    f64 = [t.numpy().astype(np.float64) for m in (bundle.gate_lora, bundle.up_lora, bundle.down_lora)
           for t in (m.lora_A, m.lora_B)]
    lo = oracle.LoRA(*f64, gate_s=2.0, up_s=2.0, down_s=2.0)
    h_np = rng.standard_normal((N, D)).astype(np.float32)
    g_np = rng.standard_normal((N, D)).astype(np.float32)
    keep = np.isin(idx, active)
    assert (~keep).any() and keep.any()
    w_kept = np.where(keep, w, 0).astype(np.float32)
    h = torch.from_numpy(h_np).cuda().requires_grad_()
    W = torch.from_numpy(w).cuda().requires_grad_()
    out = StreamedRoutedExpertsFunction.apply(h, W, torch.from_numpy(idx).cuda(), trainer, 0, bundle, active, None)
    assert_close(out.detach().cpu().numpy(), oracle.routed_forward(h_np, idx, w_kept, ex, "situ", lora=lo),
                 "streamed node fwd, dropped ids")
    out.backward(torch.from_numpy(g_np).cuda())
    want = oracle.routed_backward(h_np, idx, w_kept, ex, g_np, "situ", lora=lo)
    assert_close(h.grad.cpu().numpy(), want[0], "streamed node grad_h, dropped ids")
    gw = W.grad.cpu().numpy()
    assert np.all(gw[~keep] == 0)
    assert_close(gw[keep], want[1][keep], "streamed node grad_w, dropped ids")
    got = [t for m in (bundle.gate_lora, bundle.up_lora, bundle.down_lora) for t in m.grads[0]]
    for n, (a, b) in enumerate(zip(got, want[2])):
        assert_close(a.numpy(), b, f"streamed node LoRA grad {n}, dropped ids")


def test_many_slots_per_token(k):
    """top-k larger than one work-group's 256 threads (k = 300 of 320 experts): every grad_w slot
    is written."""
    case("k = 300 slots per token")
    rng = np.random.default_rng(27)
    E, D, F, N, topk = 320, 64, 32, 5, 300
    ex = oracle.random_experts(rng, E, D, F, 119, 123)
    idx, w = routing(rng, N, E, topk)
    h = rng.standard_normal((N, D)).astype(np.float32)
    g = rng.standard_normal((N, D)).astype(np.float32)
    L = layer_of(ex)
    H, I, W, G = (torch.from_numpy(a).cuda() for a in (h, idx, w, g))
    assert_close(k.routed_forward(H, I, W, L).cpu().numpy(), oracle.routed_forward(h, idx, w, ex), "k=300 fwd")
    gh, gw = k.routed_backward(H, I, W, L, G)
    gh64, gw64 = oracle.routed_backward(h, idx, w, ex, g)
    assert_close(gh.cpu().numpy(), gh64, "k=300 grad_h")
    assert_close(gw.cpu().numpy(), gw64, "k=300 grad_w")


def outlier_rows(rng, M, K):
    """N(0,1) rows with a few outlier channels shared by all rows (10, 30, 1e3 and 1e4 times the
    rest, both signs), the shape of a transformer residual stream."""
    x = rng.standard_normal((M, K)).astype(np.float32)
    ch = rng.choice(K, size=8, replace=False)
    mult = np.array([10, -30, 1e3, -1e3, 1e4, 30, -10, 3e3], np.float32)
    x[:, ch] *= mult
    return x


def test_outlier_activations_gemm(k, clib):
    """The single-expert product at the config-2 shape (K = 7168, R = 2048) with outlier
    channels, M = 1, 16 and 256, against the C restatement; also with the outliers confined to a
    few blocks of moderate size (x30), where they do not dominate the output."""
    rng = np.random.default_rng(28)
    K, R = 7168, 2048
    pk, sc = oracle.random_mx(rng, (R, K), 117, 121)
    P, S = torch.from_numpy(pk).cuda(), torch.from_numpy(sc).cuda()
    for M in (1, 16, 256):
        case(f"gemm with outlier channels, M={M}")
        x = outlier_rows(rng, M, K)
        y = k.gemm(torch.from_numpy(x).cuda(), P, S).cpu().numpy()
        assert_all_tokens(y, clib.gemm(x, pk, sc), f"outlier gemm M={M}", 5e-3)
        xm = rng.standard_normal((M, K)).astype(np.float32)
        xm[:, rng.choice(K, size=16, replace=False)] *= 30.0
        y = k.gemm(torch.from_numpy(xm).cuda(), P, S).cpu().numpy()
        assert_all_tokens(y, clib.gemm(xm, pk, sc), f"moderate-outlier gemm M={M}", 5e-3)


def test_outlier_activations_routed_layer(k, clib):
    """A routed layer at the BASELINE expert shape (64 experts, 256 tokens, top-8) with outlier
    channels in h, every token against the C restatement, forward and backward, each token of out
    and grad_h within the stated bar (rel-L2 5e-3). With two e4m3 terms a token whose gate/up are
    dominated by one x1e4 channel carried that channel's rounding (up to 2^-8 relative) undiluted
    (worst tokens 3.5e-3 out, 6.9e-3 grad_h, as a float64 simulation of the quantiser also gives);
    blocks whose maximum exceeds 16x the rms of the rest now get a third term. grad_w also goes
    through the down product's two-term activations: 1e-2 per token, as in the other layer tests."""
    case("routed layer with outlier channels: E=64, D=7168, F=2048, N=256, top-8")
    rng = np.random.default_rng(29)
    ex = oracle.random_experts(rng, 64, 7168, 2048, 117, 121)
    h = outlier_rows(rng, 256, 7168)
    idx, w = routing(rng, 256, 64, 8)
    g = rng.standard_normal((256, 7168)).astype(np.float32)
    L = layer_of(ex)
    H, I, W, G = (torch.from_numpy(a).cuda() for a in (h, idx, w, g))
    out = k.routed_forward(H, I, W, L).cpu().numpy()
    assert_all_tokens(out, clib.moe_forward(h, idx, w, ex), "outlier layer fwd", 5e-3)
    gh, gw = k.routed_backward(H, I, W, L, G)
    gh_c, gw_c = clib.moe_backward(h, idx, w, ex, g)
    assert_all_tokens(gh.cpu().numpy(), gh_c, "outlier layer grad_h", 5e-3)
    assert_all_tokens(gw.cpu().numpy(), gw_c, "outlier layer grad_w", 1e-2)


@pytest.mark.parametrize("fl", [False, True])
def test_outlier_activations_large_buckets(k, clib, fl):
    """Outlier channels in h with large buckets (150 and 70 rows of 243, top-1): the grouped
    gate/up work-groups (with a forward layout, the wide groups) add the third term of flagged
    blocks as the one-tile ones do; every token of out and grad_h within 5e-3 of the C restatement.
    With one slot per token grad_w is one scalar per token, a 7168-term dot product whose relative
    error is unbounded where the terms nearly cancel, so it is held to the bar as a whole tensor."""
    case(f"outlier channels, large buckets: E=4, D=7168, F=2048, top-1, forward layout={fl}")
    rng = np.random.default_rng(30 + fl)
    E, D, F = 4, 7168, 2048
    ex = oracle.random_experts(rng, E, D, F, 117, 121)
    idx = np.concatenate([np.full(c, e) for e, c in enumerate([150, 70, 20, 3])]).astype(np.int64)
    rng.shuffle(idx)
    N = idx.size
    idx = idx[:, None]
    w = rng.uniform(0.5, 1.5, (N, 1)).astype(np.float32)
    h = outlier_rows(rng, N, D)
    g = rng.standard_normal((N, D)).astype(np.float32)
    L = layer_of(ex)
    if fl:
        L.prepare_forward_layout()
    H, I, W, G = (torch.from_numpy(a).cuda() for a in (h, idx, w, g))
    out = k.routed_forward(H, I, W, L).cpu().numpy()
    assert_all_tokens(out, clib.moe_forward(h, idx, w, ex), f"outlier large fwd fl={fl}", 5e-3)
    gh, gw = k.routed_backward(H, I, W, L, G)
    gh_c, gw_c = clib.moe_backward(h, idx, w, ex, g)
    assert_all_tokens(gh.cpu().numpy(), gh_c, f"outlier large grad_h fl={fl}", 5e-3)
    assert_close(gw.cpu().numpy(), gw_c, f"outlier large grad_w fl={fl}")


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


@pytest.fixture(scope="module")
def full_layer_host(full_layer):
    """The full layer's packed bytes on the host, for the C restatement (20.96 GB)."""
    return oracle.ExpertSet(*[x.cpu().numpy() for x in full_layer.tensors()])


def per_token_rel(got, want):
    """Per-row rel-L2 (rows with a zero reference row are compared by absolute norm)."""
    num = np.linalg.norm(np.asarray(got, np.float64) - want, axis=1)
    den = np.linalg.norm(np.asarray(want, np.float64), axis=1)
    return num / np.maximum(den, 1e-30)


def assert_all_tokens(got, want, label, tol):
    """Whole-tensor rel-L2 / cosine at the stated bar, and every token's own rel-L2 below `tol`,
    so that one wrong tile, expert slot or work item cannot hide in the global figure."""
    assert_close(got, want, label)
    r = per_token_rel(got, want)
    worst = int(np.argmax(r))
    print(f"{label}: per-token rel-L2 median {np.median(r):.3e} p99 {np.percentile(r, 99):.3e} "
          f"max {r[worst]:.3e} (token {worst})")
    assert r[worst] <= tol, f"{label}: token {worst} rel-L2 {r[worst]:.3e} > {tol:.1e}"


@pytest.mark.parametrize("zipf,fl", [(False, False), (True, False), (True, True)])
def test_baseline_layer_all_tokens(k, clib, full_layer, full_layer_host, zipf, fl):
    """BASELINE configs 3/4 at full size: every one of the 1024 tokens of out, grad_h and grad_w
    against the C restatement of the reference path (lazy_trainer.py:806-880), uniform and
    Zipf-skewed routing; the Zipf layer also with its forward layout (fl), where its large buckets
    take the wide-group forward."""
    case(f"config 3/4 layer, zipf={zipf}, forward layout={fl}: fwd+bwd, all 1024 tokens vs C oracle")
    if fl:
        full_layer.prepare_forward_layout()
    rng = np.random.default_rng(21 + zipf)
    N, E, topk = 1024, 896, 8
    h = rng.standard_normal((N, 7168)).astype(np.float32)
    idx, w = routing(rng, N, E, topk, zipf=zipf)
    g = rng.standard_normal((N, 7168)).astype(np.float32)
    counts = np.bincount(idx.ravel(), minlength=E)
    print(f"active experts {int((counts > 0).sum())}, largest bucket {int(counts.max())}", flush=True)
    H, I, W, G = (torch.from_numpy(a).cuda() for a in (h, idx, w, g))
    ws = torch.empty(k.moe_workspace_bytes(N, topk, E, 7168, 2048), dtype=torch.uint8, device="cuda")
    out = k.routed_forward(H, I, W, full_layer, save_for_backward=True, workspace=ws).cpu().numpy()
    gh, gw = k.routed_backward(H, I, W, full_layer, G, reuse_forward=True, workspace=ws)
    gh, gw = gh.cpu().numpy(), gw.cpu().numpy()
    assert_all_tokens(out, clib.moe_forward(h, idx, w, full_layer_host), f"layer fwd zipf={zipf}", 5e-3)
    gh_c, gw_c = clib.moe_backward(h, idx, w, full_layer_host, g)
    full_layer.drop_forward_layout()
    assert_all_tokens(gh, gh_c, f"layer grad_h zipf={zipf}", 5e-3)
    assert_all_tokens(gw, gw_c, f"layer grad_w zipf={zipf}", 1e-2)


def test_baseline_layer_bf16_h(k, clib, full_layer, full_layer_host):
    """Config 3 with bf16 activations (config 2 names bf16 and fp32): the bf16 input against the
    C restatement fed the same values widened to fp32, all tokens, forward and backward."""
    case("config 3/4 layer, bf16 h: all 1024 tokens vs C oracle")
    rng = np.random.default_rng(24)
    N, E, topk = 1024, 896, 8
    Hb = torch.from_numpy(rng.standard_normal((N, 7168)).astype(np.float32)).bfloat16()
    h = Hb.float().numpy()
    idx, w = routing(rng, N, E, topk)
    g = rng.standard_normal((N, 7168)).astype(np.float32)
    H, I, W, G = Hb.cuda(), torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda(), torch.from_numpy(g).cuda()
    out = k.routed_forward(H, I, W, full_layer).cpu().numpy()
    assert_all_tokens(out, clib.moe_forward(h, idx, w, full_layer_host), "bf16 layer fwd", 5e-3)
    gh, gw = k.routed_backward(H, I, W, full_layer, G)
    gh_c, gw_c = clib.moe_backward(h, idx, w, full_layer_host, g)
    assert_all_tokens(gh.cpu().numpy(), gh_c, "bf16 layer grad_h", 5e-3)
    assert_all_tokens(gw.cpu().numpy(), gw_c, "bf16 layer grad_w", 1e-2)


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
