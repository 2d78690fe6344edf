"""The router's selection kernel and its gradient on the GPU, against the reference's router
fixture (router.json, 6 tokens x 128, 8 experts, top-2 with a selection bias) and the float64
oracle (oracle.router_select / router_select_backward) on the same logits.

fp32 sigmoid scores can order two experts differently from float64 when their biased scores
lie within a few ulps; such rows are compared as sets (or skipped when the k-th and (k+1)-th
choices are that close), and their number is bounded. Ties that are exact in fp32 go to the
lower expert id and are compared exactly."""
import json
import os

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NEAR = 1e-6   # biased-score gap below which fp32 and float64 may order two experts differently


@pytest.fixture(scope="module")
def k():
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    from lazylora_amd.native import kernel
    return kernel()


def case(msg):
    print(f"\n[case] {msg}", flush=True)


def arr(entry):
    return np.asarray(entry["data"], np.float64).reshape(entry["shape"])


def test_router_fixture(k):
    case("router.json through KimiK3MoERouter.forward")
    from lazylora_amd.router import KimiK3MoERouter
    with open(os.path.join(GOLDEN, "router.json")) as f:
        fx = json.load(f)
    gate, bias, x = arr(fx["gate_weight"]), arr(fx["bias"]), arr(fx["in"])
    r = KimiK3MoERouter(hidden_size=gate.shape[1], num_experts=fx["n_experts"], top_k=fx["top_k"], device="cuda")
    idx, w = r.forward(torch.tensor(x, dtype=torch.float32, device="cuda"),
                       weight=torch.tensor(gate, dtype=torch.float32, device="cuda"),
                       bias=torch.tensor(bias, dtype=torch.float32, device="cuda"))
    assert idx.dtype == torch.int64 and w.dtype == torch.float32 and idx.is_cuda
    assert idx.cpu().numpy().tolist() == arr(fx["topk_idx"]).astype(np.int64).tolist()
    assert np.allclose(w.cpu().numpy(), arr(fx["topk_weight"]), rtol=0, atol=2e-6)
    # without the bias the choice differs in the fixture's stated number of rows
    plain, _ = r.forward(torch.tensor(x, dtype=torch.float32, device="cuda"),
                         weight=torch.tensor(gate, dtype=torch.float32, device="cuda"),
                         bias=torch.zeros(fx["n_experts"], device="cuda"))
    changed = sum(set(a) != set(b) for a, b in zip(plain.cpu().tolist(), idx.cpu().tolist()))
    assert changed == fx["rows_where_bias_changed_selection"]


def compare_selection(idx, w, logits, bias, top_k, scale, renorm):
    """Exact indices where float64 leaves no near-tie; weights to 1e-5 relative everywhere the
    chosen sets agree. Returns the number of rows compared as sets or skipped."""
    want_idx, want_w = oracle.router_select(logits, bias, top_k, scale, renorm)
    s = 1.0 / (1.0 + np.exp(-np.asarray(logits, np.float64)))
    choice = s + (np.asarray(bias, np.float64) if bias is not None else 0.0)
    srt = -np.sort(-choice, axis=-1)[:, :min(top_k + 1, choice.shape[1])]
    gaps = -np.diff(srt, axis=-1)
    loose = 0
    for n in range(idx.shape[0]):
        if gaps.shape[1] and gaps[n].min() < NEAR:
            loose += 1
            if top_k < choice.shape[1] and gaps[n, top_k - 1] < NEAR:
                continue        # the k-th / (k+1)-th choice is a near-tie: the set may differ
            assert sorted(idx[n].tolist()) == sorted(want_idx[n].tolist()), n
            order = np.argsort(idx[n])
            assert np.allclose(w[n][order], want_w[n][np.argsort(want_idx[n])], rtol=1e-5, atol=1e-7), n
            continue
        assert idx[n].tolist() == want_idx[n].tolist(), (n, idx[n], want_idx[n])
        assert np.allclose(w[n], want_w[n], rtol=1e-5, atol=1e-7), n
    return loose


@pytest.mark.parametrize("N,E,top_k,renorm,scale,with_bias", [
    (1024, 896, 16, True, 1.0, True),     # the reference model's router (moe_router.py:31-37)
    (4096, 896, 8, True, 2.827, True),    # BASELINE config 3/4 routing width, scaled weights
    (7, 100, 5, False, 2.5, False),       # ragged N and E, no renormalisation, no bias
    (33, 2048, 64, True, 1.0, True),      # the wide-expert kernel variant, maximum top_k
    (5, 64, 1, True, 1.0, True),          # top_k = 1 never renormalises
    (3, 4096, 3, True, 0.5, True),        # maximum E
])
def test_selection_vs_oracle(k, N, E, top_k, renorm, scale, with_bias):
    case(f"router_topk N={N} E={E} k={top_k} renorm={renorm} scale={scale} bias={with_bias}")
    rng = np.random.default_rng(N + E + top_k)
    logits = (2.0 * rng.standard_normal((N, E))).astype(np.float32)
    bias = (0.05 * rng.standard_normal(E)).astype(np.float32) if with_bias else None
    L = torch.from_numpy(logits).cuda()
    B = torch.from_numpy(bias).cuda() if with_bias else None
    idx, w = k.router_topk(L, B, top_k, scale, renorm)
    torch.cuda.synchronize()
    idx, w = idx.cpu().numpy(), w.cpu().numpy()
    assert idx.shape == (N, top_k) and w.shape == (N, top_k)
    assert ((idx >= 0) & (idx < E)).all()
    assert all(len(set(r)) == top_k for r in idx.tolist())
    loose = compare_selection(idx, w, logits, bias, top_k, scale, renorm)
    print(f"rows with an fp32/float64 near-tie: {loose} of {N}")
    assert loose <= max(2, N // 50)
    if renorm and top_k > 1:
        assert np.allclose(w.sum(-1), scale, rtol=1e-5)


def test_exact_ties_go_to_lower_id(k):
    case("exact ties: lower expert id first, order of equal scores")
    rng = np.random.default_rng(3)
    N, E, top_k = 64, 300, 12
    logits = rng.integers(-4, 5, size=(N, E)).astype(np.float32) * 0.5   # many exact ties
    idx, w = k.router_topk(torch.from_numpy(logits).cuda(), None, top_k, 1.0, True)
    want_idx, want_w = oracle.router_select(logits, None, top_k, 1.0, True)
    assert idx.cpu().numpy().tolist() == want_idx.tolist()
    assert np.allclose(w.cpu().numpy(), want_w, rtol=1e-6)


@pytest.mark.parametrize("E", [100, 1024, 4096])
def test_nan_logits_select_real_experts(k, E):
    """NaN logits rank first, as in torch.topk; every chosen id is a real expert, including rows
    with fewer numeric scores than top_k and E filling every lane slot (1024, 4096)."""
    case(f"NaN logits E={E}")
    rng = np.random.default_rng(5)
    N, top_k = 96, 8
    logits = rng.standard_normal((N, E)).astype(np.float32)
    logits[rng.random(logits.shape) < 0.02] = np.nan
    logits[:8, :] = np.nan                        # rows with no numeric score at all
    logits[8:16, top_k // 2:] = np.nan            # rows with fewer numeric scores than top_k
    bias = (0.05 * rng.standard_normal(E)).astype(np.float32)
    idx, w = k.router_topk(torch.from_numpy(logits).cuda(), torch.from_numpy(bias).cuda(), top_k)
    idx = idx.cpu().numpy()
    assert ((idx >= 0) & (idx < E)).all()
    want_idx, _ = oracle.router_select(logits, bias, top_k)
    assert idx[:16].tolist() == want_idx[:16].tolist()   # decided by NaN ranks and ids alone
    choice = 1.0 / (1.0 + np.exp(-logits.astype(np.float64))) + bias
    loose = 0
    for r in range(16, N):
        nan = np.isnan(choice[r])
        m = min(int(nan.sum()), top_k)
        assert idx[r, :m].tolist() == want_idx[r, :m].tolist(), r
        num = np.sort(choice[r][~nan])[::-1]
        kth = top_k - m
        if kth < len(num) and kth > 0 and num[kth - 1] - num[kth] < NEAR:
            loose += 1                                   # fp32 may order the boundary pair either way
            continue
        assert sorted(idx[r, m:].tolist()) == sorted(want_idx[r, m:].tolist()), r
    assert loose <= 2


def test_selection_is_deterministic_and_zero_tokens(k):
    case("determinism over repeated calls; N = 0")
    rng = np.random.default_rng(4)
    L = torch.from_numpy(rng.standard_normal((333, 896)).astype(np.float32)).cuda()
    B = torch.from_numpy((0.1 * rng.standard_normal(896)).astype(np.float32)).cuda()
    a = k.router_topk(L, B, 16)
    b = k.router_topk(L, B, 16)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    i0, w0 = k.router_topk(torch.empty((0, 896), device="cuda"), B, 16)
    assert i0.shape == (0, 16) and w0.shape == (0, 16)


def test_argument_errors(k):
    L = torch.zeros((4, 100), device="cuda")
    with pytest.raises(ValueError):
        k.router_topk(L, None, 65)
    with pytest.raises(ValueError):
        k.router_topk(L, None, 101)
    with pytest.raises(ValueError):
        k.router_topk(torch.zeros((2, 4097), device="cuda"), None, 4)
    with pytest.raises(ValueError):
        k.router_topk(L, torch.zeros(99, device="cuda"), 4)


@pytest.mark.parametrize("E,top_k,renorm,scale", [(896, 16, True, 1.0), (100, 5, False, 2.5),
                                                  (2048, 64, True, 0.7), (64, 1, True, 1.0)])
def test_backward_vs_oracle(k, E, top_k, renorm, scale):
    case(f"router_topk_backward E={E} k={top_k} renorm={renorm} scale={scale}")
    rng = np.random.default_rng(E + top_k)
    N = 257
    logits = (2.0 * rng.standard_normal((N, E))).astype(np.float32)
    g = rng.standard_normal((N, top_k)).astype(np.float32)
    L = torch.from_numpy(logits).cuda()
    idx, _ = k.router_topk(L, None, top_k, scale, renorm)
    got = k.router_topk_backward(L, idx, torch.from_numpy(g).cuda(), scale, renorm).cpu().numpy()
    want = oracle.router_select_backward(logits, idx.cpu().numpy(), g, scale, renorm)
    assert got.shape == (N, E)
    assert np.allclose(got, want, rtol=1e-4, atol=1e-7), np.abs(got - want).max()
    assert (got[want == 0] == 0).all()


def test_autograd_through_router(k):
    """dL/dx and dL/dW through KimiK3MoERouter against torch autograd of the reference's torch
    branch (moe_router.py:86-98) in fp32 on the CPU, with the selection taken from the GPU."""
    case("autograd: x and gate weight gradients")
    from lazylora_amd.router import KimiK3MoERouter
    torch.manual_seed(0)
    N, H, E, top_k, scale = 96, 256, 128, 6, 2.5
    r = KimiK3MoERouter(hidden_size=H, num_experts=E, top_k=top_k, routed_scaling_factor=scale, device="cuda")
    with torch.no_grad():
        r.bias.copy_(0.05 * torch.randn(E))
    x = torch.randn(N, H, device="cuda", requires_grad=True)
    g = torch.randn(N, top_k, device="cuda")
    idx, w = r(x)
    (w * g).sum().backward()

    xc = x.detach().cpu().requires_grad_(True)
    wc = r.weight.detach().cpu().requires_grad_(True)
    scores = torch.sigmoid(torch.nn.functional.linear(xc, wc))
    tw = torch.gather(scores, -1, idx.cpu())
    tw = tw / (tw.sum(-1, keepdim=True) + 1e-20) * scale
    assert torch.allclose(w.detach().cpu(), tw.detach(), rtol=1e-5, atol=1e-7)
    (tw * g.cpu()).sum().backward()
    assert torch.allclose(x.grad.cpu(), xc.grad, rtol=1e-4, atol=1e-6)
    assert torch.allclose(r.weight.grad.cpu(), wc.grad, rtol=1e-4, atol=1e-6)
    assert r.bias.grad is None or not r.bias.grad.any()


def test_host_inputs_and_active_set(k):
    case("CPU tensor and NumPy inputs; get_active_expert_set")
    from lazylora_amd.router import KimiK3MoERouter, route
    rng = np.random.default_rng(6)
    x = rng.standard_normal((20, 64)).astype(np.float32)
    W = (0.1 * rng.standard_normal((32, 64))).astype(np.float32)
    i_np, w_np = route(x, W, None, top_k=4)
    assert isinstance(i_np, np.ndarray) and isinstance(w_np, np.ndarray)
    i_t, w_t = route(torch.from_numpy(x), torch.from_numpy(W), None, top_k=4)
    assert not i_t.is_cuda and np.array_equal(i_t.numpy(), i_np) and np.array_equal(w_t.numpy(), w_np)
    assert compare_selection(i_np, w_np, x.astype(np.float64) @ W.T.astype(np.float64), None, 4, 1.0, True) <= 1
    active = KimiK3MoERouter.get_active_expert_set(torch.from_numpy(i_np).cuda())
    assert active == sorted(set(i_np.ravel().tolist()))
    assert KimiK3MoERouter.get_active_expert_set(i_np) == active


def test_router_feeds_routed_layer(k):
    """Device routing straight into the routed-expert layer, no host round trip, against the
    oracle layer on the same routing."""
    case("router -> routed layer")
    from tests.conftest import assert_close
    from lazylora_amd.experts import ExpertLayer
    from lazylora_amd.router import route
    rng = np.random.default_rng(7)
    E, D, F, N, top_k = 16, 256, 128, 80, 4
    ex = oracle.random_experts(rng, E, D, F, 119, 123)
    L = ExpertLayer(*[torch.from_numpy(np.ascontiguousarray(a)).cuda()
                      for a in (ex.w1p, ex.w1s, ex.w3p, ex.w3s, ex.w2p, ex.w2s)])
    h = torch.from_numpy(rng.standard_normal((N, D)).astype(np.float32)).cuda()
    gate = torch.from_numpy((0.05 * rng.standard_normal((E, D))).astype(np.float32)).cuda()
    idx, w = route(h, gate, None, top_k=top_k)
    out = k.routed_forward(h, idx, w, L, act="situ")
    want = oracle.routed_forward(h.cpu().numpy(), idx.cpu().numpy(), w.cpu().numpy(), ex, "situ")
    assert_close(out.cpu().numpy(), want, "router -> routed forward")
