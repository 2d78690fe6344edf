"""Pins the oracle's GLUs, router and routed-layer composition against the reference's vendored
fixtures (tests/golden/*.json, checked by the reference at 1e-5 abs + 1e-4 rel, and 2e-4 abs
for the composite MoE block: lazy_lora/tests/test_reference_ops.py:52-53, :309), against torch's
own SiLU, and against central differences for every backward."""
import json
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def load(name):
    with open(os.path.join(GOLDEN, f"{name}.json")) as f:
        return json.load(f)


def arr(entry):
    return np.asarray(entry["data"], np.float64).reshape(entry["shape"])


def assert_matches(got, want, abs_tol=1e-5, rel_tol=1e-4):
    got, want = np.asarray(got, np.float64).ravel(), np.asarray(want, np.float64).ravel()
    assert got.shape == want.shape
    diff = np.abs(got - want)
    assert np.all(diff <= abs_tol + rel_tol * np.abs(want)), f"max abs diff {diff.max():.3e}"


def test_situ_glu_fixture():
    fx = load("situ_glu")
    x = arr(fx["in"])
    d = x.shape[-1] // 2
    assert fx["beta"] == oracle.SITU_BETA and fx["linear_beta"] == oracle.SITU_LINEAR_BETA
    assert_matches(oracle.glu_forward(x[..., :d], x[..., d:], "situ"), arr(fx["out"]))


def test_swiglu_matches_torch_silu():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0)
    g, u = rng.standard_normal((2, 64, 32)) * 4
    want = (torch.nn.functional.silu(torch.from_numpy(g)) * torch.from_numpy(u)).numpy()
    assert np.allclose(oracle.glu_forward(g, u, "swiglu"), want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("act", ["swiglu", "situ"])
def test_glu_backward_central_differences(act):
    rng = np.random.default_rng(1)
    g, u, go = rng.standard_normal((3, 200)) * 3
    dg, du = oracle.glu_backward(go, g, u, act)
    eps = 1e-6
    fd_g = (oracle.glu_forward(g + eps, u, act) - oracle.glu_forward(g - eps, u, act)) / (2 * eps) * go
    fd_u = (oracle.glu_forward(g, u + eps, act) - oracle.glu_forward(g, u - eps, act)) / (2 * eps) * go
    assert np.allclose(dg, fd_g, rtol=1e-6, atol=1e-8)
    assert np.allclose(du, fd_u, rtol=1e-6, atol=1e-8)


def test_router_fixture():
    fx = load("router")
    idx, w = oracle.router_forward(arr(fx["in"]), arr(fx["gate_weight"]), arr(fx["bias"]), top_k=fx["top_k"])
    want_idx = arr(fx["topk_idx"]).astype(np.int64)
    want_w = arr(fx["topk_weight"])
    got = {(r, int(i)): float(v) for r, (ii, ww) in enumerate(zip(idx, w)) for i, v in zip(ii, ww)}
    want = {(r, int(i)): float(v) for r, (ii, ww) in enumerate(zip(want_idx, want_w)) for i, v in zip(ii, ww)}
    assert sorted(got) == sorted(want)
    assert_matches([got[k] for k in sorted(got)], [want[k] for k in sorted(want)])
    # the fixture is built so that the selection bias changes the choice in some rows
    plain, _ = oracle.router_forward(arr(fx["in"]), arr(fx["gate_weight"]), None, top_k=fx["top_k"])
    changed = sum(set(a) != set(b) for a, b in zip(plain.tolist(), idx.tolist()))
    assert changed == fx["rows_where_bias_changed_selection"]


@pytest.mark.parametrize("top_k,renorm,scale", [(4, True, 1.0), (4, True, 2.5), (4, False, 1.0), (1, True, 1.0)])
def test_router_select_backward_central_differences(top_k, renorm, scale):
    """The closed-form router gradient against central differences of router_select with the
    selection held fixed (every finite-difference step keeps the same top-k)."""
    rng = np.random.default_rng(5)
    N, E = 3, 12
    logits = rng.standard_normal((N, E))
    bias = 0.1 * rng.standard_normal(E)
    idx, _ = oracle.router_select(logits, bias, top_k, scale, renorm)
    g = rng.standard_normal((N, top_k))
    got = oracle.router_select_backward(logits, idx, g, scale, renorm)
    eps = 1e-6
    fd = np.zeros_like(logits)
    for n in range(N):
        for e in range(E):
            lp, lm = logits.copy(), logits.copy()
            lp[n, e] += eps
            lm[n, e] -= eps
            ip, wp = oracle.router_select(lp, bias, top_k, scale, renorm)
            im, wm = oracle.router_select(lm, bias, top_k, scale, renorm)
            assert (ip == idx).all() and (im == idx).all()
            fd[n, e] = ((wp - wm) * g).sum() / (2 * eps)
    assert np.allclose(got, fd, rtol=1e-6, atol=1e-9)
    unchosen = np.ones_like(logits, bool)
    np.put_along_axis(unchosen, idx, False, axis=-1)
    assert (got[unchosen] == 0).all()


def test_router_select_ties_and_bias_only_in_selection():
    """Equal choices go to the lower expert id (a stable descending sort), and the weights are
    the unbiased scores: a huge bias on one expert selects it without changing its weight."""
    logits = np.zeros((1, 6))
    idx, w = oracle.router_select(logits, None, 3, 1.0, False)
    assert idx.tolist() == [[0, 1, 2]] and np.allclose(w, 0.5)
    bias = np.array([0, 0, 0, 0, 0, 100.0])
    idx, w = oracle.router_select(logits, bias, 2, 1.0, False)
    assert idx.tolist() == [[5, 0]] and np.allclose(w, 0.5)


def test_router_select_nan_ranks_first_like_torch_topk():
    """torch.topk, which KimiK3MoERouter.forward calls (moe_router.py:90), ranks NaN above every
    number. The oracle does the same: the NaN experts of a row come first (torch leaves their
    mutual order, and which of them it keeps when there are more than k, unspecified; the
    oracle takes the lowest ids), then the rest by value, exactly as torch orders them."""
    import torch
    rng = np.random.default_rng(11)
    N, E, top_k = 300, 37, 6
    logits = rng.normal(size=(N, E))
    logits[rng.random(logits.shape) < 0.08] = np.nan
    bias = 0.1 * rng.normal(size=E)
    idx, w = oracle.router_select(logits, bias, top_k)
    choice = torch.sigmoid(torch.from_numpy(logits)) + torch.from_numpy(bias)
    ti = torch.topk(choice, top_k, dim=-1, sorted=True).indices.numpy()
    nan_rows = 0
    for r in range(N):
        nan_ids = np.flatnonzero(np.isnan(choice[r].numpy()))
        m = min(len(nan_ids), top_k)
        nan_rows += m > 0
        assert set(idx[r, :m]) <= set(nan_ids) and set(ti[r, :m]) <= set(nan_ids), r
        assert idx[r, :m].tolist() == sorted(nan_ids)[:m]
        assert idx[r, m:].tolist() == ti[r, m:].tolist(), r
    assert nan_rows > N // 2
    assert ((0 <= idx) & (idx < E)).all()


def moe_params(fx):
    return {k: (arr(v) if isinstance(v, dict) else v) for k, v in fx.items()}


def test_moe_block_fixture():
    """The latent MoE block of moe.json through the oracle's composition with the fixture's
    dense expert weights (they are not MXFP4-representable)."""
    fx = load("moe")
    p = moe_params(fx)

    def dense(e):
        return tuple(p[f"experts_{e}_{m}_weight"] for m in ("w1", "w3", "w2"))

    got, _, _ = oracle.latent_moe_forward(p["in"], p, dense=dense)
    assert_matches(got, p["out"], abs_tol=2e-4)


def test_quantize_mxfp4_round_trip():
    """Representable weights survive quantisation exactly; others move by at most half a step
    of their block's grid (the largest E2M1 step is 2, times the block scale)."""
    rng = np.random.default_rng(8)
    pk, sc = oracle.random_mx(rng, (16, 128), 110, 130)
    w = oracle.dequant(pk, sc)
    qp, qs = oracle.quantize_mxfp4(w)
    assert np.array_equal(oracle.dequant(qp, qs), w)
    x = rng.standard_normal((8, 64)) * np.exp(rng.standard_normal((8, 1)))
    qp, qs = oracle.quantize_mxfp4(x)
    back = oracle.dequant(qp, qs).astype(np.float64)
    step = oracle.e8m0_table()[qs].astype(np.float64).repeat(32, axis=1)
    assert np.all(np.abs(back - x) <= step + 1e-12)
    assert np.all(np.sign(back[back != 0]) == np.sign(x[back != 0]))


@pytest.mark.parametrize("act", ["swiglu", "situ"])
def test_routed_backward_central_differences(act):
    rng = np.random.default_rng(2)
    ex = oracle.random_experts(rng, 4, 64, 32, 124, 128)
    N, k = 6, 2
    h = rng.standard_normal((N, 64))
    idx, w = oracle.softmax_topk(rng.standard_normal((N, 4)), k)
    w = w.astype(np.float64)
    g = rng.standard_normal((N, 64))
    gh, gw = oracle.routed_backward(h, idx, w, ex, g, act)

    def loss(hh, ww):
        return float((oracle.routed_forward(hh, idx, ww, ex, act) * g).sum())

    eps = 1e-6
    fd_h = np.zeros_like(h)
    for i in range(N):
        for j in range(0, 64, 7):
            d = np.zeros_like(h)
            d[i, j] = eps
            fd_h[i, j] = (loss(h + d, w) - loss(h - d, w)) / (2 * eps)
    mask = np.zeros_like(h, bool)
    mask[:, ::7] = True
    assert np.allclose(gh[mask], fd_h[mask], rtol=1e-5, atol=1e-7)
    fd_w = np.zeros_like(w)
    for i in range(N):
        for s in range(k):
            d = np.zeros_like(w)
            d[i, s] = eps
            fd_w[i, s] = (loss(h, w + d) - loss(h, w - d)) / (2 * eps)
    assert np.allclose(gw, fd_w, rtol=1e-5, atol=1e-7)


def test_routed_invariants(clib):
    rng = np.random.default_rng(3)
    ex = oracle.random_experts(rng, 8, 256, 128, 119, 123)
    N = 64
    h = rng.standard_normal((N, 256)).astype(np.float32)
    idx, w = oracle.softmax_topk(rng.standard_normal((N, 8)).astype(np.float32), 2)
    a = clib.moe_forward(h, idx, w, ex)
    # expert visiting order only changes fp32 rounding (the reference visits in disk order)
    b = clib.moe_forward(h, idx, w, ex, order=np.unique(idx)[::-1])
    assert oracle.rel_l2(a, b) < 1e-6
    # float64 composition agrees
    assert oracle.rel_l2(a, oracle.routed_forward(h, idx, w, ex)) < 1e-6
    # experts nobody chose contribute nothing; a token's output is linear in its weights
    assert np.allclose(clib.moe_forward(h, idx, 2 * w, ex), 2 * a, rtol=1e-6, atol=1e-6)
    # C backward agrees with the float64 backward
    g = rng.standard_normal((N, 256)).astype(np.float32)
    gh, gw = clib.moe_backward(h, idx, w, ex, g)
    gh64, gw64 = oracle.routed_backward(h, idx, w, ex, g)
    assert oracle.rel_l2(gh, gh64) < 1e-6 and oracle.rel_l2(gw, gw64) < 1e-6


# ------------------------------------------------------------------------------------ LoRA terms
def _lora_case(seed=9, E=4, D=64, F=32, N=6, k=2, r=3):
    rng = np.random.default_rng(seed)
    ex = oracle.random_experts(rng, E, D, F, 124, 128)
    h = rng.standard_normal((N, D))
    idx, w = oracle.softmax_topk(rng.standard_normal((N, E)), k)
    g = rng.standard_normal((N, D))
    lora = oracle.random_lora(rng, D, F, r, scale=0.2)
    return ex, h, idx, w.astype(np.float64), g, lora


@pytest.mark.parametrize("act", ["swiglu", "situ"])
def test_lora_with_zero_B_changes_nothing(act):
    """The reference initialises B to zero (lora_layer.py:82-84): the layer then equals the
    LoRA-off layer, A gets no gradient and B does."""
    ex, h, idx, w, g, lora = _lora_case()
    for name in ("gate_B", "up_B", "down_B"):
        setattr(lora, name, np.zeros_like(getattr(lora, name)))
    assert np.allclose(oracle.routed_forward(h, idx, w, ex, act, lora=lora), oracle.routed_forward(h, idx, w, ex, act))
    gh, gw, lg = oracle.routed_backward(h, idx, w, ex, g, act, lora=lora)
    gh0, gw0 = oracle.routed_backward(h, idx, w, ex, g, act)
    assert np.allclose(gh, gh0) and np.allclose(gw, gw0)
    assert all(not lg[i].any() for i in (0, 2, 4))
    assert all(np.abs(lg[i]).max() > 0 for i in (1, 3, 5))


@pytest.mark.parametrize("act", ["swiglu", "situ"])
def test_lora_equals_merged_weights(act):
    """x W^T + s (x A^T) B^T = x (W + s B A)^T: the adapters must act exactly like merged dense
    weights, in the forward and in dL/dh and dL/dw."""
    ex, h, idx, w, g, lora = _lora_case()

    def merged(e):
        W1, W3, W2 = ex.dense(e)
        return (W1 + lora.gate_s * lora.gate_B.astype(np.float64) @ lora.gate_A,
                W3 + lora.up_s * lora.up_B.astype(np.float64) @ lora.up_A,
                W2 + lora.down_s * lora.down_B.astype(np.float64) @ lora.down_A)

    got = oracle.routed_forward(h, idx, w, ex, act, lora=lora)
    assert np.allclose(got, oracle.routed_forward(h, idx, w, None, act, dense=merged), rtol=1e-10, atol=1e-12)
    assert not np.allclose(got, oracle.routed_forward(h, idx, w, ex, act))
    gh, gw, _ = oracle.routed_backward(h, idx, w, ex, g, act, lora=lora)
    mh, mw = oracle.routed_backward(h, idx, w, None, g, act, dense=merged)
    assert np.allclose(gh, mh, rtol=1e-10, atol=1e-12) and np.allclose(gw, mw, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("act", ["swiglu", "situ"])
def test_lora_gradients_central_differences(act):
    ex, h, idx, w, g, lora = _lora_case()
    _, _, lg = oracle.routed_backward(h, idx, w, ex, g, act, lora=lora)
    names = ("gate_A", "gate_B", "up_A", "up_B", "down_A", "down_B")
    eps = 1e-6
    rng = np.random.default_rng(0)
    for n, name in enumerate(names):
        base = getattr(lora, name).astype(np.float64)
        for _ in range(6):
            pos = tuple(int(rng.integers(0, s)) for s in base.shape)
            vals = []
            for sign in (1, -1):
                pert = base.copy()
                pert[pos] += sign * eps
                setattr(lora, name, pert)
                vals.append(float((oracle.routed_forward(h, idx, w, ex, act, lora=lora) * g).sum()))
            setattr(lora, name, base)
            fd = (vals[0] - vals[1]) / (2 * eps)
            assert abs(lg[n][pos] - fd) <= 1e-6 + 1e-5 * abs(fd), (name, pos, lg[n][pos], fd)
