"""The routed layer with the layer's LoRA adapters on the GPU, against the float64 oracle
(oracle.routed_forward / routed_backward with `lora`, which restate lazy_trainer.py:762-804,
:836-880 and lora_layer.py:104-139, :178-226, and are pinned on the CPU by merged-weight
equivalence and central differences).

Adapters are drawn with nonzero A and B so every LoRA term matters; the bar is the path's
rel-L2 <= 5e-3 and cosine >= 0.9999 on the outputs and on each adapter gradient."""
import types

import numpy as np
import pytest
import torch

import oracle
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu

NAMES = ("gate_A", "gate_B", "up_A", "up_B", "down_A", "down_B")


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


def adapters_of(lo: oracle.LoRA, requires_grad=False):
    """(gate, up, down) objects shaped like the reference's LazyLoRALinear."""
    mods = []
    for A, B, s in lo.adapters():
        At = torch.from_numpy(np.asarray(A, np.float32)).cuda().requires_grad_(requires_grad)
        Bt = torch.from_numpy(np.asarray(B, np.float32)).cuda().requires_grad_(requires_grad)
        mods.append(types.SimpleNamespace(lora_A=At, lora_B=Bt, scaling=s, dropout_rate=0.0))
    return tuple(mods)


def run_case(k, E, D, F, N, topk, r, act, seed, h_bf16=False, scale_lo=119, scale_hi=123, sizes=None):
    """sizes: rows per expert, routed top-1 in shuffled order (N and topk are then ignored)."""
    rng = np.random.default_rng(seed)
    ex = oracle.random_experts(rng, E, D, F, scale_lo, scale_hi)
    if sizes is not None:
        first = np.concatenate([np.full(c, e) for e, c in enumerate(sizes)]).astype(np.int64)
        rng.shuffle(first)
        N = first.size
        idx, w = first[:, None], rng.uniform(0.5, 1.5, (N, 1)).astype(np.float32)
    h = rng.standard_normal((N, D)).astype(np.float32)
    if sizes is None:
        idx, w = oracle.softmax_topk(rng.standard_normal((N, E)).astype(np.float32), topk)
    g = rng.standard_normal((N, D)).astype(np.float32)
    lo = oracle.random_lora(rng, D, F, r)
    L = layer_of(ex)
    H = torch.from_numpy(h).cuda()
    if h_bf16:
        H = H.bfloat16()
        h = H.float().cpu().numpy()
    I, W, G = (torch.from_numpy(a).cuda() for a in (idx, w, g))
    mods = adapters_of(lo)
    out = k.routed_forward(H, I, W, L, act=act, lora=mods)
    assert_close(out.cpu().numpy(), oracle.routed_forward(h, idx, w, ex, act, lora=lo), f"fwd {act} r={r}")
    gh, gw, lg = k.routed_backward(H, I, W, L, G, act=act, lora=mods)
    gh64, gw64, lg64 = oracle.routed_backward(h, idx, w, ex, g, act, lora=lo)
    assert_close(gh.cpu().numpy(), gh64, f"grad_h {act}")
    assert_close(gw.cpu().numpy(), gw64, f"grad_w {act}")
    for name, a, b in zip(NAMES, lg, lg64):
        assert a.shape == b.shape, name
        assert_close(a.cpu().numpy(), b, f"grad {name}")
    return L, H, I, W, G, mods


@pytest.mark.parametrize("act", ["swiglu", "situ"])
def test_config1_with_lora(k, act):
    """BASELINE config 1 (D 256, F 128, 8 experts, top-2, 64 tokens) with rank-16 adapters."""
    case(f"config 1 + LoRA r=16 {act}")
    run_case(k, 8, 256, 128, 64, 2, 16, act, seed=31)


@pytest.mark.parametrize("r,h_bf16", [(1, False), (8, True), (32, False)])
def test_ranks_and_dtypes(k, r, h_bf16):
    case(f"16 experts 512x256, 96 tokens top-4, LoRA r={r}, bf16 h={h_bf16}")
    run_case(k, 16, 512, 256, 96, 4, r, "situ", seed=32 + r, h_bf16=h_bf16)


@pytest.mark.parametrize("act", ["swiglu", "situ"])
def test_large_buckets_with_lora(k, act):
    """Buckets of 150, 70, 30 and 6 rows (10, 5, 2 and 1 tiles; K = 1024 and 512 keep both
    products on the path that splits them): the first two take the grouped work-groups, whose
    epilogues add the LoRA gate/up deltas and whose gradients feed the adapter gradients."""
    case(f"large buckets + LoRA r=16 {act}")
    run_case(k, 4, 1024, 512, 0, 1, 16, act, seed=47, scale_lo=118, scale_hi=122, sizes=[150, 70, 30, 6])


@pytest.mark.parametrize("F,r", [(352, 16), (352, 32), (416, 16)])
def test_ffn_not_a_multiple_of_64(k, F, r):
    """F = 352 or 416: the last 64-column block of the fused pass over the gate/up gradients is
    part valid. Its waves supply the coefficients of every rank whatever their own columns are,
    so the B_gate / B_up gradients of the last features keep ranks 8..15 (and 24..31); only the
    elements of the columns past F are zeroed."""
    case(f"2 experts 256x{F}, 120 tokens top-2, LoRA r={r}")
    run_case(k, 2, 256, F, 120, 2, r, "swiglu", seed=48 + r)


def test_expert_shape_of_the_reference(k):
    """Adapters on experts of the BASELINE shape (2048 x 7168): the long reductions (K = 7168)
    and the wide expansions run at their real sizes."""
    case("8 experts 2048x7168, 40 tokens top-2, LoRA r=16")
    run_case(k, 8, 7168, 2048, 40, 2, 16, "situ", seed=40, scale_lo=117, scale_hi=121)


def test_zero_B_is_bitwise_lora_off(k):
    """With every B = 0 (the reference's initialisation) each LoRA term adds an exact zero: the
    results equal the LoRA-off path bit for bit, and only the B gradients are nonzero."""
    case("B = 0 == LoRA off, bitwise")
    rng = np.random.default_rng(41)
    ex = oracle.random_experts(rng, 8, 256, 128, 119, 123)
    L = layer_of(ex)
    idx, w = oracle.softmax_topk(rng.standard_normal((48, 8)).astype(np.float32), 2)
    H, I, W, G = (torch.from_numpy(a).cuda() for a in (rng.standard_normal((48, 256)).astype(np.float32), idx, w,
                                                       rng.standard_normal((48, 256)).astype(np.float32)))
    lo = oracle.random_lora(rng, 256, 128, 16)
    for name in ("gate_B", "up_B", "down_B"):
        setattr(lo, name, np.zeros_like(getattr(lo, name)))
    mods = adapters_of(lo)
    assert torch.equal(k.routed_forward(H, I, W, L, lora=mods), k.routed_forward(H, I, W, L))
    gh, gw, lg = k.routed_backward(H, I, W, L, G, lora=mods)
    gh0, gw0 = k.routed_backward(H, I, W, L, G)
    assert torch.equal(gh, gh0) and torch.equal(gw, gw0)
    assert not lg[0].any() and not lg[2].any() and not lg[4].any()
    assert lg[1].abs().max() > 0 and lg[3].abs().max() > 0 and lg[5].abs().max() > 0


def test_reuse_equals_recompute_and_is_deterministic(k):
    case("LoRA backward: reused forward state == recompute; repeat calls identical")
    rng = np.random.default_rng(42)
    ex = oracle.random_experts(rng, 16, 512, 256, 117, 121)
    L = layer_of(ex)
    N, topk = 96, 4
    idx, w = oracle.softmax_topk(rng.standard_normal((N, 16)).astype(np.float32), topk)
    H, I, W, G = (torch.from_numpy(a).cuda() for a in (rng.standard_normal((N, 512)).astype(np.float32), idx, w,
                                                       rng.standard_normal((N, 512)).astype(np.float32)))
    mods = adapters_of(oracle.random_lora(rng, 512, 256, 16))
    ws = torch.empty(k.moe_workspace_bytes(N, topk, 16, 512, 256), dtype=torch.uint8, device="cuda")
    out = k.routed_forward(H, I, W, L, save_for_backward=True, workspace=ws, lora=mods)
    a = k.routed_backward(H, I, W, L, G, reuse_forward=True, workspace=ws, lora=mods)
    b = k.routed_backward(H, I, W, L, G, lora=mods)
    c = k.routed_backward(H, I, W, L, G, lora=mods)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    for x, y, z in zip(a[2], b[2], c[2]):
        assert torch.equal(x, y) and torch.equal(y, z)
    assert torch.equal(out, k.routed_forward(H, I, W, L, lora=mods))


def test_invalid_ids_with_lora(k):
    """Device ids outside [0, E) are skipped: the same as a valid id with weight 0, except that
    the skipped slot's grad_w is 0."""
    case("LoRA with expert ids outside [0, E)")
    rng = np.random.default_rng(43)
    ex = oracle.random_experts(rng, 8, 256, 128, 119, 123)
    L = layer_of(ex)
    h = rng.standard_normal((4, 256)).astype(np.float32)
    g = rng.standard_normal((4, 256)).astype(np.float32)
    idx = np.array([[0, 9], [1, 2], [3, -1], [4, 5]], np.int64)
    w = np.full((4, 2), 0.5, np.float32)
    keep, wk = idx.copy(), w.copy()
    keep[0, 1], keep[2, 1] = 0, 3
    wk[0, 1] = wk[2, 1] = 0.0
    lo = oracle.random_lora(rng, 256, 128, 4)
    mods = adapters_of(lo)
    H, G = torch.from_numpy(h).cuda(), torch.from_numpy(g).cuda()
    out = k.routed_forward(H, torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda(), L, lora=mods)
    assert_close(out.cpu().numpy(), oracle.routed_forward(h, keep, wk, ex, lora=lo), "fwd, skipped ids")
    gh, gw, lg = k.routed_backward(H, torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda(), L, G, lora=mods)
    gh64, gw64, lg64 = oracle.routed_backward(h, keep, wk, ex, g, lora=lo)
    assert_close(gh.cpu().numpy(), gh64, "grad_h, skipped ids")
    gwn = gw.cpu().numpy()
    assert gwn[0, 1] == 0 and gwn[2, 1] == 0
    valid = np.ones_like(gwn, bool)
    valid[0, 1] = valid[2, 1] = False
    assert_close(gwn[valid], gw64[valid], "grad_w, skipped ids")
    for name, a, b in zip(NAMES, lg, lg64):
        assert_close(a.cpu().numpy(), b, f"grad {name}, skipped ids")


def test_autograd_node_accumulates_adapter_grads(k):
    case("RoutedExpertsFunction with LoRA: adapter .grad accumulation")
    from lazylora_amd.routed import RoutedExpertsFunction
    rng = np.random.default_rng(44)
    ex = oracle.random_experts(rng, 8, 256, 128, 119, 123)
    L = layer_of(ex)
    idx, w = oracle.softmax_topk(rng.standard_normal((32, 8)).astype(np.float32), 2)
    h = torch.from_numpy(rng.standard_normal((32, 256)).astype(np.float32)).cuda().requires_grad_()
    I = torch.from_numpy(idx).cuda()
    W = torch.from_numpy(w).cuda().requires_grad_()
    lo = oracle.random_lora(rng, 256, 128, 8)
    mods = adapters_of(lo, requires_grad=True)
    bundle = types.SimpleNamespace(gate_lora=mods[0], up_lora=mods[1], down_lora=mods[2])
    g = torch.randn(32, 256, device="cuda")
    for _ in range(2):  # two backward passes accumulate
        out = RoutedExpertsFunction.apply(h, W, I, L, "situ", None, bundle)
        out.backward(g)
    gh, gw, lg = k.routed_backward(h.detach(), I, W.detach(), L, g, act="situ", lora=mods)
    assert torch.equal(h.grad, 2 * gh) and torch.equal(W.grad, 2 * gw)
    for n, m in enumerate(mods):
        assert torch.equal(m.lora_A.grad, 2 * lg[2 * n]) and torch.equal(m.lora_B.grad, 2 * lg[2 * n + 1])


def test_no_tokens_and_argument_errors(k):
    case("LoRA: N = 0 gives zero adapter gradients; bad adapters are rejected")
    rng = np.random.default_rng(45)
    ex = oracle.random_experts(rng, 4, 64, 32, 119, 123)
    L = layer_of(ex)
    lo = oracle.random_lora(rng, 64, 32, 4)
    mods = adapters_of(lo)
    H = torch.zeros((0, 64), device="cuda")
    I = torch.zeros((0, 2), dtype=torch.int64, device="cuda")
    W = torch.zeros((0, 2), device="cuda")
    out = k.routed_forward(H, I, W, L, lora=mods)
    assert out.shape == (0, 64)
    gh, gw, lg = k.routed_backward(H, I, W, L, torch.zeros((0, 64), device="cuda"), lora=mods)
    assert all(t.shape == m.shape and not t.any() for t, m in
               zip(lg, [mods[0].lora_A, mods[0].lora_B, mods[1].lora_A, mods[1].lora_B, mods[2].lora_A,
                        mods[2].lora_B]))
    H1 = torch.zeros((2, 64), device="cuda")
    I1 = torch.zeros((2, 2), dtype=torch.int64, device="cuda")
    W1 = torch.zeros((2, 2), device="cuda")
    big = oracle.random_lora(rng, 64, 32, 33)
    with pytest.raises(ValueError):
        k.routed_forward(H1, I1, W1, L, lora=adapters_of(big))
    drop = adapters_of(lo)
    drop[0].dropout_rate = 0.1
    with pytest.raises(ValueError):
        k.routed_forward(H1, I1, W1, L, lora=drop)
    bad = adapters_of(lo)
    bad[2].lora_B = bad[2].lora_B[:, :2]
    with pytest.raises(ValueError):
        k.routed_forward(H1, I1, W1, L, lora=bad)
