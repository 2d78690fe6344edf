"""A seeded sweep of routed-layer configurations on the GPU against the float64 oracle
(oracle.routed_forward / routed_backward, which restate lazy_trainer.py:746-880 and, with LoRA,
lora_layer.py:104-139, :178-226).

Each configuration draws the hidden and FFN sizes (multiples of 32: some multiples of 512 and
256, where the layer's forward and backward layout copies apply, some not), the expert count,
tokens, top-k, activation, the activations' dtype, the LoRA rank (0 = off), which layout copies
the layer carries, and the routing: uniform, Zipf-skewed (large buckets, which take the grouped
work-groups) or top-1 with the tokens sorted by expert (whole waves of the routing kernel then
add to one expert's counter at once). The forward, the backward recomputing the forward and,
with LoRA, the six adapter gradients are held to the path's bar (rel-L2 <= 5e-3, cosine >=
0.9999); the backward reusing the forward's saved state must equal the recomputing one bit for
bit."""
import os
import types

import numpy as np
import pytest
import torch

import oracle
from tests.conftest import REL_L2_TOL, assert_close

pytestmark = pytest.mark.gpu

# LAZYLORA_SWEEP_SCALE=n draws n times as many cases of each kind (the first ones unchanged)
SCALE = max(1, int(os.environ.get("LAZYLORA_SWEEP_SCALE", "1")))
N_CONFIGS = 120 * SCALE


@pytest.fixture(scope="module")
def k():
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    from lazylora_amd.native import kernel
    return kernel()


def draw(i):
    rng = np.random.default_rng(7000 + i)
    E = int(rng.integers(1, 17))
    D = int(rng.choice([160, 256, 512, 544, 1024, 1056, 2048]))
    F = int(rng.choice([96, 128, 256, 352, 512, 608, 1024, 2048]))
    routing = str(rng.choice(["uniform", "uniform", "zipf", "sorted"]))
    n_max = 64 if D * F > (1 << 20) else 300  # the float64 oracle's time
    return dict(
        seed=7000 + i,
        D=D,
        F=F,
        E=E,
        topk=1 if routing == "sorted" else int(rng.integers(1, min(E, 8) + 1)),
        N=int(rng.integers(1, n_max + 1)),
        act=str(rng.choice(["swiglu", "situ"])),
        bf16=bool(rng.random() < 0.3),
        r=int(rng.choice([0, 0, 1, 8, 16, 32])),
        layouts=str(rng.choice(["none", "forward", "both"])),
        routing=routing,
    )


CONFIGS = [draw(i) for i in range(N_CONFIGS)]


def label(c):
    return (f"D{c['D']}-F{c['F']}-E{c['E']}-k{c['topk']}-N{c['N']}-{c['act']}-{'bf16' if c['bf16'] else 'f32'}"
            f"-r{c['r']}-{c['layouts']}-{c['routing']}")


def adapters_of(lo):
    return tuple(types.SimpleNamespace(lora_A=torch.from_numpy(np.asarray(A, np.float32)).cuda(),
                                       lora_B=torch.from_numpy(np.asarray(B, np.float32)).cuda(), scaling=s,
                                       dropout_rate=0.0) for A, B, s in lo.adapters())


def dot_scale(h, idx, ex, g, act, lo):
    """Per (token, slot): ||g_t|| * ||down_e(h_t)|| / sqrt(D), the size of the dot product
    grad_w[t, slot] = <g_t, down_e(h_t)> for unrelated vectors (float64; ids outside [0, E): 0)."""
    scale = np.zeros(idx.shape)
    D = h.shape[1]
    for e in np.unique(idx):
        if e < 0 or e >= ex.E:
            continue
        t, sl = np.nonzero(idx == e)
        W1, W3, W2 = ex.dense(int(e))
        x = np.asarray(h[t], np.float64)
        gate, up = x @ W1.T, x @ W3.T
        if lo is not None:
            (ag, bg, sg), (au, bu, su), _ = lo.adapters()
            gate, up = gate + oracle.lora_delta(x, ag, bg, sg), up + oracle.lora_delta(x, au, bu, su)
        a = oracle.glu_forward(gate, up, act)
        down = a @ W2.T
        if lo is not None:
            down = down + oracle.lora_delta(a, lo.down_A, lo.down_B, lo.down_s)
        scale[t, sl] = np.linalg.norm(np.asarray(g[t], np.float64), axis=1) * np.linalg.norm(down, axis=1) / np.sqrt(D)
    return scale


def assert_grad_w_close(got, want, scale, label):
    """grad_w at the path's bar, with the error measured against max(||want||, ||scale||): the
    error of a computed dot <g, down> is proportional to the dot's natural size ||g|| ||down|| /
    sqrt(D), not to its value, so where the dots cancel (a few slots whose <g, down> is much smaller
    than such dots usually are, e.g. one token at top-1) their relative error is no measure of the
    products' precision. For many slots ||want|| is about ||scale|| (the dots of unrelated vectors
    have that mean square), so this is the rel-L2 bar, checked with the cosine where ||want|| is
    the larger."""
    wn, sn = float(np.linalg.norm(want)), float(np.linalg.norm(scale))
    if wn >= sn:
        assert_close(got, want, label)
        return
    err = float(np.linalg.norm(np.asarray(got, np.float64) - want))
    print(f"{label}: cancelling dots (||want|| {wn:.3e}, ||scale|| {sn:.3e}): error / ||scale|| {err / sn:.3e}")
    assert np.all(np.isfinite(np.asarray(got))), f"{label}: non-finite values"
    assert err <= REL_L2_TOL * sn, f"{label}: error {err:.3e} > {REL_L2_TOL:.1e} x ||scale|| {sn:.3e}"


def lora_a_scales(h, idx, w, ex, g, act, lo):
    """Natural sizes (Frobenius norms) of the gate_A and up_A gradients, sum over tokens t of
    c_t (x) x_t with c_tj = s * sum over the token's pairs of <B[:, j], d_gate_p> (d_up for up_A,
    lora_layer.py:178-226): each such dot has the natural size s ||B[:, j]|| ||d_gate_p|| / sqrt(F),
    so an entry's is sqrt(sum_t (that for c_tj)^2 x_td^2). d_gate, d_up per pair in float64 as the
    routed backward makes them (ids outside [0, E) add nothing)."""
    N, D = h.shape
    F = ex.F
    sq = np.zeros((2, N))  # per token: sum over j of (natural size of c_tj)^2, gate and up
    Bn = [np.linalg.norm(np.asarray(B, np.float64), axis=0) for B in (lo.gate_B, lo.up_B)]
    for e in np.unique(idx):
        if e < 0 or e >= ex.E:
            continue
        t, sl = np.nonzero(idx == e)
        W1, W3, W2 = ex.dense(int(e))
        x = np.asarray(h[t], np.float64)
        gate = x @ W1.T + oracle.lora_delta(x, lo.gate_A, lo.gate_B, lo.gate_s)
        up = x @ W3.T + oracle.lora_delta(x, lo.up_A, lo.up_B, lo.up_s)
        a = oracle.glu_forward(gate, up, act)
        d_down = np.asarray(g[t], np.float64) * np.asarray(w[t, sl], np.float64)[:, None]
        d_act = d_down @ W2 + oracle.lora_gradients(d_down, a, lo.down_A, lo.down_B, lo.down_s)[2]
        d_gate, d_up = oracle.glu_backward(d_act, gate, up, act)
        for i, (dv, sc) in enumerate(((d_gate, lo.gate_s), (d_up, lo.up_s))):
            np.add.at(sq[i], t, sc * sc * float(np.sum(Bn[i] ** 2)) * np.sum(dv * dv, axis=1) / F)
    xn2 = np.sum(np.asarray(h, np.float64) ** 2, axis=1)
    return [float(np.sqrt(np.sum(sq[i] * xn2))) for i in range(2)]


def assert_scaled_close(got, want, scale, label):
    """The path's bar with the error measured against max(||want||, scale), scale the natural size
    of a result made of dot products: the error of a computed dot follows that size, not the dot's
    value, so where the dots cancel their relative error is no measure of the products' precision;
    for many terms ||want|| is about the scale and this is the rel-L2 bar, checked with the cosine
    where ||want|| is the larger."""
    wn = float(np.linalg.norm(want))
    if wn >= scale:
        assert_close(got, want, label)
        return
    err = float(np.linalg.norm(np.asarray(got, np.float64) - want))
    print(f"{label}: cancelling dots (||want|| {wn:.3e}, scale {scale:.3e}): error / scale {err / scale:.3e}")
    assert np.all(np.isfinite(np.asarray(got))), f"{label}: non-finite values"
    assert err <= REL_L2_TOL * scale, f"{label}: error {err:.3e} > {REL_L2_TOL:.1e} x scale {scale:.3e}"


@pytest.mark.parametrize("c", CONFIGS, ids=[label(c) for c in CONFIGS])
def test_routed_layer_config(k, c):
    print(f"\n[case] shape sweep {label(c)}", flush=True)
    from lazylora_amd.experts import ExpertLayer
    rng = np.random.default_rng(c["seed"])
    D, F, E, N, topk, act = c["D"], c["F"], c["E"], c["N"], c["topk"], c["act"]
    ex = oracle.random_experts(rng, E, D, F, 118, 122)
    if c["routing"] == "sorted":
        idx = np.sort(rng.integers(0, E, N)).astype(np.int64)[:, None]
        w = rng.uniform(0.5, 1.5, (N, 1)).astype(np.float32)
    else:
        logits = rng.standard_normal((N, E)).astype(np.float32)
        if c["routing"] == "zipf":
            logits = logits + oracle.zipf_offsets(rng, E)[None, :]
        idx, w = oracle.softmax_topk(logits, topk)
    h = rng.standard_normal((N, D)).astype(np.float32)
    g = rng.standard_normal((N, D)).astype(np.float32)
    lo = oracle.random_lora(rng, D, F, c["r"]) if c["r"] else None
    L = ExpertLayer(*[torch.from_numpy(np.ascontiguousarray(a)).cuda()
                      for a in (ex.w1p, ex.w1s, ex.w3p, ex.w3s, ex.w2p, ex.w2s)])
    if c["layouts"] in ("forward", "both"):
        L.prepare_forward_layout()
    if c["layouts"] == "both":
        L.prepare_backward_layout()
    H = torch.from_numpy(h).cuda()
    if c["bf16"]:
        H = H.bfloat16()
        h = H.float().cpu().numpy()
    I, W, G = (torch.from_numpy(a).cuda() for a in (idx, w, g))
    mods = adapters_of(lo) if lo else None
    ws = torch.empty(k.moe_workspace_bytes(N, topk, E, D, F), dtype=torch.uint8, device="cuda")
    out = k.routed_forward(H, I, W, L, act=act, save_for_backward=True, workspace=ws, lora=mods)
    reuse = k.routed_backward(H, I, W, L, G, act=act, reuse_forward=True, workspace=ws, lora=mods)
    rec = k.routed_backward(H, I, W, L, G, act=act, lora=mods)
    flat = lambda r: list(r[:2]) + (list(r[2]) if mods else [])
    for i, (a, b) in enumerate(zip(flat(reuse), flat(rec))):
        assert torch.equal(a, b), f"backward result {i}: reusing the forward differs from recomputing it"
    assert_close(out.cpu().numpy(), oracle.routed_forward(h, idx, w, ex, act, lora=lo), f"fwd {label(c)}")
    want = oracle.routed_backward(h, idx, w, ex, g, act, lora=lo)
    assert_close(rec[0].cpu().numpy(), want[0], f"grad_h {label(c)}")
    assert_grad_w_close(rec[1].cpu().numpy(), want[1], dot_scale(h, idx, ex, g, act, lo), f"grad_w {label(c)}")
    if mods:
        sa = dict(zip(("gate_A", "up_A"), lora_a_scales(h, idx, w, ex, g, act, lo)))
        for name, a, b in zip(("gate_A", "gate_B", "up_A", "up_B", "down_A", "down_B"), rec[2], want[2]):
            assert a.shape == b.shape, name
            if name in sa:
                assert_scaled_close(a.cpu().numpy(), b, sa[name], f"grad {name} {label(c)}")
            else:
                assert_close(a.cpu().numpy(), b, f"grad {name} {label(c)}")


def draw_product(i):
    rng = np.random.default_rng(9000 + i)
    return dict(seed=9000 + i, M=int(rng.integers(1, 300)), K=32 * int(rng.integers(1, 129)),
                R=int(rng.integers(1, 700)), lo=int(rng.integers(100, 125)))


PRODUCTS = [draw_product(i) for i in range(60 * SCALE)]


@pytest.mark.parametrize("c", PRODUCTS, ids=[f"M{c['M']}-K{c['K']}-R{c['R']}-s{c['lo']}" for c in PRODUCTS])
def test_products_config(k, clib, c):
    """mxfp4_gemm (y = x W^T, two-term e4m3 activations) and mxfp4_gemm_t (y = dy W, exact bf16
    weights, two bf16 terms of dy) at random shapes, scales 2^(lo-127) .. 2^(lo-123), against
    the C restatement of the reference's products (mxfp4_gemm.c:64-129)."""
    print(f"\n[case] product sweep M={c['M']} K={c['K']} R={c['R']}", flush=True)
    rng = np.random.default_rng(c["seed"])
    M, K, R = c["M"], c["K"], c["R"]
    p, s = oracle.random_mx(rng, (R, K), c["lo"], c["lo"] + 4)
    x = rng.standard_normal((M, K)).astype(np.float32)
    dy = rng.standard_normal((M, R)).astype(np.float32)
    P, S = torch.from_numpy(p).cuda(), torch.from_numpy(s).cuda()
    got = k.gemm(torch.from_numpy(x).cuda(), P, S).cpu().numpy()
    assert got.shape == (M, R)
    assert_close(got, clib.gemm(x, p, s), f"gemm {M}x{K}x{R}")
    got_t = k.gemm_t(torch.from_numpy(dy).cuda(), P, S).cpu().numpy()
    assert got_t.shape == (M, K)
    assert_close(got_t, clib.gemm_t(dy, p, s), f"gemm_t {M}x{K}x{R}", rel=2e-5, cos=0.99999999)


def draw_router(i):
    rng = np.random.default_rng(11000 + i)
    E = int(rng.choice([int(rng.integers(1, 129)), int(rng.integers(129, 1025)), int(rng.integers(1025, 4097))]))
    return dict(seed=11000 + i, N=int(rng.integers(1, 600)), E=E, top_k=int(rng.integers(1, min(E, 64) + 1)),
                renorm=bool(rng.random() < 0.7), scale=float(rng.choice([1.0, 2.5, 0.7])),
                bias=bool(rng.random() < 0.6))


ROUTERS = [draw_router(i) for i in range(40 * SCALE)]


@pytest.mark.parametrize("c", ROUTERS, ids=[f"N{c['N']}-E{c['E']}-k{c['top_k']}-{'renorm' if c['renorm'] else 'raw'}"
                                           f"-s{c['scale']}-{'bias' if c['bias'] else 'nobias'}" for c in ROUTERS])
def test_router_config(k, c):
    """mxfp4_router_topk and its backward at random widths (moe_router.py:55-135): indices exact
    where float64 leaves no near-tie (sets where it does), weights to 1e-5 relative, dL/dlogits
    to 1e-4 against oracle.router_select_backward at the kernel's own choice."""
    from tests.test_gpu_router import compare_selection
    print(f"\n[case] router sweep {c}", flush=True)
    rng = np.random.default_rng(c["seed"])
    N, E, top_k, scale, renorm = c["N"], c["E"], c["top_k"], c["scale"], c["renorm"]
    logits = (2.0 * rng.standard_normal((N, E))).astype(np.float32)
    bias = (0.05 * rng.standard_normal(E)).astype(np.float32) if c["bias"] else None
    Lg = torch.from_numpy(logits).cuda()
    idx, w = k.router_topk(Lg, torch.from_numpy(bias).cuda() if c["bias"] else None, top_k, scale, renorm)
    idx_h, w_h = idx.cpu().numpy(), w.cpu().numpy()
    assert idx_h.shape == (N, top_k) and ((idx_h >= 0) & (idx_h < E)).all()
    assert all(len(set(r)) == top_k for r in idx_h.tolist())
    # rows whose top k + 1 biased scores hold an fp32 near-tie are compared as sets (many, at wide
    # E and large k, where the scores crowd below 1); every other row index for index
    loose = compare_selection(idx_h, w_h, logits, bias, top_k, scale, renorm)
    print(f"rows compared as sets: {loose} of {N}")
    g = rng.standard_normal((N, top_k)).astype(np.float32)
    got = k.router_topk_backward(Lg, idx, torch.from_numpy(g).cuda(), scale, renorm).cpu().numpy()
    want = oracle.router_select_backward(logits, idx_h, g, scale, renorm)
    assert np.allclose(got, want, rtol=1e-4, atol=1e-7), np.abs(got - want).max()


def draw_block(i):
    rng = np.random.default_rng(13000 + i)
    E = int(rng.integers(2, 17))
    return dict(seed=13000 + i, H=int(rng.choice([128, 256, 384, 512])), Dl=32 * int(rng.integers(2, 17)),
                Fm=32 * int(rng.integers(1, 9)), E=E, top_k=int(rng.integers(1, min(E, 8) + 1)),
                Ds=32 * int(rng.integers(1, 5)), N=int(rng.integers(1, 97)),
                latent_norm=bool(rng.random() < 0.7), renorm=bool(rng.random() < 0.7),
                scale=float(rng.choice([1.0, 2.5])), r=int(rng.choice([0, 0, 4, 16])))


BLOCKS = [draw_block(i) for i in range(16 * SCALE)]


@pytest.mark.parametrize("c", BLOCKS, ids=[f"H{c['H']}-Dl{c['Dl']}-F{c['Fm']}-E{c['E']}-k{c['top_k']}-N{c['N']}"
                                          f"-norm{int(c['latent_norm'])}-renorm{int(c['renorm'])}-r{c['r']}"
                                          for c in BLOCKS])
def test_latent_block_config(k, c):
    """The latent MoE block (lazy_trainer.py:689-737: router, shared expert, latent down / up
    projections, routed MXFP4 experts with the layer's LoRA adapters, RMSNorm of the routed sum)
    at random widths against oracle.latent_moe_forward on the same MXFP4 bytes; the router's
    choice equal to the oracle's (row sets where float64 sees a near-tie)."""
    from tests.test_gpu_latent_moe import block_from
    print(f"\n[case] latent block sweep {c}", flush=True)
    rng = np.random.default_rng(c["seed"])
    H, Dl, Fm, E, Ds, N = c["H"], c["Dl"], c["Fm"], c["E"], c["Ds"], c["N"]
    ex = oracle.random_experts(rng, E, Dl, Fm, 121, 125)
    g = lambda *s: rng.standard_normal(s) * 0.05
    p = {"gate_weight": g(E, H), "e_score_correction_bias": g(E), "shared_w1_weight": g(Ds, H),
         "shared_w3_weight": g(Ds, H), "shared_w2_weight": g(H, Ds), "down_weight": g(Dl, H) * 4,
         "up_weight": g(H, Dl), "norm_weight": 1 + g(Dl), "top_k": c["top_k"], "routed_scale": c["scale"],
         "renorm": int(c["renorm"]), "latent_norm": int(c["latent_norm"]), "rms_eps": 1e-5, "hidden": H}
    lo = oracle.random_lora(rng, Dl, Fm, c["r"]) if c["r"] else None
    # the layer's adapter bundle, as the reference's LayerLoRABundle (routed adapters only)
    bundle = types.SimpleNamespace(**dict(zip(("gate_lora", "up_lora", "down_lora"), adapters_of(lo)))) if lo else None
    blk = block_from(p, ex, lora=bundle)
    x = rng.standard_normal((N, H))
    out, idx, w = blk.forward(torch.tensor(x, dtype=torch.float32, device="cuda"))
    want, idx64, w64 = oracle.latent_moe_forward(x.astype(np.float32), p, experts=ex, lora=lo)
    got_idx = idx.cpu().numpy()
    same = [sorted(a) == sorted(b) for a, b in zip(got_idx.tolist(), np.asarray(idx64).tolist())]
    assert sum(not s for s in same) <= max(1, N // 50), "router choices differ from the oracle"
    if all(same):
        assert_close(out.detach().cpu().numpy(), want, f"latent block {c}")
