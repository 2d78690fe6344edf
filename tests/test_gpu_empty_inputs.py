"""Empty and all-skipped inputs on the GPU. The reference's torch composition
(lazy_trainer.py:746-880) gives empty outputs for no tokens and zero rows for tokens whose slots
select nothing; mxfp4_gemm / mxfp4_gemm_t (mxfp4_gemm.c:64-129) with M = 0 write nothing. Here:
no rows for the products; no tokens for the routed layer, with and without LoRA (the adapter
gradients are then zero); and every id outside [0, E), top-1 (whose down product writes token
rows directly, the unrouted ones zeroed) and top-3, with the outputs starting as garbage."""
import types

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


def layer(rng, E, D, F):
    from lazylora_amd.experts import ExpertLayer
    ex = oracle.random_experts(rng, E, D, F, 118, 122)
    return ExpertLayer(*[torch.from_numpy(np.ascontiguousarray(a)).cuda()
                         for a in (ex.w1p, ex.w1s, ex.w3p, ex.w3s, ex.w2p, ex.w2s)])


def adapters(rng, D, F, r):
    lo = oracle.random_lora(rng, D, F, r)
    return tuple(types.SimpleNamespace(lora_A=torch.from_numpy(np.asarray(A, np.float32)).cuda(),
                                       lora_B=torch.from_numpy(np.asarray(B, np.float32)).cuda(), scaling=s,
                                       dropout_rate=0.0) for A, B, s in lo.adapters())


def test_products_with_no_rows(k):
    print("\n[case] mxfp4_gemm / mxfp4_gemm_t with M = 0", flush=True)
    rng = np.random.default_rng(601)
    pk = torch.from_numpy(rng.integers(0, 256, (96, 256), dtype=np.uint8)).cuda()
    sc = torch.from_numpy(rng.integers(118, 123, (96, 16), dtype=np.uint8)).cuda()
    y = k.gemm(torch.empty((0, 512), device="cuda"), pk, sc)
    assert y.shape == (0, 96)
    yt = k.gemm_t(torch.empty((0, 96), device="cuda"), pk, sc)
    assert yt.shape == (0, 512)


@pytest.mark.parametrize("r", [0, 8])
def test_routed_layer_with_no_tokens(k, r):
    print(f"\n[case] routed layer with N = 0, LoRA rank {r}", flush=True)
    rng = np.random.default_rng(602 + r)
    E, D, F, topk = 6, 512, 256, 2
    L = layer(rng, E, D, F)
    mods = adapters(rng, D, F, r) if r else None
    H = torch.empty((0, D), device="cuda")
    I = torch.empty((0, topk), dtype=torch.int64, device="cuda")
    W = torch.empty((0, topk), device="cuda")
    G = torch.empty((0, D), device="cuda")
    out = k.routed_forward(H, I, W, L, lora=mods, save_for_backward=False)
    assert out.shape == (0, D)
    res = k.routed_backward(H, I, W, L, G, lora=mods)
    assert res[0].shape == (0, D) and res[1].shape == (0, topk)
    if r:
        assert len(res[2]) == 6
        for a, m in zip(res[2], (m for ad in mods for m in (ad.lora_A, ad.lora_B))):
            assert a.shape == m.shape and torch.count_nonzero(a) == 0


@pytest.mark.parametrize("topk,r", [(1, 0), (3, 0), (3, 8)])
def test_every_id_outside_the_layer(k, topk, r):
    print(f"\n[case] routed layer with every id outside [0, E), top-{topk}, LoRA rank {r}", flush=True)
    rng = np.random.default_rng(610 + topk + r)
    E, D, F, N = 6, 512, 256, 37
    L = layer(rng, E, D, F)
    mods = adapters(rng, D, F, r) if r else None
    H = torch.from_numpy(rng.standard_normal((N, D)).astype(np.float32)).cuda()
    G = torch.from_numpy(rng.standard_normal((N, D)).astype(np.float32)).cuda()
    I = torch.from_numpy(rng.choice([-1, E, E + 9], (N, topk)).astype(np.int64)).cuda()
    W = torch.from_numpy(rng.uniform(0.2, 1.0, (N, topk)).astype(np.float32)).cuda()
    ws = torch.empty(k.moe_workspace_bytes(N, topk, E, D, F), dtype=torch.uint8, device="cuda").fill_(0x7F)
    out = k.routed_forward(H, I, W, L, lora=mods, save_for_backward=True, workspace=ws)
    assert k.route_status(ws) & 1
    assert torch.count_nonzero(out) == 0
    res = k.routed_backward(H, I, W, L, G, lora=mods, reuse_forward=True, workspace=ws)
    assert torch.count_nonzero(res[0]) == 0 and torch.count_nonzero(res[1]) == 0
    if r:
        for a in res[2]:
            assert torch.count_nonzero(a) == 0
