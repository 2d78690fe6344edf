"""The library launches on the caller's stream (torch's current stream, passed as the hipStream_t
of every entry point in include/lazylora_mxfp4.h). Each call below runs on a second stream
(default priority) whose inputs are produced on that stream right before the call, behind a long
chain of unrelated work, without any synchronisation; a launch on another stream would read them
before they are written. Results must equal the default stream's bit for bit."""
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


def busy(n=24):
    """Work queued on the current stream ahead of the inputs (a few ms of fp32 products)."""
    a = torch.randn(2048, 2048, device="cuda")
    for _ in range(n):
        a = torch.tanh(a @ a * 1e-3)
    return a


def made_late(t):
    """t rewritten on the current stream after busy(): the copy lands only when busy() ends."""
    out = torch.empty_like(t)
    z = busy()[0, 0] * 0
    out.copy_(t + z.to(t.dtype))
    return out


def adapters_of(lo):
    return tuple(types.SimpleNamespace(lora_A=torch.from_numpy(np.asarray(A, np.float32)).cuda(),
                                       lora_B=torch.from_numpy(np.asarray(B, np.float32)).cuda(), scaling=s,
                                       dropout_rate=0.0) for A, B, s in lo.adapters())


def test_routed_layer_on_a_side_stream(k):
    from lazylora_amd.experts import ExpertLayer
    print("\n[case] routed forward/backward with LoRA r=8 on a side stream", flush=True)
    rng = np.random.default_rng(501)
    E, D, F, N, topk = 8, 1024, 512, 96, 2
    ex = oracle.random_experts(rng, E, D, F, 118, 122)
    L = ExpertLayer(*[torch.from_numpy(np.ascontiguousarray(a)).cuda()
                      for a in (ex.w1p, ex.w1s, ex.w3p, ex.w3s, ex.w2p, ex.w2s)])
    logits = rng.standard_normal((N, E)).astype(np.float32)
    logits[:60] += 4 * (np.arange(E) == 3)  # one bucket above 48 rows: grouped work-groups too
    idx, w = oracle.softmax_topk(logits, topk)
    H, I, W, G = (torch.from_numpy(a).cuda() for a in (rng.standard_normal((N, D)).astype(np.float32), idx, w,
                                                       rng.standard_normal((N, D)).astype(np.float32)))
    mods = adapters_of(oracle.random_lora(rng, D, F, 8))
    L.prepare_forward_layout()
    L.prepare_backward_layout()
    want_out = k.routed_forward(H, I, W, L, lora=mods)
    want = k.routed_backward(H, I, W, L, G, lora=mods)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        h2, i2, w2, g2 = made_late(H), made_late(I), made_late(W), made_late(G)
        out = k.routed_forward(h2, i2, w2, L, lora=mods)
        got = k.routed_backward(h2, i2, w2, L, g2, lora=mods)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(out, want_out)
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
    for a, b in zip(got[2], want[2]):
        assert torch.equal(a, b)


def test_layouts_and_products_on_a_side_stream(k):
    from lazylora_amd.experts import ExpertLayer
    print("\n[case] layout copies, mxfp4_gemm and mxfp4_gemm_t on a side stream", flush=True)
    rng = np.random.default_rng(502)
    M, K, R = 40, 7168, 2048
    pk = torch.from_numpy(rng.integers(0, 256, (R, K // 2), dtype=np.uint8)).cuda()
    sc = torch.from_numpy(rng.integers(118, 123, (R, K // 32), dtype=np.uint8)).cuda()
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda()
    dy = torch.from_numpy(rng.standard_normal((M, R)).astype(np.float32)).cuda()
    want_y, want_yt = k.gemm(x, pk, sc), k.gemm_t(dy, pk, sc)
    # a layer whose layout copies are built on the side stream from codes written there
    E, D, F, N = 4, 512, 256, 48
    ex = oracle.random_experts(rng, E, D, F, 118, 122)
    parts = [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (ex.w1p, ex.w1s, ex.w3p, ex.w3s, ex.w2p,
                                                                         ex.w2s)]
    idx, w = oracle.softmax_topk(rng.standard_normal((N, E)).astype(np.float32), 2)
    H, I, W = (torch.from_numpy(a).cuda() for a in (rng.standard_normal((N, D)).astype(np.float32), idx, w))
    want_out = k.routed_forward(H, I, W, ExpertLayer(*parts))
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        y = k.gemm(made_late(x), made_late(pk), made_late(sc))
        yt = k.gemm_t(made_late(dy), pk, sc)
        L = ExpertLayer(*[made_late(p) for p in parts])
        L.prepare_forward_layout()
        L.prepare_backward_layout()
        out = k.routed_forward(H, I, W, L)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(y, want_y) and torch.equal(yt, want_yt)
    assert torch.equal(out, want_out)
