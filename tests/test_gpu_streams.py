"""The library launches on the caller's stream (torch's current stream, passed as the hipStream_t
of every entry point in include/lazylora_mxfp4.h). Each call below runs on a second stream
(default priority) whose inputs are produced on that stream right before the call, behind a long
chain of unrelated work, without any synchronisation; a launch on another stream would read them
before they are written. Results must equal the default stream's bit for bit. Two calls
interleaved on two streams must also give what each gives alone (no kernel waits on another
work-group, and each call's counters and queues live in its own workspace)."""
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


def test_concurrent_calls_on_two_streams(k):
    """Two routed layers' forward and backward (each with its own workspace; one with large buckets,
    so its resident grouped work-groups and work queues share the GPU with the other call's
    kernels) interleaved on two streams with no synchronisation between them, three times over:
    every result equals the same call made alone."""
    from lazylora_amd.experts import ExpertLayer
    print("\n[case] two routed calls interleaved on two streams", flush=True)
    rng = np.random.default_rng(503)
    jobs = []
    for E, D, F, N, topk, skew in ((8, 1024, 512, 160, 2, True), (16, 512, 256, 200, 4, False)):
        ex = oracle.random_experts(rng, E, D, F, 118, 122)
        L = ExpertLayer(*[torch.from_numpy(np.ascontiguousarray(a)).cuda()
                          for a in (ex.w1p, ex.w1s, ex.w3p, ex.w3s, ex.w2p, ex.w2s)])
        L.prepare_forward_layout()
        logits = rng.standard_normal((N, E)).astype(np.float32)
        if skew:
            logits = logits + oracle.zipf_offsets(rng, E)[None, :]
        idx, w = oracle.softmax_topk(logits, topk)
        t = [torch.from_numpy(a).cuda() for a in (rng.standard_normal((N, D)).astype(np.float32), idx, w,
                                                  rng.standard_normal((N, D)).astype(np.float32))]
        ws = torch.empty(k.moe_workspace_bytes(N, topk, E, D, F), dtype=torch.uint8, device="cuda")
        jobs.append((L, t, ws))

    def run(L, t, ws):
        H, I, W, G = t
        out = k.routed_forward(H, I, W, L, save_for_backward=True, workspace=ws)
        gh, gw = k.routed_backward(H, I, W, L, G, reuse_forward=True, workspace=ws)
        return out, gh, gw

    alone = [run(*j) for j in jobs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    for _ in range(3):
        got = [None, None]
        for i in (0, 1):
            with torch.cuda.stream(streams[i]):
                got[i] = run(*jobs[i])
        for s in streams:
            torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        for a, b in zip(got, alone):
            assert all(torch.equal(x, y) for x, y in zip(a, b))
