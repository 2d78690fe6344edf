"""The routing's multi-launch path, against the float64 oracle (oracle.routed_forward /
routed_backward, restating lazy_trainer.py:746-880). Up to 65,536 (token, slot) pairs and 8,192
experts the routing runs in one work-group (counts, scan and placement with LDS atomics); past
either limit it runs as clears, a counting launch, a scan and a placement launch with device
atomics, whose bucket order differs. Both limits are crossed here, once each, with the workspace
filled with random bytes first, and the results compared with the oracle (forward, and the
backward recomputing the forward), and with ids outside [0, E) among the pairs."""
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


@pytest.mark.parametrize("E,D,F,N,topk,zipf", [
    (16, 256, 128, 9000, 8, False),   # 72,000 pairs
    (16, 256, 128, 8300, 8, True),    # 66,400 pairs, large buckets
    (8200, 64, 32, 300, 4, False),    # 8,200 experts
])
def test_multi_launch_routing(k, E, D, F, N, topk, zipf):
    from lazylora_amd.experts import ExpertLayer
    print(f"\n[case] multi-launch routing E={E} D={D} F={F} N={N} top-{topk} {'zipf' if zipf else 'uniform'}",
          flush=True)
    rng = np.random.default_rng(E + N + topk)
    ex = oracle.random_experts(rng, E, D, F, 118, 122)
    L = ExpertLayer(*[torch.from_numpy(np.ascontiguousarray(a)).cuda()
                      for a in (ex.w1p, ex.w1s, ex.w3p, ex.w3s, ex.w2p, ex.w2s)])
    logits = rng.standard_normal((N, E)).astype(np.float32)
    if zipf:
        logits = logits + oracle.zipf_offsets(rng, E)[None, :]
    idx, w = oracle.softmax_topk(logits, topk)
    bad = rng.random(idx.shape) < 0.01
    idx = np.where(bad, rng.choice([-1, E], idx.shape), idx)
    h = rng.standard_normal((N, D)).astype(np.float32)
    g = rng.standard_normal((N, D)).astype(np.float32)
    H, I, W, G = (torch.from_numpy(a).cuda() for a in (h, idx, w, g))
    ws = torch.empty(k.moe_workspace_bytes(N, topk, E, D, F), dtype=torch.uint8, device="cuda")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(N)
    ws.random_(0, 256, generator=gen)
    out = k.routed_forward(H, I, W, L, workspace=ws)
    assert k.route_status(ws) & 1  # the invalid ids were seen
    ws.random_(0, 256, generator=gen)
    gh, gw = k.routed_backward(H, I, W, L, G, workspace=ws)
    keep = np.where(bad, 0, idx)
    wk = np.where(bad, 0.0, w).astype(np.float32)
    assert_close(out.cpu().numpy(), oracle.routed_forward(h, keep, wk, ex, "swiglu"), "fwd")
    want = oracle.routed_backward(h, keep, wk, ex, g, "swiglu")
    assert_close(gh.cpu().numpy(), want[0], "grad_h")
    gwn = gw.cpu().numpy()
    assert np.all(gwn[bad] == 0.0)
    assert_close(np.where(bad, 0.0, gwn), np.where(bad, 0.0, want[1]), "grad_w")
    del L
    torch.cuda.empty_cache()
