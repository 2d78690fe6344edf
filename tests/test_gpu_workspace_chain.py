"""One routed-layer workspace shared by a chain of different calls, against the float64 oracle
(oracle.routed_forward / routed_backward, restating lazy_trainer.py:746-880 and, with LoRA,
lora_layer.py:104-139, :178-226).

The workspace is caller-owned scratch with no initial contents promised (mxfp4_moe_workspace_size
in include/lazylora_mxfp4.h): before every forward/backward pair it is filled with random bytes,
so a routing count, work-queue counter, third-term flag or adapter partial that a call relied on
finding zeroed, or left over from the call before, would show here. Per layer the calls vary
tokens, top-k, routing (uniform, Zipf-skewed, top-1 sorted by expert), activation, the
activations' dtype and the LoRA rank, and some calls carry ids outside [0, E), which contribute
nothing (their grad_w slots are 0). The backward reuses the forward's saved state from the
same workspace."""
import types

import numpy as np
import pytest
import torch

import oracle
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu

LAYERS = [  # D, F, E, layout copies, tokens at most, calls
    (1024, 512, 8, "both", 160, 10),
    (544, 352, 6, "forward", 160, 10),
    (2048, 1024, 12, "both", 64, 8),
    (256, 96, 5, "none", 200, 10),
]
K_MAX = 4


@pytest.fixture(scope="module")
def k():
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    from lazylora_amd.native import kernel
    return kernel()


def adapters_of(lo):
    return tuple(types.SimpleNamespace(lora_A=torch.from_numpy(np.asarray(A, np.float32)).cuda(),
                                       lora_B=torch.from_numpy(np.asarray(B, np.float32)).cuda(), scaling=s,
                                       dropout_rate=0.0) for A, B, s in lo.adapters())


def routing(rng, N, E, topk, kind):
    if kind == "sorted":
        idx = np.sort(rng.integers(0, E, N)).astype(np.int64)[:, None]
        return idx, rng.uniform(0.5, 1.5, (N, 1)).astype(np.float32)
    logits = rng.standard_normal((N, E)).astype(np.float32)
    if kind == "zipf":
        logits = logits + oracle.zipf_offsets(rng, E)[None, :]
    return oracle.softmax_topk(logits, topk)


@pytest.mark.parametrize("D,F,E,layouts,n_max,calls", LAYERS,
                         ids=[f"D{l[0]}-F{l[1]}-E{l[2]}-{l[3]}" for l in LAYERS])
def test_workspace_chain(k, D, F, E, layouts, n_max, calls):
    from lazylora_amd.experts import ExpertLayer
    rng = np.random.default_rng(D * 7 + F * 3 + E)
    ex = oracle.random_experts(rng, E, D, F, 118, 122)
    L = ExpertLayer(*[torch.from_numpy(np.ascontiguousarray(a)).cuda()
                      for a in (ex.w1p, ex.w1s, ex.w3p, ex.w3s, ex.w2p, ex.w2s)])
    if layouts in ("forward", "both"):
        L.prepare_forward_layout()
    if layouts == "both":
        L.prepare_backward_layout()
    ws = torch.empty(k.moe_workspace_bytes(n_max, K_MAX, E, D, F), dtype=torch.uint8, device="cuda")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(D + F + E)
    for call in range(calls):
        N = int(rng.integers(1, n_max + 1))
        kind = str(rng.choice(["uniform", "uniform", "zipf", "sorted"]))
        topk = 1 if kind == "sorted" else int(rng.integers(1, min(E, K_MAX) + 1))
        act = str(rng.choice(["swiglu", "situ"]))
        bf16 = bool(rng.random() < 0.3)
        r = int(rng.choice([0, 0, 8, 16]))
        idx, w = routing(rng, N, E, topk, kind)
        bad = np.zeros(idx.shape, bool)
        if r == 0 and rng.random() < 0.5:  # some slots with ids outside [0, E)
            bad = rng.random(idx.shape) < 0.08
            idx = np.where(bad, rng.choice([-1, E, E + 5], idx.shape), idx)
        name = (f"D{D}-F{F}-E{E}-{layouts} call {call}: N={N} k={topk} {kind} {act} "
                f"{'bf16' if bf16 else 'f32'} r={r} invalid={int(bad.sum())}")
        print(f"\n[case] workspace chain {name}", flush=True)
        h = rng.standard_normal((N, D)).astype(np.float32)
        g = rng.standard_normal((N, D)).astype(np.float32)
        lo = oracle.random_lora(rng, D, F, r) if r else None
        H = torch.from_numpy(h).cuda()
        if bf16:
            H = H.bfloat16()
            h = H.float().cpu().numpy()
        I, W, G = (torch.from_numpy(a).cuda() for a in (idx, w, g))
        mods = adapters_of(lo) if lo else None
        ws.random_(0, 256, generator=gen)  # no contents carried into the pair
        out = k.routed_forward(H, I, W, L, act=act, save_for_backward=True, workspace=ws, lora=mods)
        res = k.routed_backward(H, I, W, L, G, act=act, reuse_forward=True, workspace=ws, lora=mods)
        # the oracle sees an invalid slot as expert 0 with weight 0: no term in out or grad_h
        keep = np.where(bad, 0, idx)
        wk = np.where(bad, 0.0, w).astype(np.float32)
        assert_close(out.cpu().numpy(), oracle.routed_forward(h, keep, wk, ex, act, lora=lo), f"fwd {name}")
        want = oracle.routed_backward(h, keep, wk, ex, g, act, lora=lo)
        assert_close(res[0].cpu().numpy(), want[0], f"grad_h {name}")
        gw = res[1].cpu().numpy()
        assert np.all(gw[bad] == 0.0), f"grad_w of invalid slots {name}"
        assert_close(np.where(bad, 0.0, gw), np.where(bad, 0.0, want[1]), f"grad_w {name}")
        if mods:
            for nm, a, b in zip(("gate_A", "gate_B", "up_A", "up_B", "down_A", "down_B"), res[2], want[2]):
                assert_close(a.cpu().numpy(), b, f"grad {nm} {name}")
    del L
    torch.cuda.empty_cache()


@pytest.mark.parametrize("M,K,R", [(1, 7168, 2048), (37, 1024, 96), (256, 7168, 2048), (70, 544, 352)])
def test_product_workspaces_hold_no_state(k, M, K, R):
    """mxfp4_gemm and mxfp4_gemm_t with their workspaces filled with random bytes give the same
    bits as with fresh ones (the workspace holds the activation tiles, written before they are
    read)."""
    from lazylora_amd.native import _stream
    print(f"\n[case] product workspaces filled with random bytes, M={M} K={K} R={R}", flush=True)
    rng = np.random.default_rng(M + K + R)
    pk = torch.from_numpy(rng.integers(0, 256, (R, K // 2), dtype=np.uint8)).cuda()
    sc = torch.from_numpy(rng.integers(118, 123, (R, K // 32), dtype=np.uint8)).cuda()
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda()
    dy = torch.from_numpy(rng.standard_normal((M, R)).astype(np.float32)).cuda()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(M * K + R)
    dev = x.device
    for _ in range(2):
        nws = k.lib.mxfp4_gemm_workspace_size(M, K, R)
        ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=dev).random_(0, 256, generator=gen)
        y = torch.empty((M, R), dtype=torch.float32, device=dev)
        assert k.lib.mxfp4_gemm(y.data_ptr(), x.data_ptr(), pk.data_ptr(), sc.data_ptr(), M, K, R, ws.data_ptr(),
                                nws, _stream(dev)) == 0
        assert torch.equal(y, k.gemm(x, pk, sc))
        nws = k.lib.mxfp4_gemm_t_workspace_size(M, K, R)
        ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=dev).random_(0, 256, generator=gen)
        yt = torch.zeros((M, K), dtype=torch.float32, device=dev)
        assert k.lib.mxfp4_gemm_t(yt.data_ptr(), dy.data_ptr(), pk.data_ptr(), sc.data_ptr(), M, K, R,
                                  ws.data_ptr(), nws, _stream(dev)) == 0
        assert torch.equal(yt, k.gemm_t(dy, pk, sc))
