"""A seeded sweep of routed-layer configurations on the GPU against the float64 oracle
(oracle.routed_forward / routed_backward, which restate lazy_trainer.py:746-880 and, with LoRA,
lora_layer.py:104-139, :178-226).

Each configuration draws the hidden and FFN sizes (multiples of 32: some multiples of 512 and
256, where the layer's forward and backward layout copies apply, some not), the expert count,
tokens, top-k, activation, the activations' dtype, the LoRA rank (0 = off), which layout copies
the layer carries, and uniform or Zipf-skewed routing (the latter makes large buckets, which take
the grouped work-groups). The forward, the backward recomputing the forward and, with LoRA, the
six adapter gradients are held to the path's bar (rel-L2 <= 5e-3, cosine >= 0.9999); the
backward reusing the forward's saved state must equal the recomputing one bit for bit."""
import types

import numpy as np
import pytest
import torch

import oracle
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu

N_CONFIGS = 20


@pytest.fixture(scope="module")
def k():
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    from lazylora_amd.native import kernel
    return kernel()


def draw(i):
    rng = np.random.default_rng(7000 + i)
    E = int(rng.integers(1, 13))
    return dict(
        seed=7000 + i,
        D=int(rng.choice([256, 512, 544, 1024, 1056])),
        F=int(rng.choice([128, 256, 352, 512, 1024])),
        E=E,
        topk=int(rng.integers(1, min(E, 8) + 1)),
        N=int(rng.integers(1, 193)),
        act=str(rng.choice(["swiglu", "situ"])),
        bf16=bool(rng.random() < 0.3),
        r=int(rng.choice([0, 0, 1, 8, 16, 32])),
        layouts=str(rng.choice(["none", "forward", "both"])),
        zipf=bool(rng.random() < 0.4),
    )


CONFIGS = [draw(i) for i in range(N_CONFIGS)]


def label(c):
    return (f"D{c['D']}-F{c['F']}-E{c['E']}-k{c['topk']}-N{c['N']}-{c['act']}-{'bf16' if c['bf16'] else 'f32'}"
            f"-r{c['r']}-{c['layouts']}-{'zipf' if c['zipf'] else 'uniform'}")


def adapters_of(lo):
    return tuple(types.SimpleNamespace(lora_A=torch.from_numpy(np.asarray(A, np.float32)).cuda(),
                                       lora_B=torch.from_numpy(np.asarray(B, np.float32)).cuda(), scaling=s,
                                       dropout_rate=0.0) for A, B, s in lo.adapters())


@pytest.mark.parametrize("c", CONFIGS, ids=[label(c) for c in CONFIGS])
def test_routed_layer_config(k, c):
    print(f"\n[case] shape sweep {label(c)}", flush=True)
    from lazylora_amd.experts import ExpertLayer
    rng = np.random.default_rng(c["seed"])
    D, F, E, N, topk, act = c["D"], c["F"], c["E"], c["N"], c["topk"], c["act"]
    ex = oracle.random_experts(rng, E, D, F, 118, 122)
    logits = rng.standard_normal((N, E)).astype(np.float32)
    if c["zipf"]:
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
    assert_close(rec[1].cpu().numpy(), want[1], f"grad_w {label(c)}")
    if mods:
        for name, a, b in zip(("gate_A", "gate_B", "up_A", "up_B", "down_A", "down_B"), rec[2], want[2]):
            assert a.shape == b.shape, name
            assert_close(a.cpu().numpy(), b, f"grad {name} {label(c)}")
