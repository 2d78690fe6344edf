"""Packed checkpoint -> HBM, and layer streaming through a ring of HBM slots, on the GPU.

The loader's HBM bytes must equal the checkpoint's bytes, and the routed layer computed on them
must match the float64 oracle built from the same arrays. Streaming must give, layer by layer,
exactly the results of computing each layer from its own resident copy: any slot refilled
before the compute stream has finished reading it would show as a difference."""
import numpy as np
import pytest
import torch
from safetensors.numpy import save_file

import oracle
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def k():
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    from lazylora_amd.native import kernel
    return kernel()


def case(msg):
    print(f"\n[case] {msg}", flush=True)


def test_checkpoint_to_hbm_and_routed_forward(k, tmp_path):
    case("safetensors shards -> pinned -> HBM -> routed forward")
    from lazylora_amd.loader import EXPERT_TENSORS, PackedLayerReader, expert_tensor_name
    rng = np.random.default_rng(51)
    E, D, F, L = 12, 512, 256, 7
    ex = oracle.random_experts(rng, E, D, F, 119, 123)
    arrays = (ex.w1p, ex.w1s, ex.w3p, ex.w3s, ex.w2p, ex.w2s)
    shards = [{}, {}, {}]
    for e in rng.permutation(E):
        for suffix, slot in EXPERT_TENSORS:
            shards[e % 3][expert_tensor_name(L, int(e), suffix)] = np.ascontiguousarray(arrays[slot][e])
    for i, sh in enumerate(shards):
        save_file(sh, str(tmp_path / f"model-0000{i + 1}-of-00003.safetensors"))
    r = PackedLayerReader(str(tmp_path), threads=4)
    layer = r.load_layer(L)
    assert (layer.E, layer.D, layer.F) == (E, D, F)
    for got, want in zip(layer.tensors(), arrays):
        assert np.array_equal(got.cpu().numpy(), want)
    N, topk = 80, 4
    h = rng.standard_normal((N, D)).astype(np.float32)
    idx, w = oracle.softmax_topk(rng.standard_normal((N, E)).astype(np.float32), topk)
    out = k.routed_forward(torch.from_numpy(h).cuda(), torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda(),
                           layer, act="situ")
    assert_close(out.cpu().numpy(), oracle.routed_forward(h, idx, w, ex, "situ"), "loaded layer fwd")
    # only some experts: the rest of HBM is left alone
    part = r.load_layer(L, expert_ids=[3, 4, 5, 9])
    for got, want in zip(part.tensors(), arrays):
        assert np.array_equal(got[3:6].cpu().numpy(), want[3:6]) and np.array_equal(got[9].cpu().numpy(), want[9])
    r.close()


def make_hosts(rng, n, E, D, F):
    from lazylora_amd.experts import ExpertLayer
    from lazylora_amd.streaming import host_layer_from
    hosts, resident = [], []
    for _ in range(n):
        ex = oracle.random_experts(rng, E, D, F, 118, 123)
        t = [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (ex.w1p, ex.w1s, ex.w3p, ex.w3s, ex.w2p, ex.w2s)]
        layer = ExpertLayer(*t)
        resident.append(layer)
        hosts.append(host_layer_from(layer, pin=True))
    return hosts, resident


@pytest.mark.parametrize("slots", [2, 3])
def test_streamed_layers_equal_resident_layers(k, slots):
    case(f"LayerStreamer, {slots} slots, 6 layers, fwd+bwd per layer")
    from lazylora_amd.streaming import LayerStreamer
    rng = np.random.default_rng(52 + slots)
    E, D, F, N, topk = 16, 512, 256, 96, 4
    hosts, resident = make_hosts(rng, 3, E, D, F)
    order = [0, 1, 2, 1, 0, 2]  # host layers reused, as in a ring
    H = torch.from_numpy(rng.standard_normal((N, D)).astype(np.float32)).cuda()
    G = torch.from_numpy(rng.standard_normal((N, D)).astype(np.float32)).cuda()
    idx, w = oracle.softmax_topk(rng.standard_normal((N, E)).astype(np.float32), topk)
    I, W = torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda()
    want = [(k.routed_forward(H, I, W, resident[j]), *k.routed_backward(H, I, W, resident[j], G)) for j in order]
    s = LayerStreamer(E, D, F, slots=slots, timing=True)
    got = []
    for i, layer in s.stream(hosts[j] for j in order):
        got.append((k.routed_forward(H, I, W, layer), *k.routed_backward(H, I, W, layer, G)))
    torch.cuda.synchronize()
    assert len(got) == len(order)
    for a, b in zip(got, want):
        for x, y in zip(a, b):
            assert torch.equal(x, y)
    ms, nbytes = s.copy_stats()
    assert nbytes == len(order) * hosts[0].nbytes and ms > 0


def test_streaming_only_active_experts(k):
    case("LayerStreamer copying only each layer's active experts")
    from lazylora_amd.streaming import LayerStreamer
    rng = np.random.default_rng(60)
    E, D, F, N, topk = 32, 256, 128, 40, 2
    hosts, resident = make_hosts(rng, 2, E, D, F)
    H = torch.from_numpy(rng.standard_normal((N, D)).astype(np.float32)).cuda()
    routes = []
    for _ in range(4):
        logits = rng.standard_normal((N, E)).astype(np.float32)
        logits[:, : E // 2] -= 50.0  # only the upper half of the experts can be chosen
        routes.append(oracle.softmax_topk(logits, topk))
    order = [0, 1, 1, 0]
    s = LayerStreamer(E, D, F, slots=2)
    ids = [sorted(set(r[0].ravel().tolist())) for r in routes]
    for i, layer in s.stream((hosts[j] for j in order), expert_ids=ids):
        idx, w = routes[i]
        I, W = torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda()
        out = k.routed_forward(H, I, W, layer)
        assert torch.equal(out, k.routed_forward(H, I, W, resident[order[i]]))
    assert s.bytes_copied == sum(len(x) for x in ids) * hosts[0].nbytes // E
