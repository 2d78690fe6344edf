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


def _random_layer_into(layer, seed):
    """Fill an HBM layer with seeded MXFP4 bytes (codes uniform, scales 117..121: the config-2
    weights) on the GPU; the same seed always gives the same bytes."""
    gen = torch.Generator(device=layer.device)
    gen.manual_seed(seed)
    for t, is_scale in zip(layer.tensors(), (False, True, False, True, False, True)):
        if is_scale:
            t.random_(117, 122, generator=gen)
        else:
            t.random_(0, 256, generator=gen)
    return layer


def test_config5_full_size_stream(k, clib):
    """BASELINE config 5 at its real size: four distinct 896-expert layers of the config-2 shape
    (20.96 GB each) streamed through LayerStreamer's two HBM slots from a ring of two pinned
    host layers (expert_streamer.py:315-369 at layer granularity). Each streamed layer's forward
    for 1024 tokens (top-8) must equal, bit for bit, the forward of the same layer regenerated
    from its seed in HBM, and the first layer's whole forward must match the C restatement."""
    from lazylora_amd.experts import ExpertLayer
    from lazylora_amd.loader import HostLayer
    from lazylora_amd.streaming import LayerStreamer
    E, D, F, N, topk, n_layers = 896, 7168, 2048, 1024, 8, 4
    seeds = [501 + 17 * i for i in range(n_layers)]
    case("config 5: allocating 2 pinned host layers + 3 HBM layers (~105 GB)")
    ring = [HostLayer(E, D, F, pin=True) for _ in range(2)]
    scratch = ExpertLayer.empty(E, D, F)
    streamer = LayerStreamer(E, D, F, slots=2, timing=True)
    rng = np.random.default_rng(61)
    h = rng.standard_normal((N, D)).astype(np.float32)
    idx, w = oracle.softmax_topk(rng.standard_normal((N, E)).astype(np.float32), topk)
    H, I, W = (torch.from_numpy(a).cuda() for a in (h, idx, w))

    def host_layers():
        for i, seed in enumerate(seeds):
            torch.cuda.synchronize()  # every earlier copy out of this ring slot has completed
            _random_layer_into(scratch, seed)
            host = ring[i % 2]
            for src, dst in zip(scratch.tensors(), host.tensors):
                dst.copy_(src)
            print(f"[config5] host slot {i % 2} <- layer {i} (seed {seed})", flush=True)
            yield host

    n_seen = 0
    for i, layer in streamer.stream(host_layers()):
        out = k.routed_forward(H, I, W, layer)
        if i == 0:  # the ring slot still holds layer 0's bytes: check the whole layer on the CPU
            torch.cuda.synchronize()
            ex = oracle.ExpertSet(*[t.numpy() for t in ring[0].tensors])
            assert_close(out.cpu().numpy(), clib.moe_forward(h, idx, w, ex), "config5 layer 0 vs C oracle")
        twin = k.routed_forward(H, I, W, _random_layer_into(scratch, seeds[i]))
        assert torch.equal(out, twin), f"streamed layer {i} differs from its resident twin"
        print(f"[config5] layer {i}: streamed forward == resident forward", flush=True)
        n_seen += 1
    assert n_seen == n_layers
    ms, nbytes = streamer.copy_stats()
    assert nbytes == n_layers * ring[0].nbytes
    print(f"[config5] H2D {nbytes / 1e9:.2f} GB in {ms:.0f} ms of copy time ({nbytes / ms / 1e6:.1f} GB/s)")
    del streamer, scratch, ring
    torch.cuda.empty_cache()
