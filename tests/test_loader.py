"""The packed-checkpoint loader against the reference's on-disk format (no GPU).

Shards are written with the `safetensors` library (an independent writer and reader of the
format), laid out like the reference's checkpoint and its tiny-model generator
(scripts/make_tiny_model.py:130-160, :515-536): `model.layers.{L}.block_sparse_moe.experts.{e}.
w{1,3,2}.weight_packed / weight_scale`, U8, split over two shards with the experts not in id
order, next to BF16 tensors of the same layer. Every byte the loader places must equal the
byte the safetensors reader returns for that tensor."""
import json
import os
import struct

import numpy as np
import pytest
import torch
from safetensors.numpy import load_file, save_file

from lazylora_amd.loader import (EXPERT_TENSORS, HostLayer, PackedLayerReader, SafetensorsIndex,
                                 expert_tensor_name)

E, D, F, LAYER = 6, 64, 32, 3


def expert_arrays(rng, e):
    shapes = {"w1.weight_packed": (F, D // 2), "w1.weight_scale": (F, D // 32), "w3.weight_packed": (F, D // 2),
              "w3.weight_scale": (F, D // 32), "w2.weight_packed": (D, F // 2), "w2.weight_scale": (D, F // 32)}
    return {expert_tensor_name(LAYER, e, k): rng.integers(0, 256, s, dtype=np.uint8) for k, s in shapes.items()}


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    rng = np.random.default_rng(7)
    d = tmp_path_factory.mktemp("ckpt")
    want = {}
    shard1, shard2 = {}, {}
    for e in (4, 0, 2):
        shard1.update(expert_arrays(rng, e))
    for e in (5, 1, 3):
        shard2.update(expert_arrays(rng, e))
    gate = rng.integers(0, 65536, (E, 2 * D), dtype=np.uint16)
    shard1[f"model.layers.{LAYER}.block_sparse_moe.gate.weight"] = gate
    want.update(shard1)
    want.update(shard2)
    save_file(shard1, str(d / "model-00001-of-00002.safetensors"))
    save_file(shard2, str(d / "model-00002-of-00002.safetensors"))
    return str(d), want


def test_index_matches_the_safetensors_reader(ckpt):
    d, want = ckpt
    idx = SafetensorsIndex(d)
    assert not idx.bad_shards
    assert set(idx.tensor_locations) == set(want)
    for shard in sorted(os.listdir(d)):
        ref = load_file(os.path.join(d, shard))
        with open(os.path.join(d, shard), "rb") as f:
            blob = f.read()
        for name, arr in ref.items():
            path, start, end, shape, _ = idx.location(name)
            assert path.endswith(shard) and list(arr.shape) == shape
            assert blob[start:end] == arr.tobytes()


@pytest.mark.parametrize("threads", [1, 4])
def test_read_layer_places_every_byte(ckpt, threads):
    d, want = ckpt
    r = PackedLayerReader(d, threads=threads)
    assert r.layer_geometry(LAYER) == (D, F)
    host = HostLayer(E, D, F, pin=False)
    for t in host.tensors:
        t.fill_(0xA5)
    ids = [5, 0, 3]
    assert r.read_layer(LAYER, ids, host) == sum(want[expert_tensor_name(LAYER, e, s)].nbytes
                                                 for e in ids for s, _ in EXPERT_TENSORS)
    for e in range(E):
        for suffix, slot in EXPERT_TENSORS:
            got = host.tensors[slot][e].numpy()
            if e in ids:
                assert np.array_equal(got, want[expert_tensor_name(LAYER, e, suffix)]), (e, suffix)
            else:
                assert (got == 0xA5).all(), (e, suffix)
    r.close()


def test_disk_order_and_prefixes(ckpt, tmp_path):
    d, want = ckpt
    r = PackedLayerReader(d)
    # shard 1 holds experts 4, 0, 2 (written in that order), shard 2 holds 5, 1, 3
    order = r.sort_by_disk_order(LAYER, range(E))
    locs = [r.index.location(expert_tensor_name(LAYER, e, "w1.weight_packed"))[:2] for e in order]
    assert locs == sorted(locs)
    assert set(order[:3]) == {0, 2, 4} and set(order[3:]) == {1, 3, 5}
    # a checkpoint whose names carry the "language_model." prefix resolves the plain names
    rng = np.random.default_rng(1)
    arrs = {"language_model." + k: v for k, v in expert_arrays(rng, 0).items()}
    save_file(arrs, str(tmp_path / "model-00001-of-00001.safetensors"))
    idx = SafetensorsIndex(str(tmp_path))
    assert idx.has_tensor(expert_tensor_name(LAYER, 0, "w1.weight_packed"))


def test_bad_shards_and_format_errors(tmp_path):
    rng = np.random.default_rng(2)
    arrs = expert_arrays(rng, 0)
    save_file(arrs, str(tmp_path / "a.safetensors"))
    (tmp_path / "empty.safetensors").write_bytes(b"")
    blob = (tmp_path / "a.safetensors").read_bytes()
    (tmp_path / "truncated.safetensors").write_bytes(blob[: len(blob) // 2])
    idx = SafetensorsIndex(str(tmp_path))
    assert sorted(idx.bad_shards) == ["empty.safetensors", "truncated.safetensors"]
    r = PackedLayerReader(str(tmp_path))
    host = HostLayer(2, D, F, pin=False)
    with pytest.raises(KeyError):
        r.read_layer(LAYER, [1], host)          # expert 1 is in no shard
    with pytest.raises(ValueError):
        r.read_layer(LAYER, [2], host)          # id outside the host layer
    wrong = HostLayer(2, 2 * D, F, pin=False)
    with pytest.raises(ValueError):
        r.read_layer(LAYER, [0], wrong)         # shapes of another geometry
    # a header whose byte count disagrees with shape x dtype makes the shard unreadable
    n = struct.unpack("<Q", blob[:8])[0]
    header = json.loads(blob[8:8 + n])
    name = next(k for k in header if k != "__metadata__")
    header[name]["shape"] = [header[name]["shape"][0] + 1] + header[name]["shape"][1:]
    hb = json.dumps(header).encode()
    hb += b" " * ((-len(hb)) % 8)
    bad_dir = tmp_path / "bad"
    bad_dir.mkdir()
    (bad_dir / "x.safetensors").write_bytes(struct.pack("<Q", len(hb)) + hb + blob[8 + n:])
    assert SafetensorsIndex(str(bad_dir)).bad_shards == ["x.safetensors"]


def test_host_layer_shapes():
    h = HostLayer(3, D, F, pin=False)
    assert [tuple(t.shape) for t in h.tensors] == [(3, F, D // 2), (3, F, D // 32), (3, F, D // 2), (3, F, D // 32),
                                                   (3, D, F // 2), (3, D, F // 32)]
    assert h.nbytes == 3 * (2 * (F * D // 2 + F * D // 32) + D * F // 2 + D * F // 32)
    assert all(t.dtype == torch.uint8 for t in h.tensors)
