"""
Packed MXFP4 expert loader: safetensors shards -> host staging (pinned) -> HBM.

Mirrors the reference's read path for routed experts:
  * SafetensorsIndex (lazy_lora/streaming/mmap_loader.py:37-262): every `*.safetensors` file's
    header (<u64 little-endian length><JSON>) is parsed into name -> (shard, absolute byte range,
    shape, dtype); shards that cannot be indexed are listed in `bad_shards`; names resolve with
    the "model." / "language_model." prefix rules of `_resolve_name` (:227-239).
  * DynamicExpertStreamer._load_single_expert (lazy_lora/streaming/expert_streamer.py:215-284):
    an expert is `model.layers.{L}.block_sparse_moe.experts.{e}.w{1,3,2}.weight_packed` and
    `.weight_scale`, U8, w1 = gate, w3 = up, w2 = down, shapes [F, D/2], [F, D/32], [D, F/2],
    [D, F/32]; bytes come off the disk with pread (MmapTensorStreamer._read_range, :300-347),
    in on-disk order (sort_by_disk_order, :286-303).
Here a whole layer's requested experts are read at once, sorted by (shard, offset) so the
reads sweep forward through each file, by a small pool of threads (os.preadv releases the
interpreter lock), straight into host buffers laid out as the stacked ExpertLayer (six uint8
tensors [E, rows, cols]); pinned host buffers then go to HBM with asynchronous copies, one per
contiguous run of expert ids and tensor. Bytes are never decoded or reordered: HBM holds the
checkpoint's own bytes.
"""
import json
import os
import struct
from concurrent.futures import ThreadPoolExecutor
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from lazylora_amd.experts import ExpertLayer

DTYPE_SIZES = {"F64": 8, "F32": 4, "F16": 2, "BF16": 2, "I64": 8, "I32": 4, "I16": 2, "I8": 1, "U8": 1,
               "BOOL": 1}
MAX_HEADER = 100 * 1024 * 1024  # the reference's sanity bound on a header (mmap_loader.py:105)

# (tensor suffix, ExpertLayer slot) in the order ExpertLayer stacks them: w1 = gate, w3 = up, w2 = down
EXPERT_TENSORS = (("w1.weight_packed", 0), ("w1.weight_scale", 1), ("w3.weight_packed", 2),
                  ("w3.weight_scale", 3), ("w2.weight_packed", 4), ("w2.weight_scale", 5))


def expert_tensor_name(layer: int, expert: int, suffix: str) -> str:
    return f"model.layers.{layer}.block_sparse_moe.experts.{expert}.{suffix}"


def layer_shapes(E: int, D: int, F: int) -> Tuple[Tuple[int, ...], ...]:
    """Stacked shapes of the six tensors of a layer, in ExpertLayer order."""
    return ((E, F, D // 2), (E, F, D // 32), (E, F, D // 2), (E, F, D // 32), (E, D, F // 2), (E, D, F // 32))


class SafetensorsIndex:
    """name -> (shard path, start, end, shape, dtype) over every *.safetensors file of a directory."""

    def __init__(self, model_dir: str):
        self.model_dir = model_dir
        self.tensor_locations: Dict[str, Tuple[str, int, int, List[int], str]] = {}
        self.bad_shards: List[str] = []
        if os.path.isdir(model_dir):
            self.build_index()

    def build_index(self) -> None:
        for shard in sorted(f for f in os.listdir(self.model_dir) if f.endswith(".safetensors")):
            path = os.path.join(self.model_dir, shard)
            try:
                entries = self._parse(path)
            except (OSError, ValueError, UnicodeDecodeError):
                self.bad_shards.append(shard)
                continue
            self.tensor_locations.update(entries)

    @staticmethod
    def _parse(path: str) -> Dict[str, Tuple[str, int, int, List[int], str]]:
        size = os.path.getsize(path)
        with open(path, "rb") as f:
            raw = f.read(8)
            if len(raw) < 8:
                raise ValueError("no header length")
            n = struct.unpack("<Q", raw)[0]
            if n > MAX_HEADER or 8 + n > size:
                raise ValueError("bad header length")
            header = json.loads(f.read(n).decode("utf-8"))
        base = 8 + n
        out = {}
        for name, info in header.items():
            if name == "__metadata__":
                continue
            begin, end = info["data_offsets"]
            shape = [int(d) for d in info["shape"]]
            dtype = info["dtype"]
            count = 1
            for d in shape:
                count *= d
            if end < begin or base + end > size:
                raise ValueError(f"{name}: data range outside the file")
            if dtype in DTYPE_SIZES and end - begin != count * DTYPE_SIZES[dtype]:
                raise ValueError(f"{name}: byte count does not match shape and dtype")
            out[name] = (path, base + int(begin), base + int(end), shape, dtype)
        return out

    def _resolve_name(self, name: str) -> Optional[str]:
        """The reference's prefix rules (mmap_loader.py:227-239)."""
        if name in self.tensor_locations:
            return name
        for prefix in ("language_model.", "model.", "language_model.model."):
            if prefix + name in self.tensor_locations:
                return prefix + name
            if name.startswith("model.") and "language_model." + name in self.tensor_locations:
                return "language_model." + name
        return None

    def has_tensor(self, name: str) -> bool:
        return self._resolve_name(name) is not None

    def location(self, name: str) -> Tuple[str, int, int, List[int], str]:
        resolved = self._resolve_name(name)
        if resolved is None:
            raise KeyError(f"tensor {name!r} is not in any shard of {self.model_dir}")
        return self.tensor_locations[resolved]


class HostLayer:
    """A layer's six stacked expert tensors in host memory (pinned when a GPU is present)."""

    def __init__(self, E: int, D: int, F: int, pin: Optional[bool] = None):
        if pin is None:
            pin = torch.cuda.is_available()
        self.E, self.D, self.F = E, D, F
        self.tensors = [torch.empty(s, dtype=torch.uint8, pin_memory=pin) for s in layer_shapes(E, D, F)]

    @property
    def nbytes(self) -> int:
        return sum(t.numel() for t in self.tensors)


def _runs(ids: Sequence[int]) -> List[Tuple[int, int]]:
    """Sorted distinct ids as half-open runs [a, b)."""
    out: List[Tuple[int, int]] = []
    for e in sorted(set(int(i) for i in ids)):
        if out and out[-1][1] == e:
            out[-1] = (out[-1][0], e + 1)
        else:
            out.append((e, e + 1))
    return out


class PackedLayerReader:
    """Reads routed-expert layers of a packed MXFP4 checkpoint (the reference's on-disk format)."""

    def __init__(self, model_dir: str, threads: int = 8):
        self.index = SafetensorsIndex(model_dir)
        self.threads = max(1, threads)
        self._fds: Dict[str, int] = {}
        self.bytes_read = 0

    def close(self) -> None:
        for fd in self._fds.values():
            os.close(fd)
        self._fds.clear()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def layer_geometry(self, layer: int, expert: int = 0) -> Tuple[int, int]:
        """(D, F) of a layer from its expert's w1 packed shape [F, D/2]."""
        _, _, _, shape, _ = self.index.location(expert_tensor_name(layer, expert, "w1.weight_packed"))
        return shape[1] * 2, shape[0]

    def sort_by_disk_order(self, layer: int, expert_ids: Sequence[int]) -> List[int]:
        """Expert ids by the (shard, offset) of their w1 packed tensor (expert_streamer.py:286-303)."""
        def key(e):
            path, start, _, _, _ = self.index.location(expert_tensor_name(layer, e, "w1.weight_packed"))
            return (path, start)
        return sorted((int(e) for e in expert_ids), key=key)

    def _extents(self, layer: int, expert_ids: Sequence[int], host: HostLayer):
        """(shard, file offset, size, destination tensor, expert) for every tensor to read, in disk order."""
        shapes = layer_shapes(host.E, host.D, host.F)
        ext = []
        for e in expert_ids:
            if not 0 <= e < host.E:
                raise ValueError(f"expert id {e} outside [0, {host.E})")
            for suffix, slot in EXPERT_TENSORS:
                name = expert_tensor_name(layer, e, suffix)
                path, start, end, shape, dtype = self.index.location(name)
                if dtype != "U8":
                    raise ValueError(f"{name}: dtype {dtype}, the packed format is U8")
                if tuple(shape) != shapes[slot][1:]:
                    raise ValueError(f"{name}: shape {tuple(shape)}, expected {shapes[slot][1:]}")
                ext.append((path, start, end - start, slot, e))
        ext.sort(key=lambda x: (x[0], x[1]))
        return ext

    def _fd(self, path: str) -> int:
        fd = self._fds.get(path)
        if fd is None:
            fd = os.open(path, os.O_RDONLY)
            self._fds[path] = fd
        return fd

    def read_layer(self, layer: int, expert_ids: Sequence[int], host: HostLayer) -> int:
        """Reads the experts' six tensors into their rows of `host`; returns the bytes read."""
        ext = self._extents(layer, sorted(set(int(e) for e in expert_ids)), host)
        views = [t.numpy().reshape(t.shape[0], -1) for t in host.tensors]
        for path, *_ in ext:
            self._fd(path)

        def read(item):
            path, off, size, slot, e = item
            mv = memoryview(views[slot][e]).cast("B")
            got = 0
            while got < size:
                n = os.preadv(self._fds[path], [mv[got:size]], off + got)
                if n <= 0:
                    raise IOError(f"short read in {path} at {off + got}: wanted {size - got} more bytes")
                got += n
            return size

        if self.threads == 1 or len(ext) < 2:
            total = sum(read(x) for x in ext)
        else:
            # contiguous slices of the disk-ordered list per thread keep each thread's reads sequential
            step = (len(ext) + self.threads - 1) // self.threads
            parts = [ext[i:i + step] for i in range(0, len(ext), step)]
            with ThreadPoolExecutor(max_workers=len(parts)) as pool:
                total = sum(pool.map(lambda part: sum(read(x) for x in part), parts))
        self.bytes_read += total
        return total

    def load_layer(self, layer: int, expert_ids: Optional[Sequence[int]] = None, E: Optional[int] = None,
                   device=None) -> ExpertLayer:
        """A layer's experts (all of them by default) as an HBM-resident ExpertLayer. Experts not
        requested are left uninitialised in HBM; route only to the ones loaded."""
        D, F = self.layer_geometry(layer, 0 if expert_ids is None else int(list(expert_ids)[0]))
        if E is None:
            E = 0
            while self.index.has_tensor(expert_tensor_name(layer, E, "w1.weight_packed")):
                E += 1
        ids = list(range(E)) if expert_ids is None else list(expert_ids)
        host = HostLayer(E, D, F)
        self.read_layer(layer, ids, host)
        out = ExpertLayer.empty(E, D, F, device)
        upload(host, out, ids)
        torch.cuda.current_stream(out.device).synchronize()
        return out


def upload(host: HostLayer, dst: ExpertLayer, expert_ids: Optional[Sequence[int]] = None,
           stream: Optional[torch.cuda.Stream] = None) -> int:
    """Asynchronous host -> HBM copies of the given experts' rows (all by default) on `stream`
    (the current stream by default), one copy per contiguous run of ids and tensor. Returns the
    bytes enqueued. The host buffers must stay untouched until the copies complete. The layer's
    forward- and backward-layout copies, if any, no longer match and are dropped."""
    if (host.E, host.D, host.F) != (dst.E, dst.D, dst.F):
        raise ValueError("host and device layers differ in shape")
    dst.drop_forward_layout()
    dst.drop_backward_layout()
    runs = [(0, host.E)] if expert_ids is None else _runs(expert_ids)
    total = 0
    with torch.cuda.stream(stream) if stream is not None else _nullcontext():
        for src, d in zip(host.tensors, dst.tensors()):
            for a, b in runs:
                d[a:b].copy_(src[a:b], non_blocking=True)
                total += src[a:b].numel()
    return total


class _nullcontext:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False
