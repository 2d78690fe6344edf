"""
Out-of-core layer streaming: host-resident routed-expert layers through a ring of HBM slots.

The reference streams experts from disk one at a time, reading ahead on a background thread
so the drive keeps moving while the CPU multiplies (DynamicExpertStreamer.stream_experts,
lazy_lora/streaming/expert_streamer.py:316-369, depth 2). On MI355X a whole layer of packed
experts fits in HBM many times over, so the unit of streaming is the layer: `LayerStreamer`
keeps `slots` HBM copies of the layer geometry and, on its own copy stream (default priority),
copies layer i + slots - 1 from (pinned) host memory while the compute stream runs layer i.
Ordering is by events only: a slot is refilled after the compute stream has recorded that it
finished reading it, and the compute stream waits for the slot's copy before using it; the
host never blocks except to throttle when all slots are in flight.
"""
from collections import deque
from typing import Iterable, Iterator, List, Optional, Sequence, Tuple

import numpy as np
import torch

from lazylora_amd.experts import ExpertLayer
from lazylora_amd.loader import HostLayer, upload


class LayerStreamer:
    def __init__(self, E: int, D: int, F: int, slots: int = 2, device=None, timing: bool = False):
        if slots < 2:
            raise ValueError("streaming needs at least two HBM slots")
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.layers = [ExpertLayer.empty(E, D, F, self.device) for _ in range(slots)]
        self.copy_stream = torch.cuda.Stream(device=self.device)
        self.ready = [torch.cuda.Event() for _ in range(slots)]
        self.free = [torch.cuda.Event() for _ in range(slots)]
        self.timing = timing
        self.copy_events: List[Tuple[torch.cuda.Event, torch.cuda.Event, int]] = []
        self.bytes_copied = 0

    @property
    def slots(self) -> int:
        return len(self.layers)

    def _fill(self, slot: int, host: HostLayer, expert_ids: Optional[Sequence[int]]) -> None:
        cs = self.copy_stream
        cs.wait_event(self.free[slot])  # the compute stream has finished with the slot's last layer
        t0 = t1 = None
        if self.timing:
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record(cs)
        n = upload(host, self.layers[slot], expert_ids, stream=cs)
        if self.timing:
            t1.record(cs)
            self.copy_events.append((t0, t1, n))
        self.ready[slot].record(cs)
        self.bytes_copied += n

    def stream(self, hosts: Iterable, expert_ids: Optional[Iterable] = None) -> Iterator[Tuple[int, ExpertLayer]]:
        """Yields (i, layer in HBM) for each host layer in turn. The caller enqueues its work on
        the current stream before asking for the next layer; the slot is then handed back. With
        `expert_ids` (one id list per layer, or None per layer) only those experts are copied."""
        hosts = iter(hosts)
        ids = iter(expert_ids) if expert_ids is not None else None
        compute = torch.cuda.current_stream(self.device)
        for ev in self.free:
            ev.record(compute)
        pending = deque()
        i = 0

        def issue():
            nonlocal i
            try:
                host = next(hosts)
            except StopIteration:
                return False
            slot = i % self.slots
            self._fill(slot, host, next(ids) if ids is not None else None)
            pending.append((i, slot))
            i += 1
            return True

        for _ in range(self.slots):
            if not issue():
                break
        while pending:
            j, slot = pending.popleft()
            compute.wait_event(self.ready[slot])
            yield j, self.layers[slot]
            self.free[slot].record(compute)
            issue()

    def copy_stats(self) -> Tuple[float, int]:
        """(total ms spent in the copies recorded with timing=True, bytes). Synchronises."""
        torch.cuda.synchronize(self.device)
        ms = sum(a.elapsed_time(b) for a, b, _ in self.copy_events)
        return ms, sum(n for _, _, n in self.copy_events)


_BUNDLE_ATTRS = ("gate_packed", "gate_scale", "up_packed", "up_scale", "down_packed", "down_scale")


class BundleStager:
    """Packed ExpertWeightBundles, as the reference's streamer yields them (CPU tensors, one
    expert at a time, expert_streamer.py:27-50, :315-369), into a compact HBM layer that holds
    only the experts streamed.

    Each bundle is copied into one of `slots` pinned host buffers and from there to HBM by an
    asynchronous copy on a dedicated copy stream (default priority), so the DMA of expert i runs
    while expert i + 1 is taken from the generator and copied into the next buffer; the host
    waits only before refilling a buffer whose DMA is still running. Bundles already in pinned
    memory skip the staging copy; bundles already on the device are copied device to device.
    The pinned buffers are kept between calls (they are sized for one expert)."""

    def __init__(self, device=None, slots: int = 4):
        if slots < 2:
            raise ValueError("staging needs at least two pinned buffers")
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.slots = slots
        self.copy_stream = torch.cuda.Stream(device=self.device)
        self._buf: List[torch.Tensor] = []
        self._done = [torch.cuda.Event() for _ in range(slots)]
        self._used = [False] * slots
        self._shapes: Optional[Tuple[Tuple[int, ...], ...]] = None
        self.bytes_copied = 0

    def _buffers(self, shapes) -> None:
        if self._shapes == shapes:
            return
        for s in range(self.slots):  # buffers of another geometry: wait for their last copies
            if self._used[s]:
                self._done[s].synchronize()
        total = sum(int(np.prod(s)) for s in shapes)
        self._buf = [torch.empty(total, dtype=torch.uint8, pin_memory=True) for _ in range(self.slots)]
        self._used = [False] * self.slots
        self._shapes = shapes

    def stage(self, pairs: Iterable, capacity: int) -> Tuple[ExpertLayer, List[int]]:
        """(layer, ids): expert j of the returned layer is the bundle of expert id ids[j], in the
        order the (expert_id, bundle) pairs came. `capacity` bounds the number of pairs (the
        length of the active set). The current stream waits for the copies before it uses the
        layer; the call returns once the last DMA is queued."""
        it = iter(pairs)
        first = next(it, None)
        if first is None:
            raise ValueError("the streamer yielded no experts")
        b0 = first[1]
        shapes = tuple(tuple(getattr(b0, a).shape) for a in _BUNDLE_ATTRS)
        (F, Dh), (_, Dg), (_, _), (_, _), (D, Fh), (_, Fg) = shapes
        if Dh * 2 != D or Fh * 2 != F or Dg * 32 != D or Fg * 32 != F:
            raise ValueError(f"bundle shapes {shapes} are not a packed MXFP4 expert")
        self._buffers(shapes)
        layer = ExpertLayer.empty(max(1, capacity), D, F, self.device)
        dst = layer.tensors()
        compute = torch.cuda.current_stream(self.device)
        cs = self.copy_stream
        cs.wait_stream(compute)  # the layer's memory may have been in use on the compute stream
        ids: List[int] = []
        sizes = [int(np.prod(s)) for s in shapes]
        offs = np.concatenate([[0], np.cumsum(sizes)]).tolist()

        def put(j, eid, b):
            if j >= capacity:
                raise ValueError(f"the streamer yielded more than the {capacity} experts asked for")
            srcs = []
            for a, shp in zip(_BUNDLE_ATTRS, shapes):
                t = getattr(b, a)
                if t is None or tuple(t.shape) != shp or t.dtype != torch.uint8:
                    raise ValueError(f"expert {eid}: {a} must be uint8 {shp}, got "
                                     f"{None if t is None else (t.dtype, tuple(t.shape))}")
                srcs.append(t)
            slot = j % self.slots
            staged = all(t.is_cuda or t.is_pinned() for t in srcs)
            if not staged:
                if self._used[slot]:
                    self._done[slot].synchronize()  # its previous DMA has read the buffer
                buf = self._buf[slot]
                for t, o0, o1 in zip(srcs, offs[:-1], offs[1:]):
                    buf[o0:o1].copy_(t.reshape(-1))
                srcs = [buf[o0:o1] for o0, o1 in zip(offs[:-1], offs[1:])]
            with torch.cuda.stream(cs):
                for d, t in zip(dst, srcs):
                    d[j].view(-1).copy_(t.reshape(-1), non_blocking=True)
            if not staged:
                self._done[slot].record(cs)
                self._used[slot] = True
            ids.append(int(eid))
            self.bytes_copied += offs[-1]

        put(0, first[0], b0)
        for j, (eid, b) in enumerate(it, start=1):
            put(j, eid, b)
        if len(set(ids)) != len(ids) or min(ids) < 0:
            raise ValueError("expert ids must be distinct and non-negative")
        compute.wait_stream(cs)
        return layer, ids


def compact_ids(topk_indices: torch.Tensor, ids: Sequence[int], device) -> torch.Tensor:
    """topk_indices mapped onto a compact layer holding experts `ids` (expert ids[j] at j), on
    `device`: an id not among them becomes -1, which the routed call skips, as the reference's
    sweep over the streamed experts never visits it (lazy_trainer.py:806-834)."""
    n_map = max(ids) + 1
    emap = torch.full((n_map,), -1, dtype=torch.int64, device=device)
    emap[torch.tensor(ids, dtype=torch.int64, device=device)] = torch.arange(len(ids), device=device)
    idx = topk_indices.to(device, non_blocking=True).long()
    inside = (idx >= 0) & (idx < n_map)
    return torch.where(inside, emap[idx.clamp(0, n_map - 1)], torch.full_like(idx, -1)).contiguous()


def host_layer_from(layer: ExpertLayer, pin: Optional[bool] = None) -> HostLayer:
    """A host copy of an HBM layer (test and benchmark helper)."""
    h = HostLayer(layer.E, layer.D, layer.F, pin=pin)
    for src, dst in zip(layer.tensors(), h.tensors):
        dst.copy_(src)
    return h


def dequantize_mxfp4(weight_packed, weight_scale, group_size: int = 32, out_dtype=None):
    """Widen one packed MXFP4 matrix on the device (_dequantize_mxfp4,
    lazy_lora/streaming/expert_streamer.py:104-154): weight_packed [R, K/2] bytes (low nibble =
    even element), weight_scale [R, K/32] E8M0 bytes (or [R], one byte per row), value =
    e2m1(code) * 2^(scale - 127), a scale byte >= 253 giving +-0. Returns [R, K] in out_dtype,
    bfloat16 when None as in the reference; bf16 and fp32 come straight from the device kernels,
    other floating dtypes from the fp32 result. Torch tensors come back on their own device,
    NumPy arrays as fp32 NumPy arrays (the reference's NumPy branch; there, unlike its torch
    branch, only scale 255 is zeroed, where this zeroes >= 253 on both). Needs the MI355X
    library: raises RuntimeError when it is unavailable."""
    import numpy as np

    from lazylora_amd.native import kernel

    if group_size != 32:
        raise ValueError(f"MXFP4 groups hold 32 elements, got group_size={group_size}")
    k = kernel()
    if k is None:
        raise RuntimeError("dequantize_mxfp4 needs the MI355X MXFP4 library (kernel() is None)")
    as_numpy = isinstance(weight_packed, np.ndarray)
    p = torch.from_numpy(np.ascontiguousarray(weight_packed)) if as_numpy else weight_packed
    s = torch.from_numpy(np.ascontiguousarray(weight_scale)) if isinstance(weight_scale, np.ndarray) else weight_scale
    if p.dim() != 2:
        raise ValueError(f"weight_packed must be 2-D [R, K/2], got {tuple(p.shape)}")
    R, K = p.shape[0], p.shape[1] * 2
    if s.dim() == 1:  # one scale per row
        if s.shape[0] != R:
            raise ValueError(f"a 1-D weight_scale needs one byte per row ({R}), got {s.shape[0]}")
        s = s.reshape(R, 1).expand(R, K // 32)
    dtype = torch.float32 if as_numpy else (out_dtype or torch.bfloat16)
    w = k.dequant(p, s.contiguous(), out_dtype=dtype)
    return w.numpy() if as_numpy else w


_dequantize_mxfp4 = dequantize_mxfp4  # the reference's name, for callers that import it
