"""
One routed-expert layer's packed MXFP4 weights, resident in HBM.

The reference hands experts over one at a time as ExpertWeightBundle objects holding
(w1|w3|w2).weight_packed / weight_scale tensors
(lazy_lora/streaming/expert_streamer.py:27-50, :229-246). On MI355X a whole layer fits in HBM
many times over (one layer of the BASELINE shape is 20.96 GB of 288 GB), so the layer is kept
as six stacked, expert-major tensors and every routed-layer call reads experts by index:

    w1p, w3p : [E, F, D/2] uint8    w1s, w3s : [E, F, D/32] uint8     (gate / up, W is [F, D])
    w2p      : [E, D, F/2] uint8    w2s      : [E, D, F/32] uint8     (down, W is [D, F])

Roles follow the reference: w1 = gate, w3 = up, w2 = down (expert_streamer.py:229-246).
"""
import ctypes
import warnings
from typing import Iterable, Optional, Sequence

import torch


class ExpertLayer:
    def __init__(self, w1p, w1s, w3p, w3s, w2p, w2s, device: Optional[torch.device] = None):
        tensors = [w1p, w1s, w3p, w3s, w2p, w2s]
        for t in tensors:
            if t.dtype != torch.uint8:
                raise ValueError(f"expert tensors must be uint8, got {t.dtype}")
            if t.dim() != 3:
                raise ValueError(f"expert tensors must be stacked [E, rows, cols], got {tuple(t.shape)}")
        E, F, Dh = w1p.shape
        D = Dh * 2
        if D % 32 or F % 32:
            raise ValueError(f"D={D} and F={F} must be multiples of 32")
        want = {
            "w1p": (E, F, D // 2), "w1s": (E, F, D // 32), "w3p": (E, F, D // 2), "w3s": (E, F, D // 32),
            "w2p": (E, D, F // 2), "w2s": (E, D, F // 32),
        }
        for (name, shape), t in zip(want.items(), tensors):
            if tuple(t.shape) != shape:
                raise ValueError(f"{name} must be {shape}, got {tuple(t.shape)}")
        if device is None:
            device = w1p.device if w1p.is_cuda else torch.device("cuda", torch.cuda.current_device())
        self.device = torch.device(device)
        self.E, self.D, self.F = E, D, F
        (self.w1p, self.w1s, self.w3p, self.w3s, self.w2p, self.w2s) = [
            _aligned16(t.to(self.device, non_blocking=True).contiguous()) for t in tensors]
        self._fl = None  # forward-layout copies (W1, W3, W2; None where K is not a multiple of 512)
        self._bl = None  # backward-layout copies (W1, W3, W2; None where the shape does not allow one)

    @classmethod
    def empty(cls, E: int, D: int, F: int, device=None) -> "ExpertLayer":
        """An uninitialised layer in HBM (a destination for streamed or loaded experts)."""
        if device is None:
            device = torch.device("cuda", torch.cuda.current_device())
        shapes = ((E, F, D // 2), (E, F, D // 32), (E, F, D // 2), (E, F, D // 32), (E, D, F // 2), (E, D, F // 32))
        return cls(*[torch.empty(s, dtype=torch.uint8, device=device) for s in shapes], device=device)

    @classmethod
    def from_bundles(cls, bundles: Sequence, device=None, num_experts: Optional[int] = None) -> "ExpertLayer":
        """A layer from the reference's per-expert ExpertWeightBundle objects (packed form: the
        gate/up/down_packed and _scale attributes, expert_streamer.py:27-50).

        `bundles` is either a sequence of bundles, expert e at position e, or (expert_id,
        bundle) pairs as DynamicExpertStreamer.stream_experts yields them (in disk order, only
        the active experts, expert_streamer.py:315-369); then expert ids index a layer of
        `num_experts` experts (default: the largest id + 1) whose absent experts are zero
        weights, which no routing that only selects streamed experts reads."""
        items = list(bundles)
        pairs = bool(items) and isinstance(items[0], tuple)
        if not pairs:
            items = list(enumerate(items))
        if not items:
            raise ValueError("from_bundles needs at least one expert")
        for eid, b in items:
            if not getattr(b, "packed", b.gate_packed is not None) or b.gate_packed is None:
                raise ValueError(f"expert {eid} is not in packed MXFP4 form")
        ids = [int(eid) for eid, _ in items]
        if len(set(ids)) != len(ids) or min(ids) < 0:
            raise ValueError("expert ids must be distinct and non-negative")
        E = num_experts if num_experts is not None else max(ids) + 1
        if max(ids) >= E:
            raise ValueError(f"expert id {max(ids)} does not fit a layer of {E} experts")
        if device is None:
            device = torch.device("cuda", torch.cuda.current_device())
        attrs = ("gate_packed", "gate_scale", "up_packed", "up_scale", "down_packed", "down_scale")
        first = items[0][1]
        stacked = []
        for attr in attrs:
            t0 = getattr(first, attr)
            dst = torch.zeros((E,) + tuple(t0.shape), dtype=torch.uint8, device=device)
            for eid, b in items:
                src = getattr(b, attr)
                if tuple(src.shape) != tuple(t0.shape) or src.dtype != torch.uint8:
                    raise ValueError(f"expert {eid}: {attr} must be uint8 {tuple(t0.shape)}, "
                                     f"got {src.dtype} {tuple(src.shape)}")
                dst[eid].copy_(src, non_blocking=True)
            stacked.append(dst)
        return cls(*stacked, device=device)

    def prepare_forward_layout(self) -> int:
        """Builds the forward-layout copies of W1, W3 (when D is a multiple of 512) and W2 (when F
        is), which the routed forward's small-bucket work-groups then read with whole 1 KiB loads
        of codes and whole-line loads of scales (mxfp4_forward_layout; results are
        bit-identical). Each copy holds the packed codes and E8M0 scales it copies with the rows
        padded to a multiple of 16 (ceil(R / 16) * 16 * (K / 2 + K / 32) bytes per expert: the
        same size when R is a multiple of 16); returns the bytes added.

        The copies reflect the weights as they are now. An in-place torch write to the codes or
        scales (or rebinding the tensors) is detected before the next routed call, which then
        drops the copy with a warning; loader.upload drops it too. Writes the version counters do
        not see (through `.data`, ctypes or hipMemcpy, or by another C caller) are not detected:
        call drop_forward_layout() or prepare_forward_layout() after them, or the forward reads
        the old weights."""
        from lazylora_amd.native import kernel

        k = kernel()
        if k is None:
            raise RuntimeError("the forward layout needs the native library on a GPU")
        w13 = ((k.forward_layout(self.w1p, self.w1s), k.forward_layout(self.w3p, self.w3s)) if self.D % 512 == 0
               else (None, None))
        w2 = k.forward_layout(self.w2p, self.w2s) if self.F % 512 == 0 else None
        self._fl = (w13[0], w13[1], w2)
        self._fl_versions = self._code_versions()
        return sum(t.numel() for t in self._fl if t is not None)

    def drop_forward_layout(self) -> None:
        """Forgets the forward-layout copies (the routed calls then read the checkpoint layout)."""
        self._fl = None

    def prepare_backward_layout(self) -> int:
        """Builds the backward-layout copies of W1, W3 (when D is a multiple of 256) and W2 (when
        F is), which the routed backward's transposed products then read with four 1 KiB loads
        of codes and one 512-byte load of scales per wave and 32-row step (sixteen loads of
        pieces of eight rows otherwise; mxfp4_backward_layout; results are bit-identical). Each copy holds the codes and scales it copies: R * (K / 2 + K / 32)
        bytes per expert; returns the bytes added. Stale copies are detected and dropped like
        the forward layout's (prepare_forward_layout)."""
        from lazylora_amd.native import kernel

        k = kernel()
        if k is None:
            raise RuntimeError("the backward layout needs the native library on a GPU")
        w13 = ((k.backward_layout(self.w1p, self.w1s), k.backward_layout(self.w3p, self.w3s)) if self.D % 256 == 0
               else (None, None))
        w2 = k.backward_layout(self.w2p, self.w2s) if self.F % 256 == 0 else None
        self._bl = (w13[0], w13[1], w2)
        self._bl_versions = self._code_versions()
        return sum(t.numel() for t in self._bl if t is not None)

    def drop_backward_layout(self) -> None:
        """Forgets the backward-layout copies (the transposed products then read the checkpoint
        layout)."""
        self._bl = None

    def _code_versions(self):
        # torch counts in-place writes per tensor (a write through a view counts for its base)
        ts = (self.w1p, self.w1s, self.w3p, self.w3s, self.w2p, self.w2s)
        return tuple(t._version for t in ts) + tuple(t.data_ptr() for t in ts)

    def _fresh(self):
        """Drops (with a warning) layout copies made before an in-place write to the codes or
        scales (or a rebinding of the tensors)."""
        v = self._code_versions()
        if self._fl is not None and v != self._fl_versions:
            warnings.warn("expert weights changed after prepare_forward_layout(): the forward-layout copy is dropped "
                          "(call prepare_forward_layout() again to rebuild it)", RuntimeWarning, stacklevel=4)
            self._fl = None
        if self._bl is not None and v != self._bl_versions:
            warnings.warn("expert weights changed after prepare_backward_layout(): the backward-layout copy is "
                          "dropped (call prepare_backward_layout() again to rebuild it)", RuntimeWarning,
                          stacklevel=4)
            self._bl = None

    def forward_layout_pointers(self):
        """Host array of the three forward-layout device pointers for mxfp4_moe_*_fl, or None.
        Copies made before an in-place write to the codes (or a rebinding of the tensors) are
        stale: they are dropped, with a warning, and the call reads the checkpoint layout."""
        self._fresh()
        if self._fl is None:
            return None
        return (ctypes.c_void_p * 3)(*[t.data_ptr() if t is not None else None for t in self._fl])

    def layout_pointers(self):
        """(host pointer array, flags) for mxfp4_moe_*_fl: the three forward-layout pointers (or
        None), or, with backward-layout copies, six pointers (forward W1, W3, W2, then backward
        W1, W3, W2) and MXFP4_MOE_BWD_LAYOUT. Stale copies are dropped first, as in
        forward_layout_pointers."""
        from lazylora_amd.native import MOE_BWD_LAYOUT

        self._fresh()
        if self._bl is None:
            if self._fl is None:
                return None, 0
            return (ctypes.c_void_p * 3)(*[t.data_ptr() if t is not None else None for t in self._fl]), 0
        fl = self._fl if self._fl is not None else (None, None, None)
        return (ctypes.c_void_p * 6)(*[t.data_ptr() if t is not None else None for t in (*fl, *self._bl)]), \
            MOE_BWD_LAYOUT

    def pointers(self):
        return (self.w1p.data_ptr(), self.w1s.data_ptr(), self.w3p.data_ptr(), self.w3s.data_ptr(),
                self.w2p.data_ptr(), self.w2s.data_ptr())

    @property
    def nbytes(self) -> int:
        return sum(t.numel() for t in (self.w1p, self.w1s, self.w3p, self.w3s, self.w2p, self.w2s))

    def expert_bytes(self) -> int:
        """Packed bytes of one expert (all three matrices, codes + scales)."""
        return self.nbytes // self.E

    def tensors(self) -> Iterable[torch.Tensor]:
        return (self.w1p, self.w1s, self.w3p, self.w3s, self.w2p, self.w2s)


def _aligned16(t: torch.Tensor) -> torch.Tensor:
    """t itself when its data starts on a 16-byte boundary (the kernels' requirement for packed
    weights and scales), else an aligned copy."""
    return t if t.data_ptr() % 16 == 0 else t.clone()
