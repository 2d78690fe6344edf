"""
MXFP4 expert kernels on MI355X, with the Python interface of lazy_lora/native/__init__.py.

`kernel()` returns an `MXFP4Kernel` whose `gemm`, `gemm_t` and `dequant` take and return the
same shapes as the reference's (lazy_lora/native/__init__.py:36-74); the arithmetic runs in
hand-written gfx950 HIP kernels (liblazylora_mxfp4.so, C ABI in include/lazylora_mxfp4.h).
`routed_forward` / `routed_backward` run a whole routed-expert layer in one call each.

Differences from the reference, all deliberate:
  * results are placed on the input's device; CPU inputs are copied to the GPU and the
    result is copied back, so the unmodified CPU trainer also works;
  * shape errors raise ValueError (the reference asserts), and K % 32 != 0 is rejected
    (the reference floors K/32 and reads uninitialised memory);
  * `kernel()` returns None, with a printed warning, when the library is missing or fails to
    load or no HIP device is visible, as the reference's does (native/__init__.py:77-96), so
    callers that probe `kernel() is not None` (expert_streamer.py:206-207) take their own
    fallback. LAZYLORA_NATIVE_STRICT=1 makes those cases raise RuntimeError instead, for
    deployments where the GPU path must run. LAZYLORA_NO_NATIVE=1 returns None silently.
    Nothing here falls back to a CPU implementation: the MXFP4Kernel methods run on the GPU
    or raise.
"""
import ctypes
import os
import sys
from typing import Optional, Tuple

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblazylora_mxfp4.so")

ACT_SWIGLU = 0
ACT_SITU = 1
_ACTS = {"swiglu": ACT_SWIGLU, "situ": ACT_SITU, "situ_glu": ACT_SITU, ACT_SWIGLU: ACT_SWIGLU, ACT_SITU: ACT_SITU}

F32, BF16, I32, I64 = 0, 1, 2, 3
MOE_SAVE = 1
MOE_REUSE_FORWARD = 2
MOE_BWD_LAYOUT = 4

_lib = None
_kernel = None
_tried = False


def _load_library() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m lazylora_amd.build` "
            "(or __graft_entry__.build()) before using the MI355X kernels")
    lib = ctypes.CDLL(LIB_PATH)
    vp, ci, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    lib.mxfp4_last_error.restype = ctypes.c_char_p
    lib.mxfp4_last_error.argtypes = []
    lib.mxfp4_threads.restype = ci
    lib.mxfp4_threads.argtypes = []
    lib.mxfp4_dequant.restype = ci
    lib.mxfp4_dequant.argtypes = [vp, vp, vp, ci, ci, vp]
    lib.mxfp4_dequant_bf16.restype = ci
    lib.mxfp4_dequant_bf16.argtypes = [vp, vp, vp, ci, ci, vp]
    lib.mxfp4_gemm_workspace_size.restype = sz
    lib.mxfp4_gemm_workspace_size.argtypes = [ci, ci, ci]
    lib.mxfp4_gemm.restype = ci
    lib.mxfp4_gemm.argtypes = [vp, vp, vp, vp, ci, ci, ci, vp, sz, vp]
    lib.mxfp4_gemm_noalloc.restype = ci
    lib.mxfp4_gemm_noalloc.argtypes = [vp, vp, vp, vp, ci, ci, ci, vp]
    lib.mxfp4_gemm_t_workspace_size.restype = sz
    lib.mxfp4_gemm_t_workspace_size.argtypes = [ci, ci, ci]
    lib.mxfp4_gemm_t.restype = ci
    lib.mxfp4_gemm_t.argtypes = [vp, vp, vp, vp, ci, ci, ci, vp, sz, vp]
    lib.mxfp4_moe_workspace_size.restype = sz
    lib.mxfp4_moe_workspace_size.argtypes = [ci, ci, ci, ci, ci]
    lib.mxfp4_moe_forward.restype = ci
    lib.mxfp4_moe_forward.argtypes = [vp, vp, ci, vp, ci, vp, ci, ci, vp, vp, vp, vp, vp, vp,
                                      ci, ci, ci, ci, ci, vp, sz, vp]
    lib.mxfp4_moe_backward.restype = ci
    lib.mxfp4_moe_backward.argtypes = [vp, vp, vp, vp, ci, vp, ci, vp, ci, ci, vp, vp, vp, vp, vp, vp,
                                       ci, ci, ci, ci, ci, vp, sz, vp]
    lib.mxfp4_moe_forward_lora.restype = ci
    lib.mxfp4_moe_forward_lora.argtypes = [vp, vp, ci, vp, ci, vp, ci, ci, vp, vp, vp, vp, vp, vp,
                                           ci, ci, ci, ci, vp, vp, ci, ci, vp, sz, vp]
    lib.mxfp4_moe_backward_lora.restype = ci
    lib.mxfp4_moe_backward_lora.argtypes = [vp, vp, vp, vp, ci, vp, ci, vp, ci, ci, vp, vp, vp, vp, vp, vp,
                                            ci, ci, ci, ci, vp, vp, ci, vp, ci, vp, sz, vp]
    lib.mxfp4_moe_forward_fl.restype = ci
    lib.mxfp4_moe_forward_fl.argtypes = [vp, vp, ci, vp, ci, vp, ci, ci, vp, vp, vp, vp, vp, vp, vp,
                                         ci, ci, ci, ci, vp, vp, ci, ci, vp, sz, vp]
    lib.mxfp4_moe_backward_fl.restype = ci
    lib.mxfp4_moe_backward_fl.argtypes = [vp, vp, vp, vp, ci, vp, ci, vp, ci, ci, vp, vp, vp, vp, vp, vp, vp,
                                          ci, ci, ci, ci, vp, vp, ci, vp, ci, vp, sz, vp]
    lib.mxfp4_forward_layout_bytes.restype = sz
    lib.mxfp4_forward_layout_bytes.argtypes = [ci, ci, ci]
    lib.mxfp4_forward_layout.restype = ci
    lib.mxfp4_forward_layout.argtypes = [vp, vp, vp, ci, ci, ci, vp]
    lib.mxfp4_backward_layout_bytes.restype = sz
    lib.mxfp4_backward_layout_bytes.argtypes = [ci, ci, ci]
    lib.mxfp4_backward_layout.restype = ci
    lib.mxfp4_backward_layout.argtypes = [vp, vp, vp, ci, ci, ci, vp]
    lib.mxfp4_moe_route_status.restype = ci
    lib.mxfp4_moe_route_status.argtypes = [vp, vp, vp]
    lib.mxfp4_router_topk.restype = ci
    lib.mxfp4_router_topk.argtypes = [vp, vp, vp, vp, ci, ci, ci, ctypes.c_float, ci, vp]
    lib.mxfp4_router_topk_backward.restype = ci
    lib.mxfp4_router_topk_backward.argtypes = [vp, vp, vp, vp, ci, ci, ci, ctypes.c_float, ci, vp]
    lib.mxfp4_moe_timing.restype = ci
    lib.mxfp4_moe_timing.argtypes = [ci]
    lib.mxfp4_moe_timed_calls.restype = ci
    lib.mxfp4_moe_timed_calls.argtypes = []
    lib.mxfp4_moe_phase_times.restype = ci
    lib.mxfp4_moe_phase_times.argtypes = [ci, vp, vp, ci]
    _lib = lib
    return lib


def _check(rc: int, lib) -> None:
    if rc != 0:
        msg = lib.mxfp4_last_error().decode(errors="replace")
        if rc == -1:
            raise ValueError(msg)
        raise RuntimeError(f"MXFP4 kernel failed ({rc}): {msg}")


def _device_for(t: torch.Tensor) -> torch.device:
    if t.is_cuda:
        return t.device
    if not torch.cuda.is_available():
        raise RuntimeError("the MXFP4 kernels need a HIP device (torch.cuda.is_available() is False)")
    return torch.device("cuda", torch.cuda.current_device())


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _layouts(experts):
    """(layout pointer array or None, extra flags) of a layer for the mxfp4_moe_*_fl calls: its
    load-time layout copies (ExpertLayer.layout_pointers), or none for objects without them."""
    fn = getattr(experts, "layout_pointers", None)
    if fn is None:
        fn = getattr(experts, "forward_layout_pointers", None)
        return (fn() if fn is not None else None), 0
    return fn()


def _u8(t: torch.Tensor, dev: torch.device, name: str) -> torch.Tensor:
    if t.dtype != torch.uint8:
        raise ValueError(f"{name} must be uint8, got {t.dtype}")
    t = t.to(dev, non_blocking=True).contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


class MXFP4Kernel:
    """The reference's MXFP4Kernel (lazy_lora/native/__init__.py:19-74) on MI355X."""

    def __init__(self, lib):
        self.lib = lib

    # -- single-expert products --------------------------------------------------------------
    def gemm(self, x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
        """y[M, R] = x[M, K] @ W^T for packed W[R, K] (mxfp4_gemm.c:64-94). fp32 result."""
        if x.dim() != 2:
            raise ValueError(f"x must be 2-D [M, K], got {tuple(x.shape)}")
        M, K = x.shape
        R = packed.shape[0]
        _check_weight(packed, scales, R, K)
        dev = _device_for(x)
        xd = _aligned(x.to(dev, non_blocking=True).contiguous().float())
        p, s = _u8(packed, dev, "packed"), _u8(scales, dev, "scales")
        y = torch.empty((M, R), dtype=torch.float32, device=dev)
        if M and R:
            nws = self.lib.mxfp4_gemm_workspace_size(M, K, R)
            ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=dev)
            _check(self.lib.mxfp4_gemm(y.data_ptr(), xd.data_ptr(), p.data_ptr(), s.data_ptr(), M, K, R,
                                       ws.data_ptr(), nws, _stream(dev)), self.lib)
        return y if x.is_cuda else y.cpu()

    def gemm_t(self, dy: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
        """y[M, K] = dy[M, R] @ W for packed W[R, K] (mxfp4_gemm.c:96-129). fp32 result."""
        if dy.dim() != 2:
            raise ValueError(f"dy must be 2-D [M, R], got {tuple(dy.shape)}")
        M, R = dy.shape
        if packed.dim() != 2:
            raise ValueError(f"packed must be 2-D [R, K/2], got {tuple(packed.shape)}")
        K = packed.shape[1] * 2
        if packed.shape[0] != R:
            raise ValueError(f"dy has {R} columns but W has {packed.shape[0]} rows")
        _check_weight(packed, scales, R, K)
        dev = _device_for(dy)
        dyd = _aligned(dy.to(dev, non_blocking=True).contiguous().float())
        p, s = _u8(packed, dev, "packed"), _u8(scales, dev, "scales")
        y = torch.zeros((M, K), dtype=torch.float32, device=dev)
        if M and R:
            nws = self.lib.mxfp4_gemm_t_workspace_size(M, K, R)
            ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=dev)
            _check(self.lib.mxfp4_gemm_t(y.data_ptr(), dyd.data_ptr(), p.data_ptr(), s.data_ptr(), M, K, R,
                                         ws.data_ptr(), nws, _stream(dev)), self.lib)
        return y if dy.is_cuda else y.cpu()

    def dequant(self, packed: torch.Tensor, scales: torch.Tensor, out_dtype=torch.float32) -> torch.Tensor:
        """W[R, K] from the packed bytes, bit-exact (mxfp4_gemm.c:142-150): fp32 by default, as
        the reference's; out_dtype=torch.bfloat16 decodes straight to bf16 (the same values, each
        exact in bf16), any other floating dtype converts the fp32 result."""
        if packed.dim() != 2:
            raise ValueError(f"packed must be 2-D [R, K/2], got {tuple(packed.shape)}")
        if not out_dtype.is_floating_point:
            raise ValueError(f"out_dtype must be a floating dtype, got {out_dtype}")
        R, K = packed.shape[0], packed.shape[1] * 2
        _check_weight(packed, scales, R, K)
        dev = _device_for(packed)
        p, s = _u8(packed, dev, "packed"), _u8(scales, dev, "scales")
        bf16 = out_dtype == torch.bfloat16
        w = torch.empty((R, K), dtype=torch.bfloat16 if bf16 else torch.float32, device=dev)
        if R:
            fn = self.lib.mxfp4_dequant_bf16 if bf16 else self.lib.mxfp4_dequant
            _check(fn(w.data_ptr(), p.data_ptr(), s.data_ptr(), K, R, _stream(dev)), self.lib)
        if w.dtype != out_dtype:
            w = w.to(out_dtype)
        return w if packed.is_cuda else w.cpu()

    def threads(self) -> int:
        """Parallel width of the device (compute units), the analogue of mxfp4_threads()."""
        return int(self.lib.mxfp4_threads())

    def forward_layout(self, packed: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
        """The forward layout (mxfp4_forward_layout) of stacked packed matrices [E, R, K/2] uint8
        and their scales [E, R, K/32] uint8 in HBM, K a multiple of 512: a new flat uint8 tensor
        on the same device. No counterpart in the reference; ExpertLayer.prepare_forward_layout
        keeps these for a resident layer."""
        if packed.dtype != torch.uint8 or packed.dim() != 3 or not packed.is_cuda:
            raise ValueError("packed must be a CUDA uint8 tensor [E, R, K/2]")
        E, R, Kh = packed.shape
        K = 2 * Kh
        if K % 512:
            raise ValueError(f"the forward layout needs K to be a multiple of 512, got K={K}")
        if scales.dtype != torch.uint8 or tuple(scales.shape) != (E, R, K // 32) or scales.device != packed.device:
            raise ValueError("scales must be a uint8 tensor [E, R, K/32] on the codes' device")
        src, ssrc = packed.contiguous(), scales.contiguous()
        if src.data_ptr() % 16:
            src = src.clone()
        if ssrc.data_ptr() % 16:
            ssrc = ssrc.clone()
        n = int(self.lib.mxfp4_forward_layout_bytes(E, R, K))
        out = torch.empty(max(n, 16), dtype=torch.uint8, device=packed.device)
        _check(self.lib.mxfp4_forward_layout(out.data_ptr(), src.data_ptr(), ssrc.data_ptr(), E, R, K,
                                             _stream(packed.device)),
               self.lib)
        return out

    def backward_layout(self, packed: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
        """The backward layout (mxfp4_backward_layout) of stacked packed matrices [E, R, K/2] uint8
        and their scales [E, R, K/32] uint8 in HBM, R a multiple of 32 and K of 256: a new flat
        uint8 tensor on the same device. No counterpart in the reference;
        ExpertLayer.prepare_backward_layout keeps these for a resident layer."""
        if packed.dtype != torch.uint8 or packed.dim() != 3 or not packed.is_cuda:
            raise ValueError("packed must be a CUDA uint8 tensor [E, R, K/2]")
        E, R, Kh = packed.shape
        K = 2 * Kh
        if R % 32 or K % 256:
            raise ValueError(f"the backward layout needs R a multiple of 32 and K of 256, got R={R}, K={K}")
        if scales.dtype != torch.uint8 or tuple(scales.shape) != (E, R, K // 32) or scales.device != packed.device:
            raise ValueError("scales must be a uint8 tensor [E, R, K/32] on the codes' device")
        src, ssrc = packed.contiguous(), scales.contiguous()
        if src.data_ptr() % 16:
            src = src.clone()
        if ssrc.data_ptr() % 16:
            ssrc = ssrc.clone()
        n = int(self.lib.mxfp4_backward_layout_bytes(E, R, K))
        out = torch.empty(max(n, 16), dtype=torch.uint8, device=packed.device)
        _check(self.lib.mxfp4_backward_layout(out.data_ptr(), src.data_ptr(), ssrc.data_ptr(), E, R, K,
                                              _stream(packed.device)),
               self.lib)
        return out

    # -- routed layer ------------------------------------------------------------------------
    def routed_forward(self, h: torch.Tensor, topk_indices: torch.Tensor, topk_weights: torch.Tensor,
                       experts, act="swiglu", save_for_backward: bool = False,
                       workspace: Optional[torch.Tensor] = None, lora=None) -> torch.Tensor:
        """sum_e w_e(token) * expert_e(h) for one routed-expert layer; fp32 [N, D].

        Mirrors LazyLoRATrainer._routed_experts_forward (lazy_lora/trainer/lazy_trainer.py:806-834).
        `experts` is an ExpertLayer (stacked packed weights in HBM). `lora` is the layer's
        adapters: an object with gate_lora / up_lora / down_lora (the reference's LayerLoRABundle)
        or a (gate, up, down) sequence, each with lora_A [r, in], lora_B [out, r] and scaling
        (LazyLoRALinear, lazy_lora/core/lora_layer.py:53-97); None = LoRA off.
        """
        call = _RoutedCall(self.lib, h, topk_indices, topk_weights, experts, act, workspace)
        lo = _LoraCall(lora, call.dev, call.D, call.F)
        out = torch.empty((call.N, call.D), dtype=torch.float32, device=call.dev)
        layouts, lflags = _layouts(experts)
        _check(self.lib.mxfp4_moe_forward_fl(
            out.data_ptr(), call.h.data_ptr(), call.h_dtype, call.idx.data_ptr(), call.idx_dtype,
            call.w.data_ptr(), call.N, call.k, *experts.pointers(), layouts, experts.E,
            call.D, call.F, call.act, lo.ptrs, lo.scaling, lo.r, (MOE_SAVE if save_for_backward else 0) | lflags,
            call.ws.data_ptr(), call.nws, _stream(call.dev)), self.lib)
        return out

    def routed_backward(self, h: torch.Tensor, topk_indices: torch.Tensor, topk_weights: torch.Tensor,
                        experts, grad_out: torch.Tensor, act="swiglu", reuse_forward: bool = False,
                        workspace: Optional[torch.Tensor] = None, lora=None):
        """(dL/dh [N, D] fp32, dL/dtopk_weights [N, k] fp32) for upstream grad_out [N, D]; with
        `lora`, also the adapter gradients (gate_A, gate_B, up_A, up_B, down_A, down_B), fp32,
        summed over the experts (what the reference accumulates, lazy_trainer.py:866-876).

        Mirrors _routed_experts_backward (lazy_trainer.py:836-880). With reuse_forward=True the
        workspace must come from a routed_forward(save_for_backward=True) call on the same inputs
        and adapters; the routing and gate/up products are then not recomputed.
        """
        if reuse_forward and workspace is None:
            raise ValueError("reuse_forward=True needs the workspace of a routed_forward(save_for_backward=True) "
                             "call on the same inputs")
        call = _RoutedCall(self.lib, h, topk_indices, topk_weights, experts, act, workspace)
        lo = _LoraCall(lora, call.dev, call.D, call.F)
        if grad_out.shape != (call.N, call.D):
            raise ValueError(f"grad_out must be [{call.N}, {call.D}], got {tuple(grad_out.shape)}")
        g = _aligned(grad_out.to(call.dev, non_blocking=True).contiguous().float())
        grad_h = torch.empty((call.N, call.D), dtype=torch.float32, device=call.dev)
        grad_w = torch.empty((call.N, call.k), dtype=torch.float32, device=call.dev)
        grads = [torch.empty_like(t) for t in lo.tensors]
        gptrs = (ctypes.c_void_p * 6)(*[t.data_ptr() for t in grads]) if lo.r else None
        layouts, lflags = _layouts(experts)
        _check(self.lib.mxfp4_moe_backward_fl(
            grad_h.data_ptr(), grad_w.data_ptr(), g.data_ptr(), call.h.data_ptr(), call.h_dtype,
            call.idx.data_ptr(), call.idx_dtype, call.w.data_ptr(), call.N, call.k, *experts.pointers(),
            layouts, experts.E, call.D, call.F, call.act, lo.ptrs, lo.scaling, lo.r, gptrs,
            (MOE_REUSE_FORWARD if reuse_forward else 0) | lflags, call.ws.data_ptr(), call.nws,
            _stream(call.dev)), self.lib)
        if lo.r:
            return grad_h, grad_w, tuple(grads)
        return grad_h, grad_w

    # -- router ----------------------------------------------------------------------------
    def router_topk(self, logits: torch.Tensor, bias: Optional[torch.Tensor], top_k: int,
                    routed_scaling_factor: float = 1.0,
                    renormalize: bool = True) -> Tuple[torch.Tensor, torch.Tensor]:
        """(topk_idx [N, k] int64, topk_w [N, k] fp32) from gate logits [N, E] on the GPU: the
        selection of KimiK3MoERouter.forward (lazy_lora/core/moe_router.py:86-99)."""
        lg, N, E = self._logits(logits)
        self._router_limits(E, top_k)
        b = None
        if bias is not None:
            if tuple(bias.shape) != (E,):
                raise ValueError(f"bias must be [{E}], got {tuple(bias.shape)}")
            b = bias.to(lg.device, non_blocking=True).contiguous().float()
        idx = torch.empty((N, top_k), dtype=torch.int64, device=lg.device)
        w = torch.empty((N, top_k), dtype=torch.float32, device=lg.device)
        _check(self.lib.mxfp4_router_topk(idx.data_ptr(), w.data_ptr(), lg.data_ptr(),
                                          b.data_ptr() if b is not None else None, N, E, top_k,
                                          float(routed_scaling_factor), 1 if renormalize else 0,
                                          _stream(lg.device)), self.lib)
        return idx, w

    def router_topk_backward(self, logits: torch.Tensor, topk_idx: torch.Tensor, grad_w: torch.Tensor,
                             routed_scaling_factor: float = 1.0, renormalize: bool = True) -> torch.Tensor:
        """dL/dlogits [N, E] fp32 for dL/dtopk_w [N, k] (the autograd of moe_router.py:86-98)."""
        lg, N, E = self._logits(logits)
        if topk_idx.dim() != 2 or topk_idx.shape[0] != N:
            raise ValueError(f"topk_idx must be [{N}, k], got {tuple(topk_idx.shape)}")
        top_k = topk_idx.shape[1]
        self._router_limits(E, top_k)
        if tuple(grad_w.shape) != tuple(topk_idx.shape):
            raise ValueError("grad_w and topk_idx must have the same shape")
        idx = topk_idx.to(lg.device, non_blocking=True).contiguous().long()
        g = grad_w.to(lg.device, non_blocking=True).contiguous().float()
        out = torch.empty((N, E), dtype=torch.float32, device=lg.device)
        _check(self.lib.mxfp4_router_topk_backward(out.data_ptr(), idx.data_ptr(), g.data_ptr(), lg.data_ptr(),
                                                   N, E, top_k, float(routed_scaling_factor),
                                                   1 if renormalize else 0, _stream(lg.device)), self.lib)
        return out

    @staticmethod
    def _logits(logits: torch.Tensor):
        if logits.dim() != 2:
            raise ValueError(f"logits must be [N, E], got {tuple(logits.shape)}")
        dev = _device_for(logits)
        return logits.to(dev, non_blocking=True).contiguous().float(), logits.shape[0], logits.shape[1]

    @staticmethod
    def _router_limits(E: int, top_k: int) -> None:
        if not 0 < E <= 4096:
            raise ValueError(f"the router kernel takes 1..4096 experts, got {E}")
        if not 1 <= top_k <= min(E, 64):
            raise ValueError(f"top_k must lie in [1, min(E, 64)] = [1, {min(E, 64)}], got {top_k}")

    def moe_workspace_bytes(self, N: int, k: int, E: int, D: int, F: int) -> int:
        return int(self.lib.mxfp4_moe_workspace_size(N, k, E, D, F))

    def set_timing(self, enable: bool) -> None:
        """Record per-phase HIP events inside routed-layer calls on this thread (no syncs)."""
        _check(self.lib.mxfp4_moe_timing(1 if enable else 0), self.lib)

    def phase_times(self):
        """[(phase name, ms), ...] for every call recorded since set_timing(True) (at most the
        last 128 calls). Waits for those calls to finish."""
        out = []
        n_calls = int(self.lib.mxfp4_moe_timed_calls())
        ms = (ctypes.c_float * 16)()
        names = (ctypes.c_char_p * 16)()
        for c in range(max(0, n_calls - 128), n_calls):
            n = self.lib.mxfp4_moe_phase_times(c, ctypes.addressof(ms), ctypes.addressof(names), 16)
            if n < 0:
                _check(n, self.lib)
            out.append([(names[i].decode(), float(ms[i])) for i in range(n)])
        return out

    def route_status(self, workspace: torch.Tensor) -> int:
        """Routing flags left in a routed-layer workspace (bit 0: expert id out of range). Syncs."""
        flags = ctypes.c_int(0)
        _check(self.lib.mxfp4_moe_route_status(workspace.data_ptr(), ctypes.addressof(flags),
                                               _stream(workspace.device)), self.lib)
        return flags.value


def _check_weight(packed: torch.Tensor, scales: torch.Tensor, R: int, K: int) -> None:
    if packed.dim() != 2 or packed.shape[0] != R or packed.shape[1] * 2 != K:
        raise ValueError(f"packed must be [{R}, {K // 2}], got {tuple(packed.shape)}")
    if K % 32:
        raise ValueError(f"K = {K} is not a multiple of the MX block size 32")
    if tuple(scales.shape) != (R, K // 32):
        raise ValueError(f"scales must be [{R}, {K // 32}], got {tuple(scales.shape)}")


class _RoutedCall:
    """Validated, device-resident arguments of one routed-layer call."""

    def __init__(self, lib, h, topk_indices, topk_weights, experts, act, workspace):
        if h.dim() != 2:
            raise ValueError(f"h must be [N, D], got {tuple(h.shape)}")
        self.N, self.D = h.shape
        if self.D != experts.D:
            raise ValueError(f"h has width {self.D} but the experts take {experts.D}")
        if topk_indices.dim() != 2 or topk_indices.shape[0] != self.N:
            raise ValueError(f"topk_indices must be [{self.N}, k], got {tuple(topk_indices.shape)}")
        if tuple(topk_weights.shape) != tuple(topk_indices.shape):
            raise ValueError("topk_weights and topk_indices must have the same shape")
        if act not in _ACTS:
            raise ValueError(f"unknown activation {act!r}")
        self.k = topk_indices.shape[1]
        self.F = experts.F
        self.act = _ACTS[act]
        self.dev = experts.device
        if h.dtype == torch.bfloat16:
            self.h_dtype = BF16
        elif h.dtype == torch.float32:
            self.h_dtype = F32
        else:
            raise ValueError(f"h must be float32 or bfloat16, got {h.dtype}")
        self.h = _aligned(h.to(self.dev, non_blocking=True).contiguous())
        if topk_indices.dtype == torch.int64:
            self.idx_dtype = I64
        elif topk_indices.dtype == torch.int32:
            self.idx_dtype = I32
        else:
            raise ValueError(f"topk_indices must be int32 or int64, got {topk_indices.dtype}")
        if not topk_indices.is_cuda and topk_indices.numel():
            lo, hi = int(topk_indices.min()), int(topk_indices.max())
            if lo < 0 or hi >= experts.E:
                raise ValueError(f"expert ids must lie in [0, {experts.E}), got [{lo}, {hi}]")
        self.idx = topk_indices.to(self.dev, non_blocking=True).contiguous()
        self.w = topk_weights.to(self.dev, non_blocking=True).contiguous().float()
        self.nws = int(lib.mxfp4_moe_workspace_size(self.N, self.k, experts.E, self.D, self.F))
        if workspace is None:
            workspace = torch.empty(max(self.nws, 1), dtype=torch.uint8, device=self.dev)
        elif workspace.numel() < self.nws or workspace.dtype != torch.uint8:
            raise ValueError(f"workspace must be uint8 with at least {self.nws} bytes")
        self.ws = workspace


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """t itself when its data starts on a 16-byte boundary, else an aligned copy."""
    return t if t.data_ptr() % 16 == 0 else t.clone()


class _LoraCall:
    """Validated fp32 device copies of a layer's three adapters and their ctypes arrays."""

    def __init__(self, lora, dev, D: int, F: int):
        self.tensors, self.ptrs, self.scaling, self.r = [], None, None, 0
        if lora is None:
            return
        mods = (lora.gate_lora, lora.up_lora, lora.down_lora) if hasattr(lora, "gate_lora") else tuple(lora)
        if len(mods) != 3:
            raise ValueError("lora must hold three adapters: gate, up, down")
        ins, outs = (D, D, F), (F, F, D)
        r = None
        for mod, n_in, n_out, name in zip(mods, ins, outs, ("gate", "up", "down")):
            A, B = getattr(mod, "lora_A", None), getattr(mod, "lora_B", None)
            if A is None or B is None:
                raise ValueError(f"{name} adapter has no lora_A / lora_B (rank 0 adapters are not supported)")
            if float(getattr(mod, "dropout_rate", 0.0) or 0.0) != 0.0:
                raise ValueError("LoRA dropout is not supported: the backward recomputes the layer, so the "
                                 "reference runs with lora_dropout = 0")
            ra = A.shape[0]
            if tuple(A.shape) != (ra, n_in) or tuple(B.shape) != (n_out, ra):
                raise ValueError(f"{name} adapter must be A [r, {n_in}], B [{n_out}, r]; got "
                                 f"{tuple(A.shape)}, {tuple(B.shape)}")
            if r is None:
                r = ra
            elif ra != r:
                raise ValueError("the three adapters must share one rank")
            self.tensors += [_aligned(torch.as_tensor(A).detach().to(dev, torch.float32).contiguous()),
                             _aligned(torch.as_tensor(B).detach().to(dev, torch.float32).contiguous())]
        if not 1 <= r <= 32:
            raise ValueError(f"LoRA rank must lie in [1, 32], got {r}")
        self.r = r
        self.ptrs = (ctypes.c_void_p * 6)(*[t.data_ptr() for t in self.tensors])
        self.scaling = (ctypes.c_float * 3)(*[float(m.scaling) for m in mods])


def _unavailable(why: str) -> None:
    if os.environ.get("LAZYLORA_NATIVE_STRICT", "") == "1":
        raise RuntimeError(f"MI355X MXFP4 kernels unavailable: {why}")
    print(f"[!] MI355X MXFP4 kernels not available ({why}); callers use their fallback path",
          file=sys.stderr, flush=True)


def kernel() -> Optional[MXFP4Kernel]:
    """The MXFP4 kernel object, or None (native/__init__.py:77-97): None when
    LAZYLORA_NO_NATIVE=1, and, after one printed warning, when the library is missing or fails
    to load or no HIP device is visible (LAZYLORA_NATIVE_STRICT=1: raise RuntimeError instead).
    A failed attempt is not repeated, as in the reference."""
    global _kernel, _tried
    if os.environ.get("LAZYLORA_NO_NATIVE", "") == "1":
        return None
    if _kernel is not None:
        return _kernel
    strict = os.environ.get("LAZYLORA_NATIVE_STRICT", "") == "1"
    if _tried and not strict:
        return None
    _tried = True
    try:
        lib = _load_library()
    except (RuntimeError, OSError) as exc:
        _unavailable(str(exc))
        return None
    if not torch.cuda.is_available():
        _unavailable("no HIP device is visible")
        return None
    _kernel = MXFP4Kernel(lib)
    return _kernel
