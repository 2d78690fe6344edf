"""
The Kimi-K3 MoE router on MI355X, with the interface of lazy_lora/core/moe_router.py.

`KimiK3MoERouter.forward(x, weight, bias)` returns (topk_indices [N, k] int64, topk_weights
[N, k] fp32) like the reference (moe_router.py:55-123): the gate product logits = x . W^T runs
in fp32 in the platform BLAS (a plain dense GEMM), and the selection -- sigmoid scores, bias
added for selection only, top-k in descending order, unbiased scores gathered, renormalised
with +1e-20, scaled -- runs in one HIP kernel, one wave per token, so the indices feed the
routed-expert layer without a host round trip. Gradients flow from topk_weights back through
the logits into x (and the gate weight, if it requires grad), as torch autograd does through the
reference's torch branch; the trainer relies on that (lazy_lora/trainer/lazy_trainer.py:842-844).

Differences from the reference, all deliberate:
  * equal biased scores go to the lower expert id first (torch.topk leaves their order
    unspecified; the NumPy branch's argsort is not stable either);
  * results land on x's device (CPU and NumPy inputs are computed on the GPU and copied
    back); a missing library raises instead of falling back to a CPU path;
  * top_k <= 64 and num_experts <= 4096 (the reference configurations use 16 of 896).
"""
from typing import List, Optional, Tuple, Union

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from lazylora_amd.native import kernel


def _native():
    k = kernel()
    if k is None:
        raise RuntimeError("LAZYLORA_NO_NATIVE=1: the MI355X router is disabled")
    return k


class _Select(torch.autograd.Function):
    """Selection on device logits; backward gives dL/dlogits from dL/dtopk_weights."""

    @staticmethod
    def forward(ctx, logits, bias, top_k, scale, renormalize):
        idx, w = _native().router_topk(logits, bias, top_k, scale, renormalize)
        ctx.mark_non_differentiable(idx)
        ctx.save_for_backward(logits, idx)
        ctx.scale, ctx.renormalize = scale, renormalize
        return idx, w

    @staticmethod
    def backward(ctx, _grad_idx, grad_w):
        logits, idx = ctx.saved_tensors
        grad_logits = None
        if grad_w is not None and ctx.needs_input_grad[0]:
            grad_logits = _native().router_topk_backward(logits, idx, grad_w, ctx.scale, ctx.renormalize)
        # the bias only steers the (non-differentiable) selection: no gradient, as in torch
        return grad_logits, None, None, None, None


def route(x: Union[torch.Tensor, np.ndarray], weight: Union[torch.Tensor, np.ndarray],
          bias: Optional[Union[torch.Tensor, np.ndarray]] = None, top_k: int = 16,
          routed_scaling_factor: float = 1.0, renormalize: bool = True):
    """(topk_indices [N, k] int64, topk_weights [N, k] fp32) for tokens x [..., hidden] and gate
    weight [E, hidden] (moe_router.py:81-99). NumPy in, NumPy out; torch tensors come back on
    x's device."""
    as_numpy = isinstance(x, np.ndarray)
    xt = torch.from_numpy(np.asarray(x, np.float32)) if as_numpy else x
    if xt.is_cuda:
        dev = xt.device
    elif torch.cuda.is_available():
        dev = torch.device("cuda", torch.cuda.current_device())
    else:
        raise RuntimeError("the MI355X router needs a HIP device (torch.cuda.is_available() is False)")
    w = torch.as_tensor(weight).to(dev, torch.float32)
    if w.dim() != 2:
        raise ValueError(f"weight must be [num_experts, hidden], got {tuple(w.shape)}")
    hidden = w.shape[1]
    if xt.shape[-1] != hidden:
        raise ValueError(f"x has width {xt.shape[-1]} but the gate takes {hidden}")
    b = None if bias is None else torch.as_tensor(bias).to(dev, torch.float32)
    logits = F.linear(xt.reshape(-1, hidden).to(dev, torch.float32), w)   # [N, E] fp32
    idx, tw = _Select.apply(logits, b, int(top_k), float(routed_scaling_factor), bool(renormalize))
    if as_numpy:
        return idx.cpu().numpy(), tw.detach().cpu().numpy()
    if not xt.is_cuda:
        return idx.to(xt.device), tw.to(xt.device)
    return idx, tw


class KimiK3MoERouter(nn.Module):
    """KimiK3MoERouter (lazy_lora/core/moe_router.py:23-135) with the selection on MI355X."""

    def __init__(self, hidden_size: int = 7168, num_experts: int = 896, top_k: int = 16,
                 routed_scaling_factor: float = 1.0, renormalize: bool = True, use_bias: bool = True,
                 device: Optional[Union[str, torch.device]] = None):
        super().__init__()
        self.weight = nn.Parameter(torch.empty(num_experts, hidden_size, device=device))
        self.bias = nn.Parameter(torch.zeros(num_experts, device=device)) if use_bias else None
        nn.init.normal_(self.weight, std=0.02)
        self.hidden_size = hidden_size
        self.num_experts = num_experts
        self.top_k = top_k
        self.routed_scaling_factor = routed_scaling_factor
        self.renormalize = renormalize
        self.use_bias = use_bias

    def forward(self, x, weight=None, bias=None) -> Tuple[torch.Tensor, torch.Tensor]:
        """(topk_indices [N, top_k] int64, topk_weights [N, top_k] fp32). `weight`/`bias`
        override the module's own (each layer streams its own gate, moe_router.py:68-73)."""
        if weight is None:
            weight = self.weight
        if bias is None:
            bias = self.bias
        return route(x, weight, bias, self.top_k, self.routed_scaling_factor, self.renormalize)

    @staticmethod
    def get_active_expert_set(topk_indices) -> List[int]:
        """Sorted unique expert ids of a batch (moe_router.py:125-135)."""
        if isinstance(topk_indices, torch.Tensor):
            ids = torch.unique(topk_indices).cpu().tolist()
        else:
            ids = np.unique(np.asarray(topk_indices)).tolist()
        return sorted(int(e) for e in ids)
