"""
The routed-expert map of one MoE layer as a single autograd node, on MI355X.

Mirrors RoutedExpertsFunction and the two expert sweeps of the reference trainer
(lazy_lora/trainer/lazy_trainer.py:45-77, :806-880): forward returns the fp32
routed sum, backward returns (dL/dh_latent cast to h's dtype, dL/dtopk_weights). The expert
loops run on the GPU in a few launches each (routing histogram/scan/placement, fused
gate/up/GLU, down product with the combine weight, deterministic combine; and the three
transposed products with the GLU derivative in backward).

As in the reference, a `cached` routed sum short-circuits the forward (the backward replay,
lazy_trainer.py:60-66); here the backward can additionally reuse the forward's gate/up
activations when the same workspace is kept (save_for_backward=True), which removes the
recompute of the gate/up products that the reference performs (:859).

The layer's LoRA adapters (gate, up, down; shared by its experts, lazy_trainer.py:130-134) are
optional: their terms are added on the device and their gradients accumulated into them.
"""
from typing import Optional

import torch

from lazylora_amd.experts import ExpertLayer
from lazylora_amd.native import kernel
from lazylora_amd.streaming import BundleStager, compact_ids


def _native():
    k = kernel()
    if k is None:
        raise RuntimeError("the MI355X routed-expert path is unavailable: LAZYLORA_NO_NATIVE=1 is set, or the "
                           "native library failed to load, or no HIP device is visible (set "
                           "LAZYLORA_NATIVE_STRICT=1 to see the underlying error)")
    return k


def routed_experts_forward(h_latent: torch.Tensor, topk_indices: torch.Tensor, topk_weights: torch.Tensor,
                           layer: ExpertLayer, act: str = "swiglu", save_for_backward: bool = False,
                           workspace: Optional[torch.Tensor] = None, lora=None) -> torch.Tensor:
    """sum_e w_e(token) * expert_e(h_latent) in fp32 (lazy_trainer.py:806-834); `lora` = the
    layer's (gate, up, down) adapters or None."""
    return _native().routed_forward(h_latent, topk_indices, topk_weights, layer, act=act,
                                    save_for_backward=save_for_backward, workspace=workspace, lora=lora)


def routed_experts_backward(h_latent: torch.Tensor, topk_indices: torch.Tensor, topk_weights: torch.Tensor,
                            layer: ExpertLayer, grad_out: torch.Tensor, act: str = "swiglu",
                            reuse_forward: bool = False, workspace: Optional[torch.Tensor] = None, lora=None):
    """(dL/dh_latent, dL/dtopk_weights) (lazy_trainer.py:836-880); grad_h in h's dtype. With
    `lora` the adapters' gradients are accumulated into them as the reference does
    (accumulate_grad, lazy_trainer.py:866-876)."""
    res = _native().routed_backward(h_latent, topk_indices, topk_weights, layer, grad_out, act=act,
                                    reuse_forward=reuse_forward, workspace=workspace, lora=lora)
    if lora is not None:
        accumulate_lora_grads(lora, res[2])
    return res[0].to(h_latent.dtype), res[1].to(topk_weights.dtype)


def _adapters(lora):
    return (lora.gate_lora, lora.up_lora, lora.down_lora) if hasattr(lora, "gate_lora") else tuple(lora)


def accumulate_lora_grads(lora, grads) -> None:
    """Adds (gate_A, gate_B, up_A, up_B, down_A, down_B) gradients to the adapters: through their
    accumulate_grad when they have one (LazyLoRALinear, lora_layer.py:258-308), else into
    lora_A.grad / lora_B.grad."""
    for n, mod in enumerate(_adapters(lora)):
        gA, gB = grads[2 * n], grads[2 * n + 1]
        if hasattr(mod, "accumulate_grad"):
            mod.accumulate_grad(gA, gB)
            continue
        for p, gp in ((mod.lora_A, gA), (mod.lora_B, gB)):
            gp = gp.to(p.device, p.dtype)
            if p.grad is None:
                p.grad = gp.clone()
            else:
                p.grad.add_(gp)


class RoutedExpertsFunction(torch.autograd.Function):
    """autograd node: (h_latent, topk_weights, topk_indices, layer, act, cached, lora) -> routed
    sum. The LoRA adapters are not inputs of the node; their gradients are accumulated into them
    in backward, as the reference's node does (lazy_trainer.py:45-77, :866-876)."""

    @staticmethod
    def forward(ctx, h_latent, topk_weights, topk_indices, layer, act="swiglu", cached=None, lora=None):
        k = _native()
        ws = None
        if cached is not None:
            # the backward replay: the routed sum is already known, and the backward recomputes
            # what it needs (lazy_trainer.py:60-66)
            out = cached.to(torch.float32)
        else:
            ws = torch.empty(max(k.moe_workspace_bytes(h_latent.shape[0], topk_indices.shape[1], layer.E,
                                                       layer.D, layer.F), 1),
                             dtype=torch.uint8, device=layer.device)
            out = k.routed_forward(h_latent, topk_indices, topk_weights, layer, act=act,
                                   save_for_backward=True, workspace=ws, lora=lora)
        ctx.save_for_backward(h_latent, topk_weights, topk_indices)
        # the workspace holds the forward's routing and gate|up only until the first backward
        # has used them; a second backward (retain_graph=True) recomputes them
        ctx.layer, ctx.act, ctx.ws, ctx.lora = layer, act, ws, lora
        return out

    @staticmethod
    def backward(ctx, grad_out):
        h_latent, topk_weights, topk_indices = ctx.saved_tensors
        ws, ctx.ws = ctx.ws, None
        grad_h, grad_w = routed_experts_backward(h_latent, topk_indices, topk_weights, ctx.layer,
                                                 grad_out, act=ctx.act, reuse_forward=ws is not None,
                                                 workspace=ws, lora=ctx.lora)
        return grad_h, grad_w, None, None, None, None, None


def layer_from_stream(expert_streamer, layer_idx, active_experts, num_experts=None, device=None) -> ExpertLayer:
    """The active experts of one layer, supplied by the reference's streamer as packed
    ExpertWeightBundles (DynamicExpertStreamer.stream_experts, expert_streamer.py:315-369, in disk
    order), placed by expert id in an HBM ExpertLayer of num_experts experts (absent experts
    hold zero codes). StreamedRoutedExpertsFunction uses the compact form, stream_compact."""
    pairs = list(expert_streamer.stream_experts(layer_idx, active_experts))
    return ExpertLayer.from_bundles(pairs, device=device, num_experts=num_experts)


_stagers = {}


def _stager(device) -> BundleStager:
    dev = torch.device(device)
    if dev not in _stagers:
        _stagers[dev] = BundleStager(dev)
    return _stagers[dev]


def stream_compact(expert_streamer, layer_idx, active_experts, topk_indices, device):
    """(layer, ids on the layer): the bundles of `active_experts`, consumed from the streamer's
    generator as it yields them and staged into a compact HBM layer of only those experts
    (BundleStager), and topk_indices mapped onto it; routed ids outside the active set map to -1
    and are skipped by the routed call, as the reference's sweep over the streamed experts never
    visits them (lazy_trainer.py:806-880)."""
    active = list(active_experts)
    layer, ids = _stager(device).stage(expert_streamer.stream_experts(layer_idx, active), len(active))
    return layer, compact_ids(topk_indices, ids, device)


class StreamedRoutedExpertsFunction(torch.autograd.Function):
    """The reference node's own signature (lazy_trainer.py:45-77):
    apply(h_latent, topk_weights, topk_indices, trainer, layer_idx, bundle, active_experts, cached).

    As in the reference, the experts are streamed once in forward (skipped when `cached` holds
    the routed sum) and once more in backward, and nothing expert-sized stays alive between the
    two: each pass takes the packed bundles of `trainer.expert_streamer.stream_experts(layer_idx,
    active_experts)` as the generator yields them, stages them through pinned buffers into a
    compact HBM layer of only those experts on a copy stream (the DMA of one expert overlaps the
    next bundle's arrival), and runs the whole layer in one call. Tokens' choices outside the
    active set contribute nothing (no expert term, no adapter term, zero grad_w), as in the
    reference's sweep. The activation is SiTU-GLU and `bundle` is the layer's LoRALayerBundle
    (its gate/up/down adapters), as in _routed_experts_forward/_backward
    (lazy_trainer.py:806-880); the adapters' gradients are accumulated into them with
    accumulate_grad. The streamer must hand over packed bundles (keep_packed, which holds
    whenever kernel() is not None)."""

    @staticmethod
    def forward(ctx, h_latent, topk_weights, topk_indices, trainer, layer_idx, bundle, active_experts, cached=None):
        if cached is not None:
            out = cached.to(torch.float32)
        elif len(active_experts) == 0:  # nothing streamed: the reference's sweep adds nothing
            out = torch.zeros(h_latent.shape, dtype=torch.float32, device=h_latent.device)
        else:
            dev = _device(h_latent)
            layer, idx = stream_compact(trainer.expert_streamer, layer_idx, active_experts, topk_indices, dev)
            out = routed_experts_forward(h_latent, idx, topk_weights, layer, act="situ", lora=_lora(bundle))
            del layer
            out = out.to(h_latent.device)
        ctx.save_for_backward(h_latent, topk_weights, topk_indices)
        ctx.trainer, ctx.layer_idx, ctx.bundle, ctx.active_experts = trainer, layer_idx, bundle, active_experts
        return out

    @staticmethod
    def backward(ctx, grad_out):
        h_latent, topk_weights, topk_indices = ctx.saved_tensors
        if len(ctx.active_experts) == 0:
            return (torch.zeros_like(h_latent), torch.zeros_like(topk_weights), None, None, None, None, None, None)
        dev = _device(h_latent)
        layer, idx = stream_compact(ctx.trainer.expert_streamer, ctx.layer_idx, ctx.active_experts, topk_indices, dev)
        grad_h, grad_w = routed_experts_backward(h_latent, idx, topk_weights, layer, grad_out,
                                                 act="situ", lora=_lora(ctx.bundle))
        return (grad_h.to(h_latent.device), grad_w.to(topk_weights.device), None, None, None, None, None, None)


def _device(h_latent):
    return h_latent.device if h_latent.is_cuda else torch.device("cuda", torch.cuda.current_device())


def _lora(bundle):
    """The layer's routed-expert adapters, or None when the bundle carries none."""
    if bundle is None or getattr(bundle, "gate_lora", None) is None:
        return None
    mods = _adapters(bundle)
    if any(getattr(m, "r", 1) == 0 or getattr(m, "lora_A", None) is None for m in mods):
        return None
    return bundle
