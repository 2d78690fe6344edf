"""
The Kimi-K3 latent MoE block of one layer on MI355X, around the routed-expert kernels.

Mirrors LazyLoRATrainer._run_layer's MoE half and _moe_forward
(lazy_lora/trainer/lazy_trainer.py:689-737):
  * route: KimiK3MoERouter on the normed hidden state (moe_router.py:55-123; here the device
    router of lazylora_amd.router, so indices never leave the GPU);
  * shared expert at full width: GLU(x W1^T + LoRA, x W3^T + LoRA) W2^T + LoRA (:703-708);
  * routed experts in the latent space: h_latent = x W_down^T (:727), the routed sum
    (RoutedExpertsFunction, :728-730, the MXFP4 kernels), RMSNorm of the sum with its weight
    (RMSNormFunction, lazy_lora/streaming/trunk_streamer.py:23-34; :733), up-projection (:734);
  * out = shared + routed (:736).
The dense projections (shared expert, latent down/up) are plain GEMMs and run in the platform
BLAS through torch, in fp32; the whole block is differentiable in x (through the router's
weights too, as in the reference) and in any LoRA factor that requires grad; the routed
adapters' gradients are accumulated into them by the routed node, as in the reference.
"""
from typing import Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

from lazylora_amd.experts import ExpertLayer
from lazylora_amd.routed import RoutedExpertsFunction
from lazylora_amd.router import route

SITU_BETA, SITU_LINEAR_BETA = 4.0, 25.0  # lazy_lora/core/situ_activation.py:22-23


def glu(g: torch.Tensor, u: torch.Tensor, act: str) -> torch.Tensor:
    """SiTU-GLU (situ_activation.py:47-75) or SwiGLU, in torch (the shared expert's dense path)."""
    if act in ("situ", "situ_glu"):
        return SITU_BETA * torch.tanh(g / SITU_BETA) * torch.sigmoid(g) * (SITU_LINEAR_BETA * torch.tanh(u / SITU_LINEAR_BETA))
    if act == "swiglu":
        return F.silu(g) * u
    raise ValueError(f"unknown activation {act!r}")


def rms_norm(x: torch.Tensor, weight: Optional[torch.Tensor], eps: float = 1e-5) -> torch.Tensor:
    """RMSNormFunction.forward (trunk_streamer.py:23-34)."""
    out = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return out * weight if weight is not None else out


def lora_delta(x: torch.Tensor, mod) -> torch.Tensor:
    """forward_lora_only with dropout off (lora_layer.py:104-139): s (x A^T) B^T, fp32."""
    if mod is None:
        return 0.0
    A = mod.lora_A.to(x.device, torch.float32)
    B = mod.lora_B.to(x.device, torch.float32)
    return float(mod.scaling) * F.linear(F.linear(x, A), B)


class LatentMoEBlock:
    """One MoE layer: router, shared expert, latent projections, routed MXFP4 experts, norm.

    Weights follow the checkpoint's names (scripts/make_tiny_model.py:134-146 lists them):
    gate.weight [E, H], gate.e_score_correction_bias [E], shared_experts.{gate,up,down}_proj
    [Ds, H] / [Ds, H] / [H, Ds], routed_expert_down_proj [Dl, H], routed_expert_up_proj [H, Dl],
    routed_expert_norm [Dl]; the experts as an ExpertLayer of the latent width Dl. `lora` is the
    layer's adapter bundle (gate_lora / up_lora / down_lora for the routed experts and
    shared_gate_lora / shared_up_lora / shared_down_lora for the shared expert, any of them absent
    or None), as the reference's LayerLoRABundle (lazy_trainer.py:124-134).
    """

    def __init__(self, experts: ExpertLayer, gate_weight, gate_bias, shared_w1, shared_w3, shared_w2, latent_down,
                 latent_up, latent_norm=None, top_k: int = 16, routed_scaling_factor: float = 1.0,
                 renormalize: bool = True, act: str = "situ", rms_eps: float = 1e-5, lora=None):
        dev = experts.device
        f32 = lambda t: None if t is None else torch.as_tensor(t).to(dev, torch.float32)
        self.experts = experts
        self.gate_weight, self.gate_bias = f32(gate_weight), f32(gate_bias)
        self.shared = (f32(shared_w1), f32(shared_w3), f32(shared_w2))
        self.latent_down, self.latent_up, self.latent_norm = f32(latent_down), f32(latent_up), f32(latent_norm)
        self.top_k, self.routed_scaling_factor, self.renormalize = top_k, routed_scaling_factor, renormalize
        self.act, self.rms_eps, self.lora = act, rms_eps, lora
        H = self.gate_weight.shape[1]
        if self.latent_down.shape != (experts.D, H) or self.latent_up.shape != (H, experts.D):
            raise ValueError(f"latent projections must be [{experts.D}, {H}] and [{H}, {experts.D}]")
        self.hidden = H

    def _adapter(self, name: str):
        return getattr(self.lora, name, None) if self.lora is not None else None

    def _routed_lora(self):
        mods = tuple(self._adapter(n) for n in ("gate_lora", "up_lora", "down_lora"))
        return mods if all(m is not None for m in mods) else None

    def forward(self, h_moe_norm: torch.Tensor, cached: Optional[torch.Tensor] = None
                ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """(out in h's dtype and shape, topk_indices, topk_weights) for the normed hidden state."""
        shape, dtype = h_moe_norm.shape, h_moe_norm.dtype
        x = h_moe_norm.reshape(-1, self.hidden).to(self.experts.device, torch.float32)
        idx, w = route(x, self.gate_weight, self.gate_bias, self.top_k, self.routed_scaling_factor, self.renormalize)
        W1, W3, W2 = self.shared
        s_gate = F.linear(x, W1) + lora_delta(x, self._adapter("shared_gate_lora"))
        s_up = F.linear(x, W3) + lora_delta(x, self._adapter("shared_up_lora"))
        s_act = glu(s_gate, s_up, self.act)
        shared = F.linear(s_act, W2) + lora_delta(s_act, self._adapter("shared_down_lora"))
        h_latent = F.linear(x, self.latent_down)
        routed = RoutedExpertsFunction.apply(h_latent, w, idx, self.experts, self.act, cached, self._routed_lora())
        if self.latent_norm is not None:
            routed = rms_norm(routed, self.latent_norm, self.rms_eps)
        out = shared + F.linear(routed, self.latent_up)
        return out.reshape(shape).to(dtype), idx, w

    __call__ = forward
