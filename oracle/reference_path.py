"""
The reference trainer's routed-expert CPU path, composed as it composes it. TEST
INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg and tests/ use it; the product never does.

LazyLoRATrainer runs each active expert on the rows that chose it and picks the arithmetic by
bucket size (lazy_lora/trainer/lazy_trainer.py:746-760): up to FUSED_MAX_ROWS rows the fused
decode-and-dot C kernel (mxfp4_gemm / mxfp4_gemm_t), above that a C dequantisation of the three
matrices to fp32 followed by torch's CPU sgemm (F.linear, and d @ W in backward, :777-778,
:787, :800). Here the C kernels are this repo's restatement (oracle/mxfp4_oracle.c, bit-identical
to the reference's mxfp4_gemm.c where that runs, K <= 4096) and the dense products are torch's
CPU fp32 GEMM, as in the reference. LoRA off (the BASELINE configurations).
"""
import numpy as np
import torch
import torch.nn.functional as Fn

FUSED_MAX_ROWS = 48  # lazy_trainer.py:39-41

SITU_BETA, SITU_LBETA = 4.0, 25.0


def _glu(gate, up, act):
    if act == "swiglu":
        return Fn.silu(gate) * up
    return SITU_BETA * torch.tanh(gate / SITU_BETA) * torch.sigmoid(gate) * (SITU_LBETA * torch.tanh(up / SITU_LBETA))


def _glu_backward(d_act, gate, up, act):
    s = torch.sigmoid(gate)
    if act == "swiglu":
        return d_act * up * (s * (1.0 + gate * (1.0 - s))), d_act * gate * s
    t = torch.tanh(gate / SITU_BETA)
    a = SITU_BETA * t * s
    da = (1.0 - t * t) * s + SITU_BETA * t * s * (1.0 - s)
    tu = torch.tanh(up / SITU_LBETA)
    return d_act * (SITU_LBETA * tu) * da, d_act * a * (1.0 - tu * tu)


class _Expert:
    """One expert's matrices as _expert_matrices hands them over: fp32 dense tensors above
    FUSED_MAX_ROWS rows (three C dequantisations), else None (fused C products)."""

    def __init__(self, lib, ex, e, rows):
        self.lib = lib
        self.p = ((ex.w1p[e], ex.w1s[e]), (ex.w3p[e], ex.w3s[e]), (ex.w2p[e], ex.w2s[e]))
        self.dense = None
        if rows > FUSED_MAX_ROWS:
            self.dense = tuple(torch.from_numpy(lib.dequant(p, s)) for p, s in self.p)

    def linear(self, x, which):
        """x @ W^T (gate / up / down: which = 0 / 1 / 2)."""
        if self.dense is not None:
            return Fn.linear(x, self.dense[which])
        return torch.from_numpy(self.lib.gemm(x.numpy(), *self.p[which]))

    def dx(self, d, which):
        """d @ W."""
        if self.dense is not None:
            return d @ self.dense[which]
        return torch.from_numpy(self.lib.gemm_t(d.numpy(), *self.p[which]))

    def forward(self, x, act):
        gate, up = self.linear(x, 0), self.linear(x, 1)
        a = _glu(gate, up, act)
        return gate, up, a, self.linear(a, 2)


def _buckets(topk_idx, topk_w):
    idx = torch.as_tensor(topk_idx)
    w = torch.as_tensor(topk_w, dtype=torch.float32)
    for e in torch.unique(idx).tolist():
        mask = idx == e
        rows = mask.any(dim=-1).nonzero(as_tuple=False).squeeze(-1)
        tw = (w.index_select(0, rows) * mask.index_select(0, rows).float()).sum(-1, keepdim=True)
        yield e, rows, tw, mask.index_select(0, rows)


def routed_forward(lib, h, topk_idx, topk_w, ex, act="swiglu") -> np.ndarray:
    """_routed_experts_forward (lazy_trainer.py:806-834) with _expert_matrices' path choice."""
    h = torch.as_tensor(np.ascontiguousarray(h, np.float32))
    out = torch.zeros(h.shape, dtype=torch.float32)
    for e, rows, tw, _ in _buckets(topk_idx, topk_w):
        x = h.index_select(0, rows)
        *_, down = _Expert(lib, ex, e, rows.numel()).forward(x, act)
        out.index_add_(0, rows, down * tw)
    return out.numpy()


def routed_backward(lib, h, topk_idx, topk_w, ex, grad_out, act="swiglu"):
    """_routed_experts_backward (lazy_trainer.py:836-880), LoRA off: the forward recomputed,
    grad_w = <g, down_e> per slot, d_down = g * tw, three transposed products, GLU derivative."""
    h = torch.as_tensor(np.ascontiguousarray(h, np.float32))
    g_all = torch.as_tensor(np.ascontiguousarray(grad_out, np.float32))
    grad_h = torch.zeros(h.shape, dtype=torch.float32)
    grad_w = torch.zeros(np.shape(topk_idx), dtype=torch.float32)
    for e, rows, tw, m in _buckets(topk_idx, topk_w):
        x, g = h.index_select(0, rows), g_all.index_select(0, rows)
        ex_e = _Expert(lib, ex, e, rows.numel())
        gate, up, _a, down = ex_e.forward(x, act)
        dot = (g * down).sum(dim=-1, keepdim=True)
        grad_w.index_add_(0, rows, dot * m.float())
        d_down = g * tw
        d_gate, d_up = _glu_backward(ex_e.dx(d_down, 2), gate, up, act)
        grad_h.index_add_(0, rows, ex_e.dx(d_gate.contiguous(), 0) + ex_e.dx(d_up.contiguous(), 1))
    return grad_h.numpy(), grad_w.numpy()
