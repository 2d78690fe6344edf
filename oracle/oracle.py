"""
Float64 / NumPy restatement of LazyLoRA's routed-expert MXFP4 path. TEST INFRASTRUCTURE ONLY
(only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it).

Each function names the reference lines it restates. Reference paths are relative to the
LazyLoRA checkout.
"""
import ctypes
import math
import os
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(_HERE, "libmxfp4_oracle.so")
REF_LIB = os.path.join(_HERE, "_ref", "libmxfp4_ref.so")

# ------------------------------------------------------------------------------------ decode
# E2M1 value by 4-bit code, sign in bit 3; code 8 is -0.0
# (lazy_lora/native/mxfp4_gemm.c:33-34; lazy_lora/streaming/expert_streamer.py:57-58).
E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                 -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float32)
MAX_SAFE_E8M0 = 253  # expert_streamer.py:63; mxfp4_gemm.c:40-41


def e2m1_closed_form(code: int) -> float:
    """OCP MX E2M1: sign bit 3, exponent bits 2:1 (bias 1), mantissa bit 0; exponent 0 is subnormal."""
    sign = -1.0 if code & 8 else 1.0
    e, m = (code >> 1) & 3, code & 1
    mag = 0.5 * m if e == 0 else math.ldexp(1.0 + 0.5 * m, e - 1)
    return math.copysign(mag, sign)


def e8m0_table() -> np.ndarray:
    """2^(s-127) as float32 for s < 253, else 0 (mxfp4_gemm.c:38-43)."""
    s = np.arange(256, dtype=np.uint32)
    bits = np.where(s >= 1, s << 23, np.uint32(0x00400000)).astype(np.uint32)
    bits[MAX_SAFE_E8M0:] = 0
    return bits.view(np.float32)


_E8M0 = e8m0_table()


def unpack_codes(packed: np.ndarray) -> np.ndarray:
    """[R, K/2] bytes -> [R, K] codes, low nibble = even element (mxfp4_gemm.c:56-59)."""
    packed = np.asarray(packed, dtype=np.uint8)
    codes = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.uint8)
    codes[..., 0::2] = packed & 0x0F
    codes[..., 1::2] = packed >> 4
    return codes


def dequant(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """W [R, K] float32, exactly LUT[code] * E8M0[scale] (mxfp4_gemm.c:45-62, :142-150)."""
    codes = unpack_codes(packed)
    R, K = codes.shape
    mult = _E8M0[np.asarray(scales, dtype=np.uint8)]
    return (E2M1[codes].reshape(R, K // 32, 32) * mult[:, :, None]).reshape(R, K)


def quantize_mxfp4(w: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """(packed [R, K/2], scales [R, K/32]): the nearest MXFP4 encoding of W [R, K] (K % 32 == 0),
    a test-input generator. Per 32-block the scale is the smallest power of two 2^e with
    amax / 2^e <= 6 (no element saturates); each element takes the nearest E2M1 magnitude."""
    w = np.asarray(w, np.float64)
    R, K = w.shape
    blocks = w.reshape(R, K // 32, 32)
    amax = np.abs(blocks).max(-1)
    e = np.where(amax > 0, np.ceil(np.log2(np.where(amax > 0, amax, 6.0) / 6.0)), -127)
    sbyte = np.clip(e + 127, 0, MAX_SAFE_E8M0 - 1).astype(np.uint8)
    scale = _E8M0[sbyte].astype(np.float64)
    mags = np.abs(E2M1[:8]).astype(np.float64)
    v = np.abs(blocks) / np.where(scale > 0, scale, 1.0)[..., None]
    code = np.abs(v[..., None] - mags).argmin(-1).astype(np.uint8)
    code |= (blocks < 0).astype(np.uint8) << 3
    code = code.reshape(R, K)
    packed = (code[:, 0::2] | (code[:, 1::2] << 4)).astype(np.uint8)
    return packed, sbyte


# ------------------------------------------------------------------------------------ products
def gemm(x: np.ndarray, packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """y[M, R] = x[M, K] . W^T in float64 (the semantics of mxfp4_gemm.c:64-94)."""
    return np.asarray(x, np.float64) @ dequant(packed, scales).astype(np.float64).T


def gemm_t(dy: np.ndarray, packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """y[M, K] = dy[M, R] . W in float64 (the semantics of mxfp4_gemm.c:96-129, y zeroed first)."""
    return np.asarray(dy, np.float64) @ dequant(packed, scales).astype(np.float64)


# ------------------------------------------------------------------------------------ GLUs
SITU_BETA = 4.0         # lazy_lora/core/situ_activation.py:22
SITU_LINEAR_BETA = 25.0  # situ_activation.py:23


def _sigmoid(v):
    return 1.0 / (1.0 + np.exp(-v))


def glu_forward(gate, up, act: str):
    """SwiGLU silu(g)*u, or SiTU-GLU beta tanh(g/beta) sigmoid(g) * lb tanh(u/lb)
    (situ_activation.py:47-75). Float64."""
    g = np.asarray(gate, np.float64)
    u = np.asarray(up, np.float64)
    if act == "swiglu":
        return g * _sigmoid(g) * u
    if act == "situ":
        return SITU_BETA * np.tanh(g / SITU_BETA) * _sigmoid(g) * (SITU_LINEAR_BETA * np.tanh(u / SITU_LINEAR_BETA))
    raise ValueError(act)


def glu_backward(grad, gate, up, act: str):
    """(d gate, d up); SiTU-GLU follows situ_activation.py:78-134. Float64."""
    go = np.asarray(grad, np.float64)
    g = np.asarray(gate, np.float64)
    u = np.asarray(up, np.float64)
    s = _sigmoid(g)
    if act == "swiglu":
        return go * u * s * (1.0 + g * (1.0 - s)), go * g * s
    if act == "situ":
        t = np.tanh(g / SITU_BETA)
        a = SITU_BETA * t * s
        da = (1.0 - t * t) * s + SITU_BETA * t * s * (1.0 - s)
        tu = np.tanh(u / SITU_LINEAR_BETA)
        return go * (SITU_LINEAR_BETA * tu) * da, go * a * (1.0 - tu * tu)
    raise ValueError(act)


# ------------------------------------------------------------------------------------ router
def router_select(logits, bias=None, top_k=2, routed_scaling_factor=1.0, renormalize=True):
    """The selection half of KimiK3MoERouter.forward on given logits [N, E]
    (lazy_lora/core/moe_router.py:106-123): sigmoid scores, bias added for selection only,
    top-k (stable: equal choices go to the lower expert id; NaN ranks above every number, as in
    torch.topk), gather unbiased scores, renormalise (+1e-20) when top_k > 1, scale. Returns
    (indices [N, k] int64, weights float64)."""
    scores = _sigmoid(np.asarray(logits, np.float64))
    choice = scores + np.asarray(bias, np.float64) if bias is not None else scores
    nan = np.isnan(choice)
    # lexsort's last key is the primary one: NaN first, then descending value; stable in the id
    idx = np.lexsort((-np.where(nan, 0.0, choice), (~nan).astype(np.int8)), axis=-1)[:, :top_k]
    w = np.take_along_axis(scores, idx, axis=-1)
    if top_k > 1 and renormalize:
        w = w / (w.sum(-1, keepdims=True) + 1e-20)
    return idx.astype(np.int64), w * routed_scaling_factor


def router_forward(x, gate_weight, bias=None, top_k=2, routed_scaling_factor=1.0, renormalize=True):
    """KimiK3MoERouter.forward, NumPy branch (lazy_lora/core/moe_router.py:102-123): logits =
    x . W^T, then router_select. Returns (indices [N, k] int64, weights [N, k] float64)."""
    x = np.asarray(x, np.float64).reshape(-1, gate_weight.shape[1])
    logits = x @ np.asarray(gate_weight, np.float64).T
    return router_select(logits, bias, top_k, routed_scaling_factor, renormalize)


def router_select_backward(logits, idx, grad_w, routed_scaling_factor=1.0, renormalize=True):
    """dL/dlogits [N, E] for upstream dL/dweights grad_w [N, k], the closed-form derivative of
    router_select at fixed indices (what torch autograd computes through moe_router.py:86-98):
    with s the chosen scores, S = sum s + 1e-20 and c the scale, dL/ds_i = c (g_i / S -
    sum_j g_j s_j / S^2) when renormalising (top_k > 1), else c g_i; dL/dlogit_i = dL/ds_i s_i
    (1 - s_i); unchosen experts get 0."""
    logits = np.asarray(logits, np.float64)
    idx = np.asarray(idx, np.int64)
    g = np.asarray(grad_w, np.float64)
    s = _sigmoid(np.take_along_axis(logits, idx, axis=-1))
    if idx.shape[1] > 1 and renormalize:
        den = s.sum(-1, keepdims=True) + 1e-20
        ds = routed_scaling_factor * (g / den - (g * s).sum(-1, keepdims=True) / den ** 2)
    else:
        ds = routed_scaling_factor * g
    out = np.zeros_like(logits)
    np.put_along_axis(out, idx, ds * s * (1.0 - s), axis=-1)
    return out


def rms_norm(x, weight, eps=1e-5):
    """lazy_lora/core/attention.py:33-40."""
    x = np.asarray(x, np.float64)
    out = x / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    return out * np.asarray(weight, np.float64) if weight is not None else out


# ------------------------------------------------------------------------------------ routed layer
@dataclass
class ExpertSet:
    """Stacked packed experts: w1/w3 [E, F, D/2] + [E, F, D/32]; w2 [E, D, F/2] + [E, D, F/32]."""
    w1p: np.ndarray
    w1s: np.ndarray
    w3p: np.ndarray
    w3s: np.ndarray
    w2p: np.ndarray
    w2s: np.ndarray

    @property
    def E(self):
        return self.w1p.shape[0]

    @property
    def F(self):
        return self.w1p.shape[1]

    @property
    def D(self):
        return self.w1p.shape[2] * 2

    def dense(self, e: int):
        """(W1, W3, W2) float64 of expert e."""
        return (dequant(self.w1p[e], self.w1s[e]).astype(np.float64),
                dequant(self.w3p[e], self.w3s[e]).astype(np.float64),
                dequant(self.w2p[e], self.w2s[e]).astype(np.float64))


def _expert_rows(e, topk_idx, topk_w):
    """Tokens that chose e and their summed combine weight (lazy_trainer.py:823-829)."""
    mask = topk_idx == e
    rows = np.nonzero(mask.any(-1))[0]
    tw = (np.asarray(topk_w, np.float64)[rows] * mask[rows]).sum(-1)
    return rows, tw, mask[rows]


@dataclass
class LoRA:
    """The layer's LoRA adapters, shared by all its experts (lazy_trainer.py:130-134): A [r, in],
    B [out, r], scaling = alpha / r (lora_layer.py:53-97). Gate/up map D -> F, down F -> D."""
    gate_A: np.ndarray
    gate_B: np.ndarray
    up_A: np.ndarray
    up_B: np.ndarray
    down_A: np.ndarray
    down_B: np.ndarray
    gate_s: float = 2.0
    up_s: float = 2.0
    down_s: float = 2.0

    def adapters(self):
        return ((self.gate_A, self.gate_B, self.gate_s), (self.up_A, self.up_B, self.up_s),
                (self.down_A, self.down_B, self.down_s))


def lora_delta(x, A, B, s):
    """forward_lora_only, dropout off (lora_layer.py:104-139): s (x A^T) B^T."""
    return s * (np.asarray(x, np.float64) @ np.asarray(A, np.float64).T) @ np.asarray(B, np.float64).T


def lora_gradients(dy, x, A, B, s):
    """compute_lora_gradients (lora_layer.py:178-226) without the base term: (grad_A, grad_B,
    dx_lora) with h = x A^T, grad_B = s dy^T h, dh = s dy B, grad_A = dh^T x, dx_lora = dh A."""
    A, B = np.asarray(A, np.float64), np.asarray(B, np.float64)
    h = x @ A.T
    dh = s * dy @ B
    return dh.T @ x, s * dy.T @ h, dh @ A


def routed_forward(h, topk_idx, topk_w, experts, act: str = "swiglu", dense=None, lora=None) -> np.ndarray:
    """sum_e w_e(token) * expert_e(h) in float64 (lazy_trainer.py:806-834, and _expert_forward
    :762-791 for the LoRA terms). `dense(e) -> (W1, W3, W2)` overrides the weights (used for
    the dense moe.json fixture); `lora` is a LoRA or None."""
    h = np.asarray(h, np.float64)
    topk_idx = np.asarray(topk_idx)
    out = np.zeros(h.shape, np.float64)
    get = dense if dense is not None else experts.dense
    for e in np.unique(topk_idx):
        rows, tw, _ = _expert_rows(e, topk_idx, topk_w)
        if rows.size == 0:
            continue
        W1, W3, W2 = get(int(e))
        x = h[rows]
        gate, up = x @ W1.T, x @ W3.T
        if lora is not None:
            (ag, bg, sg), (au, bu, su), _ = lora.adapters()
            gate = gate + lora_delta(x, ag, bg, sg)
            up = up + lora_delta(x, au, bu, su)
        a = glu_forward(gate, up, act)
        down = a @ W2.T
        if lora is not None:
            down = down + lora_delta(a, lora.down_A, lora.down_B, lora.down_s)
        out[rows] += down * tw[:, None]
    return out


def routed_backward(h, topk_idx, topk_w, experts, grad_out, act: str = "swiglu", dense=None, lora=None):
    """(dL/dh [N, D], dL/dtopk_w [N, k]) in float64 (lazy_trainer.py:836-880): grad_w[t, slot] =
    <g_t, down_e(t)> for the slot that chose e; d_down = g * tw; then d_act = d_down . W2, the
    GLU derivative, and d_h = d_gate . W1 + d_up . W3. With `lora` the adapters' terms join
    each step as in compute_lora_gradients, and a third result holds the adapter gradients summed
    over the experts: (gate_A, gate_B, up_A, up_B, down_A, down_B)."""
    h = np.asarray(h, np.float64)
    g_all = np.asarray(grad_out, np.float64)
    topk_idx = np.asarray(topk_idx)
    grad_h = np.zeros(h.shape, np.float64)
    grad_w = np.zeros(topk_idx.shape, np.float64)
    get = dense if dense is not None else experts.dense
    lg = None
    if lora is not None:
        lg = [np.zeros(np.shape(m), np.float64) for m in (lora.gate_A, lora.gate_B, lora.up_A, lora.up_B,
                                                         lora.down_A, lora.down_B)]
    for e in np.unique(topk_idx):
        rows, tw, m = _expert_rows(e, topk_idx, topk_w)
        if rows.size == 0:
            continue
        W1, W3, W2 = get(int(e))
        x, g = h[rows], g_all[rows]
        gate, up = x @ W1.T, x @ W3.T
        if lora is not None:
            gate = gate + lora_delta(x, lora.gate_A, lora.gate_B, lora.gate_s)
            up = up + lora_delta(x, lora.up_A, lora.up_B, lora.up_s)
        a = glu_forward(gate, up, act)
        down = a @ W2.T
        if lora is not None:
            down = down + lora_delta(a, lora.down_A, lora.down_B, lora.down_s)
        grad_w[rows] += (g * down).sum(-1, keepdims=True) * m
        d_down = g * tw[:, None]
        d_act = d_down @ W2
        if lora is not None:
            gA, gB, dx = lora_gradients(d_down, a, lora.down_A, lora.down_B, lora.down_s)
            lg[4] += gA
            lg[5] += gB
            d_act = d_act + dx
        d_gate, d_up = glu_backward(d_act, gate, up, act)
        d_in = d_gate @ W1 + d_up @ W3
        if lora is not None:
            gA, gB, dx = lora_gradients(d_gate, x, lora.gate_A, lora.gate_B, lora.gate_s)
            lg[0] += gA
            lg[1] += gB
            d_in = d_in + dx
            gA, gB, dx = lora_gradients(d_up, x, lora.up_A, lora.up_B, lora.up_s)
            lg[2] += gA
            lg[3] += gB
            d_in = d_in + dx
        grad_h[rows] += d_in
    if lora is not None:
        return grad_h, grad_w, tuple(lg)
    return grad_h, grad_w


def latent_moe_forward(x, p, experts=None, dense=None, lora=None, act: str = "situ"):
    """Kimi-K3 latent MoE block (lazy_trainer.py:697-737) in float64, with moe.json's parameter
    names: the shared expert at full width (shared_w1/w3/w2), the router on x (gate_weight,
    e_score_correction_bias, top_k, routed_scale), the routed experts in the latent space
    (down_weight, routed sum, RMSNorm with norm_weight when latent_norm, up_weight)."""
    x = np.asarray(x, np.float64)
    flat = x.reshape(-1, int(p["hidden"]))
    a = lambda k: np.asarray(p[k], np.float64)
    shared = glu_forward(flat @ a("shared_w1_weight").T, flat @ a("shared_w3_weight").T, act) @ a("shared_w2_weight").T
    idx, w = router_forward(flat, a("gate_weight"), a("e_score_correction_bias"), top_k=int(p["top_k"]),
                            routed_scaling_factor=float(p["routed_scale"]), renormalize=bool(p.get("renorm", 1)))
    h_lat = flat @ a("down_weight").T
    routed = routed_forward(h_lat, idx, w, experts, act, dense=dense, lora=lora)
    if p.get("latent_norm", 1):
        routed = rms_norm(routed, a("norm_weight"), eps=float(p.get("rms_eps", 1e-5)))
    return (shared + routed @ a("up_weight").T).reshape(x.shape), idx, w


def random_lora(rng: np.random.Generator, D: int, F: int, r: int, scale: float = 0.05, alpha: float = 32.0) -> LoRA:
    """Adapters with nonzero A and B (the reference initialises B to zero, which would hide every
    LoRA term), scaling alpha / r."""
    s = alpha / r
    mk = lambda *shape: (scale * rng.standard_normal(shape)).astype(np.float32)
    return LoRA(mk(r, D), mk(F, r), mk(r, D), mk(F, r), mk(r, F), mk(D, r), s, s, s)


# ------------------------------------------------------------------------------------ C restatement
class CLib:
    """ctypes view of libmxfp4_oracle.so (this repo's C restatement, the CPU baseline) or of
    oracle/_ref/libmxfp4_ref.so (the reference's mxfp4_gemm.c compiled where it lies)."""

    def __init__(self, path: str, prefix: str):
        self.path = path
        self.lib = ctypes.CDLL(path)
        self.prefix = prefix
        vp, ci = ctypes.c_void_p, ctypes.c_int
        self._fn("gemm").argtypes = [vp, vp, vp, vp, ci, ci, ci]
        self._fn("gemm_t").argtypes = [vp, vp, vp, vp, ci, ci, ci]
        self._fn("dequant").argtypes = [vp, vp, vp, ci, ci]
        self._fn("threads").restype = ci
        if prefix == "oracle":
            moe = [vp, vp, vp, vp, ci, ci, vp, vp, vp, vp, vp, vp, ci, ci, vp, ci, ci]
            self.lib.oracle_moe_forward.argtypes = moe
            self.lib.oracle_moe_backward.argtypes = [vp, vp, vp] + moe[1:]

    def _fn(self, name):
        return getattr(self.lib, f"{self.prefix}_{name}")

    @staticmethod
    def _p(a: np.ndarray):
        return a.ctypes.data_as(ctypes.c_void_p)

    def threads(self) -> int:
        return int(self._fn("threads")())

    def dequant(self, packed, scales) -> np.ndarray:
        packed = np.ascontiguousarray(packed, np.uint8)
        scales = np.ascontiguousarray(scales, np.uint8)
        R, K = packed.shape[0], packed.shape[1] * 2
        out = np.empty((R, K), np.float32)
        self._fn("dequant")(self._p(out), self._p(packed), self._p(scales), K, R)
        return out

    def gemm(self, x, packed, scales) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        packed = np.ascontiguousarray(packed, np.uint8)
        scales = np.ascontiguousarray(scales, np.uint8)
        M, K = x.shape
        R = packed.shape[0]
        if self.prefix == "mxfp4" and K > 4096:
            raise ValueError("the reference's mxfp4_gemm holds at most K = 4096 (mxfp4_gemm.c:72)")
        y = np.empty((M, R), np.float32)
        self._fn("gemm")(self._p(y), self._p(x), self._p(packed), self._p(scales), M, K, R)
        return y

    def gemm_t(self, dy, packed, scales) -> np.ndarray:
        dy = np.ascontiguousarray(dy, np.float32)
        packed = np.ascontiguousarray(packed, np.uint8)
        scales = np.ascontiguousarray(scales, np.uint8)
        M, R = dy.shape
        K = packed.shape[1] * 2
        y = np.zeros((M, K), np.float32)
        self._fn("gemm_t")(self._p(y), self._p(dy), self._p(packed), self._p(scales), M, K, R)
        return y

    def _moe_args(self, h, topk_idx, topk_w, ex: ExpertSet, order):
        h = np.ascontiguousarray(h, np.float32)
        idx = np.ascontiguousarray(topk_idx, np.int64)
        w = np.ascontiguousarray(topk_w, np.float32)
        if order is None:
            order = np.unique(idx)
        order = np.ascontiguousarray(order, np.int32)
        ws = [np.ascontiguousarray(a, np.uint8) for a in (ex.w1p, ex.w1s, ex.w3p, ex.w3s, ex.w2p, ex.w2s)]
        return h, idx, w, order, ws

    def moe_forward(self, h, topk_idx, topk_w, ex: ExpertSet, act="swiglu", order=None) -> np.ndarray:
        """The routed forward composed in C: gathers, three oracle_gemm calls per expert, GLU,
        weighted index_add in `order` (default ascending ids)."""
        h, idx, w, order, ws = self._moe_args(h, topk_idx, topk_w, ex, order)
        N, k = idx.shape
        out = np.empty((N, ex.D), np.float32)
        self.lib.oracle_moe_forward(self._p(out), self._p(h), self._p(idx), self._p(w), N, k,
                                    *[self._p(a) for a in ws], ex.D, ex.F, self._p(order), len(order),
                                    ACT_CODES[act])
        return out

    def moe_backward(self, h, topk_idx, topk_w, ex: ExpertSet, grad_out, act="swiglu", order=None):
        h, idx, w, order, ws = self._moe_args(h, topk_idx, topk_w, ex, order)
        g = np.ascontiguousarray(grad_out, np.float32)
        N, k = idx.shape
        gh = np.empty((N, ex.D), np.float32)
        gw = np.empty((N, k), np.float32)
        self.lib.oracle_moe_backward(self._p(gh), self._p(gw), self._p(g), self._p(h), self._p(idx), self._p(w),
                                     N, k, *[self._p(a) for a in ws], ex.D, ex.F, self._p(order), len(order),
                                     ACT_CODES[act])
        return gh, gw


ACT_CODES = {"swiglu": 0, "situ": 1}


def oracle_lib() -> CLib:
    if not os.path.exists(ORACLE_LIB):
        raise RuntimeError(f"{ORACLE_LIB} missing: run `make -C oracle`")
    return CLib(ORACLE_LIB, "oracle")


def reference_lib() -> Optional[CLib]:
    """The reference's own mxfp4_gemm.c compiled into oracle/_ref, or None if not built."""
    return CLib(REF_LIB, "mxfp4") if os.path.exists(REF_LIB) else None


# ------------------------------------------------------------------------------------ synthetic data
def random_mx(rng: np.random.Generator, shape_rk: Tuple[int, ...], scale_lo: int, scale_hi: int):
    """Packed [..., R, K/2] with codes uniform over all 16, scales uniform in [scale_lo, scale_hi]."""
    *lead, R, K = shape_rk
    packed = rng.integers(0, 256, size=(*lead, R, K // 2), dtype=np.uint8)
    scales = rng.integers(scale_lo, scale_hi + 1, size=(*lead, R, K // 32), dtype=np.uint8)
    return packed, scales


def random_experts(rng: np.random.Generator, E: int, D: int, F: int, scale_lo: int, scale_hi: int) -> ExpertSet:
    w1p, w1s = random_mx(rng, (E, F, D), scale_lo, scale_hi)
    w3p, w3s = random_mx(rng, (E, F, D), scale_lo, scale_hi)
    w2p, w2s = random_mx(rng, (E, D, F), scale_lo, scale_hi)
    return ExpertSet(w1p, w1s, w3p, w3s, w2p, w2s)


def softmax_topk(logits: np.ndarray, k: int):
    """Top-k of the logits, weights = softmax over the selected k (= renormalised softmax)."""
    idx = np.argsort(-logits, axis=-1, kind="stable")[:, :k]
    sel = np.take_along_axis(logits, idx, axis=-1).astype(np.float64)
    w = np.exp(sel - sel.max(-1, keepdims=True))
    return idx.astype(np.int64), (w / w.sum(-1, keepdims=True)).astype(np.float32)


def zipf_offsets(rng: np.random.Generator, E: int, s: float = 1.1) -> np.ndarray:
    """Per-expert logit offset -s * ln(rank), rank a seeded permutation of 1..E."""
    rank = rng.permutation(E) + 1
    return (-s * np.log(rank)).astype(np.float32)


# ------------------------------------------------------------------------------------ metrics
def rel_l2(got, want) -> float:
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-300))


def cosine(got, want) -> float:
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    return float(got @ want / max(np.linalg.norm(got) * np.linalg.norm(want), 1e-300))
