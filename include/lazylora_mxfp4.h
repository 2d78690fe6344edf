/*
 * lazylora_mxfp4.h — C ABI of the MI355X (gfx950) MXFP4 routed-expert library.
 *
 * The first four entry points replace the reference's CPU kernels one for one
 * (lazy_lora/native/mxfp4_gemm.c, bound by ctypes in lazy_lora/native/__init__.py:19-74);
 * the routed-layer entry points replace the per-expert Python loops that drive them
 * (lazy_lora/trainer/lazy_trainer.py:806-880).
 *
 * Conventions (same as the reference, mxfp4_gemm.c:12-18):
 *   W is [R, K] row-major: packed [R, K/2] bytes (low nibble = even element), scales
 *   [R, K/32] E8M0 bytes; value = e2m1(code) * 2^(s-127); a scale byte >= 253 contributes 0.
 *   K must be a multiple of 32. All array pointers are DEVICE pointers (HBM), except where
 *   noted. Every call is asynchronous on `stream` (0 = the null stream).
 *
 * Alignment (checked; a violation returns MXFP4_EINVAL and launches nothing): packed weights
 * and scales 16 bytes (mxfp4_dequant takes any alignment, mxfp4_dequant_bf16 a 4-byte aligned out); mxfp4_gemm's x 8 bytes; mxfp4_gemm_t's dy 4 bytes and y 16 bytes; the routed layer's
 * h 8 bytes (fp32) or 4 bytes (bf16), 16 bytes with LoRA, as are grad_out and the LoRA
 * factors then. Buffers from hipMalloc or torch satisfy all of these.
 *
 * Deviations from the reference signatures, all deliberate:
 *   - every call returns int status (0 = ok, see MXFP4_E*) instead of void;
 *   - every call takes a hipStream_t, and calls that need scratch take a caller-owned
 *     device workspace plus its size (query with the *_workspace_size functions), so the
 *     library itself never allocates device memory.
 *
 * Numerics: the forward products run on the fp4-native scaled MFMA with the activations
 * split into two e4m3 terms; the transposed products decode the weights exactly to bf16 and
 * split the activation gradients into two bf16 terms. Both accumulate in fp32. Results match
 * the reference's fp32 CPU path within rel-L2 5e-3 (the tolerance stated for this path), and
 * mxfp4_dequant matches it bit for bit.
 */
#ifndef LAZYLORA_MXFP4_H
#define LAZYLORA_MXFP4_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MXFP4_OK 0
#define MXFP4_EINVAL (-1)     /* bad shape / pointer / flag; nothing was launched */
#define MXFP4_EWORKSPACE (-2) /* workspace smaller than *_workspace_size() */
#define MXFP4_EHIP (-3)       /* a HIP launch failed; see mxfp4_last_error() */

/* Activation functions of the expert GLU. */
#define MXFP4_ACT_SWIGLU 0 /* silu(gate) * up */
#define MXFP4_ACT_SITU 1   /* 4 tanh(g/4) sigmoid(g) * 25 tanh(u/25): lazy_lora/core/situ_activation.py:47-75 */

/* Dtype codes for routed-layer inputs. */
#define MXFP4_F32 0
#define MXFP4_BF16 1
#define MXFP4_I32 2
#define MXFP4_I64 3

/* Flags for the routed layer. */
#define MXFP4_MOE_SAVE 1          /* forward keeps gate|up and routing in the workspace */
#define MXFP4_MOE_REUSE_FORWARD 2 /* backward reuses them instead of recomputing */
#define MXFP4_MOE_BWD_LAYOUT 4    /* mxfp4_moe_*_fl: the layout array holds 6 entries (below) */

/* Text of the last error raised on the calling thread ("" if none). */
const char *mxfp4_last_error(void);

/* Replaces int mxfp4_threads(void) (mxfp4_gemm.c:131-138): the parallel width of the
 * device, here the compute-unit count of the current HIP device. */
int mxfp4_threads(void);

/* Replaces void mxfp4_dequant(float *out, const uint8_t *packed, const uint8_t *scales,
 * int K, int R) (mxfp4_gemm.c:142-150): out[R, K] fp32 = W, bit-exact. */
int mxfp4_dequant(float *out, const uint8_t *packed, const uint8_t *scales, int K, int R,
                  hipStream_t stream);

/* Replaces the bf16 result of _dequantize_mxfp4(weight_packed, weight_scale,
 * out_dtype=None) (lazy_lora/streaming/expert_streamer.py:104-154, whose default output dtype
 * is bfloat16): out[R, K] bf16 = W, the same values as mxfp4_dequant (each decoded value is
 * exact in bf16), scale bytes >= 253 giving +-0. out 4-byte aligned. */
int mxfp4_dequant_bf16(uint16_t *out, const uint8_t *packed, const uint8_t *scales, int K,
                       int R, hipStream_t stream);

/* Replaces void mxfp4_gemm(float *y, const float *x, const uint8_t *packed,
 * const uint8_t *scales, int M, int K, int R) (mxfp4_gemm.c:64-94):
 * y[M, R] = x[M, K] . W^T, y fully overwritten. x, y fp32 row-major contiguous. */
size_t mxfp4_gemm_workspace_size(int M, int K, int R);
int mxfp4_gemm(float *y, const float *x, const uint8_t *packed, const uint8_t *scales, int M,
               int K, int R, void *workspace, size_t workspace_bytes, hipStream_t stream);

/* mxfp4_gemm without a workspace: the same product (same kernels, bit-identical results), with
 * x's activation tiles staged in a 16 MiB device array that the library holds on each GPU it runs
 * on until the process ends. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc); it calls no hipMalloc, hipFree or allocating library routine. Limit:
 * ceil(M/16) * ceil(K/512) * 16896 bytes <= 16 MiB (M <= 1120 at K = 7168), else
 * MXFP4_EWORKSPACE and nothing is launched. All calls on one device share that array: calls
 * that overlap on one device (different streams or host threads) race and must be serialised by
 * the caller; consecutive calls on one stream are safe. */
int mxfp4_gemm_noalloc(float *y, const float *x, const uint8_t *packed, const uint8_t *scales,
                       int M, int K, int R, hipStream_t stream);

/* Replaces void mxfp4_gemm_t(float *y, const float *dy, const uint8_t *packed,
 * const uint8_t *scales, int M, int K, int R) (mxfp4_gemm.c:96-129):
 * y[M, K] += dy[M, R] . W (accumulates into y, like the reference). */
size_t mxfp4_gemm_t_workspace_size(int M, int K, int R);
int mxfp4_gemm_t(float *y, const float *dy, const uint8_t *packed, const uint8_t *scales, int M,
                 int K, int R, void *workspace, size_t workspace_bytes, hipStream_t stream);

/* Routed-expert layer forward, replacing LazyLoRATrainer._routed_experts_forward
 * (lazy_lora/trainer/lazy_trainer.py:806-834) with LoRA off:
 *   out[N, D] fp32 = sum over (t, slot) of topk_w[t, slot] * expert_e(h[t]),
 *   expert_e(x) = W2_e . act(W1_e . x, W3_e . x),  e = topk_idx[t, slot].
 * h: [N, D] fp32 or bf16 (h_dtype). topk_idx: [N, k] int32 or int64 (idx_dtype); ids outside
 * [0, E) contribute nothing. topk_w: [N, k] fp32.
 * Expert weights are stacked expert-major: w1p/w3p [E, F, D/2], w1s/w3s [E, F, D/32],
 * w2p [E, D, F/2], w2s [E, D, F/32]. D and F must be multiples of 32. */
size_t mxfp4_moe_workspace_size(int N, int k, int E, int D, int F);
int mxfp4_moe_forward(float *out, const void *h, int h_dtype, const void *topk_idx, int idx_dtype,
                      const float *topk_w, int N, int k, const uint8_t *w1p, const uint8_t *w1s,
                      const uint8_t *w3p, const uint8_t *w3s, const uint8_t *w2p,
                      const uint8_t *w2s, int E, int D, int F, int act_kind, int flags,
                      void *workspace, size_t workspace_bytes, hipStream_t stream);

/* Routed-expert layer backward, replacing _routed_experts_backward (lazy_trainer.py:836-880)
 * with LoRA off: grad_h[N, D] fp32 = dL/dh, grad_w[N, k] fp32 = dL/dtopk_w for upstream
 * grad_out[N, D] fp32. With MXFP4_MOE_REUSE_FORWARD the routing and gate|up saved by a
 * forward call made with MXFP4_MOE_SAVE on the same inputs and workspace are reused;
 * otherwise they are recomputed. */
int mxfp4_moe_backward(float *grad_h, float *grad_w, const float *grad_out, const void *h,
                       int h_dtype, const void *topk_idx, int idx_dtype, const float *topk_w,
                       int N, int k, const uint8_t *w1p, const uint8_t *w1s, const uint8_t *w3p,
                       const uint8_t *w3s, const uint8_t *w2p, const uint8_t *w2s, int E, int D,
                       int F, int act_kind, int flags, void *workspace, size_t workspace_bytes,
                       hipStream_t stream);

/* The routed layer with the layer's LoRA adapters, which all its experts share
 * (lazy_lora/trainer/lazy_trainer.py:130-134), applied as the reference applies them per expert
 * (_expert_forward, lazy_trainer.py:762-791; LazyLoRALinear.forward_lora_only,
 * lazy_lora/core/lora_layer.py:104-139; dropout off, as the reference's config sets it):
 *   gate = x W1^T + s_g (x A_g^T) B_g^T, up likewise with A_u, B_u, act = GLU(gate, up),
 *   down = act W2^T + s_d (act A_d^T) B_d^T.
 * lora: host array of 6 DEVICE pointers, fp32 row-major: A_gate [r, D], B_gate [F, r],
 * A_up [r, D], B_up [F, r], A_down [r, F], B_down [D, r]; NULL = LoRA off (then these calls are
 * mxfp4_moe_forward / mxfp4_moe_backward). lora_scaling: host array {s_g, s_u, s_d}
 * (lora_alpha / r). 1 <= lora_rank <= 32.
 * The backward also writes the adapter gradients (lora_layer.py:178-226 summed over the
 * experts, the sum the reference accumulates with accumulate_grad, lazy_trainer.py:866-876)
 * into lora_grads: host array of 6 device pointers shaped like `lora`, overwritten.
 * MXFP4_MOE_REUSE_FORWARD needs a forward made with MXFP4_MOE_SAVE and the same adapters. */
int mxfp4_moe_forward_lora(float *out, const void *h, int h_dtype, const void *topk_idx,
                           int idx_dtype, const float *topk_w, int N, int k, const uint8_t *w1p,
                           const uint8_t *w1s, const uint8_t *w3p, const uint8_t *w3s,
                           const uint8_t *w2p, const uint8_t *w2s, int E, int D, int F,
                           int act_kind, const float *const *lora, const float *lora_scaling,
                           int lora_rank, int flags, void *workspace, size_t workspace_bytes,
                           hipStream_t stream);
int mxfp4_moe_backward_lora(float *grad_h, float *grad_w, const float *grad_out, const void *h,
                            int h_dtype, const void *topk_idx, int idx_dtype,
                            const float *topk_w, int N, int k, const uint8_t *w1p,
                            const uint8_t *w1s, const uint8_t *w3p, const uint8_t *w3s,
                            const uint8_t *w2p, const uint8_t *w2s, int E, int D, int F,
                            int act_kind, const float *const *lora, const float *lora_scaling,
                            int lora_rank, float *const *lora_grads, int flags, void *workspace,
                            size_t workspace_bytes, hipStream_t stream);

/* Forward layout: a load-time copy of expert weights for the routed layer's forward products.
 * No counterpart in the reference, whose weights stay in the checkpoint layout; it is for
 * callers that keep a layer resident in HBM over many steps. For E stacked packed [R, K]
 * matrices (K a multiple of 512) with their E8M0 scales [R, K / 32], mxfp4_forward_layout writes
 * mxfp4_forward_layout_bytes(E, R, K) bytes: per expert, 16-row group and 512-element
 * super-chunk, the 4 KiB of codes that the one-tile forward work-groups read, in the order their
 * load instructions consume them (each instruction then reads 1 KiB contiguous instead of
 * 16-byte pieces of 16 rows; the large-bucket work-groups' copies read four 256-byte runs instead
 * of 16 rows' 64-byte runs), then the same blocks' scales, 256 B per group and super-chunk in the
 * order one 4-byte load per lane reads them (each scale line read once). The copy must be rebuilt
 * whenever the weights change. dst, packed and scales: 16-byte aligned, dst overlapping neither. */
size_t mxfp4_forward_layout_bytes(int E, int R, int K);
int mxfp4_forward_layout(uint8_t *dst, const uint8_t *packed, const uint8_t *scales, int E, int R,
                         int K, hipStream_t stream);

/* Backward layout: a load-time copy of expert weights for the routed layer's transposed
 * products (the backward). No counterpart in the reference; like the forward layout it is for
 * callers that keep a layer resident in HBM. For E stacked packed [R, K] matrices (R a multiple
 * of 32, K a multiple of 256) with their E8M0 scales [R, K / 32], mxfp4_backward_layout writes
 * mxfp4_backward_layout_bytes(E, R, K) bytes (the codes and scales it copies, rearranged): per
 * expert, 32-row step and 256-element stripe, the 4 KiB of codes that one wave of the transposed
 * products reads, in the order its four 16-byte loads per lane consume them (each instruction
 * reads 1 KiB contiguous instead of 8-byte or 4-byte pieces of eight rows), then the blocks'
 * scales, 256 B each, one 8-byte load per lane (instead of eight scale loads). 0 bytes / MXFP4_EINVAL for
 * other shapes. The copy must be rebuilt whenever the weights change. dst, packed and scales:
 * 16-byte aligned, dst overlapping neither. */
size_t mxfp4_backward_layout_bytes(int E, int R, int K);
int mxfp4_backward_layout(uint8_t *dst, const uint8_t *packed, const uint8_t *scales, int E, int R,
                          int K, hipStream_t stream);

/* mxfp4_moe_forward_lora / mxfp4_moe_backward_lora that also read load-time layouts: fwd_layout
 * is a host array of 3 device pointers {W1, W3, W2}, the mxfp4_forward_layout of w1p, w3p, w2p
 * (W1 and W3 both or neither; NULL entries, or a NULL array, read the checkpoint layout). An
 * entry needs its K (D for W1 and W3, F for W2) to be a multiple of 512. With
 * MXFP4_MOE_BWD_LAYOUT in flags the array holds 6 pointers: those 3, then the
 * mxfp4_backward_layout of w1p, w3p, w2p (again W1 and W3 both or neither; W1 and W3 need D a
 * multiple of 256, W2 needs F a multiple of 256), which the backward's transposed products read
 * (the forward ignores them). Results are bit-identical to the calls without layouts; w1p..w2s
 * are still read where a product has no layout copy. */
int mxfp4_moe_forward_fl(float *out, const void *h, int h_dtype, const void *topk_idx,
                         int idx_dtype, const float *topk_w, int N, int k, const uint8_t *w1p,
                         const uint8_t *w1s, const uint8_t *w3p, const uint8_t *w3s,
                         const uint8_t *w2p, const uint8_t *w2s, const uint8_t *const *fwd_layout,
                         int E, int D, int F, int act_kind, const float *const *lora,
                         const float *lora_scaling, int lora_rank, int flags, void *workspace,
                         size_t workspace_bytes, hipStream_t stream);
int mxfp4_moe_backward_fl(float *grad_h, float *grad_w, const float *grad_out, const void *h,
                          int h_dtype, const void *topk_idx, int idx_dtype, const float *topk_w,
                          int N, int k, const uint8_t *w1p, const uint8_t *w1s,
                          const uint8_t *w3p, const uint8_t *w3s, const uint8_t *w2p,
                          const uint8_t *w2s, const uint8_t *const *fwd_layout, int E, int D,
                          int F, int act_kind, const float *const *lora,
                          const float *lora_scaling, int lora_rank, float *const *lora_grads,
                          int flags, void *workspace, size_t workspace_bytes, hipStream_t stream);

/* Copies the routing status word of a routed-layer workspace to *host_flags after
 * synchronising `stream`: bit 0 set = some topk_idx entry was outside [0, E). */
int mxfp4_moe_route_status(const void *workspace, int *host_flags, hipStream_t stream);

/* Expert selection of KimiK3MoERouter.forward after the gate product
 * (lazy_lora/core/moe_router.py:81-99, the torch branch; :102-123 is the same in NumPy):
 *   scores = sigmoid(logits); choice = scores + bias (bias may be NULL: no bias);
 *   topk_idx[t, :] = the top_k experts by choice, in descending order (torch.topk(sorted=True);
 *   equal choices go to the lower expert id first);
 *   topk_w[t, j] = scores[t, topk_idx[t, j]], divided by (sum over j + 1e-20) when
 *   renormalize != 0 and top_k > 1, then multiplied by routed_scaling_factor.
 * logits [N, E] fp32 (the caller's x . W_gate^T, fp32 as in the reference), bias [E] fp32;
 * topk_idx [N, top_k] int64 and topk_w [N, top_k] fp32, the dtypes the routed-layer entry
 * points take. 1 <= top_k <= min(E, 64), E <= 4096. */
int mxfp4_router_topk(int64_t *topk_idx, float *topk_w, const float *logits, const float *bias, int N,
                      int E, int top_k, float routed_scaling_factor, int renormalize,
                      hipStream_t stream);

/* Gradient of mxfp4_router_topk's weights with respect to its logits: the autograd of the
 * torch branch (lazy_lora/core/moe_router.py:86-98) that carries dL/dtopk_w back into the
 * router's input (lazy_lora/trainer/lazy_trainer.py:842-844). grad_logits [N, E] fp32 is fully
 * written: sigmoid'(logit) times the derivative of the renormalised, scaled weights for the
 * chosen experts, 0 elsewhere. topk_idx [N, top_k] int64 as produced by mxfp4_router_topk;
 * grad_w [N, top_k] fp32. Same limits as mxfp4_router_topk. */
int mxfp4_router_topk_backward(float *grad_logits, const int64_t *topk_idx, const float *grad_w,
                               const float *logits, int N, int E, int top_k,
                               float routed_scaling_factor, int renormalize, hipStream_t stream);

/* Phase timing of the routed-layer calls made on the calling thread, the counterpart of the
 * reference's LAZYLORA_PROFILE timings (lazy_lora/trainer/lazy_trainer.py:192-194). While
 * enabled, every mxfp4_moe_forward/backward call records HIP events on its stream around
 * each phase (routing, quantisation, each product, combine) into a ring of 128 calls; nothing
 * synchronises. mxfp4_moe_timing(1) also clears the ring. mxfp4_moe_phase_times waits for call
 * number `call` (0-based since enabling) and writes up to max_phases elapsed times in ms and
 * phase names (static strings); it returns the phase count or a negative MXFP4_E* code. */
int mxfp4_moe_timing(int enable);
int mxfp4_moe_timed_calls(void);
int mxfp4_moe_phase_times(int call, float *ms, const char **names, int max_phases);

#ifdef __cplusplus
}
#endif

#endif /* LAZYLORA_MXFP4_H */
