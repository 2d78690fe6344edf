// Expert selection of the Kimi-K3 MoE router on the GPU (lazy_lora/core/moe_router.py:55-123).
//
// The gate product logits = x . W^T is a plain dense GEMM and runs in the platform BLAS; this
// kernel does the rest per token, one wave per token: scores = sigmoid(logits), the top_k
// largest of scores + bias (the bias steers selection only), the unbiased scores of the chosen
// experts renormalised by their sum + 1e-20 and multiplied by the scaling factor. The indices
// are written in descending order of the biased score, like torch.topk(sorted=True); equal
// scores go to the lower expert id first.
#include "mx_device.h"
#include "mx_kernels.h"

namespace mx {

namespace {

// (value, index) pair order for the selection: NaN first (torch.topk ranks NaN above every
// number), then the larger value, then the lower index.
__device__ __forceinline__ bool beats(float v, int i, float bv, int bi)
{
  const bool vn = v != v, bn = bv != bv;
  if (vn != bn) return vn;
  return (vn || v == bv) ? i < bi : v > bv;
}

template <int PER_LANE>
__global__ __launch_bounds__(256) void router_topk_kernel(long long* __restrict__ topk_idx, float* __restrict__ topk_w,
                                                          const float* __restrict__ logits,
                                                          const float* __restrict__ bias, int N, int E, int top_k,
                                                          float scale, int renormalize)
{
  const int lane = threadIdx.x & 63;
  const int token = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (token >= N) return;  // whole waves leave together
  const float* row = logits + (long long)token * E;

  // this lane's experts e = lane + 64 m; `open` marks the ones still selectable (present and
  // not yet chosen), so every round's winner is a real expert id whatever the scores hold
  // (NaN, infinities) as long as top_k <= E, which the host checks
  float choice[PER_LANE];
  uint64_t open = 0;
#pragma unroll
  for (int m = 0; m < PER_LANE; ++m) {
    const int e = lane + 64 * m;
    choice[m] = 0.f;
    if (e < E) {
      const float s = 1.0f / (1.0f + expf(-row[e]));
      choice[m] = bias ? s + bias[e] : s;
      open |= 1ull << m;
    }
  }

  float sum = 0.f;
  float mine = 0.f;  // lane t keeps the t-th chosen score
  int mine_idx = 0;
  for (int t = 0; t < top_k; ++t) {
    float bv = -__builtin_inff();
    int bi = 0x7fffffff;  // "none": loses to every open entry
#pragma unroll
    for (int m = 0; m < PER_LANE; ++m) {
      const int e = lane + 64 * m;
      if (((open >> m) & 1) && (bi == 0x7fffffff || beats(choice[m], e, bv, bi))) {
        bv = choice[m];
        bi = e;
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 64);
      const int oi = __shfl_xor(bi, off, 64);
      if (oi != 0x7fffffff && (bi == 0x7fffffff || beats(ov, oi, bv, bi))) {
        bv = ov;
        bi = oi;
      }
    }
    if (bi >= E) bi = 0;  // unreachable while top_k <= E; keeps the read below in bounds
    // every lane now holds the winner; its owner retires it
    if ((bi & 63) == lane) open &= ~(1ull << (bi >> 6));
    const float s = 1.0f / (1.0f + expf(-row[bi]));  // the unbiased score
    sum += s;
    if (lane == t) {
      mine = s;
      mine_idx = bi;
    }
  }
  if (lane < top_k) {
    float w = mine;
    if (renormalize && top_k > 1) w = w / (sum + 1e-20f);
    topk_idx[(long long)token * top_k + lane] = mine_idx;
    topk_w[(long long)token * top_k + lane] = w * scale;
  }
}

// Gradient of the combine weights with respect to the logits, the autograd of the torch
// branch (moe_router.py:86-98), which the trainer relies on to carry dL/dtopk_w back into the
// router's input (lazy_lora/trainer/lazy_trainer.py:842-844). With s_j the chosen scores,
// S = sum_j s_j + 1e-20 and c the scaling factor:
//   w_j = c s_j / S          (renormalised)  =>  dL/ds_i = c (g_i / S - sum_j g_j s_j / S^2)
//   w_j = c s_j              (otherwise)     =>  dL/ds_i = c g_i
// and dL/dlogit_i = dL/ds_i s_i (1 - s_i) for chosen experts, 0 for the others (the selection
// itself has no gradient, and neither has the bias). One wave per token writes its whole row.
template <int PER_LANE>
__global__ __launch_bounds__(256) void router_topk_bwd_kernel(float* __restrict__ grad_logits,
                                                              const long long* __restrict__ topk_idx,
                                                              const float* __restrict__ grad_w,
                                                              const float* __restrict__ logits, int N, int E,
                                                              int top_k, float scale, int renormalize)
{
  const int lane = threadIdx.x & 63;
  const int token = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (token >= N) return;
  const float* row = logits + (long long)token * E;

  int e = -1;
  float s = 0.f, sm = 0.f, g = 0.f;  // sm = sigmoid(-x) = 1 - s, without the cancellation of 1 - s
  if (lane < top_k) {
    const long long v = topk_idx[(long long)token * top_k + lane];
    if (v >= 0 && v < E) {
      e = (int)v;
      s = 1.0f / (1.0f + expf(-row[e]));
      sm = 1.0f / (1.0f + expf(row[e]));
      g = grad_w[(long long)token * top_k + lane];
    }
  }
  float S = s, G = g * s;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    S += __shfl_xor(S, off, 64);
    G += __shfl_xor(G, off, 64);
  }
  float ds;
  if (renormalize && top_k > 1) {
    const float den = S + 1e-20f;
    ds = scale * (g / den - G / (den * den));
  } else {
    ds = scale * g;
  }
  const float val = ds * s * sm;  // sigmoid'(x) = s (1 - s), its small factor computed directly

  float out[PER_LANE];
#pragma unroll
  for (int m = 0; m < PER_LANE; ++m) out[m] = 0.f;
  for (int j = 0; j < top_k; ++j) {
    const int ej = __shfl(e, j, 64);
    const float vj = __shfl(val, j, 64);
    if (ej >= 0 && (ej & 63) == lane) {
#pragma unroll
      for (int m = 0; m < PER_LANE; ++m)
        if (lane + 64 * m == ej) out[m] += vj;
    }
  }
  float* orow = grad_logits + (long long)token * E;
#pragma unroll
  for (int m = 0; m < PER_LANE; ++m) {
    const int c = lane + 64 * m;
    if (c < E) orow[c] = out[m];
  }
}

}  // namespace

hipError_t launch_router_topk_bwd(float* grad_logits, const long long* topk_idx, const float* grad_w,
                                  const float* logits, int N, int E, int top_k, float scale, int renormalize,
                                  hipStream_t s)
{
  if (N <= 0) return hipSuccess;
  dim3 grid((unsigned)((N + 3) / 4)), block(256);
  if (E <= 16 * 64)
    hipLaunchKernelGGL(router_topk_bwd_kernel<16>, grid, block, 0, s, grad_logits, topk_idx, grad_w, logits, N, E,
                       top_k, scale, renormalize);
  else
    hipLaunchKernelGGL(router_topk_bwd_kernel<64>, grid, block, 0, s, grad_logits, topk_idx, grad_w, logits, N, E,
                       top_k, scale, renormalize);
  return hipGetLastError();
}

hipError_t launch_router_topk(long long* topk_idx, float* topk_w, const float* logits, const float* bias, int N,
                              int E, int top_k, float scale, int renormalize, hipStream_t s)
{
  if (N <= 0) return hipSuccess;
  dim3 grid((unsigned)((N + 3) / 4)), block(256);
  if (E <= 16 * 64)
    hipLaunchKernelGGL(router_topk_kernel<16>, grid, block, 0, s, topk_idx, topk_w, logits, bias, N, E, top_k, scale,
                       renormalize);
  else
    hipLaunchKernelGGL(router_topk_kernel<64>, grid, block, 0, s, topk_idx, topk_w, logits, bias, N, E, top_k, scale,
                       renormalize);
  return hipGetLastError();
}

}  // namespace mx
