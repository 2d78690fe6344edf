// LoRA coupling of the routed-expert layer: the rank-r adapters shared by all experts of a
// layer (lazy_lora/trainer/lazy_trainer.py:130-134), applied as the reference applies them per
// expert (lazy_trainer.py:762-791, :836-880; lazy_lora/core/lora_layer.py:104-139, :178-226),
// but factored through per-token rank-r vectors so no expert-sized dense work is added:
//   gate/up delta of a pair = s B (A x_t): per token, added in the gate/up product's epilogue;
//   down delta summed over a token's pairs = s B_d (sum_p w_p A_d act_p): one rank-r vector per
//   token, expanded once;
//   adapter gradients = outer products summed over tokens or pairs.
// Three shapes of kernel do the small dense work: row dots (rows x long K -> rank-r
// coefficients), expansions (rank-r coefficients -> rows), and column-wise outer-product
// reductions (split over fixed row chunks, then added in chunk order, so results do not
// depend on scheduling). All arithmetic is fp32.
#include "mx_device.h"
#include "mx_kernels.h"

namespace mx {

namespace {

MX_DEV float bf16f(uint16_t v) { return __builtin_bit_cast(float, (uint32_t)v << 16); }

template <int KIND>
MX_DEV float src_at(const LoraMat& a, long long row, int c)
{
  if (KIND == kLoraF32) return static_cast<const float*>(a.p0)[row * a.ld + c];
  if (KIND == kLoraBF16) return bf16f(static_cast<const uint16_t*>(a.p0)[row * a.ld + c]);
  if (KIND == kLoraGLU) {
    const float* r = static_cast<const float*>(a.p0) + row * a.ld;
    return glu_fwd(r[c], r[a.F + c], a.act_kind);
  }
  const long long o = row * a.ld + c;
  return bf16f(static_cast<const uint16_t*>(a.p0)[o]) + bf16f(static_cast<const uint16_t*>(a.p1)[o]);
}

MX_DEV float factor_at(const LoraFactor& f, int j, int k)
{
  return f.kmajor ? f.m[(long long)k * f.ld + j] : f.m[(long long)j * f.ld + k];
}

// ---------------------------------------------------------------- row dots
struct RowDotArgs {
  LoraMat src;
  int rows;
  const int* rows_dev;
  int K, r, nseg;
  LoraFactor f[2];
  int koff[2];
  float* out;
};

// Two rows per wave; lane l takes k = l, l + 64, ... and keeps 64 partial sums (2 rows x 32
// coefficients). The wave then reduces them by recursive halving: at offset o each lane keeps
// the half of its values selected by lane bit o and adds its partner's copy of that half, so
// after six steps lane l holds the full sum of value l (row l / 32, coefficient l % 32).
template <int KIND>
__global__ __launch_bounds__(256) void lora_rowdot_kernel(RowDotArgs a)
{
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 2;
  int nrows = a.rows;
  if (a.rows_dev) nrows = min(nrows, *a.rows_dev);
  if (row0 >= nrows) return;  // whole waves leave together
  const bool two = row0 + 1 < nrows;
  for (int sg = 0; sg < a.nseg; ++sg) {
    const LoraFactor f = a.f[sg];
    const int koff = a.koff[sg];
    float v[64];
#pragma unroll
    for (int i = 0; i < 64; ++i) v[i] = 0.f;
    for (int k = lane; k < a.K; k += 64) {
      const float x0 = src_at<KIND>(a.src, row0, koff + k);
      const float x1 = two ? src_at<KIND>(a.src, row0 + 1, koff + k) : 0.f;
#pragma unroll
      for (int j = 0; j < kLoraMaxRank; ++j) {
        if (j < a.r) {
          const float m = factor_at(f, j, k);
          v[j] += x0 * m;
          v[32 + j] += x1 * m;
        }
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const bool up = (lane & o) != 0;
#pragma unroll
      for (int i = 0; i < o; ++i) {
        const float keep = up ? v[o + i] : v[i];
        const float give = up ? v[i] : v[o + i];
        v[i] = keep + __shfl_xor(give, o, 64);
      }
    }
    const int rr = lane >> 5, j = lane & 31;
    if (j < a.r && (rr == 0 || two)) a.out[(long long)(row0 + rr) * (a.nseg * a.r) + sg * a.r + j] = f.scale * v[0];
  }
}

// ---------------------------------------------------------------- expansions
struct ExpandArgs {
  const float* coef;
  int ldc, rows, r, nseg;
  LoraFactor f[2];
  int coff[2], col0[2], ncol[2];
  float* out;
  long long ldo;
  int Cout, accumulate;
};

__global__ __launch_bounds__(256) void lora_expand_kernel(ExpandArgs a)
{
  const int t = blockIdx.y;
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (t >= a.rows || c >= a.Cout) return;
  const float* cr = a.coef + (long long)t * a.ldc;
  float* o = a.out + (long long)t * a.ldo + c;
  float acc = a.accumulate ? *o : 0.f;
  for (int sg = 0; sg < a.nseg; ++sg) {
    const int cc = c - a.col0[sg];
    if (cc < 0 || cc >= a.ncol[sg]) continue;
    const LoraFactor f = a.f[sg];
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < kLoraMaxRank; ++j)
      if (j < a.r) s += cr[a.coff[sg] + j] * factor_at(f, j, cc);
    acc += f.scale * s;
  }
  *o = acc;
}

__global__ __launch_bounds__(256) void lora_slot_sum_kernel(const float* src, int m, const int* pair_of,
                                                            const float* topk_w, int N, int k, float* out)
{
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long long)N * m) return;
  const int t = (int)(idx / m), j = (int)(idx % m);
  float acc = 0.f;
  for (int s = 0; s < k; ++s) {
    const int p = pair_of[(long long)t * k + s];
    if (p < 0) continue;
    const float w = topk_w ? topk_w[(long long)t * k + s] : 1.0f;
    acc += w * src[(long long)p * m + j];
  }
  out[idx] = acc;
}

// ---------------------------------------------------------------- outer-product reductions
struct OuterArgs {
  LoraMat src;
  int Q;
  const int* pair_of;
  int k;
  const float* topk_w;
  const float* coef;
  int ldc, m, coef_split, coef_shift, C, chunk;
  float* partial;
};

constexpr int kOuterUnroll = 8;

// One column per thread, one row chunk per blockIdx.y; rows are taken eight at a time so
// their loads are in flight together.
template <int KIND>
__global__ __launch_bounds__(256) void lora_outer_kernel(OuterArgs a)
{
  const int c = blockIdx.x * 256 + threadIdx.x;
  const int rs = blockIdx.y;
  const int q0 = rs * a.chunk, q1 = min(q0 + a.chunk, a.Q);
  const bool cok = c < a.C;
  const int cs = cok ? c : 0;
  const int shift = (a.coef_split > 0 && cs >= a.coef_split) ? a.coef_shift : 0;
  float acc[64];
#pragma unroll
  for (int j = 0; j < 64; ++j) acc[j] = 0.f;
  for (int q = q0; q < q1; q += kOuterUnroll) {
    float x[kOuterUnroll];
    int crow[kOuterUnroll];
    bool ok[kOuterUnroll];
#pragma unroll
    for (int u = 0; u < kOuterUnroll; ++u) {
      const int qq = q + u;
      ok[u] = qq < q1;
      long long row = qq;
      crow[u] = qq;
      float wq = 1.0f;
      if (a.pair_of && ok[u]) {
        const int p = a.pair_of[qq];
        ok[u] = p >= 0;
        row = p;
        crow[u] = qq / a.k;
        if (a.topk_w) wq = a.topk_w[qq];
      }
      x[u] = ok[u] ? wq * src_at<KIND>(a.src, row, cs) : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kOuterUnroll; ++u) {
      if (!ok[u]) continue;
      const float* cr = a.coef + (long long)crow[u] * a.ldc + shift;
#pragma unroll
      for (int j = 0; j < 64; ++j)
        if (j < a.m) acc[j] += cr[j] * x[u];
    }
  }
  if (!cok) return;
  float* out = a.partial + (long long)rs * a.m * a.C;
#pragma unroll
  for (int j = 0; j < 64; ++j)
    if (j < a.m) out[(long long)j * a.C + c] = acc[j];
}

__global__ __launch_bounds__(256) void lora_outer_reduce_kernel(const float* partial, int RS, int m, int C,
                                                                LoraOuterDst d)
{
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long long)m * C) return;
  const int j = (int)(idx / C), c = (int)(idx % C);
  float s = 0.f;
  for (int rs = 0; rs < RS; ++rs) s += partial[((long long)rs * m + j) * C + c];
  const bool seg = (d.split_c > 0 && c >= d.split_c) || (d.split_j > 0 && j >= d.split_j);
  const int sg = seg ? 1 : 0;
  const int cc = (seg && d.split_c > 0) ? c - d.split_c : c;
  const int jj = (seg && d.split_j > 0) ? j - d.split_j : j;
  const long long o = d.kmajor[sg] ? (long long)cc * d.ld[sg] + jj : (long long)jj * d.ld[sg] + cc;
  d.p[sg][o] = d.scale[sg] * s;
}

// Row chunking of the outer reductions: about 1024 work-groups in all, at least 32 rows each.
void outer_chunks(int Q, int C, int& RS, int& chunk)
{
  const int colblocks = (C + 255) / 256;
  int want = (1024 + colblocks - 1) / colblocks;
  want = max(1, min(want, (Q + 31) / 32));
  chunk = (Q + want - 1) / want;
  chunk = (chunk + kOuterUnroll - 1) / kOuterUnroll * kOuterUnroll;
  RS = chunk > 0 ? (Q + chunk - 1) / chunk : 0;
}

}  // namespace

hipError_t launch_lora_rowdot(const LoraMat& src, int rows, const int* rows_dev, int K, int r, int nseg,
                              const LoraFactor* f, const int* koff, float* out, hipStream_t s)
{
  if (rows <= 0) return hipSuccess;
  RowDotArgs a = {};
  a.src = src; a.rows = rows; a.rows_dev = rows_dev; a.K = K; a.r = r; a.nseg = nseg; a.out = out;
  for (int i = 0; i < nseg; ++i) {
    a.f[i] = f[i];
    a.koff[i] = koff[i];
  }
  dim3 grid((unsigned)((rows + 7) / 8)), block(256);
  switch (src.kind) {
    case kLoraF32: hipLaunchKernelGGL(lora_rowdot_kernel<kLoraF32>, grid, block, 0, s, a); break;
    case kLoraBF16: hipLaunchKernelGGL(lora_rowdot_kernel<kLoraBF16>, grid, block, 0, s, a); break;
    case kLoraGLU: hipLaunchKernelGGL(lora_rowdot_kernel<kLoraGLU>, grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL(lora_rowdot_kernel<kLoraHiLo>, grid, block, 0, s, a); break;
  }
  return hipGetLastError();
}

hipError_t launch_lora_expand(const float* coef, int ldc, int rows, int r, int nseg, const LoraFactor* f,
                              const int* coff, const int* col0, const int* ncol, float* out, long long ldo, int Cout,
                              int accumulate, hipStream_t s)
{
  if (rows <= 0 || Cout <= 0) return hipSuccess;
  ExpandArgs a = {};
  a.coef = coef; a.ldc = ldc; a.rows = rows; a.r = r; a.nseg = nseg;
  for (int i = 0; i < nseg; ++i) {
    a.f[i] = f[i];
    a.coff[i] = coff[i];
    a.col0[i] = col0[i];
    a.ncol[i] = ncol[i];
  }
  a.out = out; a.ldo = ldo; a.Cout = Cout; a.accumulate = accumulate;
  dim3 grid((unsigned)((Cout + 255) / 256), (unsigned)rows), block(256);
  hipLaunchKernelGGL(lora_expand_kernel, grid, block, 0, s, a);
  return hipGetLastError();
}

hipError_t launch_lora_slot_sum(const float* src, int m, const int* pair_of, const float* topk_w, int N, int k,
                                float* out, hipStream_t s)
{
  const long long n = (long long)N * m;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(lora_slot_sum_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, m, pair_of,
                     topk_w, N, k, out);
  return hipGetLastError();
}

size_t lora_outer_partial_floats(int Q, int m, int C)
{
  int RS, chunk;
  outer_chunks(Q, C, RS, chunk);
  return (size_t)RS * (size_t)m * (size_t)C;
}

hipError_t launch_lora_outer(const LoraMat& src, int Q, const int* pair_of, int k, const float* topk_w,
                             const float* coef, int ldc, int m, int coef_split, int coef_shift, int C, float* partial,
                             const LoraOuterDst& dst, hipStream_t s)
{
  if (C <= 0 || m <= 0) return hipSuccess;
  int RS, chunk;
  outer_chunks(Q, C, RS, chunk);
  if (RS > 0) {
    OuterArgs a = {};
    a.src = src; a.Q = Q; a.pair_of = pair_of; a.k = k; a.topk_w = topk_w;
    a.coef = coef; a.ldc = ldc; a.m = m; a.coef_split = coef_split; a.coef_shift = coef_shift;
    a.C = C; a.chunk = chunk; a.partial = partial;
    dim3 grid((unsigned)((C + 255) / 256), (unsigned)RS), block(256);
    switch (src.kind) {
      case kLoraF32: hipLaunchKernelGGL(lora_outer_kernel<kLoraF32>, grid, block, 0, s, a); break;
      case kLoraBF16: hipLaunchKernelGGL(lora_outer_kernel<kLoraBF16>, grid, block, 0, s, a); break;
      case kLoraGLU: hipLaunchKernelGGL(lora_outer_kernel<kLoraGLU>, grid, block, 0, s, a); break;
      default: hipLaunchKernelGGL(lora_outer_kernel<kLoraHiLo>, grid, block, 0, s, a); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const long long n = (long long)m * C;
  hipLaunchKernelGGL(lora_outer_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, partial, RS, m, C,
                     dst);
  return hipGetLastError();
}

}  // namespace mx
