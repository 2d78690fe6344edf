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
MX_DEV float bf16_lo(uint32_t v) { return __builtin_bit_cast(float, v << 16); }
MX_DEV float bf16_hi(uint32_t v) { return __builtin_bit_cast(float, v & 0xffff0000u); }

// Elements (row, c .. c+3) of a source matrix as fp32; c is a multiple of 4.
template <int KIND>
MX_DEV f32x4 src4(const LoraMat& a, long long row, int c)
{
  if (KIND == kLoraF32) return *reinterpret_cast<const f32x4*>(static_cast<const float*>(a.p0) + row * a.ld + c);
  if (KIND == kLoraBF16) {
    const uint2 v = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.p0) + row * a.ld + c);
    return f32x4{bf16_lo(v.x), bf16_hi(v.x), bf16_lo(v.y), bf16_hi(v.y)};
  }
  if (KIND == kLoraGLU) {
    const float* r = static_cast<const float*>(a.p0) + row * a.ld;
    const f32x4 g = *reinterpret_cast<const f32x4*>(r + c), u = *reinterpret_cast<const f32x4*>(r + a.F + c);
    return f32x4{glu_fwd(g[0], u[0], a.act_kind), glu_fwd(g[1], u[1], a.act_kind), glu_fwd(g[2], u[2], a.act_kind),
                 glu_fwd(g[3], u[3], a.act_kind)};
  }
  const long long o = row * a.ld + c;
  const uint2 h = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.p0) + o);
  const uint2 l = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.p1) + o);
  return f32x4{bf16_lo(h.x) + bf16_lo(l.x), bf16_hi(h.x) + bf16_hi(l.x), bf16_lo(h.y) + bf16_lo(l.y),
               bf16_hi(h.y) + bf16_hi(l.y)};
}

// Streaming (nt) loads of the same elements, for the outer-product reductions, whose load
// instructions each read their lines whole and exactly once.
template <typename V>
MX_DEV V ldnt(const V* p) { return __builtin_nontemporal_load(p); }

template <int KIND>
MX_DEV f32x4 src4_nt(const LoraMat& a, long long row, int c)
{
  if (KIND == kLoraF32) return ldnt(reinterpret_cast<const f32x4*>(static_cast<const float*>(a.p0) + row * a.ld + c));
  if (KIND == kLoraBF16) {
    typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
    const u32x2v v = ldnt(reinterpret_cast<const u32x2v*>(static_cast<const uint16_t*>(a.p0) + row * a.ld + c));
    return f32x4{bf16_lo(v[0]), bf16_hi(v[0]), bf16_lo(v[1]), bf16_hi(v[1])};
  }
  if (KIND == kLoraGLU) {
    const float* r = static_cast<const float*>(a.p0) + row * a.ld;
    const f32x4 g = ldnt(reinterpret_cast<const f32x4*>(r + c)), u = ldnt(reinterpret_cast<const f32x4*>(r + a.F + c));
    return f32x4{glu_fwd(g[0], u[0], a.act_kind), glu_fwd(g[1], u[1], a.act_kind), glu_fwd(g[2], u[2], a.act_kind),
                 glu_fwd(g[3], u[3], a.act_kind)};
  }
  typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
  const long long o = row * a.ld + c;
  const u32x2v h = ldnt(reinterpret_cast<const u32x2v*>(static_cast<const uint16_t*>(a.p0) + o));
  const u32x2v l = ldnt(reinterpret_cast<const u32x2v*>(static_cast<const uint16_t*>(a.p1) + o));
  return f32x4{bf16_lo(h[0]) + bf16_lo(l[0]), bf16_hi(h[0]) + bf16_hi(l[0]), bf16_lo(h[1]) + bf16_lo(l[1]),
               bf16_hi(h[1]) + bf16_hi(l[1])};
}

MX_DEV float factor_at(const LoraFactor& f, int j, int k)
{
  return f.kmajor ? f.m[(long long)k * f.ld + j] : f.m[(long long)j * f.ld + k];
}

// f(j, k .. k+3), zero for j >= r; k is a multiple of 4.
MX_DEV f32x4 factor4(const LoraFactor& f, int j, int k, int r)
{
  if (j >= r) return f32x4{0.f, 0.f, 0.f, 0.f};
  if (!f.kmajor) return *reinterpret_cast<const f32x4*>(f.m + (long long)j * f.ld + k);
  const float* p = f.m + (long long)k * f.ld + j;
  return f32x4{p[0], p[f.ld], p[2 * f.ld], p[3 * f.ld]};
}

// fp32 matrix-core step: D[16 x 16] += A[16 x 4] B[4 x 16]. Lane l = (i = l % 16, q = l / 16)
// supplies A[i][q] and B[q][i] and holds D[4q + v][i] in element v.
MX_DEV f32x4 mfma4(float a, float b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

// ---------------------------------------------------------------- row dots
// Each wave takes one (16-row tile, segment, k-slice) and accumulates its 16 x r block of
// partial sums on the matrix cores. Lane (i, q) loads KPL consecutive k of row i (KPL = 4 for
// fp32 sources, 8 for bf16 ones, so that a load instruction reads whole 64-byte pieces of the
// 16 rows) and the same k of coefficient i (and 16 + i); one MFMA per k of the lane, each
// taking k-index q from every lane, covers the 4 KPL k of a load. The k-slices are added in
// order by lora_rowdot_reduce_kernel.
struct RowDotArgs {
  LoraMat src;
  int rows;
  const int* rows_dev;
  int K, r, nseg, S, kb_per;  // k-slices of kb_per 32-k units
  LoraFactor f[2];
  int koff[2];
  float* partial;  // [S][rows][nseg * r]
};

constexpr int kRowDotUnits = 1;  // 32-k units per step, all loads issued before the MFMAs

// Elements (row, c .. c+7) of a bf16 or hi+lo source as fp32, from 16-byte loads; c is a multiple of 8.
template <int KIND>
MX_DEV void src8(const LoraMat& a, long long row, int c, f32x4& x0, f32x4& x1)
{
  const long long o = row * a.ld + c;
  const uint4 h = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.p0) + o);
  if (KIND == kLoraBF16) {
    x0 = f32x4{bf16_lo(h.x), bf16_hi(h.x), bf16_lo(h.y), bf16_hi(h.y)};
    x1 = f32x4{bf16_lo(h.z), bf16_hi(h.z), bf16_lo(h.w), bf16_hi(h.w)};
  } else {
    const uint4 l = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.p1) + o);
    x0 = f32x4{bf16_lo(h.x) + bf16_lo(l.x), bf16_hi(h.x) + bf16_hi(l.x), bf16_lo(h.y) + bf16_lo(l.y),
               bf16_hi(h.y) + bf16_hi(l.y)};
    x1 = f32x4{bf16_lo(h.z) + bf16_lo(l.z), bf16_hi(h.z) + bf16_hi(l.z), bf16_lo(h.w) + bf16_lo(l.w),
               bf16_hi(h.w) + bf16_hi(l.w)};
  }
}

template <int KIND>
__global__ __launch_bounds__(256) void lora_rowdot_kernel(RowDotArgs a)
{
  constexpr int KPL = (KIND == kLoraBF16 || KIND == kLoraHiLo) ? 8 : 4;
  constexpr int NV = 8 / KPL;  // loads per lane per 32-k unit
  constexpr int NC = KPL / 4;  // f32x4 per load
  const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
  const int tiles = (a.rows + 15) / 16;
  const long long task = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (task >= (long long)tiles * a.nseg * a.S) return;  // whole waves leave together
  const int ks = (int)(task % a.S);
  const int sg = (int)((task / a.S) % a.nseg);
  const int tile = (int)(task / ((long long)a.S * a.nseg));
  int nrows = a.rows;
  if (a.rows_dev) nrows = min(nrows, *a.rows_dev);
  const int row = tile * 16 + i;
  const bool rok = row < nrows;
  const LoraFactor f = a.f[sg];
  const int koff = a.koff[sg];
  const bool two = a.r > 16;
  const int nu = a.K / 32;
  const int u0 = ks * a.kb_per, u1 = min(u0 + a.kb_per, nu);
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  for (int ub = u0; ub < u1; ub += kRowDotUnits) {
    f32x4 x[kRowDotUnits][NV][NC], m0[kRowDotUnits][NV][NC], m1[kRowDotUnits][NV][NC];
#pragma unroll
    for (int uu = 0; uu < kRowDotUnits; ++uu) {
      const bool in = ub + uu < u1;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const int k = (ub + uu) * 32 + v * 4 * KPL + KPL * q;
        if (KPL == 8) {
          if (rok && in) src8<KIND>(a.src, row, koff + k, x[uu][v][0], x[uu][v][NC - 1]);
          else x[uu][v][0] = x[uu][v][NC - 1] = f32x4{0.f, 0.f, 0.f, 0.f};
        } else {
          x[uu][v][0] = (rok && in) ? src4<KIND>(a.src, row, koff + k) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int t = 0; t < NC; ++t) {
          m0[uu][v][t] = in ? factor4(f, i, k + 4 * t, a.r) : f32x4{0.f, 0.f, 0.f, 0.f};
          m1[uu][v][t] = (in && two) ? factor4(f, 16 + i, k + 4 * t, a.r) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
#pragma unroll
    for (int uu = 0; uu < kRowDotUnits; ++uu)
#pragma unroll
      for (int v = 0; v < NV; ++v)
#pragma unroll
        for (int t = 0; t < NC; ++t) {
#pragma unroll
          for (int c = 0; c < 4; ++c) acc0 = mfma4(x[uu][v][t][c], m0[uu][v][t][c], acc0);
          if (two) {
#pragma unroll
            for (int c = 0; c < 4; ++c) acc1 = mfma4(x[uu][v][t][c], m1[uu][v][t][c], acc1);
          }
        }
  }
  const int m = a.nseg * a.r;
  float* out = a.partial + (long long)ks * a.rows * m + sg * a.r;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int ro = tile * 16 + 4 * q + v;
    if (ro >= a.rows) continue;
    if (i < a.r) out[(long long)ro * m + i] = acc0[v];
    if (two && 16 + i < a.r) out[(long long)ro * m + 16 + i] = acc1[v];
  }
}

__global__ __launch_bounds__(256) void lora_rowdot_reduce_kernel(const float* partial, int S, int rows, int r,
                                                                 int nseg, float scale0, float scale1, float* out)
{
  const int m = nseg * r;
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long long)rows * m) return;
  // slices added in slice order; eight loads are issued ahead of their adds
  const float* pp = partial + idx;
  const long long step = (long long)rows * m;
  float s = 0.f;
  int ks = 0;
  for (; ks + 8 <= S; ks += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = pp[(ks + u) * step];
#pragma unroll
    for (int u = 0; u < 8; ++u) s += v[u];
  }
  for (; ks < S; ++ks) s += pp[ks * step];
  out[idx] = ((int)(idx % m) < r ? scale0 : scale1) * s;
}

// k-slices of a row dot: about 4096 waves in all, at least 4 units of 32 k each.
void rowdot_slices(int rows, int K, int nseg, int& S, int& kb_per)
{
  const int tiles = (rows + 15) / 16, nu = K / 32;
  S = 4096 / max(1, tiles * nseg);
  S = max(1, min(S, nu / 4));
  kb_per = (nu + S - 1) / S;
  S = max(1, (nu + kb_per - 1) / kb_per);
}

// ---------------------------------------------------------------- expansions
// One column per thread and 16 or 32 rows per work-group, in chunks of 16: the thread loads its
// column of each segment's factor into registers once for all of the work-group's rows, and the
// work-group's coefficient rows are staged once in LDS and read back as broadcasts. Two chunks
// per work-group (the factor read once per 32 output rows) only where that still leaves
// kExpandMinBlocks work-groups: fewer, longer work-groups measured slower.
struct ExpandArgs {
  const float* coef;
  int ldc, rows, r, nseg;
  LoraFactor f[2];
  int coff[2], col0[2], ncol[2];
  int vec[2];  // k-major factor whose rows can be read as float4 (ld % 4 == 0, 16-byte aligned)
  int chunks;  // 16-row chunks per work-group
  float* out;
  long long ldo;
  int Cout, accumulate;
};

constexpr int kExpandRows = 16;
constexpr int kExpandChunks = 2;
constexpr int kExpandMinBlocks = 768;

__global__ __launch_bounds__(256) void lora_expand_kernel(ExpandArgs a)
{
  __shared__ __attribute__((aligned(16))) float sc[kExpandChunks * kExpandRows][2][kLoraMaxRank];
  const int c = blockIdx.x * 256 + threadIdx.x;
  const int span = a.chunks * kExpandRows;
  const int t0 = blockIdx.y * span;
  const int nr = min(span, a.rows - t0);
  for (int i = threadIdx.x; i < span * 2 * kLoraMaxRank; i += 256) {
    const int u = i / (2 * kLoraMaxRank), sg = (i / kLoraMaxRank) & 1, j = i % kLoraMaxRank;
    sc[u][sg][j] = (u < nr && sg < a.nseg && j < a.r) ? a.coef[(long long)(t0 + u) * a.ldc + a.coff[sg] + j] : 0.f;
  }
  __syncthreads();
  if (c >= a.Cout) return;
  float mc[2][kLoraMaxRank];
  bool in[2];
#pragma unroll
  for (int sg = 0; sg < 2; ++sg) {
    const int cc = c - a.col0[sg];
    in[sg] = sg < a.nseg && cc >= 0 && cc < a.ncol[sg];
    const LoraFactor& f = a.f[sg];
    if (in[sg] && a.vec[sg]) {
      // row cc of a k-major factor: ceil(r / 4) float4s, which stay inside the row (r <= ld, ld % 4 == 0)
      const f32x4* p = reinterpret_cast<const f32x4*>(f.m + (long long)cc * f.ld);
#pragma unroll
      for (int j4 = 0; j4 < kLoraMaxRank / 4; ++j4) {
        const f32x4 v = j4 * 4 < a.r ? p[j4] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; ++t) mc[sg][4 * j4 + t] = 4 * j4 + t < a.r ? v[t] : 0.f;
      }
    } else {
#pragma unroll
      for (int j = 0; j < kLoraMaxRank; ++j) mc[sg][j] = (in[sg] && j < a.r) ? factor_at(f, j, cc) : 0.f;
    }
  }
  for (int u0 = 0; u0 < nr; u0 += kExpandRows) {
    float acc[kExpandRows];
#pragma unroll
    for (int u = 0; u < kExpandRows; ++u)
      acc[u] = (a.accumulate && u0 + u < nr) ? a.out[(long long)(t0 + u0 + u) * a.ldo + c] : 0.f;
#pragma unroll
    for (int sg = 0; sg < 2; ++sg) {
      if (!in[sg]) continue;
      const float scale = a.f[sg].scale;
#pragma unroll
      for (int u = 0; u < kExpandRows; ++u) {
        float s = 0.f;
#pragma unroll
        for (int j4 = 0; j4 < kLoraMaxRank / 4; ++j4) {
          if (j4 * 4 < a.r) {  // uniform
            const f32x4 cv = *reinterpret_cast<const f32x4*>(&sc[u0 + u][sg][j4 * 4]);
            s += cv.x * mc[sg][j4 * 4] + cv.y * mc[sg][j4 * 4 + 1] + cv.z * mc[sg][j4 * 4 + 2] +
                 cv.w * mc[sg][j4 * 4 + 3];
          }
        }
        acc[u] += scale * s;
      }
    }
#pragma unroll
    for (int u = 0; u < kExpandRows; ++u)
      if (u0 + u < nr) a.out[(long long)(t0 + u0 + u) * a.ldo + c] = acc[u];
  }
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
// Each wave takes 64 columns and one chunk of rows; per 4 rows, lane (i, q) loads row q's
// columns 4i .. 4i+3 and that row's coefficient 16 jt + i, and four MFMAs (one per column
// phase t) accumulate G[16 jt + .., 4 i' + t]. Chunks are added in order by the reduce kernel.
constexpr int kOuterBlocks = 4;

struct OuterArgs {
  LoraMat src;
  int c_off, Q;
  const int* pair_of;
  int k;
  const float* topk_w;
  const float* coef;
  int ldc, coff, m, C, chunk, RS;
  float* partial;  // [RS][m][C]
};

template <int KIND, int JT>
__global__ __launch_bounds__(256) void lora_outer_kernel(OuterArgs a)
{
  const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
  const int ncb = (a.C + 63) / 64;
  const long long task = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (task >= (long long)ncb * a.RS) return;
  const int cb = (int)(task % ncb), rs = (int)(task / ncb);
  const int c = cb * 64 + 4 * i;
  const bool cok = c < a.C;
  const int q0 = rs * a.chunk, q1 = min(q0 + a.chunk, a.Q);
  f32x4 acc[JT][4];
#pragma unroll
  for (int jt = 0; jt < JT; ++jt)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[jt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  // four blocks of 4 rows per step: the rows' pair -> token lookups first, then every load of
  // the step's 16 rows, then the MFMAs
  for (int qb = q0; qb < q1; qb += 4 * kOuterBlocks) {
    int row[kOuterBlocks], crow[kOuterBlocks];  // row < 0: no row (past the chunk, or a dropped pair)
    float wq[kOuterBlocks];
#pragma unroll
    for (int u = 0; u < kOuterBlocks; ++u) {
      const int qq = qb + 4 * u + q;
      const bool in = qq < q1;
      row[u] = in ? qq : -1;
      crow[u] = qq;
      wq[u] = 1.0f;
      if (a.pair_of && in) {
        row[u] = a.pair_of[qq];
        crow[u] = qq / a.k;
        if (a.topk_w) wq[u] = a.topk_w[qq];
      }
    }
    f32x4 x[kOuterBlocks];
#pragma unroll
    for (int u = 0; u < kOuterBlocks; ++u)
      x[u] = (row[u] >= 0 && cok) ? src4_nt<KIND>(a.src, row[u], a.c_off + c) : f32x4{0.f, 0.f, 0.f, 0.f};
    float cf[kOuterBlocks][JT];
#pragma unroll
    for (int u = 0; u < kOuterBlocks; ++u) {
      const float* cr = a.coef + (long long)crow[u] * a.ldc + a.coff;
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) {
        const int j = jt * 16 + i;
        cf[u][jt] = (row[u] >= 0 && j < a.m) ? wq[u] * cr[j] : 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < kOuterBlocks; ++u)
#pragma unroll
      for (int jt = 0; jt < JT; ++jt)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[jt][t] = mfma4(cf[u][jt], x[u][t], acc[jt][t]);
  }
  float* out = a.partial + (long long)rs * a.m * a.C;
#pragma unroll
  for (int jt = 0; jt < JT; ++jt) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int j = jt * 16 + 4 * q + v;
      if (j < a.m && cok)
        *reinterpret_cast<f32x4*>(out + (long long)j * a.C + c) =
            f32x4{acc[jt][0][v], acc[jt][1][v], acc[jt][2][v], acc[jt][3][v]};
    }
  }
}

__global__ __launch_bounds__(256) void lora_outer_reduce_kernel(const float* partial, int RS, int m, int C,
                                                                LoraOuterDst d)
{
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long long)m * C) return;
  const int j = (int)(idx / C), c = (int)(idx % C);
  // four independent running sums (slices rs = 4i + q) keep four loads in flight per thread;
  // they are added in a fixed order, so the result does not depend on timing
  const float* pp = partial + (long long)j * C + c;
  const long long step = (long long)m * C;
  float q0 = 0.f, q1 = 0.f, q2 = 0.f, q3 = 0.f;
  int rs = 0;
  for (; rs + 16 <= RS; rs += 16) {  // the same sums, sixteen loads issued ahead of their adds
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = pp[(rs + u) * step];
#pragma unroll
    for (int u = 0; u < 16; u += 4) {
      q0 += v[u];
      q1 += v[u + 1];
      q2 += v[u + 2];
      q3 += v[u + 3];
    }
  }
  for (; rs + 4 <= RS; rs += 4) {
    q0 += pp[(rs + 0) * step];
    q1 += pp[(rs + 1) * step];
    q2 += pp[(rs + 2) * step];
    q3 += pp[(rs + 3) * step];
  }
  for (; rs < RS; ++rs) q0 += pp[rs * step];
  const float s = (q0 + q1) + (q2 + q3);
  const int sg = (d.split_j > 0 && j >= d.split_j) ? 1 : 0;
  const int jj = sg ? j - d.split_j : j;
  const long long o = d.kmajor[sg] ? (long long)c * d.ld[sg] + jj : (long long)jj * d.ld[sg] + c;
  d.p[sg][o] = d.scale[sg] * s;
}

template <int JT>
void outer_launch(int kind, dim3 grid, dim3 block, const OuterArgs& a, hipStream_t s)
{
  switch (kind) {
    case kLoraF32: hipLaunchKernelGGL((lora_outer_kernel<kLoraF32, JT>), grid, block, 0, s, a); break;
    case kLoraBF16: hipLaunchKernelGGL((lora_outer_kernel<kLoraBF16, JT>), grid, block, 0, s, a); break;
    case kLoraGLU: hipLaunchKernelGGL((lora_outer_kernel<kLoraGLU, JT>), grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL((lora_outer_kernel<kLoraHiLo, JT>), grid, block, 0, s, a); break;
  }
}

// Row chunking of the outer reductions: about 4096 waves in all, at least 16 rows each.
void outer_chunks(int Q, int C, int& RS, int& chunk)
{
  const int ncb = (C + 63) / 64;
  int want = 4096 / max(1, ncb);
  want = max(1, min(want, (Q + 15) / 16));
  chunk = (Q + want - 1) / want;
  chunk = (chunk + 4 * kOuterBlocks - 1) / (4 * kOuterBlocks) * (4 * kOuterBlocks);
  RS = chunk > 0 ? (Q + chunk - 1) / chunk : 0;
}

}  // namespace

size_t lora_rowdot_partial_floats(int rows, int K, int nseg, int r)
{
  int S, kb_per;
  rowdot_slices(rows, K, nseg, S, kb_per);
  return (size_t)S * (size_t)rows * (size_t)(nseg * r);
}

hipError_t launch_lora_rowdot(const LoraMat& src, int rows, const int* rows_dev, int K, int r, int nseg,
                              const LoraFactor* f, const int* koff, float* partial, float* out, hipStream_t s)
{
  if (rows <= 0) return hipSuccess;
  if (r > kLoraMaxRank || nseg < 1 || nseg > 2 || K % 32) return hipErrorInvalidValue;
  RowDotArgs a = {};
  a.src = src; a.rows = rows; a.rows_dev = rows_dev; a.K = K; a.r = r; a.nseg = nseg; a.partial = partial;
  rowdot_slices(rows, K, nseg, a.S, a.kb_per);
  for (int i = 0; i < nseg; ++i) {
    a.f[i] = f[i];
    a.koff[i] = koff[i];
  }
  const long long waves = (long long)((rows + 15) / 16) * nseg * a.S;
  dim3 grid((unsigned)((waves + 3) / 4)), block(256);
  switch (src.kind) {
    case kLoraF32: hipLaunchKernelGGL(lora_rowdot_kernel<kLoraF32>, grid, block, 0, s, a); break;
    case kLoraBF16: hipLaunchKernelGGL(lora_rowdot_kernel<kLoraBF16>, grid, block, 0, s, a); break;
    case kLoraGLU: hipLaunchKernelGGL(lora_rowdot_kernel<kLoraGLU>, grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL(lora_rowdot_kernel<kLoraHiLo>, grid, block, 0, s, a); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const long long n = (long long)rows * nseg * r;
  hipLaunchKernelGGL(lora_rowdot_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, partial, a.S,
                     rows, r, nseg, f[0].scale, nseg > 1 ? f[1].scale : f[0].scale, out);
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
  for (int i = 0; i < nseg; ++i)
    a.vec[i] = f[i].kmajor && f[i].ld % 4 == 0 && ((uintptr_t)f[i].m & 15) == 0;
  a.out = out; a.ldo = ldo; a.Cout = Cout; a.accumulate = accumulate;
  const int col_blocks = (Cout + 255) / 256, row_tiles = (rows + kExpandRows - 1) / kExpandRows;
  a.chunks = kExpandChunks;
  while (a.chunks > 1 && (long long)col_blocks * ((row_tiles + a.chunks - 1) / a.chunks) < kExpandMinBlocks)
    a.chunks /= 2;
  dim3 grid((unsigned)col_blocks, (unsigned)((row_tiles + a.chunks - 1) / a.chunks)), block(256);
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

hipError_t launch_lora_outer(const LoraMat& src, int c_off, int Q, const int* pair_of, int k, const float* topk_w,
                             const float* coef, int ldc, int coff, int m, int C, float* partial,
                             const LoraOuterDst& dst, hipStream_t s)
{
  if (C <= 0 || m <= 0) return hipSuccess;
  if (m > 64 || C % 4) return hipErrorInvalidValue;
  OuterArgs a = {};
  outer_chunks(Q, C, a.RS, a.chunk);
  if (a.RS > 0) {
    a.src = src; a.c_off = c_off; a.Q = Q; a.pair_of = pair_of; a.k = k; a.topk_w = topk_w;
    a.coef = coef; a.ldc = ldc; a.coff = coff; a.m = m; a.C = C; a.partial = partial;
    const long long waves = (long long)((C + 63) / 64) * a.RS;
    dim3 grid((unsigned)((waves + 3) / 4)), block(256);
    if (m <= 16) outer_launch<1>(src.kind, grid, block, a, s);
    else if (m <= 32) outer_launch<2>(src.kind, grid, block, a, s);
    else outer_launch<4>(src.kind, grid, block, a, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const long long n = (long long)m * C;
  hipLaunchKernelGGL(lora_outer_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, partial, a.RS, m,
                     C, dst);
  return hipGetLastError();
}

}  // namespace mx
