// LoRA coupling of the routed-expert layer: the rank-r adapters shared by all experts of a
// layer (lazy_lora/trainer/lazy_trainer.py:130-134), applied as the reference applies them per
// expert (lazy_trainer.py:762-791, :836-880; lazy_lora/core/lora_layer.py:104-139, :178-226),
// but factored through per-token rank-r vectors so no expert-sized dense work is added:
//   gate/up delta of a pair = s B (A x): per token, added in the gate/up product's epilogue;
//   down delta summed over a token's pairs = s B_d (sum_p w_p A_d act_p): one rank-r vector per
//   token, expanded inside the combine;
//   adapter gradients = outer products summed over tokens or pairs.
// The kernels:
//   lora_pass_kernel streams one or more of the large matrices (x, grad_out, the saved gate/up
//   pre-activations, the two-term gate/up gradients) once per stage, each work-group of 4 waves
//   running one task of one job: a row dot (64 rows x a k-slice -> rank-r coefficients, the 4
//   waves taking interleaved 32-column units and sharing nothing but the final sum), an
//   outer-product reduction (a 64-column block x a row chunk, the waves taking interleaved
//   16-row steps), or both fused over the gate/up gradients; the waves' sums are added in LDS
//   in wave order and each work-group writes one partial;
//   lora_finish_kernel adds the partials in a fixed order: row-dot partials into coefficient
//   rows (summed over each token's slots where the rows are pairs), outer-product partials into
//   the gradients;
//   lora_expand_kernel reduces per-token coefficient rows and expands them through a factor (the
//   gate/up deltas, A_down^T q), and lora_combine_kernel adds the down-projection LoRA term (and
//   in the backward A^T Dsum) while it sums each token's slot rows.
// Nothing depends on scheduling or on the order in which the routing filled the buckets, so
// results are bit-reproducible. All arithmetic is fp32.
#include "mx_device.h"
#include "mx_kernels.h"

#include <algorithm>

namespace mx {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

MX_DEV float bf16_lo(uint32_t v) { return __builtin_bit_cast(float, v << 16); }
MX_DEV float bf16_hi(uint32_t v) { return __builtin_bit_cast(float, v & 0xffff0000u); }

// Streaming (nt) loads: every line of the large matrices is read whole and once per stage.
template <typename V>
MX_DEV V ldnt(const V* p) { return __builtin_nontemporal_load(p); }

// fp32 matrix-core step: D[16 x 16] += A[16 x 4] B[4 x 16]. Lane l = (i = l % 16, q = l / 16)
// supplies A[i][q] and B[q][i] and holds D[4q + v][i] in element v.
MX_DEV f32x4 mfma4(float a, float b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

// ---------------------------------------------------------------- source elements
// Row dots read a row in 32-column units: lane (i, q) takes 8 elements of row i, element e being
// column kcol(q, e) of the unit (fp32 sources: two 16-byte loads at 4q and 16 + 4q; bf16 sources:
// one 16-byte load at 8q), so each load instruction reads whole 64-byte pieces of 16 rows.
template <int KIND>
MX_DEV int kcol(int q, int e)
{
  return (KIND == kLoraBF16 || KIND == kLoraHiLo) ? 8 * q + e : 16 * (e >> 2) + 4 * q + (e & 3);
}

template <int KIND>
struct Unit {  // raw registers of one lane's 8 elements
  u32x4 v[KIND == kLoraGLU ? 4 : (KIND == kLoraBF16 ? 1 : 2)];
};

template <int KIND>
MX_DEV Unit<KIND> unit_zero()
{
  Unit<KIND> u;
#pragma unroll
  for (int n = 0; n < (int)(sizeof(u.v) / sizeof(u.v[0])); ++n) u.v[n] = u32x4{0u, 0u, 0u, 0u};
  return u;
}

// The unit of row `row` starting at source column `col` (a multiple of 32).
template <int KIND>
MX_DEV Unit<KIND> unit_load(const LoraMat& a, long long row, int col, int q)
{
  Unit<KIND> u;
  if constexpr (KIND == kLoraF32) {
    const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const float*>(a.p0) + row * a.ld + col + 4 * q);
    u.v[0] = ldnt(p);
    u.v[1] = ldnt(p + 4);
  } else if constexpr (KIND == kLoraBF16) {
    u.v[0] = ldnt(reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.p0) + row * a.ld + col + 8 * q));
  } else if constexpr (KIND == kLoraHiLo) {
    const long long o = row * a.ld + col + 8 * q;
    u.v[0] = ldnt(reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.p0) + o));
    u.v[1] = ldnt(reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.p1) + o));
  } else {
    const float* r = static_cast<const float*>(a.p0) + row * a.ld + col + 4 * q;
    u.v[0] = ldnt(reinterpret_cast<const u32x4*>(r));
    u.v[1] = ldnt(reinterpret_cast<const u32x4*>(r + 16));
    u.v[2] = ldnt(reinterpret_cast<const u32x4*>(r + a.F));
    u.v[3] = ldnt(reinterpret_cast<const u32x4*>(r + a.F + 16));
  }
  return u;
}

template <int KIND>
MX_DEV void unit_decode(const Unit<KIND>& u, int act_kind, float x[8])
{
  if constexpr (KIND == kLoraF32) {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = bits_f(u.v[e >> 2][e & 3]);
  } else if constexpr (KIND == kLoraBF16) {
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      x[e] = bf16_lo(u.v[0][e >> 1]);
      x[e + 1] = bf16_hi(u.v[0][e >> 1]);
    }
  } else if constexpr (KIND == kLoraHiLo) {
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      x[e] = bf16_lo(u.v[0][e >> 1]) + bf16_lo(u.v[1][e >> 1]);
      x[e + 1] = bf16_hi(u.v[0][e >> 1]) + bf16_hi(u.v[1][e >> 1]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = glu_fwd(bits_f(u.v[e >> 2][e & 3]), bits_f(u.v[2 + (e >> 2)][e & 3]), act_kind);
  }
}

// Outer products read 4 consecutive columns of a row per lane (the MFMA's B operand layout).
template <int KIND>
struct Quad {
  u32x4 v[KIND == kLoraGLU ? 2 : 1];
};

template <int KIND>
MX_DEV Quad<KIND> quad_zero()
{
  Quad<KIND> u;
#pragma unroll
  for (int n = 0; n < (int)(sizeof(u.v) / sizeof(u.v[0])); ++n) u.v[n] = u32x4{0u, 0u, 0u, 0u};
  return u;
}

template <int KIND>
MX_DEV Quad<KIND> quad_load(const LoraMat& a, long long row, int col)
{
  Quad<KIND> u;
  if constexpr (KIND == kLoraF32) {
    u.v[0] = ldnt(reinterpret_cast<const u32x4*>(static_cast<const float*>(a.p0) + row * a.ld + col));
  } else if constexpr (KIND == kLoraBF16) {
    const u32x2 h = ldnt(reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(a.p0) + row * a.ld + col));
    u.v[0] = u32x4{h[0], h[1], 0u, 0u};
  } else if constexpr (KIND == kLoraHiLo) {
    const long long o = row * a.ld + col;
    const u32x2 h = ldnt(reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(a.p0) + o));
    const u32x2 l = ldnt(reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(a.p1) + o));
    u.v[0] = u32x4{h[0], h[1], l[0], l[1]};
  } else {
    const float* r = static_cast<const float*>(a.p0) + row * a.ld + col;
    u.v[0] = ldnt(reinterpret_cast<const u32x4*>(r));
    u.v[1] = ldnt(reinterpret_cast<const u32x4*>(r + a.F));
  }
  return u;
}

template <int KIND>
MX_DEV f32x4 quad_decode(const Quad<KIND>& u, int act_kind)
{
  if constexpr (KIND == kLoraF32) {
    return f32x4{bits_f(u.v[0][0]), bits_f(u.v[0][1]), bits_f(u.v[0][2]), bits_f(u.v[0][3])};
  } else if constexpr (KIND == kLoraBF16) {
    return f32x4{bf16_lo(u.v[0][0]), bf16_hi(u.v[0][0]), bf16_lo(u.v[0][1]), bf16_hi(u.v[0][1])};
  } else if constexpr (KIND == kLoraHiLo) {
    return f32x4{bf16_lo(u.v[0][0]) + bf16_lo(u.v[0][2]), bf16_hi(u.v[0][0]) + bf16_hi(u.v[0][2]),
                 bf16_lo(u.v[0][1]) + bf16_lo(u.v[0][3]), bf16_hi(u.v[0][1]) + bf16_hi(u.v[0][3])};
  } else {
    f32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = glu_fwd(bits_f(u.v[0][e]), bits_f(u.v[1][e]), act_kind);
    return r;
  }
}

// ---------------------------------------------------------------- pass kernel
// A job of the pass: a row dot or an outer product over one source (host-built by plan_job).
struct PassJob {
  int type;  // kLoraRowDot / kLoraOuter
  LoraMat src;
  int rows;              // rows of the source (tokens, or pairs in bucket order)
  const int* rows_dev;   // device count of valid rows (<= rows), or null
  int nseg, K;           // nseg segments of K columns, segment s at source column koff[s]
  int koff[2];
  int r;
  // row dot: out[row, s*r + j] (nseg 2, factor f[s]) or out[row, n*r + j] (nseg 1, factor f[n], n < nfac)
  int nfac;
  LoraFactor f[2];
  int S, kb;             // k-slices per segment, 32-column units per slice
  // outer product: G[j, s*K + c] = sum over rows q of w(q) coef(q, coff[s] + j) src(row(q), koff[s] + c)
  const float* coef;
  long long ldc;
  int coff[2];
  const int* row_of;     // non-null: q runs over (token, slot) pairs, row(q) = row_of[q] (skipped when
  int k;                 //   negative), coefficient row q / k; null: row(q) = q, coefficient row q
  const float* row_w;    // w(q) (null: 1)
  int m;                 // coefficients per segment
  int RS, chunk;         // row chunks
  int jh;                // j-halves of 32 (separate work-groups)
  float* partial;
  float* partial2;       // kLoraRowOuter: the row-dot partials
  int wg0;
};

constexpr int kMaxPassJobs = 4;
struct PassArgs {
  PassJob j[kMaxPassJobs];
  int n;
};

// Units (row dots) or 16-row steps (outer products) whose loads a wave issues before their MFMAs.
template <int KIND>
constexpr int kUnitsAhead = 2;
template <int KIND>
constexpr int kStepsAhead = 2;

// Every load below reads a valid address (rows, units, columns and coefficient indices are
// clamped into range) and nothing computes on a loaded value before the loads of its round are
// all issued; out-of-range elements are zeroed afterwards by selects, or never reach a written
// sum. (A load whose value is used inside a conditional block makes the compiler wait there for
// every load in flight.)

// The factor values lane (i, q) multiplies with its 8 unit elements: f(frow, kk0 + kcol(q, e)).
// j-major factors (rows of lora_A; base = m + frow * ld): two 16-byte loads. k-major factors
// (lora_B; base = m + frow): 8 loads, each reading 64 contiguous bytes per 16 lanes.
template <int KIND, bool KM>
MX_DEV void factor_unit(const float* base, long long ld, int kk0, int q, float out[8])
{
  if constexpr (!KM) {
    const float* b = base + kk0;
    const f32x4 a = *reinterpret_cast<const f32x4*>(b + kcol<KIND>(q, 0));
    const f32x4 c = *reinterpret_cast<const f32x4*>(b + kcol<KIND>(q, 4));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      out[e] = a[e];
      out[e + 4] = c[e];
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = base[(long long)(kk0 + kcol<KIND>(q, e)) * ld];
  }
}

// A row-dot task takes kRowTiles 16-row tiles, so each factor value a wave loads serves 64 rows
// (the factors are re-read from L2 once per 64 rows, not per 16).
constexpr int kRowTiles = 4;

template <int KIND, bool KM>
MX_DEV void rowdot_task(const PassJob& J, int t, float* red)
{
  constexpr int NT = kRowTiles;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, i = lane & 15, q = lane >> 4;
  const int slice = t % J.S;
  t /= J.S;
  const int jhalf = t % J.jh;
  t /= J.jh;
  const int seg = t % J.nseg, quad = t / J.nseg;
  int nrows = J.rows;
  if (J.rows_dev) nrows = min(nrows, *J.rows_dev);
  const int r0 = quad * 16 * NT;
  if (r0 >= nrows) return;  // the whole work-group leaves
  // rows past the end read the task's first row: only their own (unwritten) sums see them
  int srow[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) srow[n] = r0 + 16 * n + i < nrows ? r0 + 16 * n + i : r0;
  const int m_task = J.nseg == 2 ? J.r : J.nfac * J.r;
  const int jbase = 32 * jhalf;
  const int JT = min(2, (m_task - jbase + 15) / 16);
  // the lane's factor row per j-tile (clamped; columns j >= m_task of the sums are not written)
  const float* fb[2];
#pragma unroll
  for (int jt = 0; jt < 2; ++jt) {
    const int j = min(jbase + 16 * jt + i, m_task - 1);
    const int fsel = J.nseg == 2 ? seg : min(j / J.r, 1);
    const int frow = J.nseg == 2 ? j : j % J.r;
    const float* m = fsel ? J.f[1].m : J.f[0].m;
    fb[jt] = KM ? m + frow : m + (long long)frow * J.f[0].ld;
  }
  const long long fld = J.f[0].ld;
  const int nu = J.K / 32;
  const int u0 = slice * J.kb, u1 = min(u0 + J.kb, nu);
  const int scol = J.koff[seg];
  f32x4 acc[NT][2];
#pragma unroll
  for (int n = 0; n < NT; ++n) acc[n][0] = acc[n][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int unit = u0 + w; unit < u1; unit += 4) {
    Unit<KIND> raw[NT];
    float fv[2][8];
#pragma unroll
    for (int n = 0; n < NT; ++n) raw[n] = unit_load<KIND>(J.src, srow[n], scol + 32 * unit, q);
    factor_unit<KIND, KM>(fb[0], fld, 32 * unit, q, fv[0]);
    if (JT > 1) factor_unit<KIND, KM>(fb[1], fld, 32 * unit, q, fv[1]);
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      float x[8];
      unit_decode<KIND>(raw[n], J.src.act_kind, x);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[n][0] = mfma4(x[e], fv[0][e], acc[n][0]);
      if (JT > 1) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[n][1] = mfma4(x[e], fv[1][e], acc[n][1]);
      }
    }
  }
  // the 4 waves' sums, added in wave order, two tiles at a time
  const int m_out = J.nseg == 2 ? 2 * J.r : J.nfac * J.r;
  const int ocol0 = J.nseg == 2 ? seg * J.r : 0;
  float* P = J.partial + (long long)slice * J.rows * m_out;
  f32x4* R = reinterpret_cast<f32x4*>(red);  // [4 waves][2 tiles][2 j-tiles][64 lanes]
  const int l = threadIdx.x >> 2, v = threadIdx.x & 3;
#pragma unroll
  for (int n0 = 0; n0 < NT; n0 += 2) {
    if (n0 > 0) __syncthreads();
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      R[((w * 2 + n) * 2 + 0) * 64 + lane] = acc[n0 + n][0];
      R[((w * 2 + n) * 2 + 1) * 64 + lane] = acc[n0 + n][1];
    }
    __syncthreads();
#pragma unroll
    for (int n = 0; n < 2; ++n)
      for (int jt = 0; jt < JT; ++jt) {
        float s = red[(((0 * 2 + n) * 2 + jt) * 64 + l) * 4 + v];
        s += red[(((1 * 2 + n) * 2 + jt) * 64 + l) * 4 + v];
        s += red[(((2 * 2 + n) * 2 + jt) * 64 + l) * 4 + v];
        s += red[(((3 * 2 + n) * 2 + jt) * 64 + l) * 4 + v];
        const int orow = r0 + 16 * (n0 + n) + 4 * (l >> 4) + v, j = jbase + 16 * jt + (l & 15);
        if (orow < nrows && j < m_task) P[(long long)orow * m_out + ocol0 + j] = s;
      }
  }
}

template <int KIND>
MX_DEV void outer_task(const PassJob& J, int t, float* red)
{
  constexpr int U = kStepsAhead<KIND>;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, i = lane & 15, q = lane >> 4;
  const int ncb = (J.K + 63) / 64;
  const int cb = t % ncb;
  t /= ncb;
  const int jhalf = t % J.jh;
  t /= J.jh;
  const int seg = t % J.nseg, rs = t / J.nseg;
  const int q0 = rs * J.chunk, q1 = min(q0 + J.chunk, J.rows);  // may be empty: the partial is then 0
  // columns past the end read the segment's first column: only their own (unwritten) sums see them
  const int c = cb * 64 + 4 * i;
  const int scol = J.koff[seg] + (c < J.K ? c : 0);
  const int jbase = 32 * jhalf;
  const int JT = min(2, (J.m - jbase + 15) / 16);
  const float* cbase[2];
#pragma unroll
  for (int jt = 0; jt < 2; ++jt) cbase[jt] = J.coef + J.coff[seg] + min(jbase + 16 * jt + i, J.m - 1);
  f32x4 acc[2][4];
#pragma unroll
  for (int jt = 0; jt < 2; ++jt)
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[jt][u] = f32x4{0.f, 0.f, 0.f, 0.f};
  // wave w takes the 16-row steps w, w + 4, ... of the chunk, U of them per round of loads;
  // within a step, lane (i, q) reads rows 4u + q (u < 4), columns c .. c + 3. Pair sources are
  // walked in (token, slot) order, which does not depend on how the routing filled the buckets.
  for (int sb = q0 + 16 * w; sb < q1; sb += 64 * U) {
    int row[U][4];
    float wq[U][4];
#pragma unroll
    for (int uu = 0; uu < U; ++uu)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int qc = min(sb + 64 * uu + 4 * u + q, q1 - 1);
        row[uu][u] = J.row_of ? J.row_of[qc] : qc;
        wq[uu][u] = J.row_w ? J.row_w[qc] : 1.0f;
      }
    Quad<KIND> x[U][4];
    float cv[U][4][2];
#pragma unroll
    for (int uu = 0; uu < U; ++uu)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int qc = min(sb + 64 * uu + 4 * u + q, q1 - 1);
        const long long crow = J.row_of ? qc / J.k : qc;
        x[uu][u] = quad_load<KIND>(J.src, row[uu][u] >= 0 ? row[uu][u] : 0, scol);
        cv[uu][u][0] = cbase[0][crow * J.ldc];
        cv[uu][u][1] = JT > 1 ? cbase[1][crow * J.ldc] : 0.f;
      }
#pragma unroll
    for (int uu = 0; uu < U; ++uu)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bool ok = (sb + 64 * uu + 4 * u + q < q1) & (row[uu][u] >= 0);
        f32x4 xv = quad_decode<KIND>(x[uu][u], J.src.act_kind);
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[e] = ok ? xv[e] : 0.f;
        const float c0 = ok ? wq[uu][u] * cv[uu][u][0] : 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[0][e] = mfma4(c0, xv[e], acc[0][e]);
        if (JT > 1) {
          const float c1 = ok ? wq[uu][u] * cv[uu][u][1] : 0.f;
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[1][e] = mfma4(c1, xv[e], acc[1][e]);
        }
      }
  }
  // acc[jt][e][v] = G[jbase + 16 jt + 4q + v][c + e]: per v, four consecutive columns. The 4
  // waves' sums are added in LDS in wave order, one j-tile at a time.
  const long long Ctot = (long long)J.nseg * J.K;
  float* P = J.partial + (long long)rs * J.m * Ctot + (long long)seg * J.K;
  f32x4* R = reinterpret_cast<f32x4*>(red);
  const int l = threadIdx.x & 63, vv = threadIdx.x >> 6;
  for (int jt = 0; jt < JT; ++jt) {
#pragma unroll
    for (int v = 0; v < 4; ++v)
      R[(w * 4 + v) * 64 + lane] = f32x4{acc[jt][0][v], acc[jt][1][v], acc[jt][2][v], acc[jt][3][v]};
    __syncthreads();
    f32x4 s = R[(0 * 4 + vv) * 64 + l];
    s += R[(1 * 4 + vv) * 64 + l];
    s += R[(2 * 4 + vv) * 64 + l];
    s += R[(3 * 4 + vv) * 64 + l];
    const int j = jbase + 16 * jt + 4 * (l >> 4) + vv, col = cb * 64 + 4 * (l & 15);
    if (j < J.m && col < J.K) *reinterpret_cast<f32x4*>(P + (long long)j * Ctot + col) = s;
    __syncthreads();
  }
}

// Row dot and outer product fused over one pair source (nseg segments of K columns) walked in
// (token, slot) order, so each element is read once for both: per pair row the dot with the
// segment's factor (out[row, seg*r + j]), per column the outer product with coef (as outer_task).
// A work-group takes a row chunk and 256 columns of one segment; wave w owns 64 of the columns
// and walks every 16-row step of the chunk. For the row dot the wave transposes each step's
// 16 x 64 tile through its own LDS region, so that lane (i, q) supplies A[i][q] = x[row i][4s + q]
// and B[q][i] = f(j = i, column 4s + q) for the 16 column steps s (the factor operands are loaded
// once per task); the 4 waves' dots are added in LDS in wave order every kRoSteps steps and
// written as the partial of the work-group's 256-column block.
constexpr int kRoLd = 64 + 4;  // LDS row stride of a wave's transposed tile: rows start 4 banks apart
constexpr int kRoSteps = 2;    // steps per round of loads and per cross-wave sum

template <int KIND, int JT>  // JT: j-tiles of 16 (1: r <= 16)
MX_DEV void rowouter_task(const PassJob& J, int t, float* lds)
{
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, i = lane & 15, q = lane >> 4;
  const int ncb = (J.K + 255) / 256;
  const int cb = t % ncb;
  t /= ncb;
  const int seg = t % J.nseg, rs = t / J.nseg;
  const int q0 = rs * J.chunk, q1 = min(q0 + J.chunk, J.rows);  // may be empty: the outer partial is then 0
  const int cw = cb * 256 + 64 * w;  // the wave's first column in the segment
  const int c = cw + 4 * i;
  const int scol = J.koff[seg] + (c < J.K ? c : 0);
  const float* cbase[JT];
#pragma unroll
  for (int jt = 0; jt < JT; ++jt) cbase[jt] = J.coef + J.coff[seg] + min(16 * jt + i, J.m - 1);
  // row-dot factor operands fr[jt][s] = f_seg(j = 16 jt + i, column cw + 4 s + q), zero past r or K
  const float* fm = seg ? J.f[1].m : J.f[0].m;
  const long long fsc = J.f[0].kmajor ? J.f[0].ld : 1, fsj = J.f[0].kmajor ? 1 : J.f[0].ld;
  float fr[JT][16];
#pragma unroll
  for (int jt = 0; jt < JT; ++jt)
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int j = 16 * jt + i, col = cw + 4 * s + q;
      const bool ok = (j < J.r) & (col < J.K);
      const float v = fm[(ok ? col : 0) * fsc + (ok ? j : 0) * fsj];
      fr[jt][s] = ok ? v : 0.f;
    }
  f32x4 acc[JT][4];
#pragma unroll
  for (int jt = 0; jt < JT; ++jt)
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[jt][u] = f32x4{0.f, 0.f, 0.f, 0.f};
  float* tile = lds + w * 16 * kRoLd;
  f32x4* red = reinterpret_cast<f32x4*>(lds + 4 * 16 * kRoLd);  // [4 waves][kRoSteps][2][64 lanes]
  const int m_out = J.nseg * J.r;
  float* P2 = J.partial2 + (long long)cb * J.rows * m_out + seg * J.r;
  for (int sb = q0; sb < q1; sb += 16 * kRoSteps) {
    int row[kRoSteps][4];
    float wq[kRoSteps][4];
#pragma unroll
    for (int st = 0; st < kRoSteps; ++st)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int qc = min(sb + 16 * st + 4 * u + q, q1 - 1);
        row[st][u] = J.row_of[qc];
        wq[st][u] = J.row_w ? J.row_w[qc] : 1.0f;
      }
    Quad<KIND> x[kRoSteps][4];
    float cv[kRoSteps][4][JT];
#pragma unroll
    for (int st = 0; st < kRoSteps; ++st)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const long long crow = min(sb + 16 * st + 4 * u + q, q1 - 1) / J.k;
        x[st][u] = quad_load<KIND>(J.src, row[st][u] >= 0 ? row[st][u] : 0, scol);
#pragma unroll
        for (int jt = 0; jt < JT; ++jt) cv[st][u][jt] = cbase[jt][crow * J.ldc];
      }
    f32x4 dr[kRoSteps][JT];
#pragma unroll
    for (int st = 0; st < kRoSteps; ++st) {
      // outer product, and the step's tile into LDS (rows 4u + q, columns 4i .. 4i + 3)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        // the lane's row (q) and its columns (i) are checked apart: the coefficient it supplies
        // belongs to rank i of row q, whatever its own columns are, so only the elements of
        // columns past K are zeroed (they also feed the row dot through the tile)
        const bool row_ok = (sb + 16 * st + 4 * u + q < q1) & (row[st][u] >= 0);
        const bool ok = row_ok & (c < J.K);
        f32x4 xv = quad_decode<KIND>(x[st][u], J.src.act_kind);
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[e] = ok ? xv[e] : 0.f;
#pragma unroll
        for (int jt = 0; jt < JT; ++jt) {
          const float cj = row_ok ? wq[st][u] * cv[st][u][jt] : 0.f;
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[jt][e] = mfma4(cj, xv[e], acc[jt][e]);
        }
        *reinterpret_cast<f32x4*>(&tile[(4 * u + q) * kRoLd + 4 * i]) = xv;
      }
      // row dot of the step's 16 rows over the wave's 64 columns (the wave's own LDS region: its
      // LDS operations complete in order)
      float xr[16];
#pragma unroll
      for (int s = 0; s < 16; ++s) xr[s] = tile[i * kRoLd + 4 * s + q];
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) {
        dr[st][jt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 16; ++s) dr[st][jt] = mfma4(xr[s], fr[jt][s], dr[st][jt]);
      }
    }
    // the 4 waves' dots, added in wave order; lane (i', q') element v is row 4q' + v, j = i'
#pragma unroll
    for (int st = 0; st < kRoSteps; ++st)
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) red[((w * kRoSteps + st) * 2 + jt) * 64 + lane] = dr[st][jt];
    __syncthreads();
    for (int idx = threadIdx.x; idx < kRoSteps * JT * 64 * 4; idx += 256) {
      const int v = idx & 3, l = (idx >> 2) & 63, jt = (idx >> 8) % JT, st = (idx >> 8) / JT;
      const float* rf = reinterpret_cast<const float*>(red);
      float s = rf[(((0 * kRoSteps + st) * 2 + jt) * 64 + l) * 4 + v];
      s += rf[(((1 * kRoSteps + st) * 2 + jt) * 64 + l) * 4 + v];
      s += rf[(((2 * kRoSteps + st) * 2 + jt) * 64 + l) * 4 + v];
      s += rf[(((3 * kRoSteps + st) * 2 + jt) * 64 + l) * 4 + v];
      const int qq = sb + 16 * st + 4 * (l >> 4) + v, j = 16 * jt + (l & 15);
      if ((qq < q1) & (j < J.r)) {
        const int pr = J.row_of[qq];
        if (pr >= 0) P2[(long long)pr * m_out + j] = s;
      }
    }
    __syncthreads();
  }
  // the outer-product partial of the wave's 64 columns: acc[jt][e][v] = G[16 jt + 4q + v][c + e]
  const long long Ctot = (long long)J.nseg * J.K;
  float* P = J.partial + (long long)rs * J.m * Ctot + (long long)seg * J.K;
#pragma unroll
  for (int jt = 0; jt < JT; ++jt) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int j = 16 * jt + 4 * q + v;
      if ((j < J.m) & (c < J.K))
        *reinterpret_cast<f32x4*>(P + (long long)j * Ctot + c) =
            f32x4{acc[jt][0][v], acc[jt][1][v], acc[jt][2][v], acc[jt][3][v]};
    }
  }
}

__global__ __launch_bounds__(256) void lora_pass_kernel(PassArgs a)
{
  // 16 KB for the row-dot and outer reductions; a fused task also keeps its waves' tiles first
  __shared__ __attribute__((aligned(16))) float red[4 * 16 * kRoLd + 4 * kRoSteps * 2 * 64 * 4];
  int n = 0;
  while (n + 1 < a.n && (int)blockIdx.x >= a.j[n + 1].wg0) ++n;
  const PassJob& J = a.j[n];
  const int t = (int)blockIdx.x - J.wg0;
  if (J.type == kLoraRowDot) {
    const bool km = J.f[0].kmajor;
    switch (J.src.kind * 2 + (km ? 1 : 0)) {
      case kLoraF32 * 2: rowdot_task<kLoraF32, false>(J, t, red); break;
      case kLoraF32 * 2 + 1: rowdot_task<kLoraF32, true>(J, t, red); break;
      case kLoraBF16 * 2: rowdot_task<kLoraBF16, false>(J, t, red); break;
      case kLoraBF16 * 2 + 1: rowdot_task<kLoraBF16, true>(J, t, red); break;
      case kLoraGLU * 2: rowdot_task<kLoraGLU, false>(J, t, red); break;
      case kLoraGLU * 2 + 1: rowdot_task<kLoraGLU, true>(J, t, red); break;
      case kLoraHiLo * 2: rowdot_task<kLoraHiLo, false>(J, t, red); break;
      default: rowdot_task<kLoraHiLo, true>(J, t, red); break;
    }
  } else if (J.type == kLoraRowOuter) {
    rowouter_task<kLoraHiLo, 1>(J, t, red);
  } else {
    switch (J.src.kind) {
      case kLoraF32: outer_task<kLoraF32>(J, t, red); break;
      case kLoraBF16: outer_task<kLoraBF16>(J, t, red); break;
      case kLoraGLU: outer_task<kLoraGLU>(J, t, red); break;
      default: outer_task<kLoraHiLo>(J, t, red); break;
    }
  }
}

// ---------------------------------------------------------------- expansions on the matrix cores
// The LoRA term of 16 tokens x 64 columns per wave: D_s[c][t] = sum_{j < r} F_s(c - lo_s, j) *
// coef[t, coff_s + j] for the columns lo_s <= c < hi_s of segment s (0 elsewhere), F_s at
// m_s[(c - lo_s) * sc_s + j * sj_s] (k-major factors: sc = ld, sj = 1; j-major: sc = 1, sj = ld).
// As the MFMA's D[16 x 16] (rows: columns c, cols: tokens), lane (i, q) supplies A[i][q] =
// F(c0 + 16g + i, 4kk + q) and B[q][i] = coef[token i, 4kk + q] and holds the term of token i at
// columns c0 + 16g + 4q .. + 3: the layout of a float4 per lane and 16 tokens x 64 columns per wave.
struct ExpandSpec {
  const float* m[2];
  long long sc[2], sj[2];
  float scale[2];
  int coff[2], lo[2], hi[2];
  int r, nseg;
};

// (Predicates below combine with & rather than &&: short-circuit conditions become branches.)
template <int NSEG, int KK>
MX_DEV void expand_factors(const ExpandSpec& e, int c0, int lane, float fa[NSEG][4][KK])
{
  const int i = lane & 15, q = lane >> 4;
  const int r = e.r;
#pragma unroll
  for (int s = 0; s < NSEG; ++s) {
    const float* m = e.m[s];
    const long long sc = e.sc[s], sj = e.sj[s];
    const int lo = e.lo[s], hi = e.hi[s];
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const int c = c0 + 16 * g + i, j = 4 * kk + q;
        const bool ok = (c >= lo) & (c < hi) & (j < r);
        const float v = m[(ok ? c - lo : 0) * sc + (ok ? j : 0) * sj];
        fa[s][g][kk] = ok ? v : 0.f;
      }
  }
}

// The coefficient operands of token row `crow` (valid) of cf (stride ldc); zero past r or when !ok.
template <int NSEG, int KK>
MX_DEV void expand_coefs(const ExpandSpec& e, const float* cf, long long ldc, long long crow, bool ok, int lane,
                         float cb[NSEG][KK])
{
  const int q = lane >> 4;
  const int r = e.r;
#pragma unroll
  for (int s = 0; s < NSEG; ++s) {
    const float* row = cf + crow * ldc + e.coff[s];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const float v = row[min(4 * kk + q, r - 1)];
      cb[s][kk] = (ok & (4 * kk + q < r)) ? v : 0.f;
    }
  }
}

template <int NSEG, int KK>
MX_DEV void expand_mfma(const float fa[NSEG][4][KK], const float cb[NSEG][KK], f32x4 d[NSEG][4])
{
#pragma unroll
  for (int s = 0; s < NSEG; ++s)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      d[s][g] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) d[s][g] = mfma4(fa[s][g][kk], cb[s][kk], d[s][g]);
    }
}

// ---------------------------------------------------------------- finish kernel
struct FinishJob {
  int type;  // kLoraFinCoef / kLoraFinOuter
  const float* partial;
  int count;  // slices (row dots) or row chunks (outer products)
  // coefficient rows: value (row, j) = scale[j / r] * sum over slices of partial[slice, row, j], rows
  // the pair rows summed over each token's slots (times topk_w when given) if pair_of is given
  int prow, m, r;
  float scale[2];
  const int* pair_of;
  const float* topk_w;
  int k, ntok;
  float* out;  // [ntok, m]
  // outer products: G[j, c] = sum over chunks, written through dst (segments by j or by column)
  int om, Ctot, Kseg;
  LoraOuterDst dst;
  int wg0;
};

constexpr int kMaxFinishJobs = 6;
constexpr int kFinTokens = 8;  // coefficient rows per work-group
struct FinishArgs {
  FinishJob j[kMaxFinishJobs];
  int n;
};

// Coefficient rows of the work-group's tokens into J.out. Each thread takes 4 values at a time and issues all their loads (8 slices, or 8
// slots of a slice) before adding them in slice (slot) order.
MX_DEV void finish_coef(const FinishJob& J, int tb)
{
  const int t0 = tb * kFinTokens;
  const int nt = min(kFinTokens, J.ntok - t0);
  const int nv = kFinTokens * J.m;
  for (int base = 0; base < nv; base += 1024) {
    long long t[4];
    int j[4];
    float scale[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const int idx = min(base + 256 * n + (int)threadIdx.x, nv - 1);
      j[n] = idx % J.m;
      t[n] = t0 + min(idx / J.m, nt - 1);
      scale[n] = J.scale[min(j[n] / J.r, 1)];
    }
    float val[4] = {0.f, 0.f, 0.f, 0.f};
    if (J.pair_of && J.k <= 8) {
#pragma unroll 1
      for (int n = 0; n < 4; ++n) {  // one value at a time, its slots' loads together
        if (base + 256 * n + (int)threadIdx.x >= nv) break;
        int p[8];
        float wv[8], sum[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          p[s] = J.pair_of[t[n] * J.k + min(s, J.k - 1)];
          wv[s] = J.topk_w ? J.topk_w[t[n] * J.k + min(s, J.k - 1)] : 1.0f;
          sum[s] = 0.f;
        }
        for (int sl0 = 0; sl0 < J.count; sl0 += 4) {  // 4 slices of 8 slots per round of loads
          float v[4][8];
#pragma unroll
          for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int s = 0; s < 8; ++s)
              if ((s < J.k) & (sl0 + u < J.count))  // uniform
                v[u][s] = J.partial[((long long)(sl0 + u) * J.prow + max(p[s], 0)) * J.m + j[n]];
#pragma unroll
          for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int s = 0; s < 8; ++s)
              if ((s < J.k) & (sl0 + u < J.count)) sum[s] += v[u][s];
        }
#pragma unroll
        for (int s = 0; s < 8; ++s)  // a skipped slot adds +0, which leaves val (never -0) unchanged
          val[n] += ((s < J.k) & (p[s] >= 0)) ? wv[s] * (scale[n] * sum[s]) : 0.f;
      }
    } else if (J.pair_of) {
#pragma unroll
      for (int n = 0; n < 4; ++n)
        for (int s = 0; s < J.k; ++s) {
          const int p = J.pair_of[t[n] * J.k + s];
          float sum = 0.f;
          for (int sl = 0; sl < J.count; ++sl) sum += J.partial[((long long)sl * J.prow + max(p, 0)) * J.m + j[n]];
          const float wv = J.topk_w ? J.topk_w[t[n] * J.k + s] : 1.0f;
          if (p >= 0) val[n] += wv * (scale[n] * sum);
        }
    } else {
      float sum[4] = {0.f, 0.f, 0.f, 0.f};
      for (int s0 = 0; s0 < J.count; s0 += 8) {
        float v[4][8];
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
          for (int u = 0; u < 8; ++u)
            if (s0 + u < J.count)  // uniform
              v[n][u] = J.partial[((long long)(s0 + u) * J.prow + t[n]) * J.m + j[n]];
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
          for (int u = 0; u < 8; ++u)
            if (s0 + u < J.count) sum[n] += v[n][u];
      }
#pragma unroll
      for (int n = 0; n < 4; ++n) val[n] = scale[n] * sum[n];
    }
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const int idx = base + 256 * n + (int)threadIdx.x;
      if (idx >= nv) continue;
      if (idx / J.m < nt) J.out[t[n] * J.m + j[n]] = val[n];
    }
  }
}

constexpr int kTermLd = 256 + 4;  // LDS row stride of a 256-column term tile (rows start 4 banks apart)

MX_DEV void finish_outer(const FinishJob& J, int b)
{
  const long long idx = (long long)b * 256 + threadIdx.x;
  if (idx >= (long long)J.om * J.Ctot) return;
  const int j = (int)(idx / J.Ctot), c = (int)(idx % J.Ctot);
  // four running sums (chunks 4i + n) keep loads in flight; added in a fixed order
  const float* pp = J.partial + (long long)j * J.Ctot + c;
  const long long step = (long long)J.om * J.Ctot;
  float q0 = 0.f, q1 = 0.f, q2 = 0.f, q3 = 0.f;
  int rs = 0;
  for (; rs + 4 <= J.count; rs += 4) {
    q0 += pp[(rs + 0) * step];
    q1 += pp[(rs + 1) * step];
    q2 += pp[(rs + 2) * step];
    q3 += pp[(rs + 3) * step];
  }
  for (; rs < J.count; ++rs) q0 += pp[rs * step];
  const float s = (q0 + q1) + (q2 + q3);
  int sg = 0, jj = j, cc = c;
  if (J.Kseg > 0) {
    sg = c >= J.Kseg ? 1 : 0;
    cc = c - sg * J.Kseg;
  } else if (J.dst.split_j > 0 && j >= J.dst.split_j) {
    sg = 1;
    jj = j - J.dst.split_j;
  }
  const long long o = J.dst.kmajor[sg] ? (long long)cc * J.dst.ld[sg] + jj : (long long)jj * J.dst.ld[sg] + cc;
  J.dst.p[sg][o] = J.dst.scale[sg] * s;
}

__global__ __launch_bounds__(256) void lora_finish_kernel(FinishArgs a)
{
  int n = 0;
  while (n + 1 < a.n && (int)blockIdx.x >= a.j[n + 1].wg0) ++n;
  const FinishJob& J = a.j[n];
  const int b = (int)blockIdx.x - J.wg0;
  if (J.type == kLoraFinOuter) {
    finish_outer(J, b);
    return;
  }
  finish_coef(J, b);
}

// ---------------------------------------------------------------- expansions on the vector units
// out2[t, c] = scale_s * sum_{j < r} coef[t, coff_s + j] * F_s(c - lo_s, j) for c < Cexp, segment s
// = (c >= lo_1) when there are two. A thread owns 4 consecutive columns (of one segment) and keeps
// their factor values in registers (16-byte loads in either factor layout); a work-group takes
// 1024 columns and up to kExpTokens tokens (ExpandArgs::tpw), whose coefficient rows it stages in
// LDS and reads as broadcasts; each store instruction writes 1 KB of one row. The factor values
// are loaded once per work-group, so launches take as many tokens per work-group as still leave
// kExpMinGroups work-groups.
constexpr int kExpTokens = 16;
constexpr int kExpMinGroups = 512;

struct ExpandArgs {
  float* coef;  // coefficient rows [ntok, m]: read, or (with partial) written by the first column block
  int m, ntok;
  const float* partial;  // non-null: coef = scale[j / r] * sum over count slices of partial[slice, t, j]
  int count;
  float scale[2];
  float* out;
  long long ldo;
  int Cexp;
  int tpw;  // tokens per work-group, at most kExpTokens
  ExpandSpec e;
};

template <int R, bool KM>
__global__ __launch_bounds__(256) void lora_expand_kernel(ExpandArgs a)
{
  __shared__ __attribute__((aligned(16))) float sc[kExpTokens * 2 * kLoraMaxRank];
  const int c = (blockIdx.x * 256 + threadIdx.x) * 4;
  const int t0 = blockIdx.y * a.tpw;
  const int nt = min(a.tpw, a.ntok - t0);
  const ExpandSpec& e = a.e;
  const int sg = ((e.nseg > 1) & (c >= e.lo[1])) ? 1 : 0;
  const bool cok = c < a.Cexp;
  const int cc = cok ? c - e.lo[sg] : 0;
  const float* m = sg ? e.m[1] : e.m[0];
  const long long ld = KM ? (sg ? e.sc[1] : e.sc[0]) : (sg ? e.sj[1] : e.sj[0]);
  // f[u][j] = F(cc + u, j): k-major rows hold r consecutive j, j-major rows 4 consecutive columns
  float f[4][R];
  if (KM && (e.r & 3) == 0) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int j4 = 0; j4 < R / 4; ++j4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(m + (long long)(cc + u) * ld + min(4 * j4, e.r - 4));
#pragma unroll
        for (int t = 0; t < 4; ++t) f[u][4 * j4 + t] = v[t];
      }
  } else if (KM) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int j = 0; j < R; ++j) f[u][j] = m[(long long)(cc + u) * ld + min(j, e.r - 1)];
  } else {
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(m + (long long)min(j, e.r - 1) * ld + cc);
#pragma unroll
      for (int u = 0; u < 4; ++u) f[u][j] = v[u];
    }
  }
  if (!a.partial) {
    for (int i = threadIdx.x; i < nt * a.m; i += 256) sc[i] = a.coef[(long long)t0 * a.m + i];
  } else {
    // the work-group's coefficient rows from the row-dot partials (added in slice order; all of a
    // thread's loads are issued before its adds); the first column block also writes them out
    for (int i0 = 0; i0 < nt * a.m; i0 += 256) {
      const int i = min(i0 + (int)threadIdx.x, nt * a.m - 1);
      const float* pp = a.partial + (long long)t0 * a.m + i;
      const long long step = (long long)a.ntok * a.m;
      float sum = 0.f;
      for (int s0 = 0; s0 < a.count; s0 += 16) {
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u)
          if (s0 + u < a.count) v[u] = pp[(s0 + u) * step];  // uniform
#pragma unroll
        for (int u = 0; u < 16; ++u)
          if (s0 + u < a.count) sum += v[u];
      }
      const float val = a.scale[min((i % a.m) / e.r, 1)] * sum;
      if (i0 + (int)threadIdx.x < nt * a.m) {
        sc[i] = val;
        if (blockIdx.x == 0) a.coef[(long long)t0 * a.m + i] = val;
      }
    }
  }
  __syncthreads();
  const float* cs = sc + (sg ? e.coff[1] : e.coff[0]);
  const float scale = sg ? e.scale[1] : e.scale[0];
  for (int tt = 0; tt < nt; ++tt) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < R; ++j) {
      if (j < e.r) {  // uniform
        const float cj = cs[tt * a.m + j];
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[u] += cj * f[u][j];
      }
    }
    if (cok) *reinterpret_cast<f32x4*>(a.out + (long long)(t0 + tt) * a.ldo + c) = scale * acc;
  }
}

// ---------------------------------------------------------------- combines with the LoRA term
// out[t, c] = sum over the token's slots, in slot order, of rows[pair, c] + sum_s scale_s D_s[c][t]
// (the expansion above, coefficients coef[t, :]). A work-group takes 256 columns and
// kCombineTokens tokens: each wave computes the LoRA term of its 64 columns on the matrix cores
// into LDS, and sums the slot rows of 4 of the tokens over all 256 columns, a 16-byte load per
// lane and slot (1 KB of one row per load instruction); the first two tokens' rows are requested
// before the term is computed.
// Backward (grad_w non-null): also grad_w[t, s] = sum of the pair's dot partials.
constexpr int kCombineTokens = 16;

struct CombineArgs {
  float* out;
  const float* rows;
  long long ldy;
  const int* pair_of;
  int N, k, D;
  const float* coef;
  int m;
  ExpandSpec e;
  float* grad_w;
  const float* gw_part;
  int n_ct;
};

// Slot rows of two tokens at columns cc .. cc + 3 (slots past k are not read).
MX_DEV void combine_rows(const CombineArgs& a, const int p[2][8], int cc, f32x4 v[2][8])
{
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int s = 0; s < 8; ++s)
      if (s < a.k)  // uniform
        v[u][s] = ldnt(reinterpret_cast<const f32x4*>(a.rows + (long long)max(p[u][s], 0) * a.ldy + cc));
}

MX_DEV void combine_store(const CombineArgs& a, const int p[2][8], const f32x4 v[2][8], const float* term, int tb,
                          int nt, int tt0, int c, int cc)
{
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int tt = tt0 + 4 * u;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 8; ++s)
      if (s < a.k && p[u][s] >= 0) acc += v[u][s];  // slots in order; a skipped slot adds nothing
    for (int s = 8; s < a.k; ++s) {                 // more than 8 slots
      const int pp = a.pair_of[(long long)(tb + min(tt, nt - 1)) * a.k + s];
      if (pp >= 0) acc += *reinterpret_cast<const f32x4*>(a.rows + (long long)pp * a.ldy + cc);
    }
    acc += *reinterpret_cast<const f32x4*>(&term[min(tt, nt - 1) * kTermLd + 4 * lane]);
    if (tt < nt && c < a.D) *reinterpret_cast<f32x4*>(a.out + (long long)(tb + tt) * a.D + c) = acc;
  }
}

template <int NSEG, int KK>
__global__ __launch_bounds__(256) void lora_combine_kernel(CombineArgs a)
{
  __shared__ __attribute__((aligned(16))) float term[kCombineTokens * kTermLd];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, i = lane & 15, q = lane >> 4;
  const int cb = blockIdx.x * 256;
  const int tb = blockIdx.y * kCombineTokens;
  const int nt = min(kCombineTokens, a.N - tb);
  // wave w sums tokens w, w + 4 (round 0) and w + 8, w + 12 (round 1); lane owns columns c .. c + 3
  const int c = cb + 4 * lane;
  const int cc = c < a.D ? c : 0;
  int p[2][2][8];
#pragma unroll
  for (int rd = 0; rd < 2; ++rd)
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int s = 0; s < 8; ++s)
        p[rd][u][s] = a.pair_of[(long long)(tb + min(w + 8 * rd + 4 * u, nt - 1)) * a.k + min(s, a.k - 1)];
  f32x4 v[2][8];
  combine_rows(a, p[0], cc, v);
  // the LoRA term of the work-group's tokens at the wave's 64 columns
  {
    const int c0 = cb + 64 * w;
    float fa[NSEG][4][KK];
    expand_factors<NSEG, KK>(a.e, c0, lane, fa);
    const int t = tb + i;
    float cbv[NSEG][KK];
    expand_coefs<NSEG, KK>(a.e, a.coef, a.m, t < a.N ? t : a.N - 1, t < a.N, lane, cbv);
    f32x4 d[NSEG][4];
    expand_mfma<NSEG, KK>(fa, cbv, d);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      f32x4 o = a.e.scale[0] * d[0][g];
      if (NSEG > 1) o += a.e.scale[1] * d[NSEG - 1][g];
      *reinterpret_cast<f32x4*>(&term[i * kTermLd + 64 * w + 16 * g + 4 * q]) = o;
    }
  }
  __syncthreads();
  combine_store(a, p[0], v, term, tb, nt, w, c, cc);
  if (w + 8 < nt) {  // uniform
    combine_rows(a, p[1], cc, v);
    combine_store(a, p[1], v, term, tb, nt, w + 8, c, cc);
  }
  if (a.grad_w && blockIdx.x == 0) {
    for (int idx = threadIdx.x; idx < nt * a.k; idx += 256) {
      const long long ts = (long long)tb * a.k + idx;
      const int pp = a.pair_of[ts];
      float gsum = 0.f;
      if (pp >= 0)
        for (int ct = 0; ct < a.n_ct; ++ct) gsum += a.gw_part[(long long)pp * a.n_ct + ct];
      a.grad_w[ts] = gsum;
    }
  }
}

// ---------------------------------------------------------------- planning
constexpr int kPassTargetGroups = 768;

int src_bytes(int kind) { return kind == kLoraGLU ? 8 : (kind == kLoraBF16 ? 2 : 4); }

// Fills the job's work split and returns its work-group count; partial floats in *floats.
int plan_job(const LoraPassJob& d, PassJob& J, size_t floats[2])
{
  J = {};
  floats[0] = floats[1] = 0;
  J.type = d.type; J.src = d.src; J.rows = d.rows; J.rows_dev = d.rows_dev;
  J.nseg = d.nseg; J.K = d.K; J.koff[0] = d.koff[0]; J.koff[1] = d.koff[1]; J.r = d.r;
  if (d.type == kLoraRowDot) {
    const int quads = (d.rows + 16 * kRowTiles - 1) / (16 * kRowTiles);
    J.nfac = d.nfac; J.f[0] = d.f[0]; J.f[1] = d.nseg == 2 || d.nfac == 2 ? d.f[1] : d.f[0];
    const int m_task = d.nseg == 2 ? d.r : d.nfac * d.r;
    J.jh = (m_task + 31) / 32;
    const int nu = std::max(1, d.K / 32);
    const long long tasks = (long long)quads * d.nseg * J.jh;
    int S = (int)std::max(1LL, kPassTargetGroups / std::max(1LL, tasks));
    S = std::max(1, std::min(S, nu / 8));
    J.kb = (nu + S - 1) / S;
    J.S = std::max(1, (nu + J.kb - 1) / J.kb);
    const int m_out = d.nseg == 2 ? 2 * d.r : d.nfac * d.r;
    floats[0] = (size_t)J.S * (size_t)d.rows * (size_t)m_out;
    return (int)(tasks * J.S);
  }
  J.coef = d.coef; J.ldc = d.ldc; J.coff[0] = d.coff[0]; J.coff[1] = d.coff[1];
  J.row_of = d.row_of; J.k = std::max(1, d.k); J.row_w = d.row_w; J.m = d.m;
  J.jh = (d.m + 31) / 32;
  if (d.type == kLoraRowOuter) {
    J.f[0] = d.f[0]; J.f[1] = d.nseg == 2 ? d.f[1] : d.f[0];
    const int ncb = (d.K + 255) / 256;
    const long long coltasks = (long long)d.nseg * ncb;
    long long RS = std::max(1LL, kPassTargetGroups / std::max(1LL, coltasks));
    RS = std::min(RS, std::max(1LL, (long long)d.rows * src_bytes(d.src.kind) / (40LL * d.m)));
    RS = std::max(1LL, std::min(RS, (long long)(d.rows + 31) / 32));
    J.chunk = std::max(32, (int)(((d.rows + RS - 1) / RS + 31) / 32 * 32));
    J.RS = std::max(1, (d.rows + J.chunk - 1) / J.chunk);
    J.S = ncb;  // row-dot slices: one per 256-column block
    floats[0] = (size_t)J.RS * (size_t)d.m * (size_t)d.nseg * (size_t)d.K;
    floats[1] = (size_t)ncb * (size_t)d.rows * (size_t)(d.nseg * d.r);
    return (int)(coltasks * J.RS);
  }
  const int ncb = (d.K + 63) / 64;
  const long long coltasks = (long long)d.nseg * ncb * J.jh;
  // chunks: enough work-groups, partials at most about a tenth of the source's bytes
  long long RS = std::max(1LL, kPassTargetGroups / std::max(1LL, coltasks));
  RS = std::min(RS, std::max(1LL, (long long)d.rows * src_bytes(d.src.kind) / (40LL * d.m)));
  RS = std::max(1LL, std::min(RS, (long long)(d.rows + 63) / 64));
  J.chunk = std::max(64, (int)(((d.rows + RS - 1) / RS + 63) / 64 * 64));
  J.RS = std::max(1, (d.rows + J.chunk - 1) / J.chunk);  // at least one chunk: an empty one writes zeros
  floats[0] = (size_t)J.RS * (size_t)d.m * (size_t)d.nseg * (size_t)d.K;
  return (int)(coltasks * J.RS);
}

}  // namespace

size_t lora_pass_partial_floats(const LoraPassJob* jobs, int n)
{
  size_t total = 0;
  for (int i = 0; i < n; ++i) {
    PassJob J;
    size_t f[2];
    plan_job(jobs[i], J, f);
    total += (f[0] + 63) / 64 * 64 + (f[1] + 63) / 64 * 64;
  }
  return total;
}

hipError_t launch_lora_pass(const LoraPassJob* jobs, int n, float* partial, LoraPartial* parts, hipStream_t s)
{
  if (n < 1 || n > kMaxPassJobs) return hipErrorInvalidValue;
  PassArgs a = {};
  a.n = n;
  int wg = 0;
  size_t off = 0;
  for (int i = 0; i < n; ++i) {
    const LoraPassJob& d = jobs[i];
    if (d.r < 1 || d.r > kLoraMaxRank || d.nseg < 1 || d.nseg > 2 || d.K <= 0 || d.K % 32) return hipErrorInvalidValue;
    if (d.type == kLoraRowDot && (d.nfac < 1 || d.nfac > 2 || (d.nseg == 2 && d.nfac != 1))) return hipErrorInvalidValue;
    if (d.type != kLoraRowDot && (d.m < 1 || d.m > 2 * kLoraMaxRank)) return hipErrorInvalidValue;
    if (d.type == kLoraRowOuter && (d.src.kind != kLoraHiLo || !d.row_of || d.m > 16 || d.r > 16))
      return hipErrorInvalidValue;
    size_t f[2];
    const int groups = plan_job(d, a.j[i], f);
    a.j[i].partial = partial + off;
    a.j[i].wg0 = wg;
    parts[i].p = partial + off;
    parts[i].count = d.type == kLoraRowDot ? a.j[i].S : a.j[i].RS;
    off += (f[0] + 63) / 64 * 64;
    parts[i].p2 = nullptr;
    parts[i].count2 = 0;
    if (d.type == kLoraRowOuter) {
      a.j[i].partial2 = partial + off;
      parts[i].p2 = partial + off;
      parts[i].count2 = a.j[i].S;
      off += (f[1] + 63) / 64 * 64;
    }
    wg += groups;
  }
  if (wg == 0) return hipSuccess;
  hipLaunchKernelGGL(lora_pass_kernel, dim3((unsigned)wg), dim3(256), 0, s, a);
  return hipGetLastError();
}

namespace {

ExpandSpec expand_spec(int nseg, const LoraFactor* f, const int* coff, const int* lo, const int* hi, int r)
{
  ExpandSpec e = {};
  e.nseg = nseg;
  e.r = r;
  for (int s = 0; s < 2; ++s) {
    const int u = std::min(s, nseg - 1);
    e.m[s] = f[u].m;
    e.sc[s] = f[u].kmajor ? f[u].ld : 1;
    e.sj[s] = f[u].kmajor ? 1 : f[u].ld;
    e.scale[s] = f[u].scale;
    e.coff[s] = coff[u];
    e.lo[s] = lo[u];
    e.hi[s] = hi[u];
  }
  return e;
}

}  // namespace

hipError_t launch_lora_finish(const LoraFinishJob* jobs, int n, hipStream_t s)
{
  if (n < 1 || n > kMaxFinishJobs) return hipErrorInvalidValue;
  FinishArgs a = {};
  a.n = n;
  int wg = 0;
  for (int i = 0; i < n; ++i) {
    const LoraFinishJob& d = jobs[i];
    FinishJob& J = a.j[i];
    J.type = d.type; J.partial = d.part.p; J.count = d.part.count;
    J.wg0 = wg;
    if (d.type == kLoraFinCoef) {
      if (d.m > 2 * kLoraMaxRank || d.r < 1 || d.r > kLoraMaxRank) return hipErrorInvalidValue;
      J.prow = d.prow; J.m = d.m; J.r = d.r; J.scale[0] = d.scale[0]; J.scale[1] = d.scale[1];
      J.pair_of = d.pair_of; J.topk_w = d.topk_w; J.k = std::max(1, d.k); J.ntok = d.ntok; J.out = d.out;
      wg += (d.ntok + kFinTokens - 1) / kFinTokens;
    } else {
      J.om = d.om; J.Ctot = d.Ctot; J.Kseg = d.Kseg; J.dst = d.dst;
      wg += (int)(((long long)d.om * d.Ctot + 255) / 256);
    }
  }
  if (wg == 0) return hipSuccess;
  hipLaunchKernelGGL(lora_finish_kernel, dim3((unsigned)wg), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_lora_expand(float* coef, int m, int ntok, int r, float* out, long long ldo, int Cexp,
                              int Cseg, const LoraFactor* ef, const int* ecoff, hipStream_t s,
                              const LoraPartial* part, const float* part_scale)
{
  if (ntok <= 0 || Cexp <= 0) return hipSuccess;
  if (r < 1 || r > kLoraMaxRank || m > 2 * kLoraMaxRank || Cexp % 4 || ldo % 4) return hipErrorInvalidValue;
  if (Cseg <= 0) Cseg = Cexp;
  if (Cseg % 4) return hipErrorInvalidValue;
  const int nseg = Cseg < Cexp ? 2 : 1;
  if (nseg > 1 && ef[0].kmajor != ef[1].kmajor) return hipErrorInvalidValue;
  const bool km = ef[0].kmajor;
  for (int i = 0; i < nseg; ++i)  // 16-byte factor loads
    if (((uintptr_t)ef[i].m & 15) || (km ? (r % 4 == 0 && ef[i].ld % 4) : ef[i].ld % 4)) return hipErrorInvalidValue;
  ExpandArgs a = {};
  a.coef = coef; a.m = m; a.ntok = ntok; a.out = out; a.ldo = ldo; a.Cexp = Cexp;
  if (part) {
    a.partial = part->p; a.count = part->count;
    a.scale[0] = part_scale[0]; a.scale[1] = part_scale[1];
  }
  const int lo[2] = {0, Cseg}, hi[2] = {Cseg, Cexp};
  a.e = expand_spec(nseg, ef, ecoff, lo, hi, r);
  const int ncb = (Cexp / 4 + 255) / 256;
  a.tpw = kExpTokens;
  while (a.tpw > 4 && (long long)ncb * ((ntok + a.tpw - 1) / a.tpw) < kExpMinGroups) a.tpw /= 2;
  dim3 grid((unsigned)ncb, (unsigned)((ntok + a.tpw - 1) / a.tpw)), block(256);
  if (r > 16) {
    if (km) hipLaunchKernelGGL((lora_expand_kernel<32, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((lora_expand_kernel<32, false>), grid, block, 0, s, a);
  } else {
    if (km) hipLaunchKernelGGL((lora_expand_kernel<16, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((lora_expand_kernel<16, false>), grid, block, 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_lora_combine(float* out, const float* rows, long long ldy, const int* pair_of, int N, int k, int D,
                               const float* coef, int r, int nseg, const LoraFactor* f, float* grad_w,
                               const float* gw_part, int n_ct, hipStream_t s)
{
  if (N == 0 || D == 0) return hipSuccess;
  if (r < 1 || r > kLoraMaxRank || nseg < 1 || nseg > 2 || D % 4 || ldy % 4 || k < 1) return hipErrorInvalidValue;
  CombineArgs a = {};
  a.out = out; a.rows = rows; a.ldy = ldy; a.pair_of = pair_of; a.N = N; a.k = k; a.D = D;
  a.coef = coef; a.m = nseg * r;
  const int coff[2] = {0, r}, lo[2] = {0, 0}, hi[2] = {D, D};
  a.e = expand_spec(nseg, f, coff, lo, hi, r);
  a.grad_w = grad_w; a.gw_part = gw_part; a.n_ct = n_ct;
  dim3 grid((unsigned)((D + 255) / 256), (unsigned)((N + kCombineTokens - 1) / kCombineTokens)), block(256);
  if (nseg == 1) {
    if (r > 16) hipLaunchKernelGGL((lora_combine_kernel<1, 8>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((lora_combine_kernel<1, 4>), grid, block, 0, s, a);
  } else {
    if (r > 16) hipLaunchKernelGGL((lora_combine_kernel<2, 8>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((lora_combine_kernel<2, 4>), grid, block, 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace mx
