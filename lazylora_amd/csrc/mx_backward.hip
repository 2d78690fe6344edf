// Transposed MXFP4 products y[m, c] = sum_r A[m, r] W[r, c] (gfx950).
//
// The contraction runs over W's rows, the strided direction of the packed layout, and the
// E8M0 scales group W along its columns, so the scaled MFMA cannot consume W directly here.
// Each step a work-group (256 threads) cooperatively loads a 32-row x 256-column slab of W
// (every thread one 16-byte MX block = 32 columns of one row), decodes it with
// v_cvt_scalef32_pk_bf16_fp4 (bit-exact: e2m1 * 2^(s-127) is exact in bf16), and writes it
// row-major into LDS. Each wave then owns 64 output columns and pulls its B operands with
// ds_read_b64_tr_b16, which hands lane i of a 16-lane group column i of four consecutive
// rows. A (activation gradients) is split into bf16 hi + lo terms, so the products carry
// ~16 significant bits of the activation against the exact weights. The slab in LDS is
// double-buffered: one barrier per step.
//
// The whole contraction range (nseg * R rows) stays in one work-group, so every output
// element has exactly one writer and the sum order is fixed: results are deterministic.
#include "mx_device.h"
#include "mx_kernels.h"

namespace mx {

namespace {

constexpr int kSlabRows = 32;
constexpr int kSlabPitch = kBwdColsPerTile + 16;  // bf16 elements per LDS row (+32 B: spreads banks)

typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

struct WorkItem {
  int expert, row0, nrows, ct;
};

__device__ __forceinline__ bool decode_work(const int4* tiles, const int* n_tiles, int M, int n_ct,
                                            WorkItem& w)
{
  const int ntiles = tiles ? *n_tiles : (M + kFwdRowsPerTile - 1) / kFwdRowsPerTile;
  const int total = ntiles * n_ct;
  const int per_xcd = (total + 7) >> 3;
  const int slot = (int)(blockIdx.x >> 3);
  const int item = (int)(blockIdx.x & 7) * per_xcd + slot;
  if (slot >= per_xcd || item >= total) return false;
  const int t = item / n_ct;
  w.ct = item - t * n_ct;
  if (tiles) {
    const int4 tt = tiles[t];
    w.expert = tt.x;
    w.row0 = tt.y;
    w.nrows = tt.z;
  } else {
    w.expert = 0;
    w.row0 = t * kFwdRowsPerTile;
    w.nrows = min(kFwdRowsPerTile, M - w.row0);
  }
  return true;
}

// 16 fp4 bytes (32 codes of one row) -> 32 bf16 in 16 dwords, scale byte s applied exactly.
__device__ __forceinline__ void decode_block_bf16(const i32x4& raw, uint32_t s, uint32_t (&out)[16])
{
  const bool dead = s >= 253u;
  const float scale = bits_f((dead ? 127u : s) << 23);
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint32_t word = dead ? 0u : (uint32_t)raw[d];
    out[4 * d + 0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 0));
    out[4 * d + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 1));
    out[4 * d + 2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 2));
    out[4 * d + 3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 3));
  }
}

template <int MODE>
__global__ __launch_bounds__(256, 2) void bwd_kernel(BwdArgs a)
{
  __shared__ __attribute__((aligned(16))) uint16_t slab[2][kSlabRows][kSlabPitch];
  __shared__ float dotred[4][16];

  WorkItem w;
  if (!decode_work(a.tiles, a.n_tiles, a.M, a.n_ct, w)) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, g = lane >> 4;
  const int c0 = w.ct * kBwdColsPerTile;
  const int rtot = a.nseg * a.R;
  const int nsteps = (rtot + kSlabRows - 1) / kSlabRows;

  // loader role: one 16-byte MX block per thread per step
  const int lr = tid >> 3;         // slab row
  const int lc = tid & 7;          // 32-column block inside the tile
  const int lcol = c0 + lc * 32;
  const bool lcol_ok = lcol < a.C;
  const int cbs = a.C / kGroup;    // scale bytes per W row
  const long long wpitch = a.C / 2;

  auto load_raw = [&](int step, i32x4& raw, uint32_t& sc) {
    const int r = step * kSlabRows + lr;
    raw = i32x4{0, 0, 0, 0};
    sc = 127u;
    if (lcol_ok && r < rtot) {
      const int seg = r >= a.R ? 1 : 0;
      const int rr = r - seg * a.R;
      const uint8_t* P = seg ? a.wp1 : a.wp0;
      const uint8_t* S = seg ? a.ws1 : a.ws0;
      raw = ldg16(P + (long long)w.expert * a.wp_estride + (long long)rr * wpitch + lcol / 2);
      sc = S[(long long)w.expert * a.ws_estride + (long long)rr * cbs + lcol / kGroup];
    }
  };

  // A operand rows (rows past the tile end repeat the last row; never stored)
  const int ri = w.row0 + min(li, w.nrows - 1);
  const int arow = a.a_row_map ? a.a_row_map[ri] : ri;
  const uint16_t* pah = a.a_hi + (long long)arow * a.lda + 8 * g;
  const uint16_t* pal = a.a_lo + (long long)arow * a.lda + 8 * g;

  f32x4 acc[4];
#pragma unroll
  for (int cg = 0; cg < 4; ++cg) acc[cg] = f32x4{0.f, 0.f, 0.f, 0.f};

  i32x4 raw;
  uint32_t sc;
  load_raw(0, raw, sc);
  for (int s = 0; s < nsteps; ++s) {
    const int buf = s & 1;
    {
      uint32_t dec[16];
      decode_block_bf16(raw, sc, dec);
      uint32_t* dst = reinterpret_cast<uint32_t*>(&slab[buf][lr][lc * 32]);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<i32x4*>(dst + 4 * q) =
            i32x4{(int)dec[4 * q], (int)dec[4 * q + 1], (int)dec[4 * q + 2], (int)dec[4 * q + 3]};
    }
    __syncthreads();
    if (s + 1 < nsteps) load_raw(s + 1, raw, sc);

    const i32x4 ahv = ldg16(pah + s * kSlabRows);
    const i32x4 alv = ldg16(pal + s * kSlabRows);
    const bf16x8 ah = __builtin_bit_cast(bf16x8, ahv);
    const bf16x8 al = __builtin_bit_cast(bf16x8, alv);
#pragma unroll
    for (int cg = 0; cg < 4; ++cg) {
      const int col = wave * 64 + cg * 16 + 4 * (li & 3);
      const i16x4 t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_i16x4*)(&slab[buf][8 * g + (li >> 2)][col]));
      const i16x4 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_i16x4*)(&slab[buf][8 * g + 4 + (li >> 2)][col]));
      const short __attribute__((ext_vector_type(8))) bs = {t0[0], t0[1], t0[2], t0[3], t1[0], t1[1], t1[2], t1[3]};
      const bf16x8 b = __builtin_bit_cast(bf16x8, bs);
      acc[cg] = mfma_bf16(ah, b, acc[cg]);
      acc[cg] = mfma_bf16(al, b, acc[cg]);
    }
  }

  // epilogue: lane (li, g) holds rows 4g..4g+3 of column c0 + wave*64 + cg*16 + li
  if (MODE == kBwdDownT) {
    const int F = a.C;
    float dots[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int i = 4 * g + v;
      const bool row_ok = i < w.nrows;
      const int p = w.row0 + (row_ok ? i : 0);
      const float tw = a.row_w[p];
      const float* sv = a.saved + (long long)p * 2 * F;
#pragma unroll
      for (int cg = 0; cg < 4; ++cg) {
        const int f = c0 + wave * 64 + cg * 16 + li;
        if (f < F) {
          const float h = acc[cg][v];
          const float gt = sv[f], up = sv[F + f];
          dots[v] += glu_fwd(gt, up, a.act_kind) * h;
          float dg, du;
          glu_bwd(tw * h, gt, up, a.act_kind, dg, du);
          if (row_ok) {
            const long long o = (long long)p * 2 * F + f;
            const __bf16 dgh = (__bf16)dg, duh = (__bf16)du;
            a.d_hi[o] = __builtin_bit_cast(uint16_t, dgh);
            a.d_lo[o] = __builtin_bit_cast(uint16_t, (__bf16)(dg - (float)dgh));
            a.d_hi[o + F] = __builtin_bit_cast(uint16_t, duh);
            a.d_lo[o + F] = __builtin_bit_cast(uint16_t, (__bf16)(du - (float)duh));
          }
        }
      }
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float d = group16_sum(dots[v]);
      if (li == 0) dotred[wave][4 * g + v] = d;
    }
    __syncthreads();
    if (tid < 16 && tid < w.nrows) {
      const float d = dotred[0][tid] + dotred[1][tid] + dotred[2][tid] + dotred[3][tid];
      a.gw_part[(long long)(w.row0 + tid) * a.n_ct + w.ct] = d;
    }
    return;
  }

#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int i = 4 * g + v;
    if (i >= w.nrows) continue;
    float* yr = a.y + (long long)(w.row0 + i) * a.ldy;
#pragma unroll
    for (int cg = 0; cg < 4; ++cg) {
      const int col = c0 + wave * 64 + cg * 16 + li;
      if (col < a.C) {
        if (a.accumulate) yr[col] += acc[cg][v];
        else yr[col] = acc[cg][v];
      }
    }
  }
}

}  // namespace

hipError_t launch_bwd(const BwdArgs& a, int mode, int max_tiles, hipStream_t s)
{
  const long long total = (long long)max_tiles * a.n_ct;
  if (total <= 0) return hipSuccess;
  const long long blocks = (total + 7) / 8 * 8;
  dim3 grid((unsigned)blocks), block(256);
  if (mode == kBwdPlain) hipLaunchKernelGGL(bwd_kernel<kBwdPlain>, grid, block, 0, s, a);
  else if (mode == kBwdDownT) hipLaunchKernelGGL(bwd_kernel<kBwdDownT>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(bwd_kernel<kBwdGateUpT>, grid, block, 0, s, a);
  return hipGetLastError();
}

}  // namespace mx
