// Forward MXFP4 products on the fp4-native scaled MFMA (gfx950).
//
// One work-group computes a 16-row x 64-column output tile (kFwdGateUp: 16 rows x 32 gate
// features + the same 32 up features). Its four waves split the K dimension in super-chunks
// of 512 elements and reduce through LDS at the end, so every weight byte is read once per
// row tile and no wave waits on another inside the main loop.
//
// Per super-chunk c and lane (j = lane % 16, g = lane / 16), for each of the 4 column groups:
//   B: 64 contiguous bytes of weight row n = 4 MX blocks 16c+4g+q (q = 0..3), one dword of
//      scales. MFMA q consumes block 16c+4g+q from lane group g, so op_sel q picks its scale.
//   A: 128 contiguous bytes of the two-term activation row (hi, and again lo), arranged by
//      the AQ layout so that bytes [32q, 32q+32) are exactly MFMA q's A operand.
// Weights are consumed as stored: the MFMA applies the E8M0 scales and the e2m1 codes itself.
// A scale byte >= 253 zeroes its block (lazy_lora/native/mxfp4_gemm.c:16-18) before it can
// reach the MFMA, where 255 would be NaN and 253/254 would overflow.
#include "mx_device.h"
#include "mx_kernels.h"

namespace mx {

namespace {

struct WorkItem {
  int expert, row0, nrows, ct;
};

// Work-groups are issued round-robin over the 8 XCDs (blockIdx % 8). Give each XCD one
// contiguous run of work items so the tiles of one expert share that XCD's L2.
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

template <int Q>
__device__ __forceinline__ void mfma_step(f32x4 (&acc)[4], const i32x8& ah, const i32x8& al,
                                          const i32x4 (&b)[4][4], const uint32_t (&sb)[4], int sah,
                                          int sal)
{
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    acc[grp] = mfma_f8f4<Q, Q>(ah, b[grp][Q], acc[grp], sah, (int)sb[grp]);
    acc[grp] = mfma_f8f4<Q, Q>(al, b[grp][Q], acc[grp], sal, (int)sb[grp]);
  }
}

template <int MODE, bool ALIGNED>
__global__ __launch_bounds__(256, 2) void fwd_kernel(FwdArgs a)
{
  __shared__ float red[4][16][68];

  WorkItem w;
  if (!decode_work(a.tiles, a.n_tiles, a.M, a.n_ct, w)) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int nb = a.K / kGroup;

  // A row held by this lane (rows past the tile end repeat the last row; never stored)
  const int ri = w.row0 + min(j, w.nrows - 1);
  const int arow = a.a_row_map ? a.a_row_map[ri] : ri;
  const long long kp = aq_kpad(a.K);
  const uint8_t* ahi = a.a_hi + (long long)arow * kp + g * 128;
  const uint8_t* alo = a.a_lo + (long long)arow * kp + g * 128;
  const uint8_t* asc = a.a_sc + (long long)arow * aq_scale_row_bytes(a.K) + g * 8;

  const uint8_t* bp[4];
  const uint8_t* bs[4];
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    const uint8_t* P = a.wp0;
    const uint8_t* S = a.ws0;
    int n;
    if (MODE == kFwdGateUp) {
      if (grp >= 2) {
        P = a.wp1;
        S = a.ws1;
      }
      n = w.ct * 32 + (grp & 1) * 16 + j;
    } else {
      n = w.ct * kFwdColsPerTile + grp * 16 + j;
    }
    n = min(n, a.R - 1);
    bp[grp] = P + (long long)w.expert * a.wp_estride + (long long)n * (a.K / 2) + g * 64;
    bs[grp] = S + (long long)w.expert * a.ws_estride + (long long)n * nb + g * 4;
  }

  const int nsc = (nb + kChunkBlocks - 1) / kChunkBlocks;
  const int c_begin = wave * nsc / 4, c_end = (wave + 1) * nsc / 4;

  f32x4 acc[4];
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) acc[grp] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int c = c_begin; c < c_end; ++c) {
    i32x4 b[4][4];
    uint32_t sb[4];
    const bool full = ALIGNED && (c * kChunkBlocks + kChunkBlocks <= nb);
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      if (full) {
        const uint8_t* p = bp[grp] + c * 256;
#pragma unroll
        for (int q = 0; q < 4; ++q) b[grp][q] = ldg16(p + 16 * q);
        sb[grp] = *reinterpret_cast<const uint32_t*>(bs[grp] + c * 16);
      } else {
        sb[grp] = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int blk = c * kChunkBlocks + g * 4 + q;
          if (blk < nb) {
            b[grp][q] = ldg16(bp[grp] + c * 256 + 16 * q);
            sb[grp] |= (uint32_t)bs[grp][c * 16 + q] << (8 * q);
          } else {
            b[grp][q] = i32x4{0, 0, 0, 0};
            sb[grp] |= 127u << (8 * q);
          }
        }
      }
      if (any_damaged_scale(sb[grp])) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (((sb[grp] >> (8 * q)) & 0xFFu) >= 253u) {
            b[grp][q] = i32x4{0, 0, 0, 0};
            sb[grp] = (sb[grp] & ~(0xFFu << (8 * q))) | (127u << (8 * q));
          }
        }
      }
    }
    const uint8_t* ph = ahi + (long long)c * kChunk;
    const uint8_t* pl = alo + (long long)c * kChunk;
    const i32x8 ah0 = ldg32(ph), ah1 = ldg32(ph + 32), ah2 = ldg32(ph + 64), ah3 = ldg32(ph + 96);
    const i32x8 al0 = ldg32(pl), al1 = ldg32(pl + 32), al2 = ldg32(pl + 64), al3 = ldg32(pl + 96);
    const uint2 s2 = *reinterpret_cast<const uint2*>(asc + (long long)c * 32);
    mfma_step<0>(acc, ah0, al0, b, sb, (int)s2.x, (int)s2.y);
    mfma_step<1>(acc, ah1, al1, b, sb, (int)s2.x, (int)s2.y);
    mfma_step<2>(acc, ah2, al2, b, sb, (int)s2.x, (int)s2.y);
    mfma_step<3>(acc, ah3, al3, b, sb, (int)s2.x, (int)s2.y);
  }

  // split-K reduction: lane (j, g) holds rows 4g..4g+3 of column grp*16 + j
#pragma unroll
  for (int grp = 0; grp < 4; ++grp)
#pragma unroll
    for (int v = 0; v < 4; ++v) red[wave][4 * g + v][grp * 16 + j] = acc[grp][v];
  __syncthreads();

  const int i = tid >> 4;  // tile row handled in the epilogue
  const bool row_ok = i < w.nrows;
  const int row = w.row0 + (row_ok ? i : 0);

  if (MODE == kFwdGateUp) {
    const int fj = (tid & 15) * 2;
    const float g0 = red[0][i][fj] + red[1][i][fj] + red[2][i][fj] + red[3][i][fj];
    const float g1 = red[0][i][fj + 1] + red[1][i][fj + 1] + red[2][i][fj + 1] + red[3][i][fj + 1];
    const float u0 = red[0][i][32 + fj] + red[1][i][32 + fj] + red[2][i][32 + fj] + red[3][i][32 + fj];
    const float u1 = red[0][i][33 + fj] + red[1][i][33 + fj] + red[2][i][33 + fj] + red[3][i][33 + fj];
    const float a0 = glu_fwd(g0, u0, a.act_kind), a1 = glu_fwd(g1, u1, a.act_kind);
    const int F = a.R;
    const int f = w.ct * 32 + fj;
    if (a.save && row_ok) {
      float* sv = a.save + (long long)row * 2 * F;
      *reinterpret_cast<float2*>(sv + f) = make_float2(g0, g1);
      *reinterpret_cast<float2*>(sv + F + f) = make_float2(u0, u1);
    }
    const Quant2 qv = quant2_block16(a0, a1);  // all 16 lanes of the row take part
    if (row_ok) {
      const long long fp = aq_kpad(F);
      const long long off = (long long)row * fp + (f >> 9) * kChunk + aq_pos(f & 511);
      *reinterpret_cast<uint16_t*>(a.q_hi + off) = (uint16_t)qv.hi;
      *reinterpret_cast<uint16_t*>(a.q_lo + off) = (uint16_t)qv.lo;
      if ((tid & 15) == 0) {
        a.q_sc[aq_scale_off(row, F, w.ct, 0)] = (uint8_t)qv.s_hi;
        a.q_sc[aq_scale_off(row, F, w.ct, 1)] = (uint8_t)qv.s_lo;
      }
    }
    return;
  }

  const int cq = (tid & 15) * 4;
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = red[0][i][cq + e] + red[1][i][cq + e] + red[2][i][cq + e] + red[3][i][cq + e];
  if (!row_ok) return;
  if (MODE == kFwdDown) {
    const float tw = a.row_w[row];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] *= tw;
  }
  const int col = w.ct * kFwdColsPerTile + cq;
  float* yr = a.y + (long long)row * a.ldy;
  if (col + 3 < a.R && ((a.ldy & 3) == 0)) {
    *reinterpret_cast<float4*>(yr + col) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (col + e < a.R) yr[col + e] = v[e];
  }
}

}  // namespace

hipError_t launch_fwd(const FwdArgs& a, int mode, int max_tiles, hipStream_t s)
{
  const long long total = (long long)max_tiles * a.n_ct;
  if (total <= 0) return hipSuccess;
  const long long blocks = (total + 7) / 8 * 8;
  const bool aligned = (a.K % 128) == 0;
  dim3 grid((unsigned)blocks), block(256);
#define MX_LAUNCH(M, AL) hipLaunchKernelGGL((fwd_kernel<M, AL>), grid, block, 0, s, a)
  if (mode == kFwdPlain) {
    if (aligned) MX_LAUNCH(kFwdPlain, true); else MX_LAUNCH(kFwdPlain, false);
  } else if (mode == kFwdGateUp) {
    if (aligned) MX_LAUNCH(kFwdGateUp, true); else MX_LAUNCH(kFwdGateUp, false);
  } else {
    if (aligned) MX_LAUNCH(kFwdDown, true); else MX_LAUNCH(kFwdDown, false);
  }
#undef MX_LAUNCH
  return hipGetLastError();
}

}  // namespace mx
