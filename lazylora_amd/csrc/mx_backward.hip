// Transposed MXFP4 products y[m, c] = sum_r A[m, r] W[r, c] (gfx950), decoded in registers.
//
// The contraction runs over W's rows, the strided direction of the packed layout, and the
// E8M0 scales group W along its columns, so the scaled MFMA cannot consume W directly here:
// each bf16 MFMA (v_mfma_f32_16x16x32_bf16) lane needs 8 consecutive rows of ONE column. A
// wave owns a 256-column stripe over all rows and builds those operands in registers, with no
// LDS round trip:
//
//  * lane (n = l % 16, g = l / 16) loads, every 32-row step, 8 bytes of each of rows 8g..8g+7:
//    columns 16n..16n+15 of the stripe (half an MX block), plus the 8 rows' scale bytes. The 16
//    lanes of a row group read 128 contiguous bytes of a row;
//  * byte p of a row holds columns 2p and 2p+1; v_cvt_scalef32_pk_bf16_fp4 turns it into those
//    two bf16 values, exactly (e2m1 * 2^(s-127) is exact in bf16), and v_perm_b32 gathers the
//    8 rows' column-2p halves into one B operand and their column-2p+1 halves into another;
//  * so MFMA t (t = 0..15) of a step computes output columns {16n + t : n = 0..15} of the
//    stripe, and a lane's accumulators end up holding 16 CONTIGUOUS columns (4 rows each), which
//    the epilogue writes as whole 64-byte runs.
// A (activation gradients) is split into bf16 hi + lo terms, so the products carry ~16
// significant bits of the activation against the exact weights; fp32 accumulation.
//
// Per 4 KiB of weights a wave spends 64 decodes + 64 permutes (VALU) and 32 MFMAs. The four
// waves of a work-group take four neighbouring stripes of one row tile and share its A operands:
// the work-group copies them into LDS (global_load_lds, 16 steps at a time, double-buffered),
// so A costs one read per 1024 columns instead of one per 256, and one barrier per 16 steps.
// Large buckets (experts with many 16-row tiles) take items of T row tiles, which reuse every
// decoded operand for all T tiles.
//
// The whole contraction range (nseg * R rows) stays in one wave, so every output element has
// exactly one writer and the sum order is fixed: results are deterministic.
#include "mx_device.h"
#include "mx_kernels.h"

#include <algorithm>
#include <type_traits>

namespace mx {

namespace {

constexpr int kStepRows = 32;
typedef const __attribute__((address_space(4))) int* cint_ptr;

constexpr int kWaves = 4;  // waves (stripes) per work-group
// One-tile items of eight stripes (eight waves, one work-group per CU): the tile's A operands are
// copied once for 2048 columns instead of once per 1024. Used for the W2 transposed product from
// the backward layout (C a multiple of 8 stripes) when the launch has at least kWideMinItems such
// items; fewer would leave CUs idle that four-stripe items (two work-groups per CU) keep busy.
constexpr int kWideWaves = 8;
constexpr int kWideMinItems = 512;

// One work item: the NW stripes from NW * ct4 on of up to T row tiles of one expert (T = 1: a
// small-bucket tile; T > 1: part of a large-bucket group, whose tiles share every decoded
// operand).
template <int T>
struct WorkItem {
  int expert, ct4, ntl;
  int row0[T], nrows[T];
};

// The one-tile work list: the small-bucket tiles (with no large-bucket groups, every tile in
// order), read through the constant address space.
__device__ __forceinline__ bool use_small_list(const BwdArgs& a)
{
  return a.small_tiles && *(cint_ptr)a.n_groups > 0;
}
__device__ __forceinline__ int one_tile_count(const BwdArgs& a)
{
  return use_small_list(a) ? *(cint_ptr)a.n_small
                           : a.tiles ? *(cint_ptr)a.n_tiles : (a.M + kFwdRowsPerTile - 1) / kFwdRowsPerTile;
}

// Work item `it` of this work-group among items of NW stripes (items are dealt round-robin over
// the XCDs, blockIdx % 8, each XCD taking one contiguous run, in strides of the grid, so the stripe
// blocks of one tile, which read the same A rows, run on one XCD). Returns 0 when there is none
// left, 1 for an item.
template <int T, int NW>
__device__ __forceinline__ int decode_work(const BwdArgs& a, int it, WorkItem<T>& w)
{
  static_assert(T == 1, "large buckets take bwd_group_kernel");
  const bool use_small = use_small_list(a);
  const int count = one_tile_count(a);
  const int n_ct4 = (a.n_ct + NW - 1) / NW;
  const int total = count * n_ct4;
  const int per_xcd = (total + 7) >> 3;
  const int slot = (int)(blockIdx.x >> 3) + it * (int)(gridDim.x >> 3);
  const int item = (int)(blockIdx.x & 7) * per_xcd + slot;
  if (slot >= per_xcd || item >= total) return 0;
  const int i = item / n_ct4;
  w.ct4 = item - i * n_ct4;
  const int t0 = use_small ? ((cint_ptr)a.small_tiles)[i] : i;
  w.ntl = 1;
#pragma unroll
  for (int tt = 0; tt < T; ++tt) {
    const int t = t0 + (tt < w.ntl ? tt : 0);
    if (a.tiles) {
      const cint_ptr tl = (cint_ptr)(a.tiles + t);
      w.expert = tl[0];
      w.row0[tt] = tl[1];
      w.nrows[tt] = tl[2];
    } else {
      w.expert = 0;
      w.row0[tt] = t * kFwdRowsPerTile;
      w.nrows[tt] = min(kFwdRowsPerTile, a.M - w.row0[tt]);
    }
  }
  return 1;
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 8 bytes, streaming (non-temporal): weight bytes are read exactly once per wave, and the 16
// lanes of a row group consume whole 128-byte lines
MX_DEV u32x2 buf8B_nt(rsrc_t r, uint32_t off)
{
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 2));
}

// One step's weights for one lane: 8 rows x 8 bytes, and the 8 rows' scale bytes.
struct StepRaw {
  u32x2 w[8];
  uint32_t s[8];
};

// B operands of MFMAs 2P and 2P+1 from byte P of the lane's 8 rows
template <int P>
MX_DEV void decode_pair(const StepRaw& r, const float (&sf)[8], bf16x8& b0, bf16x8& b1)
{
  uint32_t d[8];
#pragma unroll
  for (int q = 0; q < 8; ++q)
    d[q] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(r.w[q][P >> 2], sf[q], P & 3));
  // d[q] = (column 2p | column 2p+1 << 16) of row q; B wants rows (2m, 2m+1) of one column
  uint32_t e[4], o[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    e[m] = __builtin_amdgcn_perm(d[2 * m + 1], d[2 * m], 0x05040100u);
    o[m] = __builtin_amdgcn_perm(d[2 * m + 1], d[2 * m], 0x07060302u);
  }
  b0 = __builtin_bit_cast(bf16x8, i32x4{(int)e[0], (int)e[1], (int)e[2], (int)e[3]});
  b1 = __builtin_bit_cast(bf16x8, i32x4{(int)o[0], (int)o[1], (int)o[2], (int)o[3]});
}

// Ring depth (steps of weights in flight per wave, each 4 KiB per wave) and A chunk (steps whose
// A operands one LDS buffer holds: kChunk x T tiles x 2 terms x 1 KiB). T > 1 items do T times
// the matrix work per step, so a shorter ring hides the loads. kChunk is a multiple of kRing.
#ifndef MX_BWD_RING
#define MX_BWD_RING 4
#endif
template <int T>
struct Cfg {
  static constexpr int kRing = MX_BWD_RING;
  static constexpr int kChunk = 16 / T;
  static constexpr int kChunkBytes = kChunk * T * 2 * 1024;
};

// BL: the weights come from the backward layout (launch_backward_layout): each 32-row step of
// a stripe is 4 KiB of codes read by four 16-byte loads per lane (each instruction 1 KiB
// contiguous) and 256 B of scales read by one 8-byte load per lane, instead of eight 8-byte
// loads from eight rows and eight scale-byte loads.
template <int MODE, int T, bool BL, int NW>
__device__ __forceinline__ void bwd_item(const BwdArgs& a, const WorkItem<T>& w, uint8_t* abuf)
{
  constexpr int kRing = Cfg<T>::kRing;
  constexpr int kChunk = Cfg<T>::kChunk;
  constexpr int kChunkBytes = Cfg<T>::kChunkBytes;
  static_assert(kChunk % kRing == 0, "a ring pass never straddles an A chunk");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int ct = w.ct4 * NW + wave;  // this wave's stripe
  const bool stripe_ok = ct < a.n_ct;    // uniform: stripes past C only help with the A copies
  const int c0 = ct * kBwdColsPerTile;
  const int rtot = a.nseg * a.R;
  const int nsteps = (rtot + kStepRows - 1) / kStepRows;
  // whole A chunks; padding steps read past the matrix (zeros)
  const int nsteps_pad = (nsteps + kChunk - 1) / kChunk * kChunk;

  const uint32_t cbs = a.C / kGroup;  // scale bytes per W row
  const uint32_t wpitch = a.C / 2;
  // this lane's 16 columns; a stripe may end past C (small C): such lanes read column 0's
  // bytes, finite weights whose products are never stored
  const int col = c0 + 16 * n;
  const int col_c = col < a.C ? col : 0;
  // Weights and scales are read through buffer resources, one per step, based at the step's
  // first row of its segment (scalar arithmetic only), so each lane's offsets stay fixed for the
  // whole item: rows at or past the segment's end (the tail of a row count that is not a
  // multiple of kStepRows, and the padding steps) fall outside the resource and read as zero
  // weights. Segments hold a multiple of kStepRows rows whenever there are two, so a step never
  // straddles them. A stripe past C gets empty resources: zeros, no memory traffic.
  const uint8_t* const wbase0 = a.wp0 + (long long)w.expert * a.wp_estride;
  const uint8_t* const sbase0 = a.ws0 + (long long)w.expert * a.ws_estride;
  const uint8_t* const wbase1 = a.nseg > 1 ? a.wp1 + (long long)w.expert * a.wp_estride : wbase0;
  const uint8_t* const sbase1 = a.nseg > 1 ? a.ws1 + (long long)w.expert * a.ws_estride : sbase0;
  uint32_t offw[8], offs[8];  // row 8g + q of a step, this lane's columns
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    offw[q] = (uint32_t)(8 * g + q) * wpitch + (uint32_t)col_c / 2;
    offs[q] = (uint32_t)(8 * g + q) * cbs + (uint32_t)col_c / kGroup;
  }

  // Backward layout: one buffer resource per segment over the expert's copy (empty for a
  // stripe past C); the step's block is (step of the segment, stripe), codes first, then the
  // scales after every block's codes. Steps past the segment's end (padding) read an empty
  // resource: zero weights.
  const int bl_nstr = a.C / kBwdColsPerTile;
  const uint32_t bl_codes = (uint32_t)(a.R / kStepRows) * (uint32_t)bl_nstr * 4096u;
  const uint32_t bl_size = stripe_ok ? bl_codes + bl_codes / 16 : 0u;
  const uint8_t* const bl0 = BL ? a.bl0 + (long long)w.expert * a.bl_estride : nullptr;
  const uint8_t* const bl1 = BL && a.nseg > 1 ? a.bl1 + (long long)w.expert * a.bl_estride : bl0;

  auto load_step = [&](int step, StepRaw& r) {
    const int row0 = step * kStepRows;
    const bool seg = a.nseg > 1 && row0 >= a.R;  // uniform
    const int rr = seg ? row0 - a.R : row0;
    if constexpr (BL) {
      const rsrc_t B = make_rsrc(seg ? bl1 : bl0, rr < a.R ? bl_size : 0u);
      const uint32_t blk = (uint32_t)(rr / kStepRows) * (uint32_t)bl_nstr + (uint32_t)ct;
#pragma unroll
      for (int u = 0; u < 4; ++u) {  // rows 8g + 2u and 8g + 2u + 1, 8 bytes each
        const i32x4 v = buf16_nt(B, (uint32_t)lane * 16u + (uint32_t)u * 1024u, blk * 4096u);
        r.w[2 * u] = u32x2{(uint32_t)v[0], (uint32_t)v[1]};
        r.w[2 * u + 1] = u32x2{(uint32_t)v[2], (uint32_t)v[3]};
      }
      const u32x2 sv = buf8B_nt(B, bl_codes + blk * 256u + (uint32_t)(lane >> 1) * 8u);
#pragma unroll
      for (int q = 0; q < 8; ++q) r.s[q] = (sv[q >> 2] >> (8 * (q & 3))) & 0xffu;
    } else {
      const int rows_left = stripe_ok ? max(a.R - rr, 0) : 0;
      const rsrc_t W = make_rsrc((seg ? wbase1 : wbase0) + (long long)rr * wpitch, (uint32_t)rows_left * wpitch);
      const rsrc_t S = make_rsrc((seg ? sbase1 : sbase0) + (long long)rr * cbs, (uint32_t)rows_left * cbs);
#pragma unroll
      for (int q = 0; q < 8; ++q) r.w[q] = buf8B_nt(W, offw[q]);
#pragma unroll
      for (int q = 0; q < 8; ++q) r.s[q] = buf8(S, offs[q]);
    }
  };
  constexpr int kStepLoads = BL ? 5 : 16;  // load instructions per step and lane

  // A operands: MFMA lane (i = n, g) takes elements 8g..8g+7 of the step's 32 contraction
  // indices of row i of each tile, hi and lo terms (16 bytes each). The work-group copies them
  // into abuf chunk by chunk: unit u = (step in chunk, tile, term) is 1 KiB, lane l's operand at
  // 16 l, exactly as a ds_read_b128 of the MFMA lanes wants it; wave w copies units w, w + 4, ...
  // Rows past a tile's end repeat its last row (never stored). Padding steps meet zero weights,
  // so their A (the last real step's, copied again) adds zero.
  const uint16_t* pa[T][2];
#pragma unroll
  for (int tt = 0; tt < T; ++tt) {
    const int ri = w.row0[tt] + min(n, w.nrows[tt] - 1);
    const long long arow = a.a_row_map ? a.a_row_map[ri] : ri;
    pa[tt][0] = a.a_hi + arow * a.lda + 8 * g;
    pa[tt][1] = a.a_lo + arow * a.lda + 8 * g;
  }
  // The copies are issued from inline assembly (the compiler does not see them, so it does not
  // drain every load in flight at each barrier); each chunk is waited for explicitly.
  auto copy_chunk = [&](int chunk) {
    uint8_t* dst = abuf + (chunk & 1) * kChunkBytes;
    static_assert(kChunk * T * 2 % NW == 0, "the A units split evenly over the waves");
#pragma unroll
    for (int k = 0; k < kChunk * T * 2 / NW; ++k) {
      const int u = k * NW + wave;
      const int si = u / (2 * T), tt = (u >> 1) % T, term = u & 1;
      const int so = min(chunk * kChunk + si, nsteps - 1) * kStepRows;
      // select tile tt's pointer without indexing (keeps pa in registers)
      const uint16_t* src = pa[0][0];
#pragma unroll
      for (int t2 = 0; t2 < T; ++t2)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          if (tt == t2 && term == h) src = pa[t2][h];
      dma16_async(src + so, dst + u * 1024);
    }
  };

  f32x4 acc[T][16];
#pragma unroll
  for (int tt = 0; tt < T; ++tt)
#pragma unroll
    for (int t = 0; t < 16; ++t) acc[tt][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  StepRaw ring[kRing];
  // issue order is pinned (the first A chunk, then the ring slot by slot) so that each step
  // waits for its own loads alone, whether it is entered from here or from the loop's back edge
  copy_chunk(0);
#pragma unroll
  for (int p = 0; p < kRing; ++p) {
    __builtin_amdgcn_sched_barrier(0);
    load_step(p, ring[p]);
  }
  __builtin_amdgcn_sched_barrier(0);

  for (int s0 = 0; s0 < nsteps_pad; s0 += kRing) {
    if (s0 % kChunk == 0) {  // uniform
      // chunk c = s0 / kChunk was copied before the weights of steps s0 .. s0 + kRing - 1 were
      // requested: with only those outstanding, this wave's part has landed; the barrier waits
      // for the other waves' parts, and every wave has finished reading the buffer that chunk
      // c + 1 now overwrites (it held chunk c - 1)
      wait_vm<(kRing * kStepLoads < 63 ? kRing * kStepLoads : 63)>();  // (the counter holds at most 63)
      __syncthreads();
      const int c = s0 / kChunk;
      if ((c + 1) * kChunk < nsteps_pad) copy_chunk(c + 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    const uint8_t* ab = abuf + ((s0 / kChunk) & 1) * kChunkBytes + lane * 16;
#pragma unroll
    for (int p = 0; p < kRing; ++p) {
      const int s = s0 + p;
      const int si = s % kChunk;
      StepRaw& r = ring[p];
      // this step's A operands from the chunk in LDS
      i32x4 ah[T], al[T];
#pragma unroll
      for (int tt = 0; tt < T; ++tt) {
        ah[tt] = *reinterpret_cast<const i32x4*>(ab + ((si * T + tt) * 2) * 1024);
        al[tt] = *reinterpret_cast<const i32x4*>(ab + ((si * T + tt) * 2 + 1) * 1024);
      }
      // scales of this step's rows as E8M0 operands of the conversion; a scale byte >= 253
      // makes its row contribute zero
      float sf[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const bool dead = r.s[q] >= 253u;
        r.w[q] = dead ? u32x2{0u, 0u} : r.w[q];
        sf[q] = bits_f((dead ? 127u : r.s[q]) << 23);
      }

      // two byte positions (four MFMA column sets) at a time: the hi terms of the four, then
      // their lo terms, so consecutive MFMAs never share an accumulator
      auto bytes = [&](auto p2c) {
        constexpr int p2 = decltype(p2c)::value;
        bf16x8 b[4];
        decode_pair<p2>(r, sf, b[0], b[1]);
        decode_pair<p2 + 1>(r, sf, b[2], b[3]);
#pragma unroll
        for (int tt = 0; tt < T; ++tt)
          if (tt < w.ntl)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              acc[tt][2 * p2 + j] = mfma_bf16(__builtin_bit_cast(bf16x8, ah[tt]), b[j], acc[tt][2 * p2 + j]);
#pragma unroll
        for (int tt = 0; tt < T; ++tt)
          if (tt < w.ntl)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              acc[tt][2 * p2 + j] = mfma_bf16(__builtin_bit_cast(bf16x8, al[tt]), b[j], acc[tt][2 * p2 + j]);
      };
      bytes(std::integral_constant<int, 0>{});
      bytes(std::integral_constant<int, 2>{});
      bytes(std::integral_constant<int, 4>{});
      bytes(std::integral_constant<int, 6>{});
      __builtin_amdgcn_sched_barrier(0);
      load_step(s + kRing, ring[p]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // epilogue, tile by tile: lane (n, g) holds rows 4g..4g+3 of columns col .. col + 15 (the
  // tile index is a compile-time constant in each call, so acc is only ever indexed statically
  // and stays in registers)
  const bool col_ok = stripe_ok && col < a.C;  // C is a multiple of 32: all 16 columns or none
  auto epilogue = [&](auto ttc) {
    constexpr int tt = decltype(ttc)::value;
    const bool live = tt < w.ntl;  // uniform
    const int row0 = w.row0[tt], nrows = live ? w.nrows[tt] : 0;
    if (MODE == kBwdDownT) {
      const int F = a.C;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = 4 * g + v;
        const bool row_ok = i < nrows;
        const int p = row0 + (row_ok ? i : 0);
        float dot = 0.f;
        if (col_ok) {
          const float tw = a.row_w[p];
          const float* sv = a.saved + (long long)p * 2 * F + col;
          // LoRA: the down adapter's A_d^T q of the row's token joins g . W2
          const float* rq = a.lora_rq ? a.lora_rq + (long long)a.a_row_map[p] * F + col : nullptr;
          uint32_t dh[8], dl[8], uh[8], ul[8];
#pragma unroll
          for (int c4 = 0; c4 < 4; ++c4) {
            const f32x4 gt4 = *reinterpret_cast<const f32x4*>(sv + 4 * c4);
            const f32x4 up4 = *reinterpret_cast<const f32x4*>(sv + F + 4 * c4);
            f32x4 rq4 = f32x4{0.f, 0.f, 0.f, 0.f};
            if (rq) rq4 = *reinterpret_cast<const f32x4*>(rq + 4 * c4);
            float dg[4], du[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float h = acc[tt][4 * c4 + e][v] + rq4[e];
              dot += glu_fwd(gt4[e], up4[e], a.act_kind) * h;
              glu_bwd(tw * h, gt4[e], up4[e], a.act_kind, dg[e], du[e]);
            }
#pragma unroll
            for (int e = 0; e < 4; e += 2) {
              const uint32_t gh = pack_bf16(dg[e], dg[e + 1]);
              const uint32_t hh = pack_bf16(du[e], du[e + 1]);
              dh[2 * c4 + e / 2] = gh;
              dl[2 * c4 + e / 2] = pack_bf16(dg[e] - bf16_lo(gh), dg[e + 1] - bf16_hi(gh));
              uh[2 * c4 + e / 2] = hh;
              ul[2 * c4 + e / 2] = pack_bf16(du[e] - bf16_lo(hh), du[e + 1] - bf16_hi(hh));
            }
          }
          if (row_ok) {
            const long long o = (long long)p * 2 * F + col;
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
              const int b = 4 * h2;
              // non-temporal: measured faster than write-back stores for these rows
              auto st = [&](const uint32_t* v, uint16_t* dst) {
                __builtin_nontemporal_store(i32x4{(int)v[b], (int)v[b + 1], (int)v[b + 2], (int)v[b + 3]},
                                            reinterpret_cast<i32x4*>(dst));
              };
              st(dh, a.d_hi + o + 8 * h2);
              st(dl, a.d_lo + o + 8 * h2);
              st(uh, a.d_hi + o + F + 8 * h2);
              st(ul, a.d_lo + o + F + 8 * h2);
            }
          }
        }
        // this stripe's part of grad_w = <act, h> for the row: the 16 lanes of the row group
        const float d = group16_sum(dot);
        if (n == 0 && row_ok && stripe_ok) a.gw_part[(long long)(row0 + i) * a.n_ct + ct] = d;
      }
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = 4 * g + v;
        if (i < nrows && col_ok) {
          float* yr = a.y + (long long)(row0 + i) * a.ldy + col;
#pragma unroll
          for (int c4 = 0; c4 < 4; ++c4) {
            f32x4 o = f32x4{acc[tt][4 * c4][v], acc[tt][4 * c4 + 1][v], acc[tt][4 * c4 + 2][v], acc[tt][4 * c4 + 3][v]};
            if (a.accumulate) o += *reinterpret_cast<const f32x4*>(yr + 4 * c4);
            *reinterpret_cast<f32x4*>(yr + 4 * c4) = o;
          }
        }
      }
    }
  };
  static_for<T>(epilogue);
}

// One work-group of kWaves waves per item (one row tile x kWaves stripes); the grid covers
// every item. With `wide` the launch has an eight-stripe companion (bwd_wide_kernel) and each
// kernel runs only when its item count suits it: this one when there are fewer than
// kWideMinItems eight-stripe items. BL: the weights come from the backward layout.
template <int MODE, bool BL>
__global__ __launch_bounds__(64 * kWaves, 2) void bwd_kernel(BwdArgs a, int wide)
{
  __shared__ __attribute__((aligned(16))) uint8_t abuf[2 * Cfg<1>::kChunkBytes];
  if (wide && one_tile_count(a) * ((a.n_ct + kWideWaves - 1) / kWideWaves) >= kWideMinItems) return;
  WorkItem<1> w;
  if (decode_work<1, kWaves>(a, 0, w) == 1) bwd_item<MODE, 1, BL, kWaves>(a, w, abuf);
}

// The same items with eight stripes (one work-group per CU; the grid covers every item); it runs
// only when there are at least kWideMinItems of them (else bwd_kernel takes the launch's items).
template <int MODE, bool BL>
__global__ __launch_bounds__(64 * kWideWaves, 1) void bwd_wide_kernel(BwdArgs a)
{
  __shared__ __attribute__((aligned(16))) uint8_t abuf[2 * Cfg<1>::kChunkBytes];
  if (one_tile_count(a) * ((a.n_ct + kWideWaves - 1) / kWideWaves) < kWideMinItems) return;
  WorkItem<1> w;
  if (decode_work<1, kWideWaves>(a, 0, w) == 1) bwd_item<MODE, 1, BL, kWideWaves>(a, w, abuf);
}

// ---------------------------------------------------------------- large buckets
// An expert with many rows would stream (and decode) its weights once per row tile. Its tiles
// come in groups of up to kGroupTiles (4) consecutive tiles; a work item is GT of them (a part of
// a group when GT is smaller) x a block of 4 GS columns: every wave decodes a GS-column stripe of
// each 32-row step once and applies it to all GT row tiles, and the item's A operands (GT tiles x
// hi/lo, 2 GT KiB per step) come through LDS for the four waves. Each weight byte is read once per 16 GT rows
// instead of once per 16, and each A fragment read from LDS feeds GS / 16 MFMAs.
//
// Lane (n, g) of a wave holds columns (GS / 16) n .. + GS / 16 - 1 of its stripe, whose weights
// are GS / 32 bytes of each of its 8 rows: with GS = 128 the lane's own dword, with GS = 64 half
// of the dword its lane pair shares. Byte p gives MFMAs 2p and 2p + 1. Scales come as the dword
// holding the lane's scale byte, so the kernel requires C % 128 == 0 (whole dwords of scales per
// row); launch_bwd sends other shapes through the one-tile kernel.
#ifndef MX_BWD_GT
#define MX_BWD_GT 4
#endif
#ifndef MX_BWD_GS
#define MX_BWD_GS 128
#endif
#ifndef MX_BWD_GRING
#define MX_BWD_GRING 2
#endif
#ifndef MX_BWD_GPER_CU
#define MX_BWD_GPER_CU 2
#endif
constexpr int kGT = MX_BWD_GT;                // row tiles per item
constexpr int kGS = MX_BWD_GS;                // columns per wave
constexpr int kGParts = kGroupTiles / kGT;    // items per group and column block
constexpr int kGCols = kWaves * kGS;          // columns per item
constexpr int kGRing = MX_BWD_GRING;          // steps of weights in flight per wave
constexpr int kGChunk = MX_BWD_GRING;         // steps per LDS A chunk (a multiple of kGRing)
constexpr int kGUnit = 1024;                  // one tile x one term x one step of A
constexpr int kGChunkBytes = kGChunk * kGT * 2 * kGUnit;
constexpr int kGBytes = kGS / 32;             // weight bytes per row and lane
static_assert(kGCols % kBwdColsPerTile == 0, "an item covers whole 256-column grad_w partials");

struct GStep {
  uint32_t w[8];  // the dword of each row holding this lane's weight bytes
  uint32_t s[8];  // the dword of each row holding this lane's scale byte
};
// The same step from the backward layout: the four 16-byte pieces of the lane pair's stripe
// columns (rows 8g + 2u and 8g + 2u + 1, the lane's dword at 4 (n % 2) of each 8-byte half) and
// the 8 scale bytes of rows 8g .. 8g + 7. The lane's dwords are picked where they are used, so
// the loads stay in flight until then.
struct GStepBL {
  i32x4 c[4];
  u32x2 s;
};

template <int P>
MX_DEV void gdecode_pair(const uint32_t (&wl)[8], const float (&sf)[8], bf16x8& b0, bf16x8& b1)
{
  uint32_t d[8];
#pragma unroll
  for (int q = 0; q < 8; ++q)
    d[q] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wl[q], sf[q], P));
  uint32_t e[4], o[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    e[m] = __builtin_amdgcn_perm(d[2 * m + 1], d[2 * m], 0x05040100u);
    o[m] = __builtin_amdgcn_perm(d[2 * m + 1], d[2 * m], 0x07060302u);
  }
  b0 = __builtin_bit_cast(bf16x8, i32x4{(int)e[0], (int)e[1], (int)e[2], (int)e[3]});
  b1 = __builtin_bit_cast(bf16x8, i32x4{(int)o[0], (int)o[1], (int)o[2], (int)o[3]});
}

// BL: the weights come from the backward layout (see bwd_item): a wave's 128 columns are half
// of a 256-column block, whose four 16-byte loads per lane give each lane pair its 8 rows x 8
// bytes (each lane keeps its 4), and one 8-byte load the rows' scale bytes: 5 loads per step
// instead of 16.
template <int MODE, bool BL>
__device__ __forceinline__ void bwd_group_item(const BwdArgs& a, int expert, int t0, int ntl, int cb, uint8_t* abuf,
                                               float* red)
{
  constexpr int T = kGT;
  constexpr int NC = kGS / 16;  // MFMA column sets = columns per lane
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int c0w = cb * kGCols + wave * kGS;  // this wave's first column
  const bool stripe_ok = c0w < a.C;          // uniform
  const int col = c0w + NC * n;
  const int rtot = a.nseg * a.R;
  const int nsteps = (rtot + kStepRows - 1) / kStepRows;
  const int nsteps_pad = (nsteps + kGChunk - 1) / kGChunk * kGChunk;
  const uint32_t cbs = a.C / kGroup, wpitch = a.C / 2;

  int row0[T], nrows[T];
#pragma unroll
  for (int tt = 0; tt < T; ++tt) {
    const cint_ptr tl = (cint_ptr)(a.tiles + t0 + (tt < ntl ? tt : 0));
    row0[tt] = tl[1];
    nrows[tt] = tt < ntl ? tl[2] : 0;
  }

  const uint8_t* const wbase0 = a.wp0 + (long long)expert * a.wp_estride;
  const uint8_t* const sbase0 = a.ws0 + (long long)expert * a.ws_estride;
  const uint8_t* const wbase1 = a.nseg > 1 ? a.wp1 + (long long)expert * a.wp_estride : wbase0;
  const uint8_t* const sbase1 = a.nseg > 1 ? a.ws1 + (long long)expert * a.ws_estride : sbase0;
  const int colc = stripe_ok ? col : 0;
  // the lane's bytes sit at byte (colc / 2) % 4 of their dword (checkpoint layout; the backward
  // layout's dwords are the lane's own)
  const uint32_t wsh = BL ? 0u : 8u * (((uint32_t)colc / 2) & 3u);
  const uint32_t ssh = BL ? 0u : 8u * (((uint32_t)colc / kGroup) & 3u);
  uint32_t offw[8], offs[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    offw[q] = ((uint32_t)(8 * g + q) * wpitch + (uint32_t)colc / 2) & ~3u;
    offs[q] = ((uint32_t)(8 * g + q) * cbs + (uint32_t)colc / kGroup) & ~3u;
  }
  // backward layout: block (step, 256-column stripe c0w / 256), this wave's half of it; the
  // lane pair's piece and scale entry (see launch_backward_layout)
  const int bl_nstr = a.C / kBwdColsPerTile;
  const uint32_t bl_codes = (uint32_t)(a.R / kStepRows) * (uint32_t)bl_nstr * 4096u;
  const uint32_t bl_size = stripe_ok ? bl_codes + bl_codes / 16 : 0u;
  const uint8_t* const bl0 = BL ? a.bl0 + (long long)expert * a.bl_estride : nullptr;
  const uint8_t* const bl1 = BL && a.nseg > 1 ? a.bl1 + (long long)expert * a.bl_estride : bl0;
  const int half = (c0w / 128) & 1;
  const uint32_t bl_lane = (uint32_t)(16 * g + 8 * half + (n >> 1)) * 16u;
  const uint32_t bl_slane = (uint32_t)(8 * g + 4 * half + (n >> 2)) * 8u;
  const bool odd = (n & 1) != 0;
  using Step = std::conditional_t<BL, GStepBL, GStep>;
  auto load_step = [&](int step, Step& r) {
    const int rs = step * kStepRows;
    const bool seg = a.nseg > 1 && rs >= a.R;  // uniform
    const int rr = seg ? rs - a.R : rs;
    if constexpr (BL) {
      const rsrc_t B = make_rsrc(seg ? bl1 : bl0, rr < a.R ? bl_size : 0u);
      const uint32_t blk = (uint32_t)(rr / kStepRows) * (uint32_t)bl_nstr + (uint32_t)(c0w / kBwdColsPerTile);
#pragma unroll
      for (int u = 0; u < 4; ++u) r.c[u] = buf16_nt(B, bl_lane, blk * 4096u + (uint32_t)u * 1024u);
      r.s = buf8B_nt(B, bl_codes + blk * 256u + bl_slane);
    } else {
      const int rows_left = stripe_ok ? max(a.R - rr, 0) : 0;
      const rsrc_t W = make_rsrc((seg ? wbase1 : wbase0) + (long long)rr * wpitch, (uint32_t)rows_left * wpitch);
      const rsrc_t S = make_rsrc((seg ? sbase1 : sbase0) + (long long)rr * cbs, (uint32_t)rows_left * cbs);
#pragma unroll
      for (int q = 0; q < 8; ++q)
        r.w[q] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(W, (int)offw[q], 0, 2);
#pragma unroll
      for (int q = 0; q < 8; ++q) r.s[q] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(S, (int)offs[q], 0, 0);
    }
  };

  // A chunk copies: unit u = (step in chunk si, tile tt, term) at ((si * T + tt) * 2 + term) KiB;
  // the four waves take the units in turn (wave w: u = w, w + 4, ...), which for every step
  // keeps each wave on one term and a fixed set of tiles
  constexpr int kUnits = kGChunk * T * 2;
  static_assert(kUnits % kWaves == 0 && (T * 2) % kWaves == 0, "units split evenly over the waves");
  constexpr int kMine = T * 2 / kWaves;  // units per step and wave
  const uint16_t* pa[kMine];
#pragma unroll
  for (int k = 0; k < kMine; ++k) {
    const int u = wave + kWaves * k;  // unit of step 0
    const int tt = (u >> 1) % T, term = u & 1;
    const int ri = row0[tt] + min(n, max(nrows[tt], 1) - 1);
    const long long arow = a.a_row_map ? a.a_row_map[ri] : ri;
    pa[k] = (term ? a.a_lo : a.a_hi) + arow * a.lda + 8 * g;
  }
  auto copy_chunk = [&](int chunk) {
    uint8_t* dst = abuf + (chunk & 1) * kGChunkBytes;
#pragma unroll
    for (int si = 0; si < kGChunk; ++si) {
      const int so = min(chunk * kGChunk + si, nsteps - 1) * kStepRows;
#pragma unroll
      for (int k = 0; k < kMine; ++k) dma16_async(pa[k] + so, dst + (si * T * 2 + wave + kWaves * k) * kGUnit);
    }
  };

  f32x4 acc[T][NC];
#pragma unroll
  for (int tt = 0; tt < T; ++tt)
#pragma unroll
    for (int t = 0; t < NC; ++t) acc[tt][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  Step ring[kGRing];
  copy_chunk(0);
#pragma unroll
  for (int p = 0; p < kGRing; ++p) {
    __builtin_amdgcn_sched_barrier(0);
    load_step(p, ring[p]);
  }
  __builtin_amdgcn_sched_barrier(0);

  constexpr int kPerStep = BL ? 5 : 16;  // vector-memory loads per step and wave
  for (int s0 = 0; s0 < nsteps_pad; s0 += kGRing) {
    if (s0 % kGChunk == 0) {  // uniform; see bwd_item for the protocol
      wait_vm<(kGRing * kPerStep < 63 ? kGRing * kPerStep : 63)>();
      __syncthreads();
      const int c = s0 / kGChunk;
      if ((c + 1) * kGChunk < nsteps_pad) copy_chunk(c + 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    const uint8_t* ab = abuf + ((s0 / kGChunk) & 1) * kGChunkBytes + lane * 16;
#pragma unroll
    for (int p = 0; p < kGRing; ++p) {
      const int si = (s0 + p) % kGChunk;
      Step& r = ring[p];
      // pin the step's loaded dwords here, so that nothing computed from them is scheduled into
      // an earlier step (which would wait for this step's loads there)
      uint32_t rw[8], rs[8];
      if constexpr (BL) {
#pragma unroll
        for (int u = 0; u < 4; ++u) asm volatile("" : "+v"(r.c[u]));
        asm volatile("" : "+v"(r.s));
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          rw[2 * u] = (uint32_t)(odd ? r.c[u][1] : r.c[u][0]);
          rw[2 * u + 1] = (uint32_t)(odd ? r.c[u][3] : r.c[u][2]);
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) rs[q] = r.s[q >> 2] >> (8 * (q & 3));
      } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          asm volatile("" : "+v"(r.w[q]));
          asm volatile("" : "+v"(r.s[q]));
          rw[q] = r.w[q];
          rs[q] = r.s[q];
        }
      }
      uint32_t wl[8];
      float sf[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const uint32_t sc = (rs[q] >> ssh) & 0xFFu;
        const bool dead = sc >= 253u;  // the row's block contributes zero
        wl[q] = dead ? 0u : rw[q] >> wsh;
        sf[q] = bits_f((dead ? 127u : sc) << 23);
      }
      bf16x8 b[NC];
      static_for<NC / 2>([&](auto pc) {
        constexpr int P = decltype(pc)::value;
        gdecode_pair<P>(wl, sf, b[2 * P], b[2 * P + 1]);
      });
      // every tile slot computes (a short part's empty slots work on copies of its first tile's
      // rows and are never stored): no branch, so the A reads of the next tiles are issued while
      // the MFMAs of the current ones run
#pragma unroll
      for (int tt = 0; tt < T; ++tt) {
        const i32x4 ah = *reinterpret_cast<const i32x4*>(ab + ((si * T + tt) * 2) * kGUnit);
        const i32x4 al = *reinterpret_cast<const i32x4*>(ab + ((si * T + tt) * 2 + 1) * kGUnit);
#pragma unroll
        for (int t = 0; t < NC; ++t) acc[tt][t] = mfma_bf16(__builtin_bit_cast(bf16x8, ah), b[t], acc[tt][t]);
#pragma unroll
        for (int t = 0; t < NC; ++t) acc[tt][t] = mfma_bf16(__builtin_bit_cast(bf16x8, al), b[t], acc[tt][t]);
      }
      __builtin_amdgcn_sched_barrier(0);
      load_step(s0 + p + kGRing, ring[p]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // epilogue: lane (n, g) holds rows 4g..4g+3 of columns col .. col + NC - 1 of every tile
  const bool col_ok = stripe_ok && col < a.C;
  auto epilogue = [&](auto ttc) {
    constexpr int tt = decltype(ttc)::value;
    const int r0 = row0[tt], nr = nrows[tt];
    if (MODE == kBwdDownT) {
      const int F = a.C;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = 4 * g + v;
        const bool row_ok = i < nr;
        const int p = r0 + (row_ok ? i : 0);
        float dot = 0.f;
        if (col_ok && row_ok) {
          const float tw = a.row_w[p];
          const float* sv = a.saved + (long long)p * 2 * F + col;
          const float* rq = a.lora_rq ? a.lora_rq + (long long)a.a_row_map[p] * F + col : nullptr;
          const long long o = (long long)p * 2 * F + col;
#pragma unroll
          for (int c4 = 0; c4 < NC / 4; ++c4) {
            const f32x4 gt4 = *reinterpret_cast<const f32x4*>(sv + 4 * c4);
            const f32x4 up4 = *reinterpret_cast<const f32x4*>(sv + F + 4 * c4);
            f32x4 rq4 = f32x4{0.f, 0.f, 0.f, 0.f};
            if (rq) rq4 = *reinterpret_cast<const f32x4*>(rq + 4 * c4);
            float dg[4], du[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float h = acc[tt][4 * c4 + e][v] + rq4[e];
              dot += glu_fwd(gt4[e], up4[e], a.act_kind) * h;
              glu_bwd(tw * h, gt4[e], up4[e], a.act_kind, dg[e], du[e]);
            }
            const uint32_t g0 = pack_bf16(dg[0], dg[1]), g1 = pack_bf16(dg[2], dg[3]);
            const uint32_t u0 = pack_bf16(du[0], du[1]), u1 = pack_bf16(du[2], du[3]);
            __builtin_nontemporal_store(u32x2{g0, g1}, reinterpret_cast<u32x2*>(a.d_hi + o + 4 * c4));
            __builtin_nontemporal_store(u32x2{pack_bf16(dg[0] - bf16_lo(g0), dg[1] - bf16_hi(g0)),
                                               pack_bf16(dg[2] - bf16_lo(g1), dg[3] - bf16_hi(g1))},
                                        reinterpret_cast<u32x2*>(a.d_lo + o + 4 * c4));
            __builtin_nontemporal_store(u32x2{u0, u1}, reinterpret_cast<u32x2*>(a.d_hi + o + F + 4 * c4));
            __builtin_nontemporal_store(u32x2{pack_bf16(du[0] - bf16_lo(u0), du[1] - bf16_hi(u0)),
                                               pack_bf16(du[2] - bf16_lo(u1), du[3] - bf16_hi(u1))},
                                        reinterpret_cast<u32x2*>(a.d_lo + o + F + 4 * c4));
          }
        }
        // the stripe's part of grad_w = <act, h>: the 16 lanes of the row group, then the waves
        const float d = group16_sum(dot);
        if (n == 0) red[(wave * T + tt) * 16 + i] = d;
      }
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = 4 * g + v;
        if (i < nr && col_ok) {
          float* yr = a.y + (long long)(r0 + i) * a.ldy + col;
#pragma unroll
          for (int c4 = 0; c4 < NC / 4; ++c4) {
            f32x4 o = f32x4{acc[tt][4 * c4][v], acc[tt][4 * c4 + 1][v], acc[tt][4 * c4 + 2][v], acc[tt][4 * c4 + 3][v]};
            if (a.accumulate) o += *reinterpret_cast<const f32x4*>(yr + 4 * c4);
            *reinterpret_cast<f32x4*>(yr + 4 * c4) = o;
          }
        }
      }
    }
  };
  static_for<T>(epilogue);
  if (MODE == kBwdDownT) {
    // grad_w partials per 256 columns: the waves of each 256-column part, in a fixed order
    constexpr int kWavesPerPart = kBwdColsPerTile / kGS;
    constexpr int kParts = kWaves / kWavesPerPart;
    __syncthreads();
    const int t = threadIdx.x;  // one (part, tile, row) per thread
    if (t < kParts * T * 16) {
      const int part = t / (T * 16), tt = (t / 16) % T, i = t & 15;
      const int ct = cb * (kGCols / kBwdColsPerTile) + part;
      if (tt < ntl && i < nrows[tt] && ct < a.n_ct) {
        float d = 0.f;
        for (int w = 0; w < kWavesPerPart; ++w) d += red[((part * kWavesPerPart + w) * T + tt) * 16 + i];
        a.gw_part[(long long)(row0[tt] + i) * a.n_ct + ct] = d;
      }
    }
  }
}

// Resident grid over the large-bucket items (group, part, column block), dealt round-robin over
// the XCDs like the one-tile items, so launches with few or no groups cost almost nothing.
template <int MODE, bool BL>
__global__ __launch_bounds__(64 * kWaves, MX_BWD_GPER_CU) void bwd_group_kernel(BwdArgs a)
{
  __shared__ __attribute__((aligned(16))) uint8_t abuf[2 * kGChunkBytes];
  __shared__ float red[kWaves * kGT * 16];
  const int ng = *(cint_ptr)a.n_groups;
  const int ncb = (a.C + kGCols - 1) / kGCols;
  const int total = ng * kGParts * ncb;
  const int per_xcd = (total + 7) >> 3;
  bool busy = false;
  for (int it = 0;; ++it) {
    const int slot = (int)(blockIdx.x >> 3) + it * (int)(gridDim.x >> 3);
    const int item = (int)(blockIdx.x & 7) * per_xcd + slot;
    if (slot >= per_xcd || item >= total) break;
    const int gp = item / ncb, cb = item - gp * ncb;
    const int gi = gp / kGParts, part = gp - gi * kGParts;
    const cint_ptr gg = (cint_ptr)(a.groups + gi);
    const int ntl = gg[2] - part * kGT;
    if (ntl <= 0) continue;  // the empty part of a short group
    if (busy) __syncthreads();  // every wave has finished reading the previous item's LDS
    bwd_group_item<MODE, BL>(a, gg[0], gg[1] + part * kGT, min(ntl, kGT), cb, abuf, red);
    busy = true;
  }
}

int resident_groups(int per_cu)
{
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  return max(8, (per_cu * cus) / 8 * 8);
}

}  // namespace

hipError_t launch_bwd(const BwdArgs& a, int mode, int max_tiles, hipStream_t s)
{
  const long long n_ct4 = (a.n_ct + kWaves - 1) / kWaves;
  const long long total = (long long)max_tiles * n_ct4;
  if (total <= 0) return hipSuccess;
  // each weight segment is addressed through one buffer resource with a 32-bit byte count
  if ((long long)a.R * (a.C / 2) >= (1LL << 32)) return hipErrorInvalidValue;
  // the epilogue's 16-byte accesses of rows assume these (true for every caller: C is a multiple
  // of 32 and the row strides are multiples of 16 elements)
  if (a.C % 32 || (a.y && a.ldy % 4) || a.lda % 8) return hipErrorInvalidValue;
  // large buckets take the grouped kernel when their scale rows are whole dwords
  const bool split = a.tiles && a.small_tiles && a.groups && a.C % 128 == 0;
  BwdArgs b = a;
  if (!split) {
    b.small_tiles = nullptr;
    b.groups = nullptr;
  }
  const bool bl = a.bl0 != nullptr && mode != kBwdPlain;
  if (bl && (!backward_layout_ok(a.R, a.C) || (a.nseg > 1 && !a.bl1))) return hipErrorInvalidValue;
  // the W2 transposed product with whole eight-stripe items: both kernels are launched, and the
  // routing's tile count (on the device) decides which of them does the work
  const long long witems = (long long)max_tiles * (a.n_ct / kWideWaves);
  const int wide = mode == kBwdDownT && bl && a.n_ct % kWideWaves == 0 && witems >= kWideMinItems;
  long long blocks = (total + 7) / 8 * 8;
  if (wide)  // bwd_kernel then runs only with fewer than kWideMinItems wide items: twice as many of its own
    blocks = (std::min<long long>(total, 2LL * kWideMinItems) + 7) / 8 * 8;
  dim3 grid((unsigned)blocks), block(64 * kWaves);
  if (mode == kBwdPlain) hipLaunchKernelGGL((bwd_kernel<kBwdPlain, false>), grid, block, 0, s, b, 0);
  else if (mode == kBwdDownT && bl) hipLaunchKernelGGL((bwd_kernel<kBwdDownT, true>), grid, block, 0, s, b, wide);
  else if (mode == kBwdDownT) hipLaunchKernelGGL((bwd_kernel<kBwdDownT, false>), grid, block, 0, s, b, wide);
  else if (bl) hipLaunchKernelGGL((bwd_kernel<kBwdGateUpT, true>), grid, block, 0, s, b, 0);
  else hipLaunchKernelGGL((bwd_kernel<kBwdGateUpT, false>), grid, block, 0, s, b, 0);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (wide) {
    dim3 wgrid((unsigned)((witems + 7) / 8 * 8)), wblock(64 * kWideWaves);
    hipLaunchKernelGGL((bwd_wide_kernel<kBwdDownT, true>), wgrid, wblock, 0, s, b);
    e = hipGetLastError();
  }
  if (e != hipSuccess || !split) return e;
  // groups come from experts of at least kGroupMinTiles tiles: at most max_tiles / kGroupMinTiles + 1
  const long long gtotal = ((long long)max_tiles / kGroupMinTiles + 1) * kGParts * ((a.C + kGCols - 1) / kGCols);
  dim3 ggrid((unsigned)std::min<long long>((gtotal + 7) / 8 * 8, resident_groups(MX_BWD_GPER_CU)));
  if (mode == kBwdPlain) hipLaunchKernelGGL((bwd_group_kernel<kBwdPlain, false>), ggrid, block, 0, s, b);
  else if (mode == kBwdDownT && bl) hipLaunchKernelGGL((bwd_group_kernel<kBwdDownT, true>), ggrid, block, 0, s, b);
  else if (mode == kBwdDownT) hipLaunchKernelGGL((bwd_group_kernel<kBwdDownT, false>), ggrid, block, 0, s, b);
  else if (bl) hipLaunchKernelGGL((bwd_group_kernel<kBwdGateUpT, true>), ggrid, block, 0, s, b);
  else hipLaunchKernelGGL((bwd_group_kernel<kBwdGateUpT, false>), ggrid, block, 0, s, b);
  return hipGetLastError();
}

bool backward_layout_ok(int R, int C)
{
  return R > 0 && C > 0 && R % kStepRows == 0 && C % kBwdColsPerTile == 0 &&
         (long long)R * C / 2 + (long long)R * C / 32 < (1LL << 32);
}

long long backward_layout_bytes(int R, int C)
{
  return backward_layout_ok(R, C) ? (long long)R * C / 2 + (long long)R * C / 32 : 0;
}

namespace {

// One thread per 16-byte piece of the backward layout of one expert's [R, C] matrix: blocks
// (step st = 32 rows, stripe c = 256 columns) in order st * nstr + c. Codes: piece (u, l) of
// block b at b * 4096 + u * 1024 + l * 16 holds, for lane l = 16 g + n, bytes 8n .. 8n + 7 of
// the stripe in rows 32 st + 8g + 2u and 32 st + 8g + 2u + 1 (8 bytes each), what that lane's
// four 16-byte loads of the step read. Scales, after every block's codes: the 256 B of block b
// hold at 8 m + q (m = 8 g + j) the scale byte of row 32 st + 8g + q for MX block 8c + j, the
// 8 bytes lanes 2m and 2m + 1 (columns 32j .. 32j + 31 of the stripe) read.
__global__ __launch_bounds__(256) void backward_layout_kernel(const uint8_t* packed, const uint8_t* scales,
                                                              uint8_t* out, int R, int C, long long per_expert,
                                                              long long total)
{
  const long long p = (long long)blockIdx.x * 256 + threadIdx.x;
  if (p >= total) return;
  const int nstr = C / kBwdColsPerTile;
  const long long e = p / per_expert;
  long long r = p - e * per_expert;
  const long long code_pieces = (long long)(R / kStepRows) * nstr * 256;
  const long long cb = (long long)C / 2, sb = (long long)C / kGroup;
  if (r < code_pieces) {
    const int l = (int)(r & 63), u = (int)((r >> 6) & 3);
    const long long blk = r >> 8;
    const int st = (int)(blk / nstr), c = (int)(blk - (long long)st * nstr);
    const int row = st * kStepRows + 8 * (l >> 4) + 2 * u;
    const uint8_t* src = packed + (e * R + row) * cb + c * 128 + 8 * (l & 15);
    const u32x2 v0 = *reinterpret_cast<const u32x2*>(src);
    const u32x2 v1 = *reinterpret_cast<const u32x2*>(src + cb);
    *reinterpret_cast<i32x4*>(out + p * 16) = i32x4{(int)v0[0], (int)v0[1], (int)v1[0], (int)v1[1]};
    return;
  }
  r -= code_pieces;  // piece k of scale block blk: entries m = 2k, 2k + 1
  const int k = (int)(r & 15);
  const long long blk = r >> 4;
  const int st = (int)(blk / nstr), c = (int)(blk - (long long)st * nstr);
  uint32_t v[4];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int m = 2 * k + h, g = m >> 3, j = m & 7;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      uint32_t word = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int row = st * kStepRows + 8 * g + 4 * half + q;
        word |= (uint32_t)scales[(e * R + row) * sb + 8 * c + j] << (8 * q);
      }
      v[2 * h + half] = word;
    }
  }
  *reinterpret_cast<i32x4*>(out + p * 16) = i32x4{(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
}

}  // namespace

hipError_t launch_backward_layout(const uint8_t* packed, const uint8_t* scales, uint8_t* out, int E, int R, int C,
                                  hipStream_t s)
{
  if (E <= 0) return hipSuccess;
  if (!backward_layout_ok(R, C)) return hipErrorInvalidValue;
  const long long per_expert = backward_layout_bytes(R, C) / 16;
  const long long total = per_expert * E;
  hipLaunchKernelGGL(backward_layout_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, packed, scales,
                     out, R, C, per_expert, total);
  return hipGetLastError();
}

}  // namespace mx
