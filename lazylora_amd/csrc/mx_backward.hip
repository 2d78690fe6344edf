// Transposed MXFP4 products y[m, c] = sum_r A[m, r] W[r, c] (gfx950).
//
// The contraction runs over W's rows, the strided direction of the packed layout, and the
// E8M0 scales group W along its columns, so the scaled MFMA cannot consume W directly here.
// Each step a work-group (256 threads) cooperatively loads a 32-row x 512-column slab of W
// (every thread two 16-byte MX blocks = 2 x 32 columns of one row), decodes it with
// v_cvt_scalef32_pk_bf16_fp4 (bit-exact: e2m1 * 2^(s-127) is exact in bf16), and writes it
// row-major (padded, see slab_off) into LDS. Each wave then owns 128 output columns and pulls
// its B operands with ds_read_b64_tr_b16, which hands lane i of a 16-lane group column i of
// four consecutive rows. A (activation gradients) is split into bf16 hi + lo terms, so the
// products carry ~16 significant bits of the activation against the exact weights. The slab
// is double-buffered (2 x 32 KiB, XOR-swizzled instead of padded, so two work-groups fit per
// CU): one barrier per step.
//
// 512 columns per work-group: the E8M0 scales of one W row sit in the same 128-byte lines
// for all column tiles, and every work-group that reads a line only for its own 16 bytes
// costs a fetch of the whole line; wider tiles cut those fetches in half.
//
// The whole contraction range (nseg * R rows) stays in one work-group, so every output
// element has exactly one writer and the sum order is fixed: results are deterministic.
#include "mx_device.h"
#include "mx_kernels.h"

#include <algorithm>

namespace mx {

namespace {

constexpr int kSlabRows = 32;
constexpr int kRowBytes = kBwdColsPerTile * 2;     // 1 KiB of bf16 per slab row, no padding
constexpr int kSlabBytes = kSlabRows * kRowBytes;  // 32 KiB; two of them per work-group

// LDS slab layout. LDS has 32 banks of 4 bytes; a ds_write_b128 is served 8 lanes per cycle
// and a ds_read_b64_tr_b16 16 lanes per cycle (both measured on the hardware). A row is 128
// "quads" of 4 bf16 (8 bytes); quad q of row r is stored at position
//   q ^ (((q >> 4) & 3) << 1) ^ ((r & 3) << 2),
// which only permutes bits 1-3 of q: aligned quad pairs stay together (16-byte writes stay
// contiguous) and every quad stays in its aligned group of 16. The 8 lanes of a write phase
// (one row, blocks lc = 0..7, same piece) then cover all 32 banks, and so do the 16 lanes of a
// transposed-read phase (4 consecutive rows x 4 quads).
__device__ __forceinline__ int quad_pos(int row, int q)
{
  return q ^ (((q >> 4) & 3) << 1) ^ ((row & 3) << 2);
}
__device__ __forceinline__ int slab_off(int row, int q)  // byte offset of quad q of row
{
  return row * kRowBytes + quad_pos(row, q) * 8;
}
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef const __attribute__((address_space(4))) int* cint_ptr;

#ifndef MX_BWD_GROUP_T
#define MX_BWD_GROUP_T 2
#endif
constexpr int kBwdGroupT = MX_BWD_GROUP_T;  // row tiles per large-bucket work item (2 or 4)

// One work item: column tile ct of up to T row tiles of one expert (T = 1: a small-bucket tile;
// T = kGroupTiles: a large-bucket group, whose tiles share every decoded slab).
template <int T>
struct WorkItem {
  int expert, ct, ntl;
  int row0[T], nrows[T], tile[T];
};

// Work item `it` of this work-group (items are dealt round-robin over the XCDs, blockIdx % 8,
// each XCD taking one contiguous run, in strides of the grid). Returns 0 when there is none
// left, 2 for an empty part of a short group, 1 for an item.
template <int T>
__device__ __forceinline__ int decode_work(const BwdArgs& a, int it, WorkItem<T>& w)
{
  // the tile lists are only read here: scalar loads through the constant address space
  int count;
  constexpr int kParts = T == 1 ? 1 : kGroupTiles / T;  // work items per group
  // with no large-bucket groups the small-bucket list is every tile in order: skip it
  const bool use_small = a.small_tiles && *(cint_ptr)a.n_groups > 0;
  if (T == 1) count = use_small ? *(cint_ptr)a.n_small
                                : a.tiles ? *(cint_ptr)a.n_tiles : (a.M + kFwdRowsPerTile - 1) / kFwdRowsPerTile;
  else count = *(cint_ptr)a.n_groups * kParts;
  const int total = count * a.n_ct;
  const int per_xcd = (total + 7) >> 3;
  const int slot = (int)(blockIdx.x >> 3) + it * (int)(gridDim.x >> 3);
  const int item = (int)(blockIdx.x & 7) * per_xcd + slot;
  if (slot >= per_xcd || item >= total) return 0;
  const int i = item / a.n_ct;
  w.ct = item - i * a.n_ct;
  int t0;
  if (T == 1) {
    t0 = use_small ? ((cint_ptr)a.small_tiles)[i] : i;
    w.ntl = 1;
  } else {
    const int part = i % kParts;
    const cint_ptr gg = (cint_ptr)(a.groups + i / kParts);
    t0 = gg[1] + part * T;
    w.ntl = min(T, gg[2] - part * T);
    if (w.ntl <= 0) return 2;  // this part of a short group is empty
  }
#pragma unroll
  for (int tt = 0; tt < T; ++tt) {
    const int t = t0 + (tt < w.ntl ? tt : 0);
    w.tile[tt] = t;
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

// 16 fp4 bytes (32 codes of one row) -> 32 bf16 in 16 dwords, scale byte s applied exactly;
// s >= 253 gives zeros.
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

// Decoded block blk (32 columns = quads 8 blk .. 8 blk + 7) of a slab row: four 16-byte writes.
__device__ __forceinline__ void store_block(uint8_t* slab, int row, int blk, const i32x4& raw, uint32_t s)
{
  uint32_t dec[16];
  decode_block_bf16(raw, s, dec);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    *reinterpret_cast<i32x4*>(slab + slab_off(row, blk * 8 + 2 * j)) =
        i32x4{(int)dec[4 * j], (int)dec[4 * j + 1], (int)dec[4 * j + 2], (int)dec[4 * j + 3]};
}

// T = 1: weight steps in flight per work-group kPrefetch = 8, two work-groups per CU. T > 1:
// T times the matrix work per step, so a shorter ring hides the loads; T = 2 still fits two
// work-groups per CU, T = 4 needs the whole register file (one per CU).
//
// Step s of the main loop, after the barrier that publishes slab s: every wave issues all of
// its transposed reads of slab s at once, then the loads that refill the rings, then decodes
// step s + 1 into the other slab buffer in two halves, each followed by half of slab s's
// MFMAs. The decode's VALU work and LDS writes thus overlap the matrix work and the read
// latency is paid once per step. The other buffer held slab s - 1, whose reads every wave
// finished (its MFMAs consumed them) before arriving at this step's barrier.
template <int MODE, int T>
__device__ __forceinline__ void bwd_item(const BwdArgs& a, const WorkItem<T>& w)
{
  constexpr int kPrefetch = T == 1 ? 8 : 4;  // even
  __shared__ __attribute__((aligned(16))) uint8_t slab[2][kSlabBytes];
  __shared__ float dotred[4][16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, g = lane >> 4;
  const int c0 = w.ct * kBwdColsPerTile;
  const int rtot = a.nseg * a.R;
  const int nsteps = (rtot + kSlabRows - 1) / kSlabRows;
  // the ring below is unrolled kPrefetch-fold; padding steps read past the matrix (zeros)
  const int nsteps_pad = (nsteps + kPrefetch - 1) / kPrefetch * kPrefetch;

  // loader role: MX blocks lc and lc + 8 of slab row lr per step, so each load instruction
  // of a wave reads whole 128-byte lines (8 rows x 8 blocks). Block lc + 8 sits 128 bytes
  // (8 scale bytes) after block lc.
  const int lr = tid >> 3;
  const int lc = tid & 7;
  const uint32_t cbs = a.C / kGroup;  // scale bytes per W row
  const uint32_t wpitch = a.C / 2;
  const int colA = c0 + lc * 32;
  const int colA_c = colA < a.C ? colA : 0;
  // Each segment of this expert is one buffer resource: rows at or past the segment's end
  // (the tail of a row count that is not a multiple of kSlabRows, and the padding steps) read
  // as zero weights. Segments hold a multiple of kSlabRows rows whenever there are two, so a
  // step never straddles them. Columns past C (lanes clamped to column 0, or block lc + 8 of a
  // partial tile) read other finite weights that no stored column uses.
  const uint8_t* const wp0 = a.wp0 + (long long)w.expert * a.wp_estride;
  const uint8_t* const wp1 = a.wp1 + (long long)w.expert * a.wp_estride;
  const uint8_t* const ws0 = a.ws0 + (long long)w.expert * a.ws_estride;
  const uint8_t* const ws1 = a.ws1 + (long long)w.expert * a.ws_estride;
  const rsrc_t rw0 = make_rsrc(wp0, (uint32_t)a.R * wpitch), rw1 = make_rsrc(wp1, (uint32_t)a.R * wpitch);
  const rsrc_t rs0_ = make_rsrc(ws0, (uint32_t)a.R * cbs), rs1_ = make_rsrc(ws1, (uint32_t)a.R * cbs);
  const uint32_t lane_w = (uint32_t)lr * wpitch + colA_c / 2;
  const uint32_t lane_s = (uint32_t)lr * cbs + colA_c / kGroup;

  // Weight bytes are read exactly once per work-group: streaming loads.
  auto load_raw = [&](int step, i32x4& r0, i32x4& r1, uint8_t& s0, uint8_t& s1) {
    const int row0 = step * kSlabRows;
    const bool seg = a.nseg > 1 && row0 >= a.R;  // uniform
    const uint32_t rr = (uint32_t)(seg ? row0 - a.R : row0);
    const rsrc_t W = seg ? rw1 : rw0;
    const rsrc_t S = seg ? rs1_ : rs0_;
    const uint32_t ow = lane_w + rr * wpitch, os = lane_s + rr * cbs;
    r0 = buf16_nt(W, ow);
    r1 = buf16_nt(W, ow + 128);
    s0 = buf8(S, os);
    s1 = buf8(S, os + 8);
  };

  // A operands. A step's A tile (T tiles x hi/lo x 16 rows x 32 bf16 = 2T KiB) is loaded
  // once per work-group, each thread its 8T bytes two steps ahead, and shared through a
  // double-buffered LDS copy written one step ahead; every wave reads its MFMA operands from
  // there (four waves loading the same operands from L2 would move as many bytes as the
  // weights). Copy layout: [tile][term][row][four 16-byte K chunks], chunk c of row r at
  // position c ^ ((r >> 1) & 3), so the 8 rows of a ds_read_b128 phase cover all banks.
  // Rows past a tile's end repeat its last row (never stored). Padding steps meet zero
  // weights, so their A (the last real step's, reloaded) adds zero.
  __shared__ __attribute__((aligned(16))) uint8_t abuf[2][T * 2048];
  constexpr int kABytes = 8 * T;  // per thread and step
  typedef int av_t __attribute__((ext_vector_type(2 * T)));
  const uint16_t* pa;
  int a_dst;
  {
    const int b0 = tid * kABytes;
    const int tt = b0 >> 11, term = (b0 >> 10) & 1, row = (b0 >> 6) & 15, kb = b0 & 63;
    int r0 = w.row0[0], nr = w.nrows[0];  // tile tt's (selected, not indexed: no stack copy)
#pragma unroll
    for (int i = 1; i < T; ++i)
      if (tt == i) r0 = w.row0[i], nr = w.nrows[i];
    const int ri = r0 + min(row, nr - 1);
    const int arow = a.a_row_map ? a.a_row_map[ri] : ri;
    pa = (term ? a.a_lo : a.a_hi) + (long long)arow * a.lda + (kb >> 1);
    a_dst = (b0 & ~63) + ((((kb >> 4) ^ (row >> 1)) & 3) << 4) + (kb & 15);
  }
  auto load_a = [&](int step) { return *reinterpret_cast<const av_t*>(pa + min(step, nsteps - 1) * kSlabRows); };
  // T <= 2: the thread's bytes lie in one 16-byte chunk. T = 4: they are two whole chunks
  // (kb = 0 or 32), each stored at its own swizzled position.
  auto store_a = [&](uint8_t* buf, const av_t& v) {
    if constexpr (kABytes <= 16) {
      *reinterpret_cast<av_t*>(buf + a_dst) = v;
    } else {
      static_assert(kABytes == 32, "T is 1, 2 or 4");
      const int b0 = tid * kABytes, row = (b0 >> 6) & 15, c0 = (b0 & 63) >> 4;
#pragma unroll
      for (int h = 0; h < 2; ++h)
        *reinterpret_cast<i32x4*>(buf + (b0 & ~63) + ((((c0 + h) ^ (row >> 1)) & 3) << 4)) =
            i32x4{v[4 * h], v[4 * h + 1], v[4 * h + 2], v[4 * h + 3]};
    }
  };
  const int a_src = li * 64 + (((g ^ (li >> 1)) & 3) << 4);  // this lane's operand chunk

  f32x4 acc[T][8];
#pragma unroll
  for (int tt = 0; tt < T; ++tt)
#pragma unroll
    for (int cg = 0; cg < 8; ++cg) acc[tt][cg] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Pipeline: the raw blocks of the next kPrefetch steps are in flight in a register ring.
  // Within a step the A load is issued before the ring refill.
  i32x4 ring0[kPrefetch], ring1[kPrefetch];
  uint8_t rs0[kPrefetch], rs1[kPrefetch];
  // Issue order is pinned (A first, then the ring slot by slot) so the loop head can wait
  // for slot 0 alone, whether it is entered from here or from the back edge.
  av_t acur = load_a(0);
  store_a(abuf[0], acur);
  acur = load_a(1);
#pragma unroll
  for (int p = 0; p < kPrefetch; ++p) {
    __builtin_amdgcn_sched_barrier(0);
    load_raw(p, ring0[p], ring1[p], rs0[p], rs1[p]);
  }
  __builtin_amdgcn_sched_barrier(0);
  // slab 0 (and A copy 0 above); the previous item's last reads of these buffers ended before
  // the caller's barrier
  store_block(slab[0], lr, lc, ring0[0], rs0[0]);
  store_block(slab[0], lr, lc + 8, ring1[0], rs1[0]);

  for (int s0 = 0; s0 < nsteps_pad; s0 += kPrefetch) {
#pragma unroll
    for (int p = 0; p < kPrefetch; ++p) {
      const int s = s0 + p;
      const uint8_t* const sl = slab[p & 1];  // kPrefetch is even, so this is slab[s & 1]
      uint8_t* const sn_buf = slab[(p + 1) & 1];
      const uint8_t* const ab = abuf[p & 1];
      uint8_t* const an_buf = abuf[(p + 1) & 1];
      const int q = (p + 1) % kPrefetch;     // ring slot of step s + 1
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
      // B operands of this wave's 8 column groups: rows 8g..8g+7 of column cg*16 + li
      bf16x8 b[8];
#pragma unroll
      for (int cg = 0; cg < 8; ++cg) {
        const int qd = wave * 32 + cg * 4 + (li & 3);
        const i16x4 t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_i16x4*)(&sl[slab_off(8 * g + (li >> 2), qd)]));
        const i16x4 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_i16x4*)(&sl[slab_off(8 * g + 4 + (li >> 2), qd)]));
        const short __attribute__((ext_vector_type(8))) bs = {t0[0], t0[1], t0[2], t0[3], t1[0], t1[1], t1[2], t1[3]};
        b[cg] = __builtin_bit_cast(bf16x8, bs);
      }
      i32x4 ahv[T], alv[T];
#pragma unroll
      for (int tt = 0; tt < T; ++tt) {
        ahv[tt] = *reinterpret_cast<const i32x4*>(ab + tt * 2048 + a_src);
        alv[tt] = *reinterpret_cast<const i32x4*>(ab + tt * 2048 + 1024 + a_src);
      }
      const av_t anext = load_a(s + 2);
      __builtin_amdgcn_sched_barrier(0);
      load_raw(s + kPrefetch, ring0[p], ring1[p], rs0[p], rs1[p]);
      __builtin_amdgcn_sched_barrier(0);
      // The decode / MFMA half of the step runs at a raised wave priority: of the two waves on a
      // SIMD, the one in this phase is issued first, so it finishes its step while the other
      // waits at its barrier or on its transposed reads, and the two phases overlap instead of
      // alternating in lockstep (2-3% faster than the default level; raising it over the reads
      // instead, or over only the MFMAs or only the decode, is not).
      __builtin_amdgcn_s_setprio(1);

      // two halves: decode half h of step s + 1, then the MFMAs of column groups 4h..4h+3,
      // the hi terms of each pair of groups (and of every tile) before their lo terms
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if (h == 0) {
          store_block(sn_buf, lr, lc, ring0[q], rs0[q]);
          store_a(an_buf, acur);  // step s + 1's A
        } else {
          store_block(sn_buf, lr, lc + 8, ring1[q], rs1[q]);
        }
#pragma unroll
        for (int cp = 4 * h; cp < 4 * h + 4; cp += 2) {
#pragma unroll
          for (int e = 0; e < 2; ++e)
#pragma unroll
            for (int tt = 0; tt < T; ++tt)
              if (tt < w.ntl) acc[tt][cp + e] = mfma_bf16(__builtin_bit_cast(bf16x8, ahv[tt]), b[cp + e], acc[tt][cp + e]);
#pragma unroll
          for (int e = 0; e < 2; ++e)
#pragma unroll
            for (int tt = 0; tt < T; ++tt)
              if (tt < w.ntl) acc[tt][cp + e] = mfma_bf16(__builtin_bit_cast(bf16x8, alv[tt]), b[cp + e], acc[tt][cp + e]);
        }
      }
      __builtin_amdgcn_s_setprio(0);
      acur = anext;
    }
  }

  // epilogue, tile by tile: lane (li, g) holds rows 4g..4g+3 of column c0 + wave*128 + cg*16 + li
  // (conditionals rather than break / continue, so the loop unrolls and acc stays in registers)
#pragma unroll
  for (int tt = 0; tt < T; ++tt) {
    const bool live = tt < w.ntl;  // uniform
    const int row0 = w.row0[tt], nrows = w.nrows[tt];
    if (MODE == kBwdDownT) {
      const int F = a.C;
      float dots[4] = {0.f, 0.f, 0.f, 0.f};
      if (live) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int i = 4 * g + v;
          const bool row_ok = i < nrows;
          const int p = row0 + (row_ok ? i : 0);
          const float tw = a.row_w[p];
          const float* sv = a.saved + (long long)p * 2 * F;
          // LoRA: the down adapter's A_d^T q of the row's token joins g . W2
          const float* rq = a.lora_rq ? a.lora_rq + (long long)a.a_row_map[p] * F : nullptr;
#pragma unroll
          for (int cg = 0; cg < 8; ++cg) {
            const int f = c0 + wave * 128 + cg * 16 + li;
            if (f < F) {
              const float h = rq ? acc[tt][cg][v] + rq[f] : acc[tt][cg][v];
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
      }
      if (live) {
        if (tt > 0) __syncthreads();  // the previous tile's partial dots have been read
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float d = group16_sum(dots[v]);
          if (li == 0) dotred[wave][4 * g + v] = d;
        }
        __syncthreads();
        if (tid < 16 && tid < nrows) {
          const float d = dotred[0][tid] + dotred[1][tid] + dotred[2][tid] + dotred[3][tid];
          a.gw_part[(long long)(row0 + tid) * a.n_ct + w.ct] = d;
        }
      }
    } else if (live) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = 4 * g + v;
        if (i < nrows) {
          float* yr = a.y + (long long)(row0 + i) * a.ldy;
#pragma unroll
          for (int cg = 0; cg < 8; ++cg) {
            const int col = c0 + wave * 128 + cg * 16 + li;
            if (col < a.C) {
              if (a.accumulate) yr[col] += acc[tt][cg][v];
              else yr[col] = acc[tt][cg][v];
            }
          }
        }
      }
    }
  }
}

// T = 1: one item per work-group (the grid covers every item). T > 1: a resident grid that
// loops over the large-bucket items, so launches with few or no groups cost almost nothing.
template <int MODE, int T>
__global__ __launch_bounds__(256, T <= 2 ? 2 : 1) void bwd_kernel(BwdArgs a)
{
  WorkItem<T> w;
  if constexpr (T == 1) {
    if (decode_work<T>(a, 0, w) == 1) bwd_item<MODE, T>(a, w);
    return;
  }
  bool busy = false;
  for (int it = 0;; ++it) {
    const int st = decode_work<T>(a, it, w);
    if (st == 0) break;
    if (st == 2) continue;
    if (busy) __syncthreads();  // the previous item's LDS reads are complete
    bwd_item<MODE, T>(a, w);
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
  const long long total = (long long)max_tiles * a.n_ct;
  if (total <= 0) return hipSuccess;
  // each weight segment is addressed through one buffer resource with a 32-bit byte count
  if ((long long)a.R * (a.C / 2) >= (1LL << 32)) return hipErrorInvalidValue;
  const bool split = a.tiles && a.small_tiles && a.groups;
  BwdArgs b = a;
  if (!split) {
    b.small_tiles = nullptr;
    b.groups = nullptr;
  }
  const long long blocks = (total + 7) / 8 * 8;
  dim3 grid((unsigned)blocks), block(256);
  if (mode == kBwdPlain) hipLaunchKernelGGL((bwd_kernel<kBwdPlain, 1>), grid, block, 0, s, b);
  else if (mode == kBwdDownT) hipLaunchKernelGGL((bwd_kernel<kBwdDownT, 1>), grid, block, 0, s, b);
  else hipLaunchKernelGGL((bwd_kernel<kBwdGateUpT, 1>), grid, block, 0, s, b);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !split) return e;
  // groups come from experts of at least kGroupMinTiles tiles: at most max_tiles / 2 of them,
  // each split into kGroupTiles / kBwdGroupT work items
  const long long gtotal = ((long long)max_tiles / 2 + 1) * (kGroupTiles / kBwdGroupT) * a.n_ct;
  dim3 ggrid((unsigned)std::min<long long>((gtotal + 7) / 8 * 8, resident_groups(kBwdGroupT <= 2 ? 2 : 1)));
  if (mode == kBwdPlain) hipLaunchKernelGGL((bwd_kernel<kBwdPlain, kBwdGroupT>), ggrid, block, 0, s, b);
  else if (mode == kBwdDownT) hipLaunchKernelGGL((bwd_kernel<kBwdDownT, kBwdGroupT>), ggrid, block, 0, s, b);
  else hipLaunchKernelGGL((bwd_kernel<kBwdGateUpT, kBwdGroupT>), ggrid, block, 0, s, b);
  return hipGetLastError();
}

}  // namespace mx
