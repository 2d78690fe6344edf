// Forward MXFP4 products on the fp4-native scaled MFMA (gfx950).
//
// Each wave computes one 16-row x 64-column output tile over the whole K range
// (kFwdGateUp: 16 rows x 32 gate features + the same 32 up features). A work-group holds the
// four waves of four neighbouring column tiles of the same row tile (eight for the routed
// products from a forward layout, which then run their large-bucket items in the same launch,
// fwd_fused_kernel): they share the tile's activations, which the work-group copies into LDS
// once per super-chunk. Every weight byte is read once per row tile.
//
// Per super-chunk c (512 K elements) and lane (j = lane % 16, g = lane / 16), for each of the
// 4 column groups of 16 weight rows:
//   B: 64 contiguous bytes of weight row n = 4 MX blocks 16c+4g+q (q = 0..3), one dword of
//      scales. MFMA q consumes block 16c+4g+q from lane group g, so op_sel q picks its scale.
//      With a forward layout (launch_forward_layout) the same 16-byte pieces come from a copy
//      that holds each MFMA's operand as one contiguous KiB: whole lines per load instruction,
//      each read once, with the streaming hint.
//   A: the two-term activations of the tile in the AT layout: for each (q, plane, piece) one
//      contiguous KiB, and one 8-byte scale pair per lane.
// Weights are consumed as stored: the MFMA applies the E8M0 scales and the e2m1 codes itself.
// A scale byte >= 253 zeroes its block (lazy_lora/native/mxfp4_gemm.c:16-18) before it can
// reach the MFMA, where 255 would be NaN and 253/254 would overflow.
//
// Fast path (K a multiple of 512), one step per super-chunk:
//   wait for this step's data, barrier -> read A(c) and this chunk's weight scales from LDS
//   -> request B(c+1) into the other register buffer and DMA A(c+1) into the other LDS
//   buffer -> 32 MFMAs on chunk c while the requests are in flight.
// Weight scales are staged per wave in LDS, 8 super-chunks (128 B of every row) at a time:
// reading each chunk's 16 B straight from memory would fetch every 128 B scale line up to
// 8 times, because the weight stream evicts it from L2 between chunks.
#include "mx_device.h"
#include "mx_kernels.h"

#include <algorithm>

namespace mx {

namespace {

constexpr int kWavesPerGroup = 4;
constexpr int kAtLdsBytes = kAtCodeBytes + 1024;   // one super-chunk of A; its scale DMA writes 1 KiB
constexpr int kScaleWin = 8;                       // super-chunks per staged scale window
constexpr int kScaleRowBytes = 16 * kScaleWin;     // 128 B of scales per weight row
constexpr int kScaleWaveBytes = 64 * kScaleRowBytes;

struct FwdLds {
  uint8_t a[2][kAtLdsBytes];
  uint8_t s[kWavesPerGroup][kScaleWaveBytes];
};

struct WorkItem {
  int tile, expert, row0, nrows, ct;
  int ct0;      // first column tile of the work-group (its NW waves take ct0 .. ct0 + NW - 1)
  bool active;  // false: this wave's column tile is past the end; it only helps with the copies
};

// The grid is persistent (about two work-groups per CU) and work-groups are issued round-robin
// over the 8 XCDs (blockIdx % 8). Each XCD owns one contiguous run of work items, so the tiles
// of one expert share that XCD's L2; its work-groups take the run's items in turn (iteration
// `it` of slot s takes item s + it * slots). Returns false for the whole work-group at once.
typedef const __attribute__((address_space(4))) int* cint_ptr;

__device__ __forceinline__ bool decode_work(const int4* tiles, const int* n_tiles, const int* small_tiles,
                                            const int* n_small, const int* n_groups, int M, int n_ct, int wave,
                                            int it, WorkItem& w, int nw = kWavesPerGroup)
{
  // The tile lists are written before this kernel and only read here: scalar loads through the
  // constant address space, which do not wait for this work-group's outstanding stores.
  // with no large-bucket groups the small-bucket list is every tile in order: skip it
  const bool use_small = small_tiles && *(cint_ptr)n_groups > 0;
  const int ntiles = use_small ? *(cint_ptr)n_small
                               : tiles ? *(cint_ptr)n_tiles : (M + kFwdRowsPerTile - 1) / kFwdRowsPerTile;
  const int n_cg = (n_ct + nw - 1) / nw;
  const int total = ntiles * n_cg;
  const int per_xcd = (total + 7) >> 3;
  const int k = (int)(blockIdx.x >> 3) + it * (int)(gridDim.x >> 3);
  const int item = (int)(blockIdx.x & 7) * per_xcd + k;
  if (k >= per_xcd || item >= total) return false;
  const int i = item / n_cg;
  const int t = use_small ? ((cint_ptr)small_tiles)[i] : i;
  w.tile = t;
  w.ct0 = (item - i * n_cg) * nw;
  const int ct = w.ct0 + wave;
  w.active = ct < n_ct;
  w.ct = w.active ? ct : n_ct - 1;
  if (tiles) {
    const cint_ptr tt = (cint_ptr)(tiles + t);
    w.expert = tt[0];
    w.row0 = tt[1];
    w.nrows = tt[2];
  } else {
    w.expert = 0;
    w.row0 = t * kFwdRowsPerTile;
    w.nrows = min(kFwdRowsPerTile, M - w.row0);
  }
  return true;
}

__device__ __forceinline__ i32x8 cat8(const i32x4& x, const i32x4& y)
{
  return i32x8{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
}
__device__ __forceinline__ i32x8 cat8_ld(const uint8_t* p0, const uint8_t* p1)
{
  return cat8(*reinterpret_cast<const i32x4*>(p0), *reinterpret_cast<const i32x4*>(p1));
}

// ---------------------------------------------------------------- third term of x
// The flag bytes of super-chunks 4g..4g+3 and 16+4g..16+4g+3 of X3 row `row` (null: an unused
// slot, no flags), as lane (i, g) of a tile loads them for x3_mask.
__device__ __forceinline__ uint2 x3_flags(const FwdArgs& a, const uint8_t* row, int lane)
{
  if (!row) return uint2{0u, 0u};
  const int g = lane >> 4;
  const uint8_t* f = row + (long long)at_nchunks(a.K) * 528;
  return uint2{*reinterpret_cast<const uint32_t*>(f + 4 * g), *reinterpret_cast<const uint32_t*>(f + 16 + 4 * g)};
}
// Bit c of the result (uniform): some row slot of the tile has a third term in super-chunk c
// (quant3_block16); the lanes' flag bytes (x3_flags) OR-ed over the wave.
__device__ __forceinline__ uint32_t x3_mask(uint2 d, int lane)
{
  const int g = lane >> 4;
  uint32_t m = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) m |= (((d.x >> (8 * j)) & 1u) << (4 * g + j)) | (((d.y >> (8 * j)) & 1u) << (16 + 4 * g + j));
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) m |= (uint32_t)__shfl_xor((int)m, o, 64);
  return __builtin_amdgcn_readfirstlane(m);
}
// X3 row of tile slot i (null when the slot is unused)
__device__ __forceinline__ const uint8_t* x3_slot_row(const FwdArgs& a, int row0, int nrows, int i)
{
  return i < nrows ? a.x3 + (long long)a.row_token[row0 + i] * a.x3_row_bytes : nullptr;
}
// Whether X3 row `row` has a third term in super-chunk c (codes and scales are written only then)
__device__ __forceinline__ bool x3_row_flag(const FwdArgs& a, const uint8_t* row, int c)
{
  return row && row[(long long)at_nchunks(a.K) * 528 + c] != 0;
}

// The third-term operand of lane (i, g) for MFMA q of super-chunk c in the one-tile block order
// (MFMA q's logical block lb is block 4 lb + q): bytes 0-15 from block 4 (g / 2) + q, bytes 16-31
// from block 8 + 4 (g / 2) + q, elements 16 (g % 2) .. of each; `row` is the X3 row.
__device__ __forceinline__ i32x8 x3_operand(const uint8_t* row, int c, int q, int g)
{
  const uint8_t* p = row + c * 512 + (g >> 1) * 128 + q * 32 + (g & 1) * 16;
  return cat8_ld(p, p + 256);
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

// Zero every weight block whose scale byte is >= 253 and give it scale 2^0. Branch-free, so
// the block (and the compiler's placement of loads and waits) stays in one piece.
__device__ __forceinline__ void sanitize(i32x4 (&b)[4][4], uint32_t (&s)[4])
{
#pragma unroll
  for (int grp = 0; grp < 4; ++grp)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bool dead = ((s[grp] >> (8 * q)) & 0xFFu) >= 253u;
      b[grp][q] = dead ? i32x4{0, 0, 0, 0} : b[grp][q];
      s[grp] = dead ? (s[grp] & ~(0xFFu << (8 * q))) | (127u << (8 * q)) : s[grp];
    }
}

// The fast path's version: such scale bytes do not occur in checkpoints written by a
// quantiser, so the masking above runs only when some lane of the wave has one (a uniform
// branch); the test is three operations per scale dword.
__device__ __forceinline__ void sanitize_if_damaged(i32x4 (&b)[4][4], uint32_t (&s)[4])
{
  const uint32_t d = damaged_scale_bits(s[0]) | damaged_scale_bits(s[1]) | damaged_scale_bits(s[2]) |
                     damaged_scale_bits(s[3]);
  if (__builtin_amdgcn_ballot_w64(d != 0u) != 0) sanitize(b, s);
}



// Where lane (i = lane % 16, g = lane / 16) of a one-tile work-group finds its A: piece u
// (= (q * 2 + plane) * 2 + piece) of super-chunk c at base + c * kC + u * kU, its scale dwords
// (plane 0, plane 1) at sbase + c * kC and + kS. AT: the tile's block. XT (the routed gate/up
// product): the row of the slot's token (the all-zero row for unused slots), whose pieces sit
// 64 bytes apart. Grouped work-groups read AT tiles: they re-read A for every column tile, and
// 1 KiB runs from one tile serve that better than 64-byte runs from 16 rows.
template <bool XT>
struct ASrc {
  static constexpr int kC = XT ? kXtChunkBytes : kAtChunkBytes;
  static constexpr int kU = XT ? 64 : 1024;
  static constexpr int kS = XT ? 16 : 4;
  const uint8_t* base;   // the lane's piece 0 of super-chunk 0
  const uint8_t* sbase;  // the lane's plane-0 scale dword of super-chunk 0

  __device__ __forceinline__ ASrc(const FwdArgs& a, const WorkItem& w, int lane)
  {
    if constexpr (XT) {
      const int i = lane & 15, g = lane >> 4;
      const int tok = i < w.nrows ? a.row_token[w.row0 + i] : a.a_zero_row;
      const uint8_t* row = a.a_rows + (long long)tok * a.a_row_bytes;
      base = row + g * 16;
      sbase = row + kXtCodeBytes + g * 4;
    } else {
      const uint8_t* t = a.a_tiles + (long long)w.tile * at_tile_bytes(a.K);
      base = t + lane * 16;
      sbase = t + kAtCodeBytes + lane * 8;
    }
  }
  __device__ __forceinline__ const uint8_t* unit(int c, int u) const { return base + (long long)c * kC + u * kU; }
  __device__ __forceinline__ uint2 scales(int c) const
  {
    const uint8_t* p = sbase + (long long)c * kC;
    if constexpr (XT)
      return uint2{*reinterpret_cast<const uint32_t*>(p), *reinterpret_cast<const uint32_t*>(p + kS)};
    else
      return *reinterpret_cast<const uint2*>(p);
  }
};

// Epilogue of the fast path. The waves stage the work-group's outputs in the (now idle)
// activation buffers of LDS, then write them with 16-byte stores that cover whole runs of
// memory: scattered 1-byte and 4-byte stores of the same data cost the weight stream about a
// tenth of its bandwidth. The stores are non-temporal (streamed past the caches), which costs the
// weight stream less than ordinary write-back stores. Lane (j, g) holds rows 4g+v (v = 0..3) of columns grp*16 + j.
constexpr int kStagePitch = 260;  // floats per staged row: 256 + 4 keeps the row starts on distinct banks

template <int MODE, int NW = kWavesPerGroup>
__device__ __forceinline__ void epilogue_staged(const FwdArgs& a, const WorkItem& w, int wave, int lane,
                                                const f32x4 (&acc)[4], const float (&tw)[4], FwdLds& lds)
{
  const int j = lane & 15, g = lane >> 4;
  const int t = wave * 64 + lane;
  if (MODE == kFwdGateUp) {
    // Each group of four waves (half h of an eight-wave work-group) stages 128 features:
    // act codes [q = wave % 4][plane][half][row 0..15][16 B] then scales [row][plane][q], the AT
    // byte order of those features (super-chunk c, block group gl), and gate|up fp32 rows
    // [row][gate 128 | up 128]; half 1 (eight waves, forward layout) stages its rows in the
    // scale-window LDS, which the forward layout leaves unused.
    static_assert(NW == 4 || NW == 8, "four or eight waves");
    const int h = NW == 8 ? wave >> 2 : 0, wq = wave & 3;
    uint8_t* sq = lds.a[0] + h * 4608;
    float* ss = reinterpret_cast<float*>(h == 0 ? lds.a[1] : lds.s[0]);
    const int F = a.R;
    // LoRA gate/up delta of each row's token: the four rows' token indices, then their sixteen
    // delta values, each requested together (two round trips to memory rather than eight)
    float dl[4][4] = {};
    if (a.lora_delta && w.active) {
      int tok[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) tok[v] = 4 * g + v < w.nrows ? a.row_token[w.row0 + 4 * g + v] : -1;
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (tok[v] >= 0) {
          const float* d = a.lora_delta + (long long)tok[v] * 2 * F + w.ct * 32 + j;
          dl[v][0] = d[0];
          dl[v][1] = d[16];
          dl[v][2] = d[F];
          dl[v][3] = d[F + 16];
        }
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int i = 4 * g + v;
      float ga = acc[0][v], gb = acc[1][v], ua = acc[2][v], ub = acc[3][v];
      if (a.lora_delta) {
        ga += dl[v][0];
        gb += dl[v][1];
        ua += dl[v][2];
        ub += dl[v][3];
      }
      Quant2 q = quant2_block16(glu_fwd(ga, ua, a.act_kind), glu_fwd(gb, ub, a.act_kind));
      if (!w.active) q = Quant2{0, 0, 0, 0};  // features past F: the padding of the layout is zero
      sq[((wq * 2 + 0) * 2 + 0) * 256 + i * 16 + j] = (uint8_t)q.hi;
      sq[((wq * 2 + 0) * 2 + 1) * 256 + i * 16 + j] = (uint8_t)(q.hi >> 8);
      sq[((wq * 2 + 1) * 2 + 0) * 256 + i * 16 + j] = (uint8_t)q.lo;
      sq[((wq * 2 + 1) * 2 + 1) * 256 + i * 16 + j] = (uint8_t)(q.lo >> 8);
      if (j == 0) {
        sq[4096 + i * 8 + wq] = (uint8_t)q.s_hi;
        sq[4096 + i * 8 + 4 + wq] = (uint8_t)q.s_lo;
      }
      if (a.save) {
        float* r = ss + i * kStagePitch + wq * 32 + j;
        r[0] = ga;
        r[16] = gb;
        r[128] = ua;
        r[144] = ub;
      }
    }
    __syncthreads();
    const int f_wg = w.ct0 * 32 + 128 * h;  // first feature of the half, a multiple of 128
    const int c = f_wg >> 9, gl = (f_wg >> 7) & 3;
    uint8_t* qbase = a.q_tiles + (long long)w.tile * at_tile_bytes(F) + (long long)c * kAtChunkBytes;
    {
      const int th = wq * 64 + lane;  // thread of the half
      const int run = th >> 5, off = (th & 31) * 16;  // run = q * 2 + plane: 512 B each
      __builtin_nontemporal_store(*reinterpret_cast<const i32x4*>(sq + run * 512 + off),
                                  reinterpret_cast<i32x4*>(qbase + (run * 2 + (gl >> 1)) * 1024 + (gl & 1) * 512 + off));
      if (th < 8)
        *reinterpret_cast<i32x4*>(qbase + kAtCodeBytes + gl * 128 + th * 16) =
            *reinterpret_cast<const i32x4*>(sq + 4096 + th * 16);
    }
    if (a.save) {
      const int part = lane >> 5, idx = (lane & 31) * 4, f = f_wg + idx;
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int r = it * 4 + wq;
        if (r < w.nrows && f < F)
          __builtin_nontemporal_store(*reinterpret_cast<const f32x4*>(ss + r * kStagePitch + part * 128 + idx),
                                      reinterpret_cast<f32x4*>(a.save + (long long)(w.row0 + r) * 2 * F + part * F + f));
      }
    }
    return;
  }

  // kFwdPlain / kFwdDown: [row][64 NW columns of the work-group] fp32
  constexpr int kPitch = NW * 64 + 4;
  static_assert(16 * kPitch * 4 <= (int)sizeof(lds.a), "the staged rows fit the activation buffers");
  float* ss = reinterpret_cast<float*>(lds.a[0]);
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const float wv = MODE == kFwdDown ? tw[v] : 1.0f;
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) ss[(4 * g + v) * kPitch + wave * 64 + grp * 16 + j] = acc[grp][v] * wv;
  }
  __syncthreads();
  const bool vec = ((a.ldy & 3) == 0) && ((reinterpret_cast<uintptr_t>(a.y) & 15) == 0);
#pragma unroll
  for (int it = 0; it < 16 / NW; ++it) {
    const int r = it * NW + wave;
    if (r >= w.nrows) continue;
    const int orow = a.y_rows ? a.y_rows[w.row0 + r] : w.row0 + r;
    float* yr = a.y + (long long)orow * a.ldy;
#pragma unroll
    for (int h = 0; h < NW / 4; ++h) {
      const int col = w.ct0 * kFwdColsPerTile + h * 256 + lane * 4;
      const f32x4 val = *reinterpret_cast<const f32x4*>(ss + r * kPitch + h * 256 + lane * 4);
      if (vec && col + 4 <= a.R) {
        __builtin_nontemporal_store(val, reinterpret_cast<f32x4*>(yr + col));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (col + e < a.R) yr[col + e] = val[e];
      }
    }
  }
}

// Epilogue straight from the accumulators (one wave, no LDS): lane (j, g) holds rows 4g+v
// (v = 0..3) of columns grp*16 + j.
template <int MODE>
__device__ __forceinline__ void epilogue_direct(const FwdArgs& a, const WorkItem& w, int lane, const f32x4 (&acc)[4],
                                                const float (&tw)[4])
{
  const int j = lane & 15, g = lane >> 4;
  if (MODE == kFwdGateUp) {
    // rows 4g+v: gate features j and 16+j (groups 0, 1), up features the same (groups 2, 3)
    const int F = a.R;
    const int f0 = w.ct * 32;
    uint8_t* qt = a.q_tiles + (long long)w.tile * at_tile_bytes(F);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int i = 4 * g + v;
      float ga = acc[0][v], gb = acc[1][v], ua = acc[2][v], ub = acc[3][v];
      if (a.lora_delta && i < w.nrows) {  // LoRA gate/up delta of the row's token
        const float* dl = a.lora_delta + (long long)a.row_token[w.row0 + i] * 2 * F + f0 + j;
        ga += dl[0];
        gb += dl[16];
        ua += dl[F];
        ub += dl[F + 16];
      }
      const float a0 = glu_fwd(ga, ua, a.act_kind), a1 = glu_fwd(gb, ub, a.act_kind);
      if (a.save && i < w.nrows) {
        float* sv = a.save + (long long)(w.row0 + i) * 2 * F;
        sv[f0 + j] = ga;
        sv[f0 + 16 + j] = gb;
        sv[F + f0 + j] = ua;
        sv[F + f0 + 16 + j] = ub;
      }
      // act -> the down product's A operand (AT layout, same tile). Unused row slots carry
      // zeros (their inputs were zero), which is what the layout expects.
      const Quant2 q = quant2_block16(a0, a1);  // the 16 lanes of row i hold its 32 features
      qt[at_code_off(i, f0 + j, 0)] = (uint8_t)q.hi;
      qt[at_code_off(i, f0 + 16 + j, 0)] = (uint8_t)(q.hi >> 8);
      qt[at_code_off(i, f0 + j, 1)] = (uint8_t)q.lo;
      qt[at_code_off(i, f0 + 16 + j, 1)] = (uint8_t)(q.lo >> 8);
      if (j == 0) {
        qt[at_scale_off(i, f0, 0)] = (uint8_t)q.s_hi;
        qt[at_scale_off(i, f0, 1)] = (uint8_t)q.s_lo;
      }
    }
    return;
  }

#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int i = 4 * g + v;
    if (i >= w.nrows) continue;
    const int row = w.row0 + i;
    const float wv = MODE == kFwdDown ? tw[v] : 1.0f;
    float* yr = a.y + (long long)(a.y_rows ? a.y_rows[row] : row) * a.ldy;
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      const int col = w.ct * kFwdColsPerTile + grp * 16 + j;
      if (col < a.R) yr[col] = acc[grp][v] * wv;
    }
  }
}


// One work item: the 16 x 64 tile (w.tile, w.ct) over all of K, then its epilogue.
// FL: the weights come from the forward layout (fl0 / fl1), one 1 KiB block per load instruction
// NW waves per work-group (column tiles per item): 4, or 8 for the routed products from the
// forward layout, whose work-groups then hold a CU alone and copy each tile's activations once
// per 8 column tiles instead of once per 4. lds: the work-group's copies and staging (fast path).
template <int MODE, bool FAST, bool FL, int NW = kWavesPerGroup>
__device__ __forceinline__ void fwd_item(const FwdArgs& a, const WorkItem& w, int wave, int lane, FwdLds& lds)
{
  static_assert(NW == kWavesPerGroup || (FL && MODE != kFwdPlain), "eight waves: the routed products' forward layout path");
  static_assert(FAST || !FL, "the forward layout is read by the fast path only");
  const int j = lane & 15, g = lane >> 4;
  const int nb = a.K / kGroup;
  const int nsc = at_nchunks(a.K);
  constexpr bool kXt = MODE == kFwdGateUp;
  const ASrc<kXt> as(a, w, lane);

  // first weight row of column group grp, and that group's packed / scale bases
  auto grp_row = [&](int grp) {
    return MODE == kFwdGateUp ? w.ct * 32 + (grp & 1) * 16 : w.ct * kFwdColsPerTile + grp * 16;
  };
  auto grp_wp = [&](int grp) {
    return (MODE == kFwdGateUp && grp >= 2 ? a.wp1 : a.wp0) + (long long)w.expert * a.wp_estride;
  };
  auto grp_ws = [&](int grp) {
    return (MODE == kFwdGateUp && grp >= 2 ? a.ws1 : a.ws0) + (long long)w.expert * a.ws_estride;
  };

  // weight row n of group grp at wrow[grp] (uniform) + boff[grp] (this lane's 32-bit offset)
  const uint8_t* wrow[4];
  uint32_t boff[4];
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    const int rb = min(grp_row(grp), a.R - 1);  // rows past the end repeat the last row
    wrow[grp] = grp_wp(grp) + (long long)rb * (a.K / 2);
    boff[grp] = (uint32_t)(min(j, a.R - 1 - rb) * (a.K / 2) + g * 64);
  }

  f32x4 acc[4];
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) acc[grp] = f32x4{0.f, 0.f, 0.f, 0.f};
  float tw[4];  // kFwdDown: combine weights of this lane's output rows, requested with the first loads

  // gate/up: the third term of x where the tile's rows have one (super-chunks of m3, rare); its
  // operands come straight from the X3 rows of the slots' tokens
  // The flag loads are issued here and reduced at the first chunk, after the pipeline's first
  // loads: their latency hides behind those.
  uint32_t m3 = 0;
  uint2 f3 = uint2{0u, 0u};
  const bool use3 = MODE == kFwdGateUp && a.x3 != nullptr && *(cint_ptr)a.x3_any != 0;
  if (use3) f3 = x3_flags(a, x3_slot_row(a, w.row0, w.nrows, j), lane);
  auto third_term = [&](int c, const i32x4 (&b)[4][4], const uint32_t (&sb)[4]) {
    int l = lane;  // lane-derived values recomputed here: nothing of this stays live across the loop
    asm volatile("" : "+v"(l));
    const uint8_t* row = x3_slot_row(a, w.row0, w.nrows, l & 15);
    const bool mine = x3_row_flag(a, row, c);  // this lane's row has a third term in chunk c
    const uint32_t s3 = mine ? *reinterpret_cast<const uint32_t*>(row + (long long)nsc * 512 + c * 16 + 4 * g) : 0x7F7F7F7Fu;
    static_for<4>([&](auto qc) {
      constexpr int q = decltype(qc)::value;
      const i32x8 a3 = mine ? x3_operand(row, c, q, g) : i32x8{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int grp = 0; grp < 4; ++grp) acc[grp] = mfma_f8f4<q, q>(a3, b[grp][q], acc[grp], (int)s3, (int)sb[grp]);
    });
  };

  auto load_b = [&](int c, i32x4 (&b)[4][4]) {
#pragma unroll
    for (int grp = 0; grp < 4; ++grp)
#pragma unroll
      for (int q = 0; q < 4; ++q) b[grp][q] = ldg16(wrow[grp] + c * 256 + boff[grp] + 16 * q);
  };

  if constexpr (FAST) {
    uint8_t* const sw = lds.s[wave];

    // A(c) -> lds.a[buf]: wave w copies KiB units 4w..4w+3 of the codes (lane l's 16 bytes of
    // unit u at u * 1024 + 16 l); wave 0 also copies the scales: AT, the tile's 512 B as they
    // lie (lane l's two dwords at 8 l; its upper 32 lanes repeat them into the spare half KiB),
    // XT, the lanes' plane-0 dwords at 4 l and plane-1 dwords at 256 + 4 l
    auto issue_a = [&](int c, int buf) {
#pragma unroll
      for (int u = 0; u < 16 / NW; ++u) {
        const int unit = (16 / NW) * wave + u;
        dma16_async(as.unit(c, unit), &lds.a[buf][unit * 1024]);
      }
      if (wave == 0) {
        if constexpr (kXt) {
          const uint8_t* ss = as.sbase + (long long)c * as.kC;
          dma4_async(ss, &lds.a[buf][kAtCodeBytes]);
          dma4_async(ss + as.kS, &lds.a[buf][kAtCodeBytes + 256]);
        } else {
          dma16_async(as.unit(c, 0) - lane * 16 + kAtCodeBytes + (lane & 31) * 16, &lds.a[buf][kAtCodeBytes]);
        }
      }
    };
    // scale window win -> sw: instruction i covers rows 8i..8i+7 of this wave's 64, lane l
    // copies 16 B (one super-chunk) of row 8i + l/8 into slot l%8 of that row; the slot holds
    // chunk 8 win + ((l%8) ^ (row & 7)) (clamped to the row), so the 16 rows read together
    // below spread over all 32 banks instead of sharing one (addresses are rebuilt at each call
    // from uniform bases and 32-bit lane offsets rather than held in registers across the
    // steps in between)
    auto issue_scales = [&](int win) {
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const int cc = min(win * kScaleWin + ((ln & 7) ^ (ln >> 3)), nsc - 1);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int grp = i >> 1;
        const uint32_t off = (uint32_t)(min(grp_row(grp) + 8 * (i & 1) + (ln >> 3), a.R - 1) * nb + cc * 16);
        dma16_async(grp_ws(grp) + off, sw + i * 1024);
      }
    };
    // weights of chunk c through one buffer resource per column group: a fixed per-lane offset
    // + 256 c (uniform) + 16 q (immediate). A chunk past the last is requested from an empty
    // resource: zeros, no memory traffic, and the same count of loads in vmcnt.
    // Forward layout: the column group's 16 rows are row group rg, whose chunk c is the 4 KiB at
    // (rg * nsc + c) * 4096 and holds MFMA q's operand at q * 1024, lane l's 16 B at l * 16: the
    // same bytes, each load instruction one contiguous 1 KiB.
    rsrc_t wr[4], wr_none[4];
    rsrc_t sr[4];  // forward layout: the row group's weight-scale blocks
    uint32_t woff[4];
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      if constexpr (FL) {
        // the resource starts at the row group, so the lane offset is the same for all four
        const int rg = min(grp_row(grp), a.R - 1) / 16;
        const int nrg = (a.R + 15) / 16;
        const uint8_t* ebase = (MODE == kFwdGateUp && grp >= 2 ? a.fl1 : a.fl0) + (long long)w.expert * a.fl_estride;
        const uint8_t* base = ebase + (long long)rg * nsc * 4096;
        wr[grp] = make_rsrc(base, (uint32_t)(nrg - rg) * (uint32_t)nsc * 4096u);
        wr_none[grp] = make_rsrc(base, 0);
        woff[grp] = (uint32_t)lane * 16u;
        sr[grp] = make_rsrc(ebase + (long long)nrg * nsc * 4096 + (long long)rg * nsc * 256,
                            (uint32_t)(nrg - rg) * (uint32_t)nsc * 256u);
      } else {
        const uint8_t* base = grp_wp(grp);
        wr[grp] = make_rsrc(base, (uint32_t)a.R * (uint32_t)(a.K / 2));
        wr_none[grp] = make_rsrc(base, 0);
        woff[grp] = (uint32_t)(wrow[grp] - base) + boff[grp];
      }
    }
    // forward layout: with a chunk's weights, the lanes' scale dwords of it (block (rg, c) holds
    // lane l's dword at 4 l, one whole 256 B per instruction); a chunk past the last reads nothing
    auto load_b_buf = [&](int c, i32x4 (&b)[4][4], uint32_t (&sbuf)[4]) {
      const bool live = c < nsc;  // uniform
#pragma unroll
      for (int grp = 0; grp < 4; ++grp)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if constexpr (FL)  // each line read once, whole, by one instruction: streaming hint
            b[grp][q] = buf16_nt(live ? wr[grp] : wr_none[grp], woff[grp] + 1024 * q, (uint32_t)c * 4096);
          else
            b[grp][q] = buf16(live ? wr[grp] : wr_none[grp], woff[grp] + 16 * q, (uint32_t)c * 256);
        }
      if constexpr (FL) {
#pragma unroll
        for (int grp = 0; grp < 4; ++grp)
          sbuf[grp] = buf4_nt(live ? sr[grp] : wr_none[grp], (uint32_t)lane * 4u, (uint32_t)c * 256);
      }
    };
    constexpr int kChunkLoads = FL ? 20 : 16;  // vector loads per chunk of weights (and FL scales)

    // Two chunks of weights in flight: a buffer is refilled with chunk c + 2 as soon as chunk
    // c's MFMAs have read it, and chunk c + 1's loads are in flight meanwhile. The activation
    // copy and scale window of chunk c are requested at the top of chunk c - 1, before the 16
    // weight loads of chunk c + 1 (issued at the end of chunk c - 1), so at the top of chunk c
    // everything but those 16 has landed. The copies are issued from
    // inline assembly: a copy the compiler knows of makes it drain every load at each barrier.
    auto step = [&](int c, i32x4 (&cur)[4][4], uint32_t (&cur_s)[4]) {
      wait_vm<kChunkLoads>();
      __syncthreads();
      // everything this chunk needs from LDS, before any new copy into LDS is requested
      uint32_t sb[4];
#pragma unroll
      for (int grp = 0; grp < 4; ++grp) {
        if constexpr (FL) {
          sb[grp] = cur_s[grp];
        } else {
          sb[grp] = *reinterpret_cast<const uint32_t*>(sw + (grp * 16 + j) * kScaleRowBytes +
                                                       (((c % kScaleWin) ^ (j & 7)) * 16) + g * 4);
        }
      }
      const uint8_t* la = &lds.a[c & 1][lane * 16];
      i32x8 ah[4], al[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        ah[q] = cat8(*reinterpret_cast<const i32x4*>(la + q * 4096), *reinterpret_cast<const i32x4*>(la + q * 4096 + 1024));
        al[q] = cat8(*reinterpret_cast<const i32x4*>(la + q * 4096 + 2048), *reinterpret_cast<const i32x4*>(la + q * 4096 + 3072));
      }
      const uint8_t* ls = &lds.a[c & 1][kAtCodeBytes];
      const uint2 s2 = kXt ? uint2{*reinterpret_cast<const uint32_t*>(ls + lane * 4),
                                  *reinterpret_cast<const uint32_t*>(ls + 256 + lane * 4)}
                          : *reinterpret_cast<const uint2*>(ls + lane * 8);
      wait_lgkm0();
      // chunk c's weights are complete (wait_vm above)
#pragma unroll
      for (int grp = 0; grp < 4; ++grp) {
#pragma unroll
        for (int q = 0; q < 4; ++q) pin(cur[grp][q]);
        if constexpr (FL) pin(sb[grp]);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (c + 1 < nsc) {
        issue_a(c + 1, (c + 1) & 1);
        if (!FL && (c + 1) % kScaleWin == 0) issue_scales((c + 1) / kScaleWin);
      }
      __builtin_amdgcn_sched_barrier(0);
      sanitize_if_damaged(cur, sb);
      mfma_step<0>(acc, ah[0], al[0], cur, sb, (int)s2.x, (int)s2.y);
      mfma_step<1>(acc, ah[1], al[1], cur, sb, (int)s2.x, (int)s2.y);
      mfma_step<2>(acc, ah[2], al[2], cur, sb, (int)s2.x, (int)s2.y);
      mfma_step<3>(acc, ah[3], al[3], cur, sb, (int)s2.x, (int)s2.y);
      __builtin_amdgcn_sched_barrier(0);
      load_b_buf(c + 2, cur, cur_s);
    };

    if (MODE == kFwdDown)
#pragma unroll
      for (int v = 0; v < 4; ++v) tw[v] = a.row_w[w.row0 + min(4 * g + v, w.nrows - 1)];
    i32x4 b0[4][4], b1[4][4];
    uint32_t s0[4], s1[4];
    load_b_buf(0, b0, s0);
    if (!FL) issue_scales(0);
    issue_a(0, 0);
    load_b_buf(1, b1, s1);
    // the flag loads were issued before the first chunk's loads, which the first step waits for
    if (use3) m3 = x3_mask(f3, lane);
    for (int c = 0;;) {
      step(c, b0, s0);
      if (++c >= nsc) break;
      step(c, b1, s1);
      if (++c >= nsc) break;
    }
    wait_vm0();  // (no copy is in flight past the last chunk; kept explicit for the epilogue)
    // gate/up: the third term of the flagged super-chunks (rare), after the pipelined loop so that
    // it adds nothing to the loop's registers; their weights are loaded again (checkpoint layout)
    for (uint32_t mm = m3 & (nsc >= kX3Flags ? ~0u : ((1u << nsc) - 1u)); mm; mm &= mm - 1) {
      const int c = __builtin_ctz(mm);
      int l = lane;  // addresses rebuilt from the lane: nothing of this stays live across the loop
      asm volatile("" : "+v"(l));
      i32x4 b[4][4];
      uint32_t sb[4];
#pragma unroll
      for (int grp = 0; grp < 4; ++grp) {
        const long long n = min(grp_row(grp) + (l & 15), a.R - 1);
        sb[grp] = *reinterpret_cast<const uint32_t*>(grp_ws(grp) + n * nb + c * 16 + (l >> 4) * 4);
        const uint8_t* wr0 = grp_wp(grp) + n * (a.K / 2) + c * 256 + (l >> 4) * 64;
#pragma unroll
        for (int q = 0; q < 4; ++q) b[grp][q] = ldg16(wr0 + 16 * q);
      }
      sanitize(b, sb);
      third_term(c, b, sb);
    }
  } else {
    if (MODE == kFwdDown)
#pragma unroll
      for (int v = 0; v < 4; ++v) tw[v] = a.row_w[w.row0 + min(4 * g + v, w.nrows - 1)];
    // any K (a multiple of 32): straight loads, blocks past the end of the row load nothing
    // and carry a zero operand with scale 2^0 (their activations are zero too)
    const uint8_t* bs[4];
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      const int n = min(grp_row(grp) + j, a.R - 1);
      bs[grp] = grp_ws(grp) + (long long)n * nb + g * 4;
    }
    for (int c = 0; c < nsc; ++c) {
      i32x4 b[4][4];
      uint32_t sb[4];
#pragma unroll
      for (int grp = 0; grp < 4; ++grp) {
        sb[grp] = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int blk = c * kChunkBlocks + g * 4 + q;
          if (blk < nb) {
            b[grp][q] = ldg16(wrow[grp] + c * 256 + boff[grp] + 16 * q);
            sb[grp] |= (uint32_t)bs[grp][c * 16 + q] << (8 * q);
          } else {
            b[grp][q] = i32x4{0, 0, 0, 0};
            sb[grp] |= 127u << (8 * q);
          }
        }
      }
      i32x8 ah[4], al[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        ah[q] = cat8(ldg16(as.unit(c, 4 * q)), ldg16(as.unit(c, 4 * q + 1)));
        al[q] = cat8(ldg16(as.unit(c, 4 * q + 2)), ldg16(as.unit(c, 4 * q + 3)));
      }
      const uint2 s2 = as.scales(c);
      sanitize(b, sb);
      mfma_step<0>(acc, ah[0], al[0], b, sb, (int)s2.x, (int)s2.y);
      mfma_step<1>(acc, ah[1], al[1], b, sb, (int)s2.x, (int)s2.y);
      mfma_step<2>(acc, ah[2], al[2], b, sb, (int)s2.x, (int)s2.y);
      mfma_step<3>(acc, ah[3], al[3], b, sb, (int)s2.x, (int)s2.y);
      if (use3 && c == 0) m3 = x3_mask(f3, lane);
      if (c < kX3Flags && ((m3 >> c) & 1u)) third_term(c, b, sb);  // uniform
    }
  }

  if constexpr (FAST) {
    __syncthreads();  // every wave is done with the last chunk's LDS data
    epilogue_staged<MODE, NW>(a, w, wave, lane, acc, tw, lds);
    return;
  }

  if (w.active) epilogue_direct<MODE>(a, w, lane, acc, tw);
}

template <int MODE, bool FAST, bool FL, int NW = kWavesPerGroup>
__global__ __launch_bounds__(64 * NW, NW == kWavesPerGroup ? 2 : 1) void fwd_kernel(FwdArgs a)
{
  __shared__ FwdLds lds;  // used by the fast path only
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keeps control flow scalar
  WorkItem w;
  for (int it = 0; decode_work(a.tiles, a.n_tiles, a.small_tiles, a.n_small, a.n_groups, a.M, a.n_ct, wave, it, w, NW); ++it) {
    // the previous item's reads of LDS are complete before this item's copies land there;
    // its output stores drain while this item's first loads are in flight
    if (FAST && it > 0) __syncthreads();
    // recompute lane-derived addresses per item instead of holding them across items
    int l = lane;
    asm volatile("" : "+v"(l));
    fwd_item<MODE, FAST, FL, NW>(a, w, wave, l, lds);
  }
}

// ---------------------------------------------------------------- large buckets
// An expert with many rows would re-read each weight byte once per 16-row tile. Its tiles come
// in groups of up to kGroupTiles (4). A work item is one group (up to 64 rows) x eight column
// tiles (wave w takes column tile 8 fb + w: 512 weight rows in all); a work-group of eight waves
// holds the CU's LDS alone. Both operands go through LDS one K-quarter (one MFMA's 128 K) at a
// time: per quarter the work-group copies the 16 KiB of activations of its four tiles and the
// 32 KiB of weight codes of its 512 rows, three quarters deep (the one being read and two in
// flight), and each wave issues 4 tiles x 4 column groups x 2 terms = 32 MFMAs against them.
// Every weight byte is read once per group and every activation byte once per 512 weight rows.
//
// Block order: MFMA q of super-chunk c takes blocks 16c + 4q .. 16c + 4q + 3 (lane group g takes
// block 4q + g), not the one-tile kernels' 16c + 4g + q. The quarter's weight bytes of a row are
// then one contiguous 64 B (half a cache line, whose other half the next quarter takes) instead
// of four 16 B pieces spread over two lines, each line requested again by all four quarters.
// The activations keep the AT layout: a quarter's operand is gathered from it in 256 B runs
// (every run fetched once per item), and the scale bytes of blocks 4q + g, q = 0..3, are packed
// into one register per lane at the first quarter of each super-chunk.
constexpr int kGmT = 4;                        // row tiles per item
constexpr int kGmWaves = 8;                    // column tiles per item
constexpr int kGmRows = kGmWaves * 64;         // weight rows per item
constexpr int kGmA = kGmT * 4096;              // A bytes per quarter: [tile][plane][piece][lane][16 B]
constexpr int kGmW = kGmRows * 64;             // W bytes per quarter: [row][block][16 B]
constexpr int kGmRing = 3;                     // quarters in LDS: the one read and two in flight
static_assert(kGmT >= kGroupTiles, "an item holds a whole group");
struct GemmLds {
  uint8_t q[kGmRing][kGmA + kGmW];             // quarter buffers
  uint8_t sw[kGmRows * 16];                    // weight scales of a super-chunk: [row][16 B]
  uint8_t sa[kGmT * 512];                      // activation scales of a super-chunk: [tile][512 B]
};

// FL: weight codes from the forward layout (fl0 / fl1): the same bytes land in the same LDS
// places, each copy instruction reading four 256-byte runs instead of 16 rows' 64-byte runs
template <int MODE, bool FL>
__device__ __forceinline__ void fwd_gemm_item(const FwdArgs& a, int expert, int t0, int ntl, int fb, int wave,
                                              int lane, GemmLds& lds)
{
  constexpr int T = kGmT;
  const int g = lane >> 4;
  const int nb = a.K / kGroup;
  const int nsc = at_nchunks(a.K);

  WorkItem w[T];  // slots past the group's end repeat its last tile and are not stored
#pragma unroll
  for (int tt = 0; tt < T; ++tt) {
    w[tt].tile = t0 + min(tt, ntl - 1);
    const cint_ptr tl = (cint_ptr)(a.tiles + w[tt].tile);
    w[tt].expert = expert;
    w[tt].row0 = tl[1];
    w[tt].nrows = tl[2];
    w[tt].ct0 = fb * kGmWaves;
    const int ct = fb * kGmWaves + wave;
    w[tt].active = ct < a.n_ct;
    w[tt].ct = w[tt].active ? ct : a.n_ct - 1;
  }

  // weight row n of item row r (0..511): wave r / 64's column tile, column group cg = (r / 16) % 4
  // (gate/up: groups 2, 3 are W3's rows); bases of the group's matrix
  auto w_n = [&](int r) {
    const int ct = min(fb * kGmWaves + (r >> 6), a.n_ct - 1), cg = (r >> 4) & 3, i = r & 15;
    return MODE == kFwdGateUp ? min(ct * 32 + (cg & 1) * 16 + i, a.R - 1) : min(ct * kFwdColsPerTile + cg * 16 + i, a.R - 1);
  };
  auto w_base = [&](int cg) {
    return (MODE == kFwdGateUp && cg >= 2 ? a.wp1 : a.wp0) + (long long)expert * a.wp_estride;
  };
  auto s_base = [&](int cg) {
    return (MODE == kFwdGateUp && cg >= 2 ? a.ws1 : a.ws0) + (long long)expert * a.ws_estride;
  };
  // the copies of quarter q of super-chunk c into buffer buf, six per wave: blocks 4q .. 4q + 3
  // of rows 64 wave .. + 63 of W (four instructions of 16 rows x 64 B) and the KiB units
  // (plane wave % 2, pieces 0, 1) of tile wave / 2's operand, each gathered from four 256 B runs
  // of the AT layout; at q = 0 also the super-chunk's weight scales of its 64 rows and half
  // (wave % 2) of tile wave / 2's 512 B of activation scales
  auto issue = [&](int c, int q, int buf) {
    int l = lane;
    asm volatile("" : "+v"(l));
#pragma unroll
    for (int k = 0; k < 4; ++k) {  // instruction k: column group k of this wave's tile
      const int r = wave * 64 + k * 16 + (l >> 2), b = l & 3;
      if constexpr (FL) {
        // row l / 4 of the group's 16 (row group rg of the layout), block 4q + b: piece b of its
        // super-chunk c, lane 16 q + l / 4
        const int ct = min(fb * kGmWaves + wave, a.n_ct - 1);
        const int row0 = MODE == kFwdGateUp ? ct * 32 + (k & 1) * 16 : ct * kFwdColsPerTile + k * 16;
        const uint32_t rg = (uint32_t)(min(row0, a.R - 1) / 16);
        const uint8_t* base = (MODE == kFwdGateUp && k >= 2 ? a.fl1 : a.fl0) + (long long)expert * a.fl_estride;
        dma16_async_s_nt(base, (rg * (uint32_t)nsc + (uint32_t)c) * 4096u + (uint32_t)(b * 1024 + (16 * q + (l >> 2)) * 16),
                         &lds.q[buf][kGmA + (wave * 64 + k * 16) * 64]);
      } else {
        dma16_async_s(w_base(k), (uint32_t)w_n(r) * (uint32_t)(a.K / 2) + (uint32_t)(c * 256 + (4 * q + b) * 16),
                      &lds.q[buf][kGmA + (wave * 64 + k * 16) * 64]);
      }
    }
    {
      const int tt = wave >> 1;
      const uint8_t* at = a.a_tiles + (long long)(t0 + min(tt, ntl - 1)) * at_tile_bytes(a.K) +
                          (long long)c * kAtChunkBytes;
      const int plane = wave & 1, g = l >> 4, i = l & 15;
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        // lane (i, g) of piece k holds block 4q + 2k + g / 2, elements 16 (g % 2) .. + 15, which
        // the AT layout keeps as logical block q of its MFMA 2k + g / 2: piece q / 2 of lane
        // 16 (2 (q % 2) + g % 2) + i
        const int src = ((((2 * k + (g >> 1)) * 2 + plane) * 2 + (q >> 1)) * 64 + 16 * (2 * (q & 1) + (g & 1)) + i) * 16;
        dma16_async_s(at, (uint32_t)src, &lds.q[buf][tt * 4096 + (2 * plane + k) * 1024]);
      }
    }
    if (q == 0) {  // two more copies: 8 in all
      const int r = wave * 64 + l;
      const uint8_t* ps = s_base((r >> 4) & 3) + (long long)w_n(r) * nb;
      dma16_async(ps + c * 16, &lds.sw[wave * 64 * 16]);
      const int tt = wave >> 1, h = wave & 1;
      const uint8_t* at = a.a_tiles + (long long)(t0 + min(tt, ntl - 1)) * at_tile_bytes(a.K) +
                          (long long)c * kAtChunkBytes + kAtCodeBytes + h * 256;
      dma4_async(at + l * 4, &lds.sa[tt * 512 + h * 256]);
    }
  };

  f32x4 acc[T][4];
#pragma unroll
  for (int tt = 0; tt < T; ++tt)
#pragma unroll
    for (int cg = 0; cg < 4; ++cg) acc[tt][cg] = f32x4{0.f, 0.f, 0.f, 0.f};
  float tw[T][4];
  if (MODE == kFwdDown)
#pragma unroll
    for (int tt = 0; tt < T; ++tt)
#pragma unroll
      for (int v = 0; v < 4; ++v) tw[tt][v] = a.row_w[w[tt].row0 + min(4 * g + v, w[tt].nrows - 1)];
  // gate/up: third-term masks of the tiles (bit c: super-chunk c, rare) and their union
  uint32_t m3[T], m3_any = 0;
  const bool use3 = MODE == kFwdGateUp && a.x3 != nullptr && *(cint_ptr)a.x3_any != 0;
#pragma unroll
  for (int tt = 0; tt < T; ++tt) {
    m3[tt] = 0;
    if (use3 && tt < ntl) {
      m3[tt] = x3_mask(x3_flags(a, x3_slot_row(a, w[tt].row0, w[tt].nrows, lane & 15), lane), lane);
      m3_any |= m3[tt];
    }
  }

  // One step per quarter s (super-chunk s / 4, MFMA q = s % 4): wait for its copies (the
  // next quarter's stay in flight), barrier, request quarter s + 2 into the buffer step s - 1
  // read, 32 MFMAs. At q = 0 the wave takes the super-chunk's scales into registers, which frees
  // their single LDS copy for the next super-chunk's, requested two steps later. The scale dwords
  // are shifted so that byte q is byte 0: the MFMAs' scale selectors stay constant and one copy
  // of the step serves all four quarters.
  const int ns = 4 * nsc;
  issue(0, 0, 0);
  if (ns > 1) issue(0, 1, 1);
  uint32_t rw[4], ra[T][2];
  for (int s = 0; s < ns; ++s) {
    const int c = s >> 2, q = s & 3;
    if (s + 1 >= ns) wait_vm0();
    else if (((s + 1) & 3) == 0) wait_vm<8>();
    else wait_vm<6>();
    __syncthreads();
    if (s + 2 < ns) issue((s + 2) >> 2, (s + 2) & 3, (s + 2) % kGmRing);
    __builtin_amdgcn_sched_barrier(0);
    // lane-derived LDS offsets are rebuilt here each step rather than held across the loop
    int l = lane;
    asm volatile("" : "+v"(l));
    const int jl = l & 15, gl = l >> 4;
    if (q == 0) {  // byte q of each register: the scale of block 4q + g (g = this lane's group)
      // byte g of x, y, z, w -> bytes 0..3: two byte permutes (selector 12 gives zero) and an or
      const uint32_t lo = 0x0C0C0000u | ((4u + gl) << 8) | (uint32_t)gl, hi = (lo << 16) | 0x0C0Cu;
      auto gather = [&](uint32_t x, uint32_t y, uint32_t z, uint32_t w) {
        return __builtin_amdgcn_perm(y, x, lo) | __builtin_amdgcn_perm(w, z, hi);
      };
#pragma unroll
      for (int cg = 0; cg < 4; ++cg) {
        const uint4 d = *reinterpret_cast<const uint4*>(&lds.sw[(wave * 64 + cg * 16 + jl) * 16]);
        rw[cg] = gather(d.x, d.y, d.z, d.w);
      }
#pragma unroll
      for (int tt = 0; tt < T; ++tt) {  // AT holds block 4qq + g's scales at lane 16qq + i, byte g
        uint2 s2[4];
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) s2[qq] = *reinterpret_cast<const uint2*>(&lds.sa[tt * 512 + (16 * qq + jl) * 8]);
        ra[tt][0] = gather(s2[0].x, s2[1].x, s2[2].x, s2[3].x);
        ra[tt][1] = gather(s2[0].y, s2[1].y, s2[2].y, s2[3].y);
      }
    }
    const uint8_t* lq = lds.q[s % kGmRing];
    uint32_t sb[4];
    i32x4 b[4];
#pragma unroll
    for (int cg = 0; cg < 4; ++cg) {
      const int r = wave * 64 + cg * 16 + jl;
      sb[cg] = rw[cg] >> (8 * q);
      b[cg] = *reinterpret_cast<const i32x4*>(lq + kGmA + (r * 4 + gl) * 16);
      const bool dead = (sb[cg] & 0xFFu) >= 253u;  // zero block, scale 2^0
      b[cg] = dead ? i32x4{0, 0, 0, 0} : b[cg];
      sb[cg] = dead ? 127u : sb[cg];
    }
#pragma unroll
    for (int tt = 0; tt < T; ++tt) {
      const uint8_t* pa = lq + tt * 4096 + l * 16;
      const i32x8 ah = cat8(*reinterpret_cast<const i32x4*>(pa), *reinterpret_cast<const i32x4*>(pa + 1024));
      const i32x8 al = cat8(*reinterpret_cast<const i32x4*>(pa + 2048), *reinterpret_cast<const i32x4*>(pa + 3072));
      const int sah = (int)(ra[tt][0] >> (8 * q)), sal = (int)(ra[tt][1] >> (8 * q));
#pragma unroll
      for (int cg = 0; cg < 4; ++cg) {
        acc[tt][cg] = mfma_f8f4<0, 0>(ah, b[cg], acc[tt][cg], sah, (int)sb[cg]);
        acc[tt][cg] = mfma_f8f4<0, 0>(al, b[cg], acc[tt][cg], sal, (int)sb[cg]);
      }
    }
    // third-term MFMAs of flagged tiles (a slow path): in this block order MFMA q's logical
    // block lb is block 4q + lb, so lane (i, g) takes blocks 4q + g / 2 and 4q + 2 + g / 2,
    // elements 16 (g % 2) .., and the scale of block 4q + g
    if (c < kX3Flags && ((m3_any >> c) & 1u)) {  // uniform
#pragma unroll
      for (int tt = 0; tt < T; ++tt) {
        if (tt < ntl && ((m3[tt] >> c) & 1u)) {
          const uint8_t* row = x3_slot_row(a, w[tt].row0, w[tt].nrows, jl);
          const bool mine = x3_row_flag(a, row, c);
          const uint8_t* p = mine ? row + c * 512 + q * 128 + (gl >> 1) * 32 + (gl & 1) * 16 : nullptr;
          const i32x8 a3 = mine ? cat8_ld(p, p + 64) : i32x8{0, 0, 0, 0, 0, 0, 0, 0};
          const int s3 = mine ? (int)row[(long long)nsc * 512 + c * 16 + 4 * q + gl] : 127;
#pragma unroll
          for (int cg = 0; cg < 4; ++cg) acc[tt][cg] = mfma_f8f4<0, 0>(a3, b[cg], acc[tt][cg], s3, (int)sb[cg]);
        }
      }
    }
  }
  wait_vm0();
#pragma unroll
  for (int tt = 0; tt < T; ++tt)
    if (tt < ntl && w[tt].active) epilogue_direct<MODE>(a, w[tt], lane, acc[tt], tw[tt]);
}

// Resident grid over the items (group, block of eight column tiles), feature blocks outermost,
// dealt over the XCDs in contiguous runs: the work-groups on one XCD at a time take neighbouring
// groups (mostly of one expert) at the same columns, so they share the weights through its L2.
template <int MODE, bool FL>
__global__ __launch_bounds__(64 * kGmWaves, 1) void fwd_gemm_kernel(FwdArgs a)
{
  __shared__ GemmLds lds;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ng = *(cint_ptr)a.n_groups;
  const int nfb = (a.n_ct + kGmWaves - 1) / kGmWaves;
  const int total = ng * nfb;
  const int per_xcd = (total + 7) >> 3;
  for (int it = 0;; ++it) {
    const int slot = (int)(blockIdx.x >> 3) + it * (int)(gridDim.x >> 3);
    const int item = (int)(blockIdx.x & 7) * per_xcd + slot;
    if (slot >= per_xcd || item >= total) break;
    const int fb = item / ng, gi = item - fb * ng;
    const cint_ptr gg = (cint_ptr)(a.groups + gi);
    if (it > 0) __syncthreads();  // every wave is done with the previous item's LDS
    int l = lane;
    asm volatile("" : "+v"(l));
    fwd_gemm_item<MODE, FL>(a, gg[0], gg[1], gg[2], fb, wave, l, lds);
  }
}

// ---------------------------------------------------------------- large buckets, forward layout
// With a forward layout the large buckets take wider items: one wide group (up to
// kWideGroupTiles = 8 row tiles, 128 rows) x eight column tiles (512 weight rows, 64 per wave of
// an eight-wave work-group that holds the CU alone). Each wave loads its own weight operands
// straight into registers, one contiguous KiB per MFMA operand block of the forward layout
// (two quarters in flight); only the activations go through LDS, one quarter (8 tiles x 4 KiB,
// copied from the AT layout as it lies) at a time, double-buffered. Per quarter a wave issues
// 8 tiles x 4 column groups x 2 terms = 64 MFMAs, for 64 KiB the CU reads (32 KiB of
// activations, 32 KiB of weights): half the bytes per MFMA of the four-tile items, whose rate
// the CU's reads in flight bound. Block order and lane layouts are the one-tile kernels' (MFMA q
// takes blocks 4g + q), so both operands are copied as they lie. Each super-chunk's activation
// scales (8 tiles x 512 B) go through LDS; the weight scales of four super-chunks at a time
// (64 B per row) through a per-wave LDS window.
//
// Per quarter s (super-chunk s / 4, MFMA q = s % 4): wait until only the weight loads of quarter
// s + 1 are outstanding, barrier, request the activation copy of quarter s + 1 (and, when due,
// the next super-chunk's activation scales and the next scale window), 64 MFMAs, then the weight
// loads of quarter s + 2 into the registers quarter s has just read. The copies are issued from
// inline assembly, so the compiler counts only the weight loads, and its own wait for quarter s's
// weights (vmcnt 4: quarter s + 1's four loads) is the one above.
constexpr int kWgT = kWideGroupTiles;  // row tiles per item
constexpr int kWgWaves = 8;            // column tiles per item (one per wave)
constexpr int kWgA = kWgT * 4096;      // activation bytes per quarter
constexpr int kWgWin = 4;              // super-chunks per weight-scale window
struct WideLds {
  uint8_t a[2][kWgA];                      // quarter buffers: [tile][plane][piece][lane][16 B]
  uint8_t sa[2][kWgT][1024];               // super-chunk activation scales: [c % 2][tile][lane][plane][4 B], + a spare half
  uint8_t sw[kWgWaves][64 * 16 * kWgWin];  // weight-scale windows: [wave][row 0..63][super-chunk 0..3][16 B]
};

template <int MODE>
__device__ __forceinline__ void fwd_wide_item(const FwdArgs& a, int expert, int t0, int ntl, int fb, int wave,
                                              int lane, WideLds& lds)
{
  constexpr int T = kWgT;
  const int g = lane >> 4;
  const int nb = a.K / kGroup;
  const int nsc = a.K / kChunk;  // the fast path: K is a multiple of 512
  const int ns = 4 * nsc;
  const int ct_raw = fb * kWgWaves + wave;
  const bool active = ct_raw < a.n_ct;
  const int ct = active ? ct_raw : a.n_ct - 1;

  // first weight row of column group cg (gate/up: groups 2, 3 are W3's rows)
  auto grp_row = [&](int cg) { return MODE == kFwdGateUp ? ct * 32 + (cg & 1) * 16 : ct * kFwdColsPerTile + cg * 16; };
  auto s_base = [&](int cg) {
    return (MODE == kFwdGateUp && cg >= 2 ? a.ws1 : a.ws0) + (long long)expert * a.ws_estride;
  };
  // weight operands: column group cg is row group rg = row0 / 16 of the forward layout, whose
  // quarter s is the KiB at s * 1024 (lane l's 16 B at l * 16); past the last quarter an empty
  // resource returns zeros without memory traffic and keeps the load count
  rsrc_t wr[4];
#pragma unroll
  for (int cg = 0; cg < 4; ++cg) {
    const int rg = min(grp_row(cg), a.R - 1) / 16;
    const uint8_t* base = (MODE == kFwdGateUp && cg >= 2 ? a.fl1 : a.fl0) + (long long)expert * a.fl_estride +
                          (long long)rg * nsc * 4096;
    wr[cg] = make_rsrc(base, (uint32_t)((a.R + 15) / 16 - rg) * (uint32_t)nsc * 4096u);
  }
  const rsrc_t wr_none = make_rsrc(a.fl0, 0);
  auto load_b = [&](int s, i32x4 (&b)[4]) {
    const bool live = s < ns;  // uniform
#pragma unroll
    for (int cg = 0; cg < 4; ++cg) b[cg] = buf16_nt(live ? wr[cg] : wr_none, (uint32_t)lane * 16u, (uint32_t)s * 1024u);
  };
  // activation copies: wave w takes tile w (the group's last tile past its end)
  const uint8_t* my_tile = a.a_tiles + (long long)(t0 + min(wave, ntl - 1)) * at_tile_bytes(a.K);
  auto issue_a = [&](int s) {
    const uint8_t* src = my_tile + (long long)(s >> 2) * kAtChunkBytes + (s & 3) * 4096;
#pragma unroll
    for (int u = 0; u < 4; ++u) dma16_async_s(src, (uint32_t)(lane * 16 + u * 1024), &lds.a[s & 1][wave * 4096 + u * 1024]);
  };
  auto issue_sa = [&](int c) {  // lanes 32..63 repeat lanes 0..31 into the spare half
    dma16_async_s(my_tile + (long long)c * kAtChunkBytes + kAtCodeBytes, (uint32_t)((lane & 31) * 16),
                  &lds.sa[c & 1][wave][0]);
  };
  // weight-scale window `win`: instruction k copies column group k's 16 rows, lane l 16 B of row
  // l / 4 (super-chunk 4 win + l % 4) to row * 64 + (l % 4) * 16
  auto issue_sw = [&](int win) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int n = min(grp_row(k) + (lane >> 2), a.R - 1);
      const int cc = min(win * kWgWin + (lane & 3), nsc - 1);
      dma16_async_s(s_base(k), (uint32_t)(n * nb + cc * 16), &lds.sw[wave][k * 1024]);
    }
  };

  f32x4 acc[T][4];
#pragma unroll
  for (int tt = 0; tt < T; ++tt)
#pragma unroll
    for (int cg = 0; cg < 4; ++cg) acc[tt][cg] = f32x4{0.f, 0.f, 0.f, 0.f};

  // the previous item's epilogue stores complete here, in a wait the compiler sees: with stores
  // of unknown completion order pending it would wait for every load at the loop's head
  __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0)
  // gate/up: third-term masks of the tiles (m3[tt], bit c: super-chunk c, rare) and their union
  uint32_t m3[T], m3_any = 0;
  const bool use3 = MODE == kFwdGateUp && a.x3 != nullptr && *(cint_ptr)a.x3_any != 0;
#pragma unroll
  for (int tt = 0; tt < T; ++tt) {
    m3[tt] = 0;
    if (use3 && tt < ntl) {
      const cint_ptr tl = (cint_ptr)(a.tiles + t0 + tt);
      m3[tt] = x3_mask(x3_flags(a, x3_slot_row(a, tl[1], tl[2], lane & 15), lane), lane);
      m3_any |= m3[tt];
    }
  }
  // tile tt's third-term MFMAs of quarter (c, q), operands straight from the X3 rows (a slow path)
  auto third_term = [&](int c, auto Q, const i32x4 (&b)[4], const uint32_t (&sb)[4]) {
    constexpr int q = decltype(Q)::value;
#pragma unroll
    for (int tt = 0; tt < T; ++tt) {
      if (tt < ntl && ((m3[tt] >> c) & 1u)) {
        const cint_ptr tl = (cint_ptr)(a.tiles + t0 + tt);
        const uint8_t* row = x3_slot_row(a, tl[1], tl[2], lane & 15);
        const bool mine = x3_row_flag(a, row, c);
        const uint32_t s3 = mine ? *reinterpret_cast<const uint32_t*>(row + (long long)nsc * 512 + c * 16 + 4 * g) : 0x7F7F7F7Fu;
        const i32x8 a3 = mine ? x3_operand(row, c, q, g) : i32x8{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int cg = 0; cg < 4; ++cg) acc[tt][cg] = mfma_f8f4<q, q>(a3, b[cg], acc[tt][cg], (int)s3, (int)sb[cg]);
      }
    }
  };

  issue_sw(0);
  issue_sa(0);
  issue_a(0);
  i32x4 b0[4], b1[4];
  uint32_t rw[4];  // this super-chunk's weight scale dwords (byte q: block 4g + q)
  bool damaged = false;

  auto step = [&](int c, auto Q, i32x4 (&b)[4], bool tail) {
    constexpr int q = decltype(Q)::value;
    const int s = 4 * c + q;
    wait_vm<4>();
    __syncthreads();
#pragma unroll
    for (int cg = 0; cg < 4; ++cg) pin(b[cg]);
    int l = lane;
    asm volatile("" : "+v"(l));
    if constexpr (q == 0) {
      const int j = l & 15;
      uint32_t d = 0;
#pragma unroll
      for (int cg = 0; cg < 4; ++cg) {
        rw[cg] = *reinterpret_cast<const uint32_t*>(&lds.sw[wave][(cg * 16 + j) * 64 + (c % kWgWin) * 16 + (l >> 4) * 4]);
        d |= damaged_scale_bits(rw[cg]);
      }
      wait_lgkm0();  // before any copy may overwrite the window read here
      damaged = __builtin_amdgcn_ballot_w64(d != 0u) != 0;
    }
    __builtin_amdgcn_sched_barrier(0);
    if (s + 1 < ns) {
      issue_a(s + 1);
      if (((s + 1) & 3) == 0) issue_sa((s + 1) >> 2);
      // the next window, after this wave's last read of the current one (super-chunk 4 win + 3, q = 0)
      const int win = s / (4 * kWgWin);
      if (s % (4 * kWgWin) == 4 * (kWgWin - 1) + 1 && (win + 1) * kWgWin < nsc) issue_sw(win + 1);
    }
    __builtin_amdgcn_sched_barrier(0);
    uint32_t sb[4];
#pragma unroll
    for (int cg = 0; cg < 4; ++cg) sb[cg] = rw[cg];
    if (damaged) {  // scale bytes >= 253: zero block, scale 2^0 (uniform branch, rare)
#pragma unroll
      for (int cg = 0; cg < 4; ++cg) {
        const bool dead = ((rw[cg] >> (8 * q)) & 0xFFu) >= 253u;
        b[cg] = dead ? i32x4{0, 0, 0, 0} : b[cg];
        sb[cg] = dead ? (rw[cg] & ~(0xFFu << (8 * q))) | (127u << (8 * q)) : rw[cg];
      }
    }
    // tile tt's operands are read from LDS while tile tt - 1's MFMAs run (one tile ahead)
    const uint8_t* la = &lds.a[q & 1][l * 16];
    const uint8_t* ls = &lds.sa[c & 1][0][l * 8];
    auto read_a = [&](int tt, i32x8& ah, i32x8& al, uint2& sc) {
      const uint8_t* pa = la + tt * 4096;
      ah = cat8(*reinterpret_cast<const i32x4*>(pa), *reinterpret_cast<const i32x4*>(pa + 1024));
      al = cat8(*reinterpret_cast<const i32x4*>(pa + 2048), *reinterpret_cast<const i32x4*>(pa + 3072));
      sc = *reinterpret_cast<const uint2*>(ls + tt * 1024);
    };
    i32x8 ah, al, nh, nl;
    uint2 sc, nsc2;
    read_a(0, nh, nl, nsc2);
#pragma unroll
    for (int tt = 0; tt < T; ++tt) {
      ah = nh;
      al = nl;
      sc = nsc2;
      if (tt + 1 < T) read_a(tt + 1, nh, nl, nsc2);
      if (tt < ntl) {
        // the four hi-term MFMAs, then the four lo-term ones: each lo MFMA reads the accumulator
        // its hi MFMA wrote three instructions earlier rather than right before it
        f32x4 t4[4];
#pragma unroll
        for (int cg = 0; cg < 4; ++cg) t4[cg] = mfma_f8f4<q, q>(ah, b[cg], acc[tt][cg], (int)sc.x, (int)sb[cg]);
#pragma unroll
        for (int cg = 0; cg < 4; ++cg) acc[tt][cg] = mfma_f8f4<q, q>(al, b[cg], t4[cg], (int)sc.y, (int)sb[cg]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (c < kX3Flags && ((m3_any >> c) & 1u)) third_term(c, Q, b, sb);  // uniform
    if (tail) load_b(s + 2, b);
  };

  // The last step of a super-chunk leaves its weight loads (quarter s + 2) to the head of the
  // next iteration, so only one register buffer is in flight across the loop's back edge: with
  // two, the compiler waits for both at the loop head.
  load_b(0, b0);
  for (int c = 0; c < nsc; ++c) {
    load_b(4 * c + 1, b1);
    step(c, std::integral_constant<int, 0>{}, b0, true);
    step(c, std::integral_constant<int, 1>{}, b1, true);
    step(c, std::integral_constant<int, 2>{}, b0, true);
    step(c, std::integral_constant<int, 3>{}, b1, false);
  }
  wait_vm0();
  if (!active) return;
#pragma unroll
  for (int tt = 0; tt < T; ++tt) {
    if (tt >= ntl) break;
    WorkItem w;
    w.tile = t0 + tt;
    const cint_ptr tl = (cint_ptr)(a.tiles + w.tile);
    w.expert = expert;
    w.row0 = tl[1];
    w.nrows = tl[2];
    w.ct0 = fb * kWgWaves;
    w.ct = ct;
    w.active = true;
    float tw[4];
    if (MODE == kFwdDown)
#pragma unroll
      for (int v = 0; v < 4; ++v) tw[v] = a.row_w[w.row0 + min(4 * g + v, w.nrows - 1)];
    epilogue_direct<MODE>(a, w, lane, acc[tt], tw);
  }
}

// Resident grid (one eight-wave work-group per CU) over the items (wide group, block of eight
// column tiles). Items vary in cost (a partial group has fewer tiles, and its MFMAs for the
// missing tiles are skipped), so the work-groups take them from a work counter in list order:
// the full groups' items first, then the partial groups', which fill in behind them. Consecutive
// items are the eight column blocks of one group, which run at about the same time and share its
// activations.
template <int MODE>
__global__ __launch_bounds__(64 * kWgWaves, 1) void fwd_wide_kernel(FwdArgs a)
{
  __shared__ WideLds lds;
  __shared__ int s_item;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ng = *(cint_ptr)a.n_wgroups;
  if (ng == 0) return;  // no large buckets: the whole grid leaves without touching the queue
  const int nfb = (a.n_ct + kWgWaves - 1) / kWgWaves;
  const int total = ng * nfb;
  for (;;) {
    const int item = queue_next(a.wcounter, &s_item);  // also: every wave is done with the previous item's LDS
    if (item >= total) break;
    const int gi = item / nfb, fb = item - gi * nfb;
    const cint_ptr gg = (cint_ptr)(a.wgroups + gi);
    int l = lane;
    asm volatile("" : "+v"(l));
    fwd_wide_item<MODE>(a, gg[0], gg[1], gg[2], fb, wave, l, lds);
  }
  queue_leave(a.wcounter);
}

// Both bucket kinds of a routed product from the forward layout in one launch of eight-wave
// work-groups (one per CU, the shape of both kernels above): each work-group runs its one-tile
// items (fwd_kernel<MODE, true, true, 8>) and then takes large-bucket items from the work queue
// (fwd_wide_kernel), so the large items fill the slots that the one-tile items' last round leaves
// idle, and a routing without large buckets pays for no second launch. Same items, same
// arithmetic: the results are those of the two launches.
union FusedLds {
  FwdLds f;
  WideLds w;
};

template <int MODE>
__global__ __launch_bounds__(64 * kWgWaves, 1) void fwd_fused_kernel(FwdArgs a)
{
  static_assert(kWgWaves == 8, "the one-tile items run in eight-wave work-groups");
  __shared__ FusedLds lds;
  __shared__ int s_item;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  WorkItem w;
  for (int it = 0; decode_work(a.tiles, a.n_tiles, a.small_tiles, a.n_small, a.n_groups, a.M, a.n_ct, wave, it, w, 8); ++it) {
    if (it > 0) __syncthreads();
    int l = lane;
    asm volatile("" : "+v"(l));
    fwd_item<MODE, true, true, 8>(a, w, wave, l, lds.f);
  }
  const int ng = *(cint_ptr)a.n_wgroups;
  if (ng == 0) return;  // no large buckets: the work queue is not touched
  const int nfb = (a.n_ct + kWgWaves - 1) / kWgWaves;
  const int total = ng * nfb;
  for (;;) {
    const int item = queue_next(a.wcounter, &s_item);  // also: every wave is done with the LDS before
    if (item >= total) break;
    const int gi = item / nfb, fb = item - gi * nfb;
    const cint_ptr gg = (cint_ptr)(a.wgroups + gi);
    int l = lane;
    asm volatile("" : "+v"(l));
    fwd_wide_item<MODE>(a, gg[0], gg[1], gg[2], fb, wave, l, lds.w);
  }
  queue_leave(a.wcounter);
}

// Work-groups that fit on the device at once (two per CU: the LDS and register budgets of
// fwd_kernel), rounded down to a multiple of the 8 XCDs.
int resident_groups()
{
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  return max(8, (2 * cus) / 8 * 8);
}

// The fast path addresses a weight matrix through one buffer resource (32-bit byte counts and
// offsets); larger matrices, and K not a multiple of 512, take the general path.
bool fast_path(int R, int K) { return K > 0 && (K % kChunk) == 0 && (long long)R * (K / 2) < (1LL << 32); }

}  // namespace

bool fwd_bucket_split(int R, int K) { return fast_path(R, K); }

hipError_t launch_fwd(const FwdArgs& a, int mode, int max_tiles, hipStream_t s)
{
  const long long n_cg = (a.n_ct + kWavesPerGroup - 1) / kWavesPerGroup;
  const long long total = (long long)max_tiles * n_cg;
  if (total <= 0) return hipSuccess;
  const long long blocks = std::min<long long>((total + 7) / 8 * 8, resident_groups());
  // the down product from the forward layout: eight column tiles per work-group, one per CU
  const long long n_cg8 = (a.n_ct + 7) / 8;
  const long long blocks8 = std::min<long long>(((long long)max_tiles * n_cg8 + 7) / 8 * 8, resident_groups() / 16 * 8);
  const bool fast = fast_path(a.R, a.K);
  // the bucket split needs the tile list and the fast path; otherwise every tile takes fwd_kernel
  const bool split = fwd_bucket_split(a.R, a.K) && a.tiles && a.small_tiles && a.groups;
  FwdArgs b = a;
  if (!split) {
    b.small_tiles = nullptr;
    b.groups = nullptr;
    b.wgroups = nullptr;
  }
  // both work-group shapes read the forward layout when every matrix of the product has one
  // (and its byte count fits a buffer resource, as for the checkpoint layout)
  const bool fl = fast && mode != kFwdPlain && a.fl0 && (mode != kFwdGateUp || a.fl1) &&
                  forward_layout_bytes(a.R, a.K) < (1LL << 32);
  // both bucket kinds in one launch: eight-wave one-tile items and wide large-bucket items
  const bool fused = fl && a.n_ct % 8 == 0 && split && b.wgroups && b.wcounter;
  dim3 grid((unsigned)blocks), block(64 * kWavesPerGroup);
#define MX_LAUNCH(M, F, L) hipLaunchKernelGGL((fwd_kernel<M, F, L>), grid, block, 0, s, b)
  if (mode == kFwdPlain) {
    if (fast) MX_LAUNCH(kFwdPlain, true, false); else MX_LAUNCH(kFwdPlain, false, false);
  } else if (fused) {
    if (mode == kFwdGateUp) hipLaunchKernelGGL((fwd_fused_kernel<kFwdGateUp>), dim3((unsigned)blocks8), dim3(512), 0, s, b);
    else hipLaunchKernelGGL((fwd_fused_kernel<kFwdDown>), dim3((unsigned)blocks8), dim3(512), 0, s, b);
    return hipGetLastError();
  } else if (mode == kFwdGateUp) {
    if (fl && a.n_ct % 8 == 0)
      hipLaunchKernelGGL((fwd_kernel<kFwdGateUp, true, true, 8>), dim3((unsigned)blocks8), dim3(512), 0, s, b);
    else if (fl) MX_LAUNCH(kFwdGateUp, true, true);
    else if (fast) MX_LAUNCH(kFwdGateUp, true, false);
    else MX_LAUNCH(kFwdGateUp, false, false);
  } else {
    if (fl && a.n_ct % 8 == 0)
      hipLaunchKernelGGL((fwd_kernel<kFwdDown, true, true, 8>), dim3((unsigned)blocks8), dim3(512), 0, s, b);
    else if (fl) MX_LAUNCH(kFwdDown, true, true);
    else if (fast) MX_LAUNCH(kFwdDown, true, false);
    else MX_LAUNCH(kFwdDown, false, false);
  }
#undef MX_LAUNCH
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !split) return e;
  dim3 mgrid((unsigned)(resident_groups() / 16 * 8)), mblock(64 * kGmWaves);  // one per CU, a multiple of 8
  if (fl && b.wgroups && b.wcounter && mode != kFwdPlain) {  // wide groups, weights straight from the forward layout
    dim3 wblock(64 * kWgWaves);
    if (mode == kFwdGateUp) hipLaunchKernelGGL((fwd_wide_kernel<kFwdGateUp>), mgrid, wblock, 0, s, b);
    else hipLaunchKernelGGL((fwd_wide_kernel<kFwdDown>), mgrid, wblock, 0, s, b);
    return hipGetLastError();
  }
  if (mode == kFwdGateUp) {
    if (fl) hipLaunchKernelGGL((fwd_gemm_kernel<kFwdGateUp, true>), mgrid, mblock, 0, s, b);
    else hipLaunchKernelGGL((fwd_gemm_kernel<kFwdGateUp, false>), mgrid, mblock, 0, s, b);
  } else if (mode == kFwdDown) {
    if (fl) hipLaunchKernelGGL((fwd_gemm_kernel<kFwdDown, true>), mgrid, mblock, 0, s, b);
    else hipLaunchKernelGGL((fwd_gemm_kernel<kFwdDown, false>), mgrid, mblock, 0, s, b);
  } else {
    hipLaunchKernelGGL((fwd_gemm_kernel<kFwdPlain, false>), mgrid, mblock, 0, s, b);
  }
  return hipGetLastError();
}

long long forward_layout_bytes(int R, int K)
{
  return (long long)((R + 15) / 16) * (K / kChunk) * (4096 + 256);
}

namespace {

// One thread per 16-byte piece of the forward layout. Codes: piece l of operand block q of
// super-chunk c of row group rg (at byte ((rg * nsc + c) * 4 + q) * 1024 + l * 16 of the expert's
// layout) is MX block 4 (l / 16) + q of that super-chunk of row 16 rg + l % 16, the 16 bytes lane l
// of the one-tile kernels reads for MFMA q. Scales, after the codes of all row groups: the 256 B of
// (rg, c) at ((nrg * nsc) * 4096 + (rg * nsc + c) * 256) hold lane l's scale dword (blocks
// 4 (l / 16) .. + 3 of super-chunk c of row 16 rg + l % 16) at 4 l. Rows past R repeat row R - 1,
// as those kernels' loads do.
__global__ __launch_bounds__(256) void forward_layout_kernel(const uint8_t* packed, const uint8_t* scales,
                                                             uint8_t* out, int R, int K, long long per_expert,
                                                             long long total)
{
  const long long p = (long long)blockIdx.x * 256 + threadIdx.x;
  if (p >= total) return;
  const int nsc = K / kChunk;
  const long long e = p / per_expert;
  long long r = p - e * per_expert;
  const long long code_pieces = (long long)((R + 15) / 16) * nsc * 256;
  if (r < code_pieces) {
    const int l = (int)(r & 63);
    r >>= 6;
    const int q = (int)(r & 3);
    r >>= 2;
    const int rg = (int)(r / nsc), c = (int)(r - (long long)rg * nsc);
    const int row = min(rg * 16 + (l & 15), R - 1);
    const uint8_t* src = packed + (e * R + row) * (long long)(K / 2) + c * 256 + (4 * (l >> 4) + q) * 16;
    *reinterpret_cast<i32x4*>(out + p * 16) = *reinterpret_cast<const i32x4*>(src);
    return;
  }
  r -= code_pieces;  // piece k of scale block (rg, c): the dwords of lanes 4k .. 4k + 3
  const int k = (int)(r & 15);
  r >>= 4;
  const int rg = (int)(r / nsc), c = (int)(r - (long long)rg * nsc);
  i32x4 v;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int l = 4 * k + u;
    const int row = min(rg * 16 + (l & 15), R - 1);
    v[u] = *reinterpret_cast<const int*>(scales + (e * R + row) * (long long)(K / 32) + c * 16 + 4 * (l >> 4));
  }
  *reinterpret_cast<i32x4*>(out + p * 16) = v;
}

}  // namespace

hipError_t launch_forward_layout(const uint8_t* packed, const uint8_t* scales, uint8_t* out, int E, int R, int K,
                                 hipStream_t s)
{
  if (E <= 0 || R <= 0) return hipSuccess;
  if (K <= 0 || K % kChunk) return hipErrorInvalidValue;
  const long long per_expert = forward_layout_bytes(R, K) / 16;
  const long long total = per_expert * E;
  hipLaunchKernelGGL(forward_layout_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, packed, scales,
                     out, R, K, per_expert, total);
  return hipGetLastError();
}

}  // namespace mx
