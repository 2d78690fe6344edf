// Forward MXFP4 products on the fp4-native scaled MFMA (gfx950).
//
// Each wave computes one 16-row x 64-column output tile over the whole K range
// (kFwdGateUp: 16 rows x 32 gate features + the same 32 up features). A work-group holds the
// four waves of four neighbouring column tiles of the same row tile: they share the tile's
// activations, which the work-group copies into LDS once per super-chunk. Every weight byte
// is read once per row tile.
//
// Per super-chunk c (512 K elements) and lane (j = lane % 16, g = lane / 16), for each of the
// 4 column groups of 16 weight rows:
//   B: 64 contiguous bytes of weight row n = 4 MX blocks 16c+4g+q (q = 0..3), one dword of
//      scales. MFMA q consumes block 16c+4g+q from lane group g, so op_sel q picks its scale.
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
  int ct0;      // first column tile of the work-group (its four waves take ct0 .. ct0 + 3)
  bool active;  // false: this wave's column tile is past the end; it only helps with the copies
};

// The grid is persistent (about two work-groups per CU) and work-groups are issued round-robin
// over the 8 XCDs (blockIdx % 8). Each XCD owns one contiguous run of work items, so the tiles
// of one expert share that XCD's L2; its work-groups take the run's items in turn (iteration
// `it` of slot s takes item s + it * slots). Returns false for the whole work-group at once.
typedef const __attribute__((address_space(4))) int* cint_ptr;

__device__ __forceinline__ bool decode_work(const int4* tiles, const int* n_tiles, const int* small_tiles,
                                            const int* n_small, const int* n_groups, int M, int n_ct, int wave,
                                            int it, WorkItem& w)
{
  // The tile lists are written before this kernel and only read here: scalar loads through the
  // constant address space, which do not wait for this work-group's outstanding stores.
  // with no large-bucket groups the small-bucket list is every tile in order: skip it
  const bool use_small = small_tiles && *(cint_ptr)n_groups > 0;
  const int ntiles = use_small ? *(cint_ptr)n_small
                               : tiles ? *(cint_ptr)n_tiles : (M + kFwdRowsPerTile - 1) / kFwdRowsPerTile;
  const int n_cg = (n_ct + kWavesPerGroup - 1) / kWavesPerGroup;
  const int total = ntiles * n_cg;
  const int per_xcd = (total + 7) >> 3;
  const int k = (int)(blockIdx.x >> 3) + it * (int)(gridDim.x >> 3);
  const int item = (int)(blockIdx.x & 7) * per_xcd + k;
  if (k >= per_xcd || item >= total) return false;
  const int i = item / n_cg;
  const int t = use_small ? ((cint_ptr)small_tiles)[i] : i;
  w.tile = t;
  w.ct0 = (item - i * n_cg) * kWavesPerGroup;
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

__device__ __forceinline__ i32x8 cat8(const i32x4& x, const i32x4& y)
{
  return i32x8{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
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

// Epilogue of the fast path. The four waves stage the work-group's outputs in the (now idle)
// activation buffers of LDS, then write them with 16-byte stores that cover whole runs of
// memory: scattered 1-byte and 4-byte stores of the same data cost the weight stream about a
// tenth of its bandwidth. The stores are non-temporal (streamed past the caches), which costs the
// weight stream less than ordinary write-back stores. Lane (j, g) holds rows 4g+v (v = 0..3) of columns grp*16 + j.
constexpr int kStagePitch = 260;  // floats per staged row: 256 + 4 keeps the row starts on distinct banks

template <int MODE>
__device__ __forceinline__ void epilogue_staged(const FwdArgs& a, const WorkItem& w, int wave, int lane,
                                                const f32x4 (&acc)[4], const float (&tw)[4], FwdLds& lds)
{
  const int j = lane & 15, g = lane >> 4;
  const int t = wave * 64 + lane;
  if (MODE == kFwdGateUp) {
    // act codes: [q = wave][plane][half][row 0..15][16 B] then scales [row][plane][q]; this is
    // the AT byte order of the work-group's 128 features (super-chunk c, block group gl)
    uint8_t* sq = lds.a[0];
    float* ss = reinterpret_cast<float*>(lds.a[1]);  // [row][gate 128 | up 128] fp32
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
      sq[((wave * 2 + 0) * 2 + 0) * 256 + i * 16 + j] = (uint8_t)q.hi;
      sq[((wave * 2 + 0) * 2 + 1) * 256 + i * 16 + j] = (uint8_t)(q.hi >> 8);
      sq[((wave * 2 + 1) * 2 + 0) * 256 + i * 16 + j] = (uint8_t)q.lo;
      sq[((wave * 2 + 1) * 2 + 1) * 256 + i * 16 + j] = (uint8_t)(q.lo >> 8);
      if (j == 0) {
        sq[4096 + i * 8 + wave] = (uint8_t)q.s_hi;
        sq[4096 + i * 8 + 4 + wave] = (uint8_t)q.s_lo;
      }
      if (a.save) {
        float* r = ss + i * kStagePitch + wave * 32 + j;
        r[0] = ga;
        r[16] = gb;
        r[128] = ua;
        r[144] = ub;
      }
    }
    __syncthreads();
    const int f_wg = w.ct0 * 32;  // first feature of the work-group, a multiple of 128
    const int c = f_wg >> 9, gl = (f_wg >> 7) & 3;
    uint8_t* qbase = a.q_tiles + (long long)w.tile * at_tile_bytes(F) + (long long)c * kAtChunkBytes;
    {
      const int run = t >> 5, off = (t & 31) * 16;  // run = q * 2 + plane: 512 B each
      __builtin_nontemporal_store(*reinterpret_cast<const i32x4*>(sq + run * 512 + off),
                                  reinterpret_cast<i32x4*>(qbase + (run * 2 + (gl >> 1)) * 1024 + (gl & 1) * 512 + off));
      if (t < 8)
        *reinterpret_cast<i32x4*>(qbase + kAtCodeBytes + gl * 128 + t * 16) =
            *reinterpret_cast<const i32x4*>(sq + 4096 + t * 16);
    }
    if (a.save) {
      const int part = lane >> 5, idx = (lane & 31) * 4, f = f_wg + idx;
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int r = it * 4 + wave;
        if (r < w.nrows && f < F)
          __builtin_nontemporal_store(*reinterpret_cast<const f32x4*>(ss + r * kStagePitch + part * 128 + idx),
                                      reinterpret_cast<f32x4*>(a.save + (long long)(w.row0 + r) * 2 * F + part * F + f));
      }
    }
    return;
  }

  // kFwdPlain / kFwdDown: [row][256 columns of the work-group] fp32
  float* ss = reinterpret_cast<float*>(lds.a[0]);
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const float wv = MODE == kFwdDown ? tw[v] : 1.0f;
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) ss[(4 * g + v) * kStagePitch + wave * 64 + grp * 16 + j] = acc[grp][v] * wv;
  }
  __syncthreads();
  const int col = w.ct0 * kFwdColsPerTile + lane * 4;
  const bool vec = ((a.ldy & 3) == 0) && ((reinterpret_cast<uintptr_t>(a.y) & 15) == 0);
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int r = it * 4 + wave;
    if (r >= w.nrows) continue;
    const f32x4 val = *reinterpret_cast<const f32x4*>(ss + r * kStagePitch + lane * 4);
    float* yr = a.y + (long long)(w.row0 + r) * a.ldy;
    if (vec && col + 4 <= a.R) {
      __builtin_nontemporal_store(val, reinterpret_cast<f32x4*>(yr + col));
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (col + e < a.R) yr[col + e] = val[e];
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
    float* yr = a.y + (long long)row * a.ldy;
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      const int col = w.ct * kFwdColsPerTile + grp * 16 + j;
      if (col < a.R) yr[col] = acc[grp][v] * wv;
    }
  }
}


// One work item: the 16 x 64 tile (w.tile, w.ct) over all of K, then its epilogue.
template <int MODE, bool FAST>
__device__ __forceinline__ void fwd_item(const FwdArgs& a, const WorkItem& w, int wave, int lane)
{
  __shared__ FwdLds lds;  // used by the fast path only
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
      for (int u = 0; u < 4; ++u) {
        const int unit = 4 * wave + u;
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
    rsrc_t wr[4], wr_none[4];
    uint32_t woff[4];
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      const uint8_t* base = grp_wp(grp);
      wr[grp] = make_rsrc(base, (uint32_t)a.R * (uint32_t)(a.K / 2));
      wr_none[grp] = make_rsrc(base, 0);
      woff[grp] = (uint32_t)(wrow[grp] - base) + boff[grp];
    }
    auto load_b_buf = [&](int c, i32x4 (&b)[4][4]) {
      const bool live = c < nsc;  // uniform
#pragma unroll
      for (int grp = 0; grp < 4; ++grp)
#pragma unroll
        for (int q = 0; q < 4; ++q) b[grp][q] = buf16(live ? wr[grp] : wr_none[grp], woff[grp] + 16 * q, (uint32_t)c * 256);
    };

    // Two chunks of weights in flight: a buffer is refilled with chunk c + 2 as soon as chunk
    // c's MFMAs have read it, and chunk c + 1's loads are in flight meanwhile. The activation
    // copy and scale window of chunk c are requested at the top of chunk c - 1, before the 16
    // weight loads of chunk c + 1 (issued at the end of chunk c - 1), so at the top of chunk c
    // everything but those 16 has landed. The copies are issued from
    // inline assembly: a copy the compiler knows of makes it drain every load at each barrier.
    auto step = [&](int c, i32x4 (&cur)[4][4]) {
      wait_vm<16>();
      __syncthreads();
      // everything this chunk needs from LDS, before any new copy into LDS is requested
      uint32_t sb[4];
#pragma unroll
      for (int grp = 0; grp < 4; ++grp)
        sb[grp] = *reinterpret_cast<const uint32_t*>(sw + (grp * 16 + j) * kScaleRowBytes +
                                                     (((c % kScaleWin) ^ (j & 7)) * 16) + g * 4);
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
      for (int grp = 0; grp < 4; ++grp)
#pragma unroll
        for (int q = 0; q < 4; ++q) pin(cur[grp][q]);
      __builtin_amdgcn_sched_barrier(0);
      if (c + 1 < nsc) {
        issue_a(c + 1, (c + 1) & 1);
        if ((c + 1) % kScaleWin == 0) issue_scales((c + 1) / kScaleWin);
      }
      __builtin_amdgcn_sched_barrier(0);
      sanitize_if_damaged(cur, sb);
      mfma_step<0>(acc, ah[0], al[0], cur, sb, (int)s2.x, (int)s2.y);
      mfma_step<1>(acc, ah[1], al[1], cur, sb, (int)s2.x, (int)s2.y);
      mfma_step<2>(acc, ah[2], al[2], cur, sb, (int)s2.x, (int)s2.y);
      mfma_step<3>(acc, ah[3], al[3], cur, sb, (int)s2.x, (int)s2.y);
      __builtin_amdgcn_sched_barrier(0);
      load_b_buf(c + 2, cur);
    };

    if (MODE == kFwdDown)
#pragma unroll
      for (int v = 0; v < 4; ++v) tw[v] = a.row_w[w.row0 + min(4 * g + v, w.nrows - 1)];
    i32x4 b0[4][4], b1[4][4];
    load_b_buf(0, b0);
    issue_scales(0);
    issue_a(0, 0);
    load_b_buf(1, b1);
    for (int c = 0;;) {
      step(c, b0);
      if (++c >= nsc) break;
      step(c, b1);
      if (++c >= nsc) break;
    }
    wait_vm0();  // (no copy is in flight past the last chunk; kept explicit for the epilogue)
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
    }
  }

  if constexpr (FAST) {
    __syncthreads();  // every wave is done with the last chunk's LDS data
    epilogue_staged<MODE>(a, w, wave, lane, acc, tw, lds);
    return;
  }

  if (w.active) epilogue_direct<MODE>(a, w, lane, acc, tw);
}

template <int MODE, bool FAST>
__global__ __launch_bounds__(256, 2) void fwd_kernel(FwdArgs a)
{
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keeps control flow scalar
  WorkItem w;
  for (int it = 0; decode_work(a.tiles, a.n_tiles, a.small_tiles, a.n_small, a.n_groups, a.M, a.n_ct, wave, it, w); ++it) {
    // the previous item's reads of LDS are complete before this item's copies land there;
    // its output stores drain while this item's first loads are in flight
    if (FAST && it > 0) __syncthreads();
    // recompute lane-derived addresses per item instead of holding them across items
    int l = lane;
    asm volatile("" : "+v"(l));
    fwd_item<MODE, FAST>(a, w, wave, l);
  }
}

// ---------------------------------------------------------------- large buckets
// An expert with many rows would re-read each weight byte once per 16-row tile. Its tiles come
// in groups of up to kGroupTiles (4): a work-group takes one column tile of a group's tiles, wave
// w takes row tile w, and the column tile's weights go through LDS once per super-chunk for all
// four waves (64 weight rows x 256 B of codes, plus 16 B of scales per row). Each wave streams its
// own tile's activations from memory one super-chunk ahead.
//
// LDS layout of the codes: row rr (0..63, = column group * 16 + row in group) holds its 16
// 16-byte units at unit rr * 16 + (u ^ (rr & 7)); the XOR spreads the eight rows read together
// by one 128-bit LDS instruction over all 32 banks. The copies place units with LDS DMA, which
// writes a wave's 64 lanes to one contiguous KiB, so the swizzle is applied to the source
// addresses: LDS unit p of an instruction fetches unit (p % 16) ^ (rr & 7) of row rr.
constexpr int kGrpRows = 64;
constexpr int kGrpCodeBytes = kGrpRows * 256;
constexpr int kGrpLdsBytes = kGrpCodeBytes + kGrpRows * 16;

struct GroupLds {
  uint8_t b[2][kGrpLdsBytes];
};

// Item `it` of this work-group: (group, part of four of its up to kGroupTiles tiles, column
// tile). Returns 0 when there is none left, 2 for the empty part of a short group, 1 for an item.
constexpr int kGrpParts = kGroupTiles / kWavesPerGroup;

__device__ __forceinline__ int decode_group(const FwdArgs& a, int wave, int it, WorkItem& w)
{
  const int ng = *(cint_ptr)a.n_groups;
  const int total = ng * kGrpParts * a.n_ct;
  const int per_xcd = (total + 7) >> 3;
  const int k = (int)(blockIdx.x >> 3) + it * (int)(gridDim.x >> 3);
  const int item = (int)(blockIdx.x & 7) * per_xcd + k;
  if (k >= per_xcd || item >= total) return 0;
  const int gp = item / a.n_ct;
  w.ct = item - gp * a.n_ct;
  w.ct0 = w.ct;
  const int gi = gp / kGrpParts, part = gp - gi * kGrpParts;
  const cint_ptr gg = (cint_ptr)(a.groups + gi);
  w.expert = gg[0];
  const int t0 = gg[1] + part * kWavesPerGroup, nt = gg[2] - part * kWavesPerGroup;
  if (nt <= 0) return 2;
  w.active = wave < nt;
  w.tile = t0 + (w.active ? wave : 0);
  const cint_ptr tt = (cint_ptr)(a.tiles + w.tile);
  w.row0 = tt[1];
  w.nrows = tt[2];
  return 1;
}

template <int MODE>
__device__ __forceinline__ void fwd_group_item(const FwdArgs& a, const WorkItem& w, int wave, int lane)
{
  __shared__ GroupLds lds;
  const int j = lane & 15, g = lane >> 4;
  const int nb = a.K / kGroup;
  const int nsc = at_nchunks(a.K);
  const uint8_t* const at_tile = a.a_tiles + (long long)w.tile * at_tile_bytes(a.K);

  auto grp_row = [&](int grp) {
    return MODE == kFwdGateUp ? w.ct * 32 + (grp & 1) * 16 : w.ct * kFwdColsPerTile + grp * 16;
  };
  auto grp_wp = [&](int grp) {
    return (MODE == kFwdGateUp && grp >= 2 ? a.wp1 : a.wp0) + (long long)w.expert * a.wp_estride;
  };
  auto grp_ws = [&](int grp) {
    return (MODE == kFwdGateUp && grp >= 2 ? a.ws1 : a.ws0) + (long long)w.expert * a.ws_estride;
  };

  // B(c) -> lds.b[buf]: instruction u of wave `wave` covers rows 4 (4 wave + u) .. +3; wave 0
  // also copies the 64 rows' 16 scale bytes of the chunk
  auto issue_b = [&](int c, int buf) {
    int ln = lane;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int rr = (4 * wave + u) * 4 + (ln >> 4);
      const int grp = rr >> 4;
      const int n = min(grp_row(grp) + (rr & 15), a.R - 1);
      const uint32_t off = (uint32_t)(n * (a.K / 2) + c * 256 + (((ln & 15) ^ (rr & 7)) << 4));
      dma16(grp_wp(grp) + off, &lds.b[buf][(4 * wave + u) * 1024]);
    }
    if (wave == 0) {
      const int grp = ln >> 4;
      const int n = min(grp_row(grp) + (ln & 15), a.R - 1);
      dma16(grp_ws(grp) + (uint32_t)(n * nb + c * 16), &lds.b[buf][kGrpCodeBytes]);
    }
  };
  struct AChunk {
    i32x4 v[16];
    uint2 s;
  };
  auto load_a = [&](int c, AChunk& x) {
    const uint8_t* p = at_tile + (long long)c * kAtChunkBytes + lane * 16;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int h = 0; h < 4; ++h) x.v[4 * q + h] = ldg16(p + q * 4096 + h * 1024);
    x.s = *reinterpret_cast<const uint2*>(at_tile + (long long)c * kAtChunkBytes + kAtCodeBytes + lane * 8);
  };

  f32x4 acc[4];
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) acc[grp] = f32x4{0.f, 0.f, 0.f, 0.f};
  float tw[4];
  if (MODE == kFwdDown)
#pragma unroll
    for (int v = 0; v < 4; ++v) tw[v] = a.row_w[w.row0 + min(4 * g + v, w.nrows - 1)];

  auto step = [&](int c, AChunk& cur, AChunk& nxt) {
    wait_vm0();
    __syncthreads();
    const uint8_t* lb = lds.b[c & 1];
    i32x4 b[4][4];
    uint32_t sb[4];
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      const int rr = grp * 16 + j;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        b[grp][q] = *reinterpret_cast<const i32x4*>(lb + (rr * 16 + ((g * 4 + q) ^ (rr & 7))) * 16);
      sb[grp] = *reinterpret_cast<const uint32_t*>(lb + kGrpCodeBytes + rr * 16 + g * 4);
    }
    wait_lgkm0();
    __builtin_amdgcn_sched_barrier(0);
    if (c + 1 < nsc) {
      issue_b(c + 1, (c + 1) & 1);
      if (w.active) load_a(c + 1, nxt);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (w.active) {
      sanitize(b, sb);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const i32x8 ah = cat8(cur.v[4 * q], cur.v[4 * q + 1]), al = cat8(cur.v[4 * q + 2], cur.v[4 * q + 3]);
        if (q == 0) mfma_step<0>(acc, ah, al, b, sb, (int)cur.s.x, (int)cur.s.y);
        if (q == 1) mfma_step<1>(acc, ah, al, b, sb, (int)cur.s.x, (int)cur.s.y);
        if (q == 2) mfma_step<2>(acc, ah, al, b, sb, (int)cur.s.x, (int)cur.s.y);
        if (q == 3) mfma_step<3>(acc, ah, al, b, sb, (int)cur.s.x, (int)cur.s.y);
      }
    }
  };

  AChunk a0, a1;
  issue_b(0, 0);
  if (w.active) load_a(0, a0);
  for (int c = 0;;) {
    step(c, a0, a1);
    if (++c >= nsc) break;
    step(c, a1, a0);
    if (++c >= nsc) break;
  }
  if (w.active) epilogue_direct<MODE>(a, w, lane, acc, tw);
}

template <int MODE>
__global__ __launch_bounds__(256, 2) void fwd_group_kernel(FwdArgs a)
{
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  WorkItem w;
  bool busy = false;
  for (int it = 0;; ++it) {
    const int st = decode_group(a, wave, it, w);
    if (st == 0) break;
    if (st == 2) continue;
    if (busy) __syncthreads();  // every wave is done with the previous item's LDS buffers
    int l = lane;
    asm volatile("" : "+v"(l));
    fwd_group_item<MODE>(a, w, wave, l);
    busy = true;
  }
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

}  // namespace

hipError_t launch_fwd(const FwdArgs& a, int mode, int max_tiles, hipStream_t s)
{
  const long long n_cg = (a.n_ct + kWavesPerGroup - 1) / kWavesPerGroup;
  const long long total = (long long)max_tiles * n_cg;
  if (total <= 0) return hipSuccess;
  const long long blocks = std::min<long long>((total + 7) / 8 * 8, resident_groups());
  // the fast path addresses a weight matrix through one buffer resource (32-bit byte counts and
  // offsets); larger matrices take the general path
  const bool fast = (a.K % kChunk) == 0 && (long long)a.R * (a.K / 2) < (1LL << 32);
  // the bucket split needs the tile list and the fast path; otherwise every tile takes fwd_kernel
  const bool split = fast && a.tiles && a.small_tiles && a.groups;
  FwdArgs b = a;
  if (!split) {
    b.small_tiles = nullptr;
    b.groups = nullptr;
  }
  dim3 grid((unsigned)blocks), block(64 * kWavesPerGroup);
#define MX_LAUNCH(M, F) hipLaunchKernelGGL((fwd_kernel<M, F>), grid, block, 0, s, b)
  if (mode == kFwdPlain) {
    if (fast) MX_LAUNCH(kFwdPlain, true); else MX_LAUNCH(kFwdPlain, false);
  } else if (mode == kFwdGateUp) {
    if (fast) MX_LAUNCH(kFwdGateUp, true); else MX_LAUNCH(kFwdGateUp, false);
  } else {
    if (fast) MX_LAUNCH(kFwdDown, true); else MX_LAUNCH(kFwdDown, false);
  }
#undef MX_LAUNCH
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !split) return e;
  dim3 ggrid((unsigned)resident_groups());
  if (mode == kFwdGateUp) hipLaunchKernelGGL(fwd_group_kernel<kFwdGateUp>, ggrid, block, 0, s, b);
  else if (mode == kFwdDown) hipLaunchKernelGGL(fwd_group_kernel<kFwdDown>, ggrid, block, 0, s, b);
  else hipLaunchKernelGGL(fwd_group_kernel<kFwdPlain>, ggrid, block, 0, s, b);
  return hipGetLastError();
}

}  // namespace mx
