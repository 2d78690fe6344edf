// Elementwise, routing and combine kernels around the MXFP4 products.
#include "mx_device.h"
#include "mx_kernels.h"

namespace mx {

namespace {

// ---------------------------------------------------------------- activation quantisation
// The third term of one row's super-chunk c (c < kX3Flags) into its X3 row, by the 16 lanes of
// the row: the codes and scales only when some block of the chunk is flagged (readers use them
// only then), the chunk's flag byte always.
MX_DEV void x3_store(uint8_t* x3r, int nsc, int c, int l16, const Quant3 (&q3)[kChunkBlocks], bool any3, int* x3_any)
{
  // the call-wide "some block has a third term" flag, which lets the products skip every
  // third-term step: one atomic per wave that has a flagged row, by the first such lane
  const uint64_t fl = __builtin_amdgcn_ballot_w64(any3 && l16 == 0);
  if (fl != 0 && (int)(threadIdx.x & 63) == __builtin_ctzll(fl)) atomicOr(x3_any, 1);
  if (any3) {
#pragma unroll
    for (int b = 0; b < kChunkBlocks; ++b) {
      *reinterpret_cast<uint16_t*>(x3r + c * kChunk + b * kGroup + 2 * l16) = (uint16_t)q3[b].th;
      if (l16 == 0) x3r[(long long)nsc * 512 + c * 16 + b] = (uint8_t)q3[b].s_th;
    }
  }
  if (l16 == 0) x3r[(long long)nsc * 528 + c] = any3 ? 1 : 0;
}

// One work-group per (tile, super-chunk). Its 16 lane groups take the 16 row slots; each walks
// the 16 blocks of the chunk, quantises them to two e4m3 terms and writes codes and scales into
// an LDS copy of the chunk in the AT layout; the work-group then writes the chunk out with
// contiguous 16-byte stores. Slots past the tile's row count, and K positions past the row
// end, get zeros.
// One (tile, super-chunk) of quant_tiles_kernel: tile t holds rows row0 .. row0 + nrows - 1 of
// the row map (or of x); chunk is the work-group's LDS staging copy.
template <bool BF16>
MX_DEV void quant_tile_chunk(const void* x, long long ldx, int rows, int K, int t, int c, int row0, int nrows,
                             const int* row_map, const uint8_t* xt, const int* meta, uint8_t* out, uint8_t* x3,
                             int* x3_any, uint8_t* chunk)
{
  const int nsc = at_nchunks(K);
  const int i = threadIdx.x >> 4, l16 = threadIdx.x & 15;
  const long long cbase = (long long)c * kAtChunkBytes;  // at_*_off are tile-relative
  if (xt && !(meta[2] == 0 && meta[3] > 0)) {
    // The token-major rows are written (quant_rows_kernel runs before this kernel and quantises
    // each token's row with the same blocks, so they hold the same codes): tile unit u, lane
    // 16g + i is piece (u, g) of the row of slot i's token (the zero row `rows` for unused
    // slots), and lane 16g + i's scale dword of a plane is that row's dword (plane, g).
    uint8_t* dst = out + (long long)t * at_tile_bytes(K) + cbase;
    const long long rb = xt_row_bytes(K);
    for (int p = threadIdx.x; p < 1024; p += 256) {
      const int u = p >> 6, l = p & 63, ii = l & 15, g = l >> 4;
      const long long tok = ii < nrows ? row_map[row0 + ii] : rows;
      *reinterpret_cast<i32x4*>(dst + u * 1024 + l * 16) =
          *reinterpret_cast<const i32x4*>(xt + tok * rb + (long long)c * kXtChunkBytes + (u * 4 + g) * 16);
    }
    if (threadIdx.x < 128) {
      const int l = threadIdx.x >> 1, plane = threadIdx.x & 1, ii = l & 15, g = l >> 4;
      const long long tok = ii < nrows ? row_map[row0 + ii] : rows;
      *reinterpret_cast<uint32_t*>(dst + kAtCodeBytes + l * 8 + plane * 4) = *reinterpret_cast<const uint32_t*>(
          xt + tok * rb + (long long)c * kXtChunkBytes + kXtCodeBytes + (plane * 4 + g) * 4);
    }
    return;
  }
  const bool valid = i < nrows;
  const long long src = valid ? (row_map ? row_map[row0 + i] : row0 + i) : 0;
  // all 16 blocks' loads are issued before the first is quantised
  float v0[kChunkBlocks], v1[kChunkBlocks];
#pragma unroll
  for (int b = 0; b < kChunkBlocks; ++b) {
    const int k = c * kChunk + b * kGroup + 2 * l16;
    v0[b] = 0.f;
    v1[b] = 0.f;
    if (valid && k < K) {
      if (BF16) {
        const uint32_t u = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(x) + src * ldx + k);
        v0[b] = bf16_lo(u);
        v1[b] = bf16_hi(u);
      } else {
        const float2 f = *reinterpret_cast<const float2*>(reinterpret_cast<const float*>(x) + src * ldx + k);
        v0[b] = f.x;
        v1[b] = f.y;
      }
    }
  }
  // x3 (the routed gate/up product when the token-major rows are skipped): also the third term
  // of the slot's token row (a token in several tiles gets the same bytes each time)
  const bool third = x3 && valid && c < kX3Flags;
  Quant3 q3[kChunkBlocks];
  bool any3 = false;
#pragma unroll
  for (int b = 0; b < kChunkBlocks; ++b) {
    const int k = c * kChunk + b * kGroup + 2 * l16;
    const Quant2 q = quant2_block16(v0[b], v1[b]);
    *reinterpret_cast<uint16_t*>(chunk + (at_code_off(i, k, 0) - cbase)) = (uint16_t)q.hi;
    *reinterpret_cast<uint16_t*>(chunk + (at_code_off(i, k, 1) - cbase)) = (uint16_t)q.lo;
    if (l16 == 0) {
      chunk[at_scale_off(i, k, 0) - cbase] = (uint8_t)q.s_hi;
      chunk[at_scale_off(i, k, 1) - cbase] = (uint8_t)q.s_lo;
    }
    q3[b] = third ? quant3_block16(v0[b], v1[b], q) : Quant3{0u, 127u, false};
    any3 |= q3[b].flag;
  }
  if (third) x3_store(x3 + src * x3_row_bytes(K), nsc, c, l16, q3, any3, x3_any);
  __syncthreads();
  uint8_t* dst = out + (long long)t * at_tile_bytes(K) + cbase;
  for (int o = threadIdx.x * 16; o < kAtChunkBytes; o += 256 * 16)
    *reinterpret_cast<i32x4*>(dst + o) = *reinterpret_cast<const i32x4*>(chunk + o);
}

template <bool BF16>
__global__ __launch_bounds__(256) void quant_tiles_kernel(const void* x, long long ldx, int rows, int K,
                                                          const int4* tiles, const int* n_tiles, const int* row_map,
                                                          int large_only, const int4* groups, const int* n_groups,
                                                          const uint8_t* xt, const int* meta, uint8_t* out,
                                                          uint8_t* x3, int* x3_any)
{
  __shared__ __attribute__((aligned(16))) uint8_t chunk[kAtChunkBytes];
  const int nsc = at_nchunks(K);
  if (groups) {
    // the large buckets' tiles, by groups: a resident grid loops over (group, tile, super-chunk),
    // so a routing without large buckets costs one read of the group count per work-group
    const int total = *n_groups * kGroupTiles * nsc;
    for (int wi = blockIdx.x; wi < total; wi += gridDim.x) {
      const int g = wi / (kGroupTiles * nsc), r = wi - g * (kGroupTiles * nsc);
      const int ti = r / nsc, c = r - ti * nsc;
      const int4 gr = groups[g];
      if (ti >= gr.z) continue;  // uniform
      const int t = gr.y + ti;
      const int4 tt = tiles[t];
      __syncthreads();  // the previous item's reads of chunk are complete
      quant_tile_chunk<BF16>(x, ldx, rows, K, t, c, tt.y, tt.z, row_map, xt, meta, out, x3, x3_any, chunk);
    }
    return;
  }
  const int t = (int)(blockIdx.x / nsc), c = (int)(blockIdx.x - (long long)t * nsc);
  const int ntiles = tiles ? *n_tiles : (rows + kFwdRowsPerTile - 1) / kFwdRowsPerTile;
  if (t >= ntiles) return;  // the whole work-group
  int row0, nrows;
  if (tiles) {
    const int4 tt = tiles[t];
    if (large_only && tt.w == 0) return;  // the whole work-group: a small bucket's tile
    row0 = tt.y;
    nrows = tt.z;
  } else {
    row0 = t * kFwdRowsPerTile;
    nrows = min(kFwdRowsPerTile, rows - row0);
  }
  quant_tile_chunk<BF16>(x, ldx, rows, K, t, c, row0, nrows, row_map, xt, meta, out, x3, x3_any, chunk);
}

// ---------------------------------------------------------------- fp32 -> bf16 hi + lo
__global__ __launch_bounds__(256) void split_bf16_kernel(const float* x, long long ldx, int rows, int K,
                                                         int Kpad, uint16_t* hi, uint16_t* lo)
{
  const long long idx = ((long long)blockIdx.x * 256 + threadIdx.x) * 2;
  const long long total = (long long)rows * Kpad;
  if (idx >= total) return;
  const int row = (int)(idx / Kpad);
  const int k = (int)(idx - (long long)row * Kpad);
  float v0 = 0.f, v1 = 0.f;
  if (k < K) v0 = x[row * ldx + k];
  if (k + 1 < K) v1 = x[row * ldx + k + 1];
  const uint32_t h = pack_bf16(v0, v1);
  const uint32_t l = pack_bf16(v0 - bf16_lo(h), v1 - bf16_hi(h));
  *reinterpret_cast<uint32_t*>(hi + idx) = h;
  *reinterpret_cast<uint32_t*>(lo + idx) = l;
}

// ---------------------------------------------------------------- exact dequantisation
// out[R, K] = decoded W (lazy_lora/native/mxfp4_gemm.c:142-150), fp32 or bf16
// (lazy_lora/streaming/expert_streamer.py:104-154, whose default output is bf16). The hardware
// fp4 -> bf16 conversion is exact for scale bytes 0..252, and so is either output (bf16 widens to
// fp32 by a 16-bit shift); bytes >= 253 give +-0 with the code's sign, as LUT[code] * 0.0f does.
template <bool BF16>
__global__ __launch_bounds__(256) void dequant_kernel(void* out, const uint8_t* packed, const uint8_t* scales, int K,
                                                      int R)
{
  const long long blk = (long long)blockIdx.x * 256 + threadIdx.x;  // one 32-element block
  const int nb = K / kGroup;
  if (blk >= (long long)R * nb) return;
  const int r = (int)(blk / nb);
  const int b = (int)(blk - (long long)r * nb);
  const uint8_t* src = packed + (long long)r * (K / 2) + b * 16;
  uint32_t words[4];
  if ((reinterpret_cast<uintptr_t>(src) & 15) == 0) {
    const i32x4 v = ldg16(src);
    words[0] = (uint32_t)v[0]; words[1] = (uint32_t)v[1]; words[2] = (uint32_t)v[2]; words[3] = (uint32_t)v[3];
  } else {
#pragma unroll
    for (int d = 0; d < 4; ++d)
      words[d] = (uint32_t)src[4 * d] | ((uint32_t)src[4 * d + 1] << 8) | ((uint32_t)src[4 * d + 2] << 16) |
                 ((uint32_t)src[4 * d + 3] << 24);
  }
  const uint32_t s = scales[(long long)r * nb + b];
  const long long e0 = (long long)r * K + b * kGroup;  // first output element of the block
  // the block's 32 values as 16 bf16 pairs (element 2n in the low half of pair n)
  uint32_t pr[16];
  if (s >= 253u) {
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int n = 0; n < 4; ++n)  // the sign bits (bit 3) of codes 2n and 2n + 1 of word d
        pr[4 * d + n] = (((words[d] >> (8 * n)) & 8u) << 12) | (((words[d] >> (8 * n + 4)) & 8u) << 28);
  } else {
    const float scale = bits_f(s << 23);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      pr[4 * d + 0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(words[d], scale, 0));
      pr[4 * d + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(words[d], scale, 1));
      pr[4 * d + 2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(words[d], scale, 2));
      pr[4 * d + 3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(words[d], scale, 3));
    }
  }
  if (BF16) {
    uint32_t* dst = reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(out) + e0);
#pragma unroll
    for (int n = 0; n < 16; ++n) dst[n] = pr[n];
  } else {
    float* dst = static_cast<float*>(out) + e0;
#pragma unroll
    for (int n = 0; n < 16; ++n) {
      dst[2 * n] = bf16_lo(pr[n]);
      dst[2 * n + 1] = bf16_hi(pr[n]);
    }
  }
}

constexpr int kQuantResidentBlocks = 1536;  // resident grid of quant_tiles over the large buckets: six per CU

// ---------------------------------------------------------------- routing
// (token, slot) pairs are bucketed by expert: counts -> exclusive offsets -> placement.
// The order of pairs inside a bucket is left to atomics; nothing downstream depends on it,
// because every row of a product is computed independently and the combine gathers each
// token's slots in slot order.
__device__ __forceinline__ int read_idx(const void* idx, int idx64, long long p)
{
  return idx64 ? (int)reinterpret_cast<const long long*>(idx)[p] : reinterpret_cast<const int*>(idx)[p];
}

// counter[e] += 1 for every lane with `valid` set; returns the lane's slot (the counter's old value
// plus the lane's rank among the wave's lanes with the same e). The lanes of the first
// kAggRounds distinct experts of the wave add with one atomic per expert (buckets shared by many
// lanes of a wave, as when tokens come sorted by expert, would otherwise serialise on one
// address); any lanes left take one atomic each.
__device__ __forceinline__ int wave_bucket_add(int* counter, int e, bool valid)
{
  constexpr int kAggRounds = 2;
  const int lane = (int)(threadIdx.x & 63);
  uint64_t todo = __builtin_amdgcn_ballot_w64(valid);
  int pos = -1;
#pragma unroll
  for (int r = 0; r < kAggRounds; ++r) {
    if (todo == 0) break;
    const int leader = __builtin_ctzll(todo);
    const int el = __builtin_amdgcn_readlane(e, leader);
    const bool mine = valid && e == el;
    const uint64_t m = __builtin_amdgcn_ballot_w64(mine);
    int base = 0;
    if (lane == leader) base = atomicAdd(&counter[el], __popcll(m));
    base = __builtin_amdgcn_readlane(base, leader);
    if (mine) pos = base + __popcll(m & ((1ull << lane) - 1ull));
    todo &= ~m;
  }
  if (valid && pos < 0) pos = atomicAdd(&counter[e], 1);
  return pos;
}

// An LDS counter add for route_one_kernel: when every valid lane of the wave routes to one expert
// (tokens sorted by expert), one atomic for the wave; otherwise one per lane (distinct experts
// across the wave, the usual case, gain nothing from aggregation). Called by the whole wave.
__device__ __forceinline__ int lds_bucket_add(int* counter, int e, bool valid)
{
  const int lane = (int)(threadIdx.x & 63);
  const uint64_t vm = __builtin_amdgcn_ballot_w64(valid);
  if (vm == 0) return -1;
  const int leader = __builtin_ctzll(vm);
  const int el = __builtin_amdgcn_readlane(e, leader);
  if (__builtin_amdgcn_ballot_w64(valid && e == el) == vm) {  // uniform
    int base = 0;
    if (lane == leader) base = atomicAdd(&counter[el], __popcll(vm));
    base = __builtin_amdgcn_readlane(base, leader);
    return valid ? base + __popcll(vm & ((1ull << lane) - 1ull)) : -1;
  }
  return valid ? atomicAdd(&counter[e], 1) : -1;
}

__global__ __launch_bounds__(256) void route_count_kernel(const void* idx, int idx64, int P, int E, int* counts,
                                                          int* meta)
{
  const int p = blockIdx.x * 256 + threadIdx.x;
  const long long raw = p < P ? (idx64 ? reinterpret_cast<const long long*>(idx)[p] : reinterpret_cast<const int*>(idx)[p]) : 0;
  const bool valid = p < P && raw >= 0 && raw < E;
  if (p < P && !valid) atomicOr(&meta[1], 1);
  wave_bucket_add(counts, valid ? (int)raw : 0, valid);
}

// Single work-group: exclusive scan of counts and of per-expert tile counts, tile list. An
// expert with at least kGroupMinTiles tiles (a large bucket) also gets its tiles listed as
// groups of up to kGroupTiles consecutive tiles, and again as wide groups of up to
// kWideGroupTiles: every full wide group first (expert order), then the experts' last, partial
// ones, so that a work queue taking them in order hands out the largest items first. The other
// experts' tile indices go to the small-bucket list. meta = {tiles, flags, small tiles, groups,
// wide groups, full wide groups}. cursor[e] gets offsets[e] (cursor may be counts itself: each
// expert's count is read before its cursor is written, by the same thread).
__device__ __forceinline__ void route_scan(const int* counts, int E, int* offsets, int* cursor, int4* tiles,
                                           int* small_tiles, int4* groups, int4* wgroups, int* meta, int* s_rows,
                                           int* s_tiles, int* s_small, int* s_groups, int* s_wgroups, int* s_wpart)
{
  const int t = threadIdx.x;
  const int per = (E + 1023) / 1024;
  const int e0 = min(t * per, E), e1 = min(e0 + per, E);
  int rows = 0, nt = 0, ns = 0, ng = 0, nw = 0, np = 0;  // nw: full wide groups, np: partial ones
  for (int e = e0; e < e1; ++e) {
    const int et = (counts[e] + kFwdRowsPerTile - 1) / kFwdRowsPerTile;
    rows += counts[e];
    nt += et;
    if (et >= kGroupMinTiles) {
      ng += (et + kGroupTiles - 1) / kGroupTiles;
      nw += et / kWideGroupTiles;
      np += et % kWideGroupTiles ? 1 : 0;
    } else {
      ns += et;
    }
  }
  s_rows[t] = rows;
  s_tiles[t] = nt;
  s_small[t] = ns;
  s_groups[t] = ng;
  s_wgroups[t] = nw;
  s_wpart[t] = np;
  __syncthreads();
  for (int d = 1; d < 1024; d <<= 1) {  // Hillis-Steele inclusive scans
    const int a = t >= d ? s_rows[t - d] : 0;
    const int b = t >= d ? s_tiles[t - d] : 0;
    const int c = t >= d ? s_small[t - d] : 0;
    const int g = t >= d ? s_groups[t - d] : 0;
    const int w = t >= d ? s_wgroups[t - d] : 0;
    const int v = t >= d ? s_wpart[t - d] : 0;
    __syncthreads();
    s_rows[t] += a;
    s_tiles[t] += b;
    s_small[t] += c;
    s_groups[t] += g;
    s_wgroups[t] += w;
    s_wpart[t] += v;
    __syncthreads();
  }
  const int n_full = s_wgroups[1023];
  int row_off = s_rows[t] - rows, tile_off = s_tiles[t] - nt, small_off = s_small[t] - ns, group_off = s_groups[t] - ng,
      wgroup_off = s_wgroups[t] - nw, wpart_off = n_full + s_wpart[t] - np;
  for (int e = e0; e < e1; ++e) {
    const int c = counts[e];
    const int et = (c + kFwdRowsPerTile - 1) / kFwdRowsPerTile;
    offsets[e] = row_off;
    cursor[e] = row_off;
    if (et >= kGroupMinTiles) {
      for (int g = 0; g < et; g += kGroupTiles) groups[group_off++] = make_int4(e, tile_off + g, min(kGroupTiles, et - g), 0);
      for (int g = 0; g + kWideGroupTiles <= et; g += kWideGroupTiles)
        wgroups[wgroup_off++] = make_int4(e, tile_off + g, kWideGroupTiles, 0);
      if (et % kWideGroupTiles)
        wgroups[wpart_off++] = make_int4(e, tile_off + et / kWideGroupTiles * kWideGroupTiles, et % kWideGroupTiles, 0);
    } else {
      for (int m = 0; m < et; ++m) small_tiles[small_off++] = tile_off + m;
    }
    for (int m = 0; m < c; m += kFwdRowsPerTile)
      tiles[tile_off++] = make_int4(e, row_off + m, min(kFwdRowsPerTile, c - m), et >= kGroupMinTiles ? 1 : 0);
    row_off += c;
  }
  if (t == 1023) {
    offsets[E] = s_rows[1023];
    meta[0] = s_tiles[1023];
    meta[2] = s_small[1023];
    meta[3] = s_groups[1023];
    meta[4] = s_wgroups[1023] + s_wpart[1023];
    meta[5] = s_wgroups[1023];
  }
}

__global__ __launch_bounds__(1024) void route_scan_kernel(const int* counts, int E, int* offsets, int* cursor,
                                                          int4* tiles, int* small_tiles, int4* groups, int4* wgroups,
                                                          int* meta)
{
  __shared__ int s[6][1024];
  route_scan(counts, E, offsets, cursor, tiles, small_tiles, groups, wgroups, meta, s[0], s[1], s[2], s[3], s[4], s[5]);
}

// The whole routing in one work-group (P <= kRouteOneP pairs, E <= kRouteOneE experts): counts
// with LDS atomics, the scan above (cursors in LDS), then the placement with LDS atomics; all 16
// meta words are written. Replaces five launches (two clears, count, scan, place) when the pairs
// are few. A wave whose pairs all go to one expert (tokens sorted by expert) adds to its counter
// once rather than serialising 64 atomics on one address, and up to kRouteStageP pairs the
// placed token and weight of each bucket position are staged in LDS and written out in position
// order (contiguous stores) rather than scattered from the one CU.
constexpr int kRouteOneP = 65536;
constexpr int kRouteOneE = 8192;
constexpr int kRouteStageP = 8192;

__global__ __launch_bounds__(1024) void route_one_kernel(const void* idx, int idx64, const float* w, int P, int k,
                                                         int E, int* counts, int* offsets, int4* tiles,
                                                         int* small_tiles, int4* groups, int4* wgroups, int* meta,
                                                         int* pair_token, float* pair_w, int* pair_of)
{
  __shared__ int s[6][1024];
  __shared__ int s_cnt[kRouteOneE];
  __shared__ int s_tok[kRouteStageP];
  __shared__ float s_w[kRouteStageP];
  __shared__ int s_bad;
  const int t = threadIdx.x;
  const bool stage = P <= kRouteStageP;
  for (int e = t; e < E; e += 1024) s_cnt[e] = 0;
  if (t == 0) s_bad = 0;
  __syncthreads();
  // 8 pairs per thread and round, their index loads all issued before the atomics
  for (int p0 = 0; p0 < P; p0 += 8 * 1024) {
    int raw[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int p = p0 + u * 1024 + t;
      raw[u] = p < P ? read_idx(idx, idx64, p) : 0;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {  // wave-aggregated: pairs of one expert in a wave add once
      const bool in = p0 + u * 1024 + t < P;
      const bool valid = in && raw[u] >= 0 && raw[u] < E;
      if (in && !valid) s_bad = 1;
      lds_bucket_add(s_cnt, valid ? raw[u] : 0, valid);
    }
  }
  __syncthreads();
  for (int e = t; e < E; e += 1024) counts[e] = s_cnt[e];
  // meta: the scan writes words 0 and 2..5; the flags word and words 6..15 (the products' flags
  // and work-queue counters, which start at zero) are written here
  if (t == 1) meta[1] = s_bad;
  if (t >= 6 && t < 16) meta[t] = 0;
  route_scan(s_cnt, E, offsets, s_cnt, tiles, small_tiles, groups, wgroups, meta, s[0], s[1], s[2], s[3], s[4], s[5]);
  __syncthreads();
  for (int p0 = 0; p0 < P; p0 += 8 * 1024) {
    int raw[8];
    float wv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int p = min(p0 + u * 1024 + t, P - 1);
      raw[u] = read_idx(idx, idx64, p);
      wv[u] = w[p];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int p = p0 + u * 1024 + t;
      const bool valid = p < P && raw[u] >= 0 && raw[u] < E;
      const int pos = lds_bucket_add(s_cnt, valid ? raw[u] : 0, valid);
      if (p >= P) continue;
      if (!valid) {
        pair_of[p] = -1;
        continue;
      }
      if (stage) {
        s_tok[pos] = p / k;
        s_w[pos] = wv[u];
      } else {
        pair_token[pos] = p / k;
        pair_w[pos] = wv[u];
      }
      pair_of[p] = pos;
    }
  }
  if (stage) {
    __syncthreads();
    const int placed = s[0][1023];  // the scan's total: pairs with a valid expert id
    for (int i = t; i < placed; i += 1024) {
      pair_token[i] = s_tok[i];
      pair_w[i] = s_w[i];
    }
  }
}

__global__ __launch_bounds__(256) void route_place_kernel(const void* idx, int idx64, const float* w, int P, int k,
                                                          int E, int* cursor, int* pair_token, float* pair_w,
                                                          int* pair_of)
{
  const int p = blockIdx.x * 256 + threadIdx.x;
  const long long raw = p < P ? (idx64 ? reinterpret_cast<const long long*>(idx)[p] : reinterpret_cast<const int*>(idx)[p]) : 0;
  const bool valid = p < P && raw >= 0 && raw < E;
  const int pos = wave_bucket_add(cursor, valid ? (int)raw : 0, valid);
  if (p >= P) return;
  if (!valid) {
    pair_of[p] = -1;
    return;
  }
  pair_token[pos] = p / k;
  pair_w[pos] = w[p];
  pair_of[p] = pos;
}

// ---------------------------------------------------------------- combines
// out[t, :] = sum over the token's slots, in slot order, of the pair rows (already weighted).
// sum over a token's slots, in slot order, of 4 columns of its pairs' rows (p < 0: no row).
// Up to 8 slots the row loads are all issued before the adds; each row is read once (streaming).
MX_DEV float4 slot_sum4(const float* rows, long long ld, const int* slots, int k, int d)
{
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (k <= 8) {
    int p[8];
    f32x4 v[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) p[s] = s < k ? slots[s] : -1;
#pragma unroll
    for (int s = 0; s < 8; ++s)
      v[s] = p[s] >= 0 ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(rows + (long long)p[s] * ld + d))
                       : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 8; ++s)
      if (p[s] >= 0) acc += v[s];  // a skipped slot adds nothing (not even +0, which would turn -0 into +0)
  } else {
    for (int s = 0; s < k; ++s) {
      const int q = slots[s];
      if (q >= 0) acc += *reinterpret_cast<const f32x4*>(rows + (long long)q * ld + d);
    }
  }
  return make_float4(acc[0], acc[1], acc[2], acc[3]);
}

// Top-1 routing writes each token's row straight from the down product; a token whose id was
// outside [0, E) has no pair row and gets zeros here instead (one work-group per 64 tokens; rows
// are written only for such tokens).
__global__ __launch_bounds__(256) void zero_unrouted_kernel(float* out, long long ldo, int D, const int* pair_of,
                                                            int N)
{
  const int t0 = blockIdx.x * 64;
  const int t = t0 + (int)(threadIdx.x & 63);
  const bool bad = t < N && pair_of[t] < 0;
  uint64_t m = __builtin_amdgcn_ballot_w64(bad);  // the same in every wave
  while (m) {
    const int r = t0 + __builtin_ctzll(m);
    m &= m - 1;
    for (int d = threadIdx.x; d < D; d += 256) out[(long long)r * ldo + d] = 0.f;
  }
}

__global__ __launch_bounds__(256) void combine_kernel(float* out, const float* ypair, long long ldy,
                                                      const int* pair_of, int N, int k, int D)
{
  const int t = blockIdx.y;
  const int d = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (t >= N || d >= D) return;
  *reinterpret_cast<float4*>(out + (long long)t * D + d) = slot_sum4(ypair, ldy, pair_of + (long long)t * k, k, d);
}

__global__ __launch_bounds__(256) void combine_bwd_kernel(float* grad_h, float* grad_w, const float* dxpair,
                                                          long long ldy, const float* gw_part, int n_ct,
                                                          const int* pair_of, int N, int k, int D)
{
  const int t = blockIdx.y;
  const int d = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (t >= N) return;
  if (blockIdx.x == 0) {
    for (int s = threadIdx.x; s < k; s += 256) {
      const int p = pair_of[t * k + s];
      float gsum = 0.f;
      if (p >= 0)
        for (int c = 0; c < n_ct; ++c) gsum += gw_part[(long long)p * n_ct + c];
      grad_w[t * k + s] = gsum;
    }
  }
  if (d >= D) return;
  *reinterpret_cast<float4*>(grad_h + (long long)t * D + d) = slot_sum4(dxpair, ldy, pair_of + (long long)t * k, k, d);
}

// The same quantisation into the XT layout: one work-group per (16 rows, super-chunk), rows
// r0 .. r0 + 15 of x; rows at or past `rows` (at least the one that follows the last) get zeros,
// the row a tile's unused slots read. Only the one-tile work-groups read this layout: with the
// routing's meta (non-null), a layer whose buckets are all large (groups, no small tiles) skips it.
// x3 (non-null): also the third term of the flagged blocks (quant3_block16) in the X3 layout,
// written whether or not XT is skipped (every gate/up work-group reads it).
template <bool BF16>
__global__ __launch_bounds__(256) void quant_rows_kernel(const void* x, long long ldx, int rows, int K,
                                                         const int* meta, uint8_t* out, uint8_t* x3, int* x3_any)
{
  if (meta && meta[2] == 0 && meta[3] > 0) return;  // the whole grid (quant_tiles writes X3 then)
  __shared__ __attribute__((aligned(16))) uint8_t chunk[16 * kXtChunkBytes];
  const int nsc = at_nchunks(K);
  const int rg = (int)(blockIdx.x / nsc), c = (int)(blockIdx.x - (long long)rg * nsc);
  const int i = threadIdx.x >> 4, l16 = threadIdx.x & 15;
  const int row = rg * 16 + i;
  const bool valid = row < rows;
  const int cbase = c * kXtChunkBytes;  // xt_*_off are row-relative
  float v0[kChunkBlocks], v1[kChunkBlocks];
#pragma unroll
  for (int b = 0; b < kChunkBlocks; ++b) {
    const int k = c * kChunk + b * kGroup + 2 * l16;
    v0[b] = 0.f;
    v1[b] = 0.f;
    if (valid && k < K) {
      if (BF16) {
        const uint32_t u = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(x) + (long long)row * ldx + k);
        v0[b] = bf16_lo(u);
        v1[b] = bf16_hi(u);
      } else {
        const float2 f = *reinterpret_cast<const float2*>(reinterpret_cast<const float*>(x) + (long long)row * ldx + k);
        v0[b] = f.x;
        v1[b] = f.y;
      }
    }
  }
  uint8_t* mine = chunk + i * kXtChunkBytes;
  const bool third = x3 && c < kX3Flags;
  Quant3 q3[kChunkBlocks];
  bool any3 = false;
#pragma unroll
  for (int b = 0; b < kChunkBlocks; ++b) {
    const int k = c * kChunk + b * kGroup + 2 * l16;
    const Quant2 q = quant2_block16(v0[b], v1[b]);
    *reinterpret_cast<uint16_t*>(mine + (xt_code_off(k, 0) - cbase)) = (uint16_t)q.hi;
    *reinterpret_cast<uint16_t*>(mine + (xt_code_off(k, 1) - cbase)) = (uint16_t)q.lo;
    if (l16 == 0) {
      mine[xt_scale_off(k, 0) - cbase] = (uint8_t)q.s_hi;
      mine[xt_scale_off(k, 1) - cbase] = (uint8_t)q.s_lo;
    }
    q3[b] = third ? quant3_block16(v0[b], v1[b], q) : Quant3{0u, 127u, false};
    any3 |= q3[b].flag;
  }
  if (third) x3_store(x3 + (long long)row * x3_row_bytes(K), nsc, c, l16, q3, any3, x3_any);
  __syncthreads();
  // 16 rows x 66 sixteen-byte units, each row's chunk contiguous in memory
  const long long rb = xt_row_bytes(K);
  for (int u = threadIdx.x; u < 16 * (kXtChunkBytes / 16); u += 256) {
    const int rr = u / (kXtChunkBytes / 16), o = (u - rr * (kXtChunkBytes / 16)) * 16;
    *reinterpret_cast<i32x4*>(out + (long long)(rg * 16 + rr) * rb + cbase + o) =
        *reinterpret_cast<const i32x4*>(chunk + rr * kXtChunkBytes + o);
  }
}

__global__ __launch_bounds__(256) void zero_kernel(uint32_t* p, long long n_words)
{
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n_words; i += (long long)gridDim.x * 256) p[i] = 0u;
}

}  // namespace

hipError_t launch_quant_tiles(const void* x, int x_bf16, long long ldx, int rows, int K, const int4* tiles,
                              const int* n_tiles, int max_tiles, const int* row_map, int large_only, const uint8_t* xt,
                              const int* meta, uint8_t* out, uint8_t* x3, int* x3_any, hipStream_t s,
                              const int4* groups, const int* n_groups)
{
  long long blocks = (long long)max_tiles * at_nchunks(K);  // (tile, super-chunk) work-groups
  if (blocks == 0) return hipSuccess;
  if (xt && (!meta || !row_map || !tiles)) return hipErrorInvalidValue;
  if (x3 && (!row_map || !x3_any)) return hipErrorInvalidValue;
  if (groups && (!large_only || !tiles || !n_groups)) return hipErrorInvalidValue;
  if (groups) blocks = std::min(blocks, (long long)kQuantResidentBlocks);  // a resident grid over the groups
  dim3 grid((unsigned)blocks), block(256);
  if (x_bf16)
    hipLaunchKernelGGL(quant_tiles_kernel<true>, grid, block, 0, s, x, ldx, rows, K, tiles, n_tiles, row_map,
                       large_only, groups, n_groups, xt, meta, out, x3, x3_any);
  else
    hipLaunchKernelGGL(quant_tiles_kernel<false>, grid, block, 0, s, x, ldx, rows, K, tiles, n_tiles, row_map,
                       large_only, groups, n_groups, xt, meta, out, x3, x3_any);
  return hipGetLastError();
}

hipError_t launch_quant_rows(const void* x, int x_bf16, long long ldx, int rows, int K, const int* meta, uint8_t* out,
                             uint8_t* x3, int* x3_any, hipStream_t s)
{
  const long long groups = (long long)xt_rows(rows) / 16 * at_nchunks(K);  // (16 rows, super-chunk)
  if (groups == 0) return hipSuccess;
  if (x3 && !x3_any) return hipErrorInvalidValue;
  dim3 grid((unsigned)groups), block(256);
  if (x_bf16) hipLaunchKernelGGL(quant_rows_kernel<true>, grid, block, 0, s, x, ldx, rows, K, meta, out, x3, x3_any);
  else hipLaunchKernelGGL(quant_rows_kernel<false>, grid, block, 0, s, x, ldx, rows, K, meta, out, x3, x3_any);
  return hipGetLastError();
}

hipError_t launch_split_bf16(const float* x, long long ldx, int rows, int K, int Kpad, uint16_t* hi, uint16_t* lo,
                             hipStream_t s)
{
  const long long pairs = (long long)rows * Kpad / 2;
  if (pairs == 0) return hipSuccess;
  dim3 grid((unsigned)((pairs + 255) / 256)), block(256);
  hipLaunchKernelGGL(split_bf16_kernel, grid, block, 0, s, x, ldx, rows, K, Kpad, hi, lo);
  return hipGetLastError();
}

hipError_t launch_dequant(void* out, int out_bf16, const uint8_t* packed, const uint8_t* scales, int K, int R,
                          hipStream_t s)
{
  const long long blocks = (long long)R * (K / kGroup);
  if (blocks == 0) return hipSuccess;
  dim3 grid((unsigned)((blocks + 255) / 256)), block(256);
  if (out_bf16) hipLaunchKernelGGL(dequant_kernel<true>, grid, block, 0, s, out, packed, scales, K, R);
  else hipLaunchKernelGGL(dequant_kernel<false>, grid, block, 0, s, out, packed, scales, K, R);
  return hipGetLastError();
}

hipError_t launch_zero(void* p, size_t bytes, hipStream_t s)
{
  const long long words = (long long)(bytes / 4);
  if (words == 0) return hipSuccess;
  long long blocks = (words + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(zero_kernel, dim3((unsigned)blocks), dim3(256), 0, s, reinterpret_cast<uint32_t*>(p), words);
  return hipGetLastError();
}

hipError_t launch_route(const void* topk_idx, int idx64, const float* topk_w, int N, int k, int E, int* counts,
                        int* offsets, int* cursor, int4* tiles, int* small_tiles, int4* groups, int4* wgroups,
                        int* meta, int* pair_token, float* pair_w, int* pair_of, hipStream_t s)
{
  const int P = N * k;
  if (P <= kRouteOneP && E <= kRouteOneE) {
    hipLaunchKernelGGL(route_one_kernel, dim3(1), dim3(1024), 0, s, topk_idx, idx64, topk_w, P, k, E, counts, offsets,
                       tiles, small_tiles, groups, wgroups, meta, pair_token, pair_w, pair_of);
    return hipGetLastError();
  }
  hipError_t e = launch_zero(counts, sizeof(int) * (size_t)E, s);
  if (e != hipSuccess) return e;
  e = launch_zero(meta, sizeof(int) * 16, s);
  if (e != hipSuccess) return e;
  if (P > 0) hipLaunchKernelGGL(route_count_kernel, dim3((P + 255) / 256), dim3(256), 0, s, topk_idx, idx64, P, E, counts, meta);
  hipLaunchKernelGGL(route_scan_kernel, dim3(1), dim3(1024), 0, s, counts, E, offsets, cursor, tiles, small_tiles,
                     groups, wgroups, meta);
  if (P > 0)
    hipLaunchKernelGGL(route_place_kernel, dim3((P + 255) / 256), dim3(256), 0, s, topk_idx, idx64, topk_w, P, k, E,
                       cursor, pair_token, pair_w, pair_of);
  return hipGetLastError();
}

hipError_t launch_combine(float* out, const float* ypair, long long ldy, const int* pair_of, int N, int k, int D,
                          hipStream_t s)
{
  if (N == 0 || D == 0) return hipSuccess;
  dim3 grid((unsigned)((D / 4 + 255) / 256), (unsigned)N), block(256);
  hipLaunchKernelGGL(combine_kernel, grid, block, 0, s, out, ypair, ldy, pair_of, N, k, D);
  return hipGetLastError();
}

hipError_t launch_zero_unrouted(float* out, long long ldo, int D, const int* pair_of, int N, hipStream_t s)
{
  if (N <= 0 || D <= 0) return hipSuccess;
  hipLaunchKernelGGL(zero_unrouted_kernel, dim3((unsigned)((N + 63) / 64)), dim3(256), 0, s, out, ldo, D, pair_of, N);
  return hipGetLastError();
}

hipError_t launch_combine_bwd(float* grad_h, float* grad_w, const float* dxpair, long long ldy, const float* gw_part,
                              int n_ct, const int* pair_of, int N, int k, int D, hipStream_t s)
{
  if (N == 0) return hipSuccess;
  dim3 grid((unsigned)((D / 4 + 255) / 256 > 0 ? (D / 4 + 255) / 256 : 1), (unsigned)N), block(256);
  hipLaunchKernelGGL(combine_bwd_kernel, grid, block, 0, s, grad_h, grad_w, dxpair, ldy, gw_part, n_ct, pair_of, N,
                     k, D);
  return hipGetLastError();
}

}  // namespace mx
