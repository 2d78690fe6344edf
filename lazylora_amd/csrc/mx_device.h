// Device-side building blocks shared by the MXFP4 kernels (gfx950 / MI355X only).
//
// Conventions used by every kernel in this directory:
//  * A weight matrix W is logically [R, K] and stored the way LazyLoRA's checkpoints and
//    lazy_lora/native/mxfp4_gemm.c:12-15 store it: packed [R, K/2] bytes, low nibble = even
//    element, plus scales [R, K/32] E8M0 bytes. A scale byte >= 253 makes its 32-element
//    group contribute zero (mxfp4_gemm.c:16-18).
//  * Activations that feed the forward products are held as a two-term e4m3 split
//    ("AT" layout, see below): x ~= (hi + lo) with each term carrying its own E8M0 scale per
//    32-element block. hi alone keeps 4 significant bits; hi + lo keeps ~8, which puts the
//    rounding error of an activation below that of bf16.
//  * The forward products run on v_mfma_scale_f32_16x16x128_f8f6f4 with A = e4m3 activations
//    and B = the packed fp4 weights exactly as stored, so weights are never decoded in the
//    forward pass. Lane layouts (measured on the hardware):
//      B (fp4, 4 VGPRs): lane (j = l%16, g = l/16) holds logical K [32g, 32g+32) of column j,
//                        i.e. one whole 16-byte MX block; its scale is the lane's own byte.
//      A (fp8, 8 VGPRs): lane (i = l%16, g) holds logical K [16g, 16g+16) in bytes 0-15 and
//                        [64+16g, 64+16g+16) in bytes 16-31; the lane's scale byte applies
//                        to logical block g of row i.
//      C: lane (j, g) holds rows 4g..4g+3 of column j.
//    op_sel q (0..3) picks byte q of the 32-bit scale register for A and B alike.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

#define MX_DEV __device__ __forceinline__

namespace mx {

constexpr int kGroup = 32;        // elements per MX block
constexpr int kChunk = 512;       // K elements per "super-chunk" of the forward main loop
constexpr int kChunkBlocks = 16;  // MX blocks per super-chunk

// ------------------------------------------------------------------ AT activation layout
// The A operand of the forward products is stored tile-major, in exactly the order the MFMA
// lanes consume it, so every activation load instruction of a wave reads 1 KiB contiguous.
// Rows are grouped in tiles of 16 (the work tiles of the product; unused slots hold zeros).
// K is cut into super-chunks of 512 elements (16 MX blocks). The forward loop gives MFMA q
// (q = 0..3) of super-chunk c the blocks 16c + 4b + q as its logical blocks b = 0..3, so a
// weight lane's 4 operands are 4 consecutive MX blocks of one row.
//
// Per (tile, super-chunk) there are 16 KiB of codes and 512 B of scales:
//   codes  [q 0..3][plane hi/lo][piece 0..1][lane 0..63][16 B]
//   scales [lane 0..63][plane hi/lo][4 B: byte q = scale of block 16c + 4g + q]
// Lane l = 16g + i serves row i of the tile. Its MFMA-q operand is piece 0 (logical K
// [16g, 16g+16): block b = g/2, elements 16(g%2)..+16) then piece 1 (logical K [64+16g, ..):
// block b = 2 + g/2). Its scale register holds the scale of logical block b = g.
constexpr int kAtCodeBytes = 16384;
constexpr int kAtChunkBytes = kAtCodeBytes + 512;

__host__ __device__ inline int at_nchunks(int K) { return (K + kChunk - 1) / kChunk; }
__host__ __device__ inline long long at_tile_bytes(int K) { return (long long)at_nchunks(K) * kAtChunkBytes; }

// Byte offset, inside a tile, of elements e..e+1 (e even) of a row slot i and K index k,
// for one plane; and of the scale byte of the 32-element block holding k.
MX_DEV long long at_code_off(int i, int k, int plane)
{
  const int c = k >> 9, b = (k >> 5) & 15, e = k & 31;
  const int q = b & 3, gl = b >> 2;             // logical block of MFMA q
  const int piece = gl >> 1;
  const int g = 2 * (gl & 1) + (e >> 4);        // lane group holding these 16 elements
  return (long long)c * kAtChunkBytes + ((q * 2 + plane) * 2 + piece) * 1024 + (16 * g + i) * 16 + (e & 15);
}
MX_DEV long long at_scale_off(int i, int k, int plane)
{
  const int c = k >> 9, b = (k >> 5) & 15;
  const int q = b & 3, g = b >> 2;
  return (long long)c * kAtChunkBytes + kAtCodeBytes + (16 * g + i) * 8 + plane * 4 + q;
}

// ------------------------------------------------------------------ XT activation layout
// The same codes and scales stored once per row of x instead of once per work tile ("XT",
// token-major): the one-tile work-groups of the routed gate/up product gather each tile lane's
// pieces from the row of its token, so a token chosen by k experts is quantised and stored once,
// not k times. Per (row,
// super-chunk): 1024 B of codes [q][plane][piece][g][16 B] (the 16-byte piece that tile lane
// 16g + i takes from row i), then 32 B of scales [plane][g][4 B: byte q].
constexpr int kXtCodeBytes = 1024;
constexpr int kXtChunkBytes = kXtCodeBytes + 32;

__host__ __device__ inline long long xt_row_bytes(int K) { return (long long)at_nchunks(K) * kXtChunkBytes; }

// Byte offset, inside a row, of elements k..k+1 (k even) for one plane, and of the scale byte
// of the 32-element block holding k (the per-lane offsets of at_code_off / at_scale_off).
MX_DEV int xt_code_off(int k, int plane)
{
  const int c = k >> 9, b = (k >> 5) & 15, e = k & 31;
  const int q = b & 3, gl = b >> 2;
  const int piece = gl >> 1;
  const int g = 2 * (gl & 1) + (e >> 4);
  return c * kXtChunkBytes + (((q * 2 + plane) * 2 + piece) * 4 + g) * 16 + (e & 15);
}
MX_DEV int xt_scale_off(int k, int plane)
{
  const int c = k >> 9, b = (k >> 5) & 15;
  const int q = b & 3, g = b >> 2;
  return c * kXtChunkBytes + kXtCodeBytes + (plane * 4 + g) * 4 + q;
}

// ------------------------------------------------------------------ X3: the third term of x
// Token-major, per row x3_row_bytes(K) bytes: the third-term codes in natural element order (one
// e4m3 byte per element, at_nchunks(K) * 512), the third-term block scales (16 bytes per
// super-chunk, block b at b), then one flag byte per super-chunk (kX3Flags of them: 1 when a
// block of that super-chunk has a third term). Blocks without a third term hold zero codes. The
// third term covers the first kX3Flags super-chunks (K <= 16384); later blocks keep two terms.
constexpr int kX3Flags = 32;
__host__ __device__ inline long long x3_row_bytes(int K) { return (long long)at_nchunks(K) * 528 + kX3Flags; }

// ------------------------------------------------------------------ small helpers
MX_DEV float bits_f(uint32_t u) { return __builtin_bit_cast(float, u); }
MX_DEV uint32_t f_bits(float f) { return __builtin_bit_cast(uint32_t, f); }

// Reductions over the 16 lanes of a lane group (lanes 16n..16n+15, one DPP row), as a butterfly
// on DPP lane moves inside the VALU (a cross-lane shuffle would be an LDS permute with its round
// trip): quad_perm [1,0,3,2] gives lane ^ 1 and [2,3,0,1] lane ^ 2; after those two steps every
// quad holds one value, so row_half_mirror (7 - lane within 8) brings the other quad's value as
// lane ^ 4 would, and row_mirror (15 - lane) then the other half-row's as lane ^ 8 would. Every
// lane adds the same two operands at each step, so all 16 end with the same bits.
template <int CTRL>
MX_DEV float dpp_lane(float v)
{
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror
constexpr int kDppMirror = 0x140;      // row_mirror

MX_DEV float group16_max(float v)
{
  v = fmaxf(v, dpp_lane<kDppXor1>(v));
  v = fmaxf(v, dpp_lane<kDppXor2>(v));
  v = fmaxf(v, dpp_lane<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_lane<kDppMirror>(v));
  return v;
}
MX_DEV float group16_sum(float v)
{
  v += dpp_lane<kDppXor1>(v);
  v += dpp_lane<kDppXor2>(v);
  v += dpp_lane<kDppHalfMirror>(v);
  v += dpp_lane<kDppMirror>(v);
  return v;
}

// Two-term e4m3 quantisation of one 32-element block held 2 values per lane over 16
// consecutive lanes. hi uses scale 2^(s_hi-127) chosen from the block maximum so that
// |x / scale| < 256 (e4m3 max is 448); lo quantises the exact residual the same way.
// Returns bytes (hi0 | hi1 << 8) and (lo0 | lo1 << 8) and the two scale bytes.
struct Quant2 {
  uint32_t hi, lo;
  uint32_t s_hi, s_lo;
  float amax;  // the block's max |x|
};
MX_DEV Quant2 quant2_block16(float v0, float v1)
{
  Quant2 r;
  const float amax = group16_max(fmaxf(fabsf(v0), fabsf(v1)));
  const int eb = (int)((f_bits(amax) >> 23) & 0xFF);
  const int sb = eb > 7 ? eb - 7 : 0;
  const float inv = bits_f((uint32_t)(254 - sb) << 23);       // 2^(127 - sb)
  const float y0 = v0 * inv, y1 = v1 * inv;
  const uint32_t q = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(y0, y1, 0, false) & 0xFFFFu;
  const float d0 = y0 - __builtin_amdgcn_cvt_f32_fp8((int)q, 0);
  const float d1 = y1 - __builtin_amdgcn_cvt_f32_fp8((int)q, 1);
  const float dmax = group16_max(fmaxf(fabsf(d0), fabsf(d1)));
  const int ed = (int)((f_bits(dmax) >> 23) & 0xFF);
  uint32_t ql = 0;
  int sl = 127;
  if (ed >= 27) {  // residual above 2^-100 of the hi scale: worth a second term
    const int t = sb + ed - 134;
    sl = t > 0 ? t : 0;
    const float m = bits_f((uint32_t)(127 + sb - sl) << 23);  // 2^(sb - sl)
    ql = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(d0 * m, d1 * m, 0, false) & 0xFFFFu;
  }
  r.hi = q;
  r.lo = ql;
  r.s_hi = (uint32_t)sb;
  r.s_lo = (uint32_t)sl;
  r.amax = amax;
  return r;
}

// A third e4m3 term for blocks that two terms leave short. Two terms keep ~8 significant bits of
// the block maximum; when one element dominates its block (max |x| > 16 x the rms of the other
// 31) it usually dominates the row's dot products too (an outlier channel), and its rounding
// (up to 2^-8 relative) then shows undiluted in that token's outputs. Such blocks are flagged and
// get a third term: the residual after hi + lo, quantised again with its own scale (~12 bits for
// the maximum). For every other block the third term is zero and its flag is clear.
// Returns the third term's bytes (element 2n | 2n+1 << 8 of the lane), its scale byte and the flag
// (the same on all 16 lanes of the block). q2 is the block's two-term result.
struct Quant3 {
  uint32_t th, s_th;
  bool flag;
};
MX_DEV Quant3 quant3_block16(float v0, float v1, const Quant2& q2)
{
  Quant3 r{0u, 127u, false};
  // in the hi term's scaled domain (|y| < 256): the flag and the residual after hi + lo
  const float inv = bits_f((uint32_t)(254 - (int)q2.s_hi) << 23);  // 2^(127 - s_hi)
  const float y0 = v0 * inv, y1 = v1 * inv;
  const float m = q2.amax * inv;
  const float ss = group16_sum(y0 * y0 + y1 * y1);
  // max > 16 rms(rest) <=> 31 m^2 > 256 (ss - m^2) <=> 287 m^2 > 256 ss
  r.flag = 287.0f * m * m > 256.0f * ss;
  if (!r.flag) return r;
  const float hi0 = __builtin_amdgcn_cvt_f32_fp8((int)q2.hi, 0), hi1 = __builtin_amdgcn_cvt_f32_fp8((int)q2.hi, 1);
  // lo's codes scaled by 2^(s_hi - s_lo) in the hi domain
  const float lsc = bits_f((uint32_t)(127 + (int)q2.s_lo - (int)q2.s_hi) << 23);
  const float lo0 = __builtin_amdgcn_cvt_f32_fp8((int)q2.lo, 0) * lsc, lo1 = __builtin_amdgcn_cvt_f32_fp8((int)q2.lo, 1) * lsc;
  const float d0 = (y0 - hi0) - lo0, d1 = (y1 - hi1) - lo1;
  const float dmax = group16_max(fmaxf(fabsf(d0), fabsf(d1)));
  const int ed = (int)((f_bits(dmax) >> 23) & 0xFF);
  if (ed < 27) return r;  // nothing left worth a term (the block is exact in two terms)
  // scale 2^(t - 127) relative to x: the residual's maximum maps into [128, 256)
  const int t = (int)q2.s_hi + ed - 134;
  const int st = t > 0 ? t : 0;
  const float mm = bits_f((uint32_t)(127 + (int)q2.s_hi - st) << 23);  // 2^(s_hi - st)
  r.th = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(d0 * mm, d1 * mm, 0, false) & 0xFFFFu;
  r.s_th = (uint32_t)st;
  return r;
}

// True when any of the 4 scale bytes of w is >= 253.
MX_DEV bool any_damaged_scale(uint32_t w)
{
  return ((w & 0xFFu) >= 253u) | (((w >> 8) & 0xFFu) >= 253u) | (((w >> 16) & 0xFFu) >= 253u) |
         ((w >> 24) >= 253u);
}
// Bit 7 of each byte of the result is set when that byte of w is >= 253 (0xFD..0xFF): its top
// bit is set and its low 7 bits are >= 125, so adding 3 to them carries into bit 7.
MX_DEV uint32_t damaged_scale_bits(uint32_t w)
{
  return w & ((w & 0x7F7F7F7Fu) + 0x03030303u) & 0x80808080u;
}

// Scaled MFMA, A = e4m3 (format 0), B = fp4 (format 4). QA / QB pick the scale bytes.
template <int QA, int QB>
MX_DEV f32x4 mfma_f8f4(const i32x8& a, const i32x4& b, f32x4 c, int sa, int sb)
{
  const i32x8 b8 = {b[0], b[1], b[2], b[3], 0, 0, 0, 0};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b8, c, 0, 4, QA, sa, QB, sb);
}

MX_DEV f32x4 mfma_bf16(const bf16x8& a, const bf16x8& b, f32x4 c)
{
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

MX_DEV i32x4 ldg16(const void* p) { return *reinterpret_cast<const i32x4*>(p); }
// Streaming (non-temporal) load for data read exactly once, such as the expert weights: it
// does not push reused lines (activations, scale rows shared by work-groups) out of L2. Only
// for loads whose instruction consumes every byte of its cache lines: a line that a later
// instruction reads again is fetched again.
MX_DEV i32x4 ldg16_nt(const void* p) { return __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(p)); }

// Buffer resources: a base address and a byte count held in SGPRs. A buffer load whose VGPR
// offset plus immediate offset is at or past the count returns zeros instead of touching
// memory (the SGPR offset is not range-checked, so variable offsets go in the VGPR one).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
MX_DEV rsrc_t make_rsrc(const void* base, uint32_t bytes)
{
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// voff: per-lane (range-checked) offset, soff: uniform offset added to it (not range-checked)
MX_DEV i32x4 buf16(rsrc_t r, uint32_t voff, uint32_t soff)
{
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
}
// 16 bytes, streaming (non-temporal, as ldg16_nt)
MX_DEV i32x4 buf16_nt(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 2); }
// Streaming (nt) load with a scalar offset: for bytes each read exactly once, by whole lines.
MX_DEV i32x4 buf16_nt(rsrc_t r, uint32_t voff, uint32_t soff)
{
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 2);
}
MX_DEV uint8_t buf8(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b8(r, (int)off, 0, 0); }
MX_DEV uint32_t buf4_nt(rsrc_t r, uint32_t voff, uint32_t soff)
{
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 2);
}

// f(integral_constant<int, i>) for i = 0 .. N-1
template <int N, int I = 0, typename Fn>
MX_DEV void static_for(Fn&& f)
{
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, I + 1>(f);
  }
}

// Direct global -> LDS copy (global_load_lds_dwordx4): lane l's 16 bytes from src land at
// lds + 16 l. lds must be the same for the whole wave. Completion is counted by vmcnt.
MX_DEV void dma16(const void* src, void* lds)
{
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}
// The same copy issued from inline assembly. While a copy the compiler knows of is in
// flight, it makes every barrier wait for all outstanding loads (vmcnt(0)), which drains any
// deeper load pipeline at each barrier; this one it does not see. The caller must wait for it
// itself (wait_vm<N>) before the copied bytes are read, and nothing else may rely on M0.
MX_DEV void dma16_async(const void* src, void* lds)
{
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0) : "memory");
}
// The same copy with a uniform 64-bit base and a per-lane 32-bit byte offset (the saddr form:
// one VGPR per address instead of two).
MX_DEV void dma16_async_s(const void* base, uint32_t voff, void* lds)
{
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds);
  const uint64_t b = (uint64_t)(uintptr_t)base;
  const uint32_t blo = __builtin_amdgcn_readfirstlane((uint32_t)b), bhi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  const uint64_t bs = ((uint64_t)bhi << 32) | blo;
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(bs), "s"(m0) : "memory");
}
// dma16_async_s with the streaming (nt) hint, for bytes each copied exactly once, by whole lines.
MX_DEV void dma16_async_s_nt(const void* base, uint32_t voff, void* lds)
{
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds);
  const uint64_t b = (uint64_t)(uintptr_t)base;
  const uint32_t blo = __builtin_amdgcn_readfirstlane((uint32_t)b), bhi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  const uint64_t bs = ((uint64_t)bhi << 32) | blo;
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(bs), "s"(m0) : "memory");
}
// The 4-byte form (global_load_lds_dword): lane l's 4 bytes land at lds + 4 l.
MX_DEV void dma4_async(const void* src, void* lds)
{
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(m0) : "memory");
}
// Mark registers as redefined here (no instruction). After an explicit wait_vm that has already
// completed the loads behind them, this keeps the compiler from placing its own wait for those
// loads further down, where copies it does not know of (dma16_async) would be counted as well
// and the wait would hold for later loads too.
MX_DEV void pin(i32x4& x) { asm volatile("" : "+v"(x)); }
MX_DEV void pin(uint32_t& x) { asm volatile("" : "+v"(x)); }

// Wait until at most N vector-memory operations of this wave are outstanding (they retire in
// issue order, so everything but the last N issued is complete).
template <int N>
MX_DEV void wait_vm()
{
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
MX_DEV void wait_vm0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
MX_DEV void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Work queue of a resident grid. counter[0] hands out items in order (one atomic per work-group
// and item); counter[1] counts the work-groups that have found the queue empty, and the last of
// them resets both to zero, so the next launch on the same counters starts from item 0 without
// a clearing launch. Every work-group of the grid must call queue_leave once, after its loop.
MX_DEV int queue_next(int* counter, int* s_item)
{
  __syncthreads();  // every wave is done with the previous item (and with *s_item)
  if (threadIdx.x == 0) *s_item = atomicAdd(counter, 1);
  __syncthreads();
  return __builtin_amdgcn_readfirstlane(*s_item);
}
MX_DEV void queue_leave(int* counter)
{
  if (threadIdx.x == 0 && atomicAdd(counter + 1, 1) == (int)gridDim.x - 1) {
    atomicExch(counter, 0);
    atomicExch(counter + 1, 0);
  }
}

// bf16 helpers (round to nearest even, as v_cvt_pk_bf16_f32 does)
MX_DEV uint32_t pack_bf16(float a, float b)
{
  const __bf16 x = (__bf16)a, y = (__bf16)b;
  return (uint32_t)__builtin_bit_cast(uint16_t, x) | ((uint32_t)__builtin_bit_cast(uint16_t, y) << 16);
}
MX_DEV float bf16_lo(uint32_t u) { return bits_f(u << 16); }
MX_DEV float bf16_hi(uint32_t u) { return bits_f(u & 0xFFFF0000u); }

// ------------------------------------------------------------------ GLU epilogues
// kind 0: SwiGLU  silu(g) * u
// kind 1: SiTU-GLU  4 tanh(g/4) sigmoid(g) * 25 tanh(u/25)  (lazy_lora/core/situ_activation.py:47-75)
constexpr float kSituBeta = 4.0f;
constexpr float kSituLinearBeta = 25.0f;

MX_DEV float sigmoid_f(float v) { return 1.0f / (1.0f + __expf(-v)); }
MX_DEV float tanh_f(float v) { return tanhf(v); }

MX_DEV float glu_fwd(float g, float u, int kind)
{
  const float s = sigmoid_f(g);
  if (kind == 0) return g * s * u;
  return kSituBeta * tanh_f(g / kSituBeta) * s * (kSituLinearBeta * tanh_f(u / kSituLinearBeta));
}

// (d gate, d up) for upstream grad go (situ_activation.py:78-134 for kind 1)
MX_DEV void glu_bwd(float go, float g, float u, int kind, float& dg, float& du)
{
  const float s = sigmoid_f(g);
  if (kind == 0) {
    dg = go * u * (s * (1.0f + g * (1.0f - s)));
    du = go * g * s;
    return;
  }
  const float t = tanh_f(g / kSituBeta);
  const float a = kSituBeta * t * s;
  const float da = (1.0f - t * t) * s + kSituBeta * t * s * (1.0f - s);
  const float tu = tanh_f(u / kSituLinearBeta);
  dg = go * (kSituLinearBeta * tu) * da;
  du = go * a * (1.0f - tu * tu);
}

}  // namespace mx
