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
constexpr int kPrefetch = 8;  // weight steps in flight per work-group (even)

typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

struct WorkItem {
  int expert, row0, nrows, ct;
};

__device__ __forceinline__ bool decode_work(const int4* tiles, const int* n_tiles, int M, int n_ct,
                                            WorkItem& w)
{
  // the tile list is only read here: scalar loads through the constant address space
  typedef const __attribute__((address_space(4))) int* cint_ptr;
  const int ntiles = tiles ? *(cint_ptr)n_tiles : (M + kFwdRowsPerTile - 1) / kFwdRowsPerTile;
  const int total = ntiles * n_ct;
  const int per_xcd = (total + 7) >> 3;
  const int slot = (int)(blockIdx.x >> 3);
  const int item = (int)(blockIdx.x & 7) * per_xcd + slot;
  if (slot >= per_xcd || item >= total) return false;
  const int t = item / n_ct;
  w.ct = item - t * n_ct;
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

template <int MODE>
__global__ __launch_bounds__(256, 2) void bwd_kernel(BwdArgs a)
{
  __shared__ __attribute__((aligned(16))) uint8_t slab[2][kSlabBytes];
  __shared__ float dotred[4][16];

  WorkItem w;
  if (!decode_work(a.tiles, a.n_tiles, a.M, a.n_ct, w)) return;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, g = lane >> 4;
  const int c0 = w.ct * kBwdColsPerTile;
  const int rtot = a.nseg * a.R;
  const int nsteps = (rtot + kSlabRows - 1) / kSlabRows;
  // the ring below is unrolled kPrefetch-fold; padding steps load nothing useful (zero weights)
  const int nsteps_pad = (nsteps + kPrefetch - 1) / kPrefetch * kPrefetch;

  // loader role: MX blocks lc and lc + 8 of slab row lr per step, so each load instruction
  // of a wave reads whole 128-byte lines (8 rows x 8 blocks)
  const int lr = tid >> 3;
  const int lc = tid & 7;
  const int cbs = a.C / kGroup;    // scale bytes per W row
  const long long wpitch = a.C / 2;
  const int colA = c0 + lc * 32, colB = c0 + (lc + 8) * 32;
  const int colA_c = colA < a.C ? colA : 0, colB_c = colB < a.C ? colB : 0;
  const long long wbase = (long long)w.expert * a.wp_estride;
  const long long sbase = (long long)w.expert * a.ws_estride;

  // Always issues the loads, with rows and columns clamped into the matrix, so the wait
  // counters stay exact and nothing touches the loaded data before its decode step. Clamped
  // blocks are harmless: columns >= C are never stored, and rows >= nseg*R meet zero
  // activations (zero padding of A, or the padding steps below). Rows >= R read the second
  // segment (W3 after W1). Weight bytes are read exactly once: streaming loads.
  auto load_raw = [&](int step, i32x4& r0, i32x4& r1, uint8_t& s0, uint8_t& s1) {
    const int r = min(step * kSlabRows + lr, rtot - 1);
    const bool seg = r >= a.R;
    const int rr = seg ? r - a.R : r;
    const uint8_t* P = (seg ? a.wp1 : a.wp0) + wbase + (long long)rr * wpitch;
    const uint8_t* S = (seg ? a.ws1 : a.ws0) + sbase + (long long)rr * cbs;
    r0 = ldg16_nt(P + colA_c / 2);
    r1 = ldg16_nt(P + colB_c / 2);
    s0 = S[colA_c / kGroup];
    s1 = S[colB_c / kGroup];
  };

  // A operand rows (rows past the tile end repeat the last row; never stored)
  const int ri = w.row0 + min(li, w.nrows - 1);
  const int arow = a.a_row_map ? a.a_row_map[ri] : ri;
  const uint16_t* pah = a.a_hi + (long long)arow * a.lda + 8 * g;
  const uint16_t* pal = a.a_lo + (long long)arow * a.lda + 8 * g;

  f32x4 acc[8];
#pragma unroll
  for (int cg = 0; cg < 8; ++cg) acc[cg] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Pipeline: the raw blocks of the next kPrefetch steps are in flight in a register ring.
  // Within a step the next step's A loads are issued before the ring refill, so waiting for
  // A (vmcnt is an in-order counter) never waits for the far-ahead weight loads.
  i32x4 ring0[kPrefetch], ring1[kPrefetch];
  uint8_t rs0[kPrefetch], rs1[kPrefetch];
  // Issue order is pinned (A first, then the ring slot by slot) so the loop head can wait
  // for slot 0 alone, whether it is entered from here or from the back edge.
  i32x4 ahv = ldg16(pah), alv = ldg16(pal);
#pragma unroll
  for (int p = 0; p < kPrefetch; ++p) {
    __builtin_amdgcn_sched_barrier(0);
    load_raw(p, ring0[p], ring1[p], rs0[p], rs1[p]);
  }
  __builtin_amdgcn_sched_barrier(0);

  for (int s0 = 0; s0 < nsteps_pad; s0 += kPrefetch) {
#pragma unroll
    for (int p = 0; p < kPrefetch; ++p) {
      const int s = s0 + p;
      uint8_t* const sl = slab[p & 1];  // kPrefetch is even, so this is slab[s & 1]
      // keep later steps' use of the ring (and so their waits) below this point
      __builtin_amdgcn_sched_barrier(0);
      // this buffer was last read two steps ago; the barrier of the previous step ordered
      // those reads before these writes
      store_block(sl, lr, lc, ring0[p], rs0[p]);
      store_block(sl, lr, lc + 8, ring1[p], rs1[p]);
      __syncthreads();
      const int sn = min(s + 1, nsteps - 1);
      const i32x4 ahn = ldg16(pah + sn * kSlabRows);
      const i32x4 aln = ldg16(pal + sn * kSlabRows);
      __builtin_amdgcn_sched_barrier(0);
      load_raw(s + kPrefetch, ring0[p], ring1[p], rs0[p], rs1[p]);
      __builtin_amdgcn_sched_barrier(0);

      // padding steps (s >= nsteps) see clamped weights: zero their activations instead
      const bool real = s < nsteps;
      const bf16x8 ah = __builtin_bit_cast(bf16x8, real ? ahv : i32x4{0, 0, 0, 0});
      const bf16x8 al = __builtin_bit_cast(bf16x8, real ? alv : i32x4{0, 0, 0, 0});
      // B operands of this wave's 8 column groups (rows 8g..8g+7 of column cg*16 + li), each
      // read just before its two MFMAs
#pragma unroll
      for (int cg = 0; cg < 8; ++cg) {
        const int q = wave * 32 + cg * 4 + (li & 3);
        const i16x4 t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_i16x4*)(&sl[slab_off(8 * g + (li >> 2), q)]));
        const i16x4 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_i16x4*)(&sl[slab_off(8 * g + 4 + (li >> 2), q)]));
        const short __attribute__((ext_vector_type(8))) bs = {t0[0], t0[1], t0[2], t0[3], t1[0], t1[1], t1[2], t1[3]};
        const bf16x8 b = __builtin_bit_cast(bf16x8, bs);
        acc[cg] = mfma_bf16(ah, b, acc[cg]);
        acc[cg] = mfma_bf16(al, b, acc[cg]);
      }
      ahv = ahn;
      alv = aln;
    }
  }

  // epilogue: lane (li, g) holds rows 4g..4g+3 of column c0 + wave*128 + cg*16 + li
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
      // LoRA: the down adapter's A_d^T q of the row's token joins g . W2
      const float* rq = a.lora_rq ? a.lora_rq + (long long)a.a_row_map[p] * F : nullptr;
#pragma unroll
      for (int cg = 0; cg < 8; ++cg) {
        const int f = c0 + wave * 128 + cg * 16 + li;
        if (f < F) {
          const float h = rq ? acc[cg][v] + rq[f] : acc[cg][v];
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
    for (int cg = 0; cg < 8; ++cg) {
      const int col = c0 + wave * 128 + cg * 16 + li;
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
