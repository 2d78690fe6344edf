// Kernel argument blocks and launch helpers shared by the .hip translation units.
// Host-visible; no torch types.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mx {

// ---------------------------------------------------------------- forward products
enum FwdMode : int {
  kFwdPlain = 0,   // y[row, n] = A[row] . W[n]
  kFwdGateUp = 1,  // act = GLU(A . W1^T, A . W3^T) -> two-term e4m3 act (+ optional fp32 gate|up)
  kFwdDown = 2,    // y_pair[p, n] = tw[p] * (act[p] . W2[n])
};

struct FwdArgs {
  const uint8_t* wp0;  // packed W (or W1 for kFwdGateUp), expert-major
  const uint8_t* ws0;
  const uint8_t* wp1;  // W3 for kFwdGateUp
  const uint8_t* ws1;
  long long wp_estride;  // bytes between experts in wp*
  long long ws_estride;  // bytes between experts in ws*
  int R, K;              // each W is [R, K]
  // A operand: two-term e4m3 activations in the AT layout, one block of at_tile_bytes(K)
  // per work tile (tile t of the list below)
  const uint8_t* a_tiles;
  // kFwdGateUp, one-tile work-groups: A in the XT layout instead; pair row p reads row
  // row_token[p] of a_rows (rows a_row_bytes apart), a tile's unused slots row a_zero_row. Its
  // grouped work-groups read a_tiles, of which only the large buckets' tiles need be written.
  const uint8_t* a_rows;
  long long a_row_bytes;
  int a_zero_row;
  // work: tiles[t] = {expert, first row, row count <= 16, 1 in a large bucket}; null = dense, rows 16t.. of M
  const int4* tiles;
  const int* n_tiles;
  int M;
  int n_ct;  // column tiles per row tile
  // outputs
  float* y;
  long long ldy;
  const int* y_rows;     // output row of each row (null: the row itself; top-1 routing writes tokens)
  const float* row_w;    // kFwdDown: combine weight per row
  uint8_t* q_tiles;      // kFwdGateUp: act in the AT layout with K = R (= F), same tiles
  float* save;           // kFwdGateUp: [rows, 2R] gate | up in fp32, or null
  int act_kind;
  // token of each pair row (XT gather); with LoRA, gate|up of row p gain
  // lora_delta[row_token[p], 0:2R) before the GLU
  const int* row_token;
  const float* lora_delta;  // [tokens, 2R] fp32, or null
  // kFwdGateUp: the third term of x (X3 layout, rows as a_rows, x3_row_bytes apart), or null, and
  // the call-wide flag (non-zero: some block has a third term; zero: the products skip it all)
  const uint8_t* x3;
  long long x3_row_bytes;
  const int* x3_any;
  // Bucket split (with a tile list and K a multiple of 512): the tiles of small buckets
  // (indices into `tiles`) take the one-row-tile work-groups; large-bucket groups of up to
  // kGroupTiles tiles ({expert, first tile, tiles, 0}) take work-groups that share each column
  // tile's weights over the group's row tiles. Null small_tiles: every tile takes the first shape.
  const int* small_tiles;
  const int* n_small;
  const int4* groups;
  const int* n_groups;
  // The same large-bucket tiles as wide groups of up to kWideGroupTiles tiles, taken instead of
  // `groups` by the large-bucket work-groups that read a forward layout (null: use `groups`).
  const int4* wgroups;
  const int* n_wgroups;
  int* wcounter;  // the wide-group launch's work queue: 2 ints, zero before the first launch (queue_next)
  // Forward layout (launch_forward_layout) of W (W1 for kFwdGateUp) and W3, or null: the
  // one-tile fast path's work-groups then read their weight codes and scales from it in whole
  // lines, the wide large-bucket work-groups their codes (the general path, the wide groups'
  // scales and the rare third-term pass always read wp* / ws*).
  const uint8_t* fl0;
  const uint8_t* fl1;
  long long fl_estride;  // bytes between experts in fl*
};

// Forward layout of E stacked packed [R, K] matrices (K a multiple of 512) and their E8M0 scales
// [R, K / 32], per expert forward_layout_bytes(R, K) bytes, nrg = ceil(R / 16) row groups and
// nsc = K / 512 super-chunks: codes, the 4 KiB at (rg * nsc + c) * 4096 hold super-chunk c of the
// 16 rows 16 rg .., MFMA q's operand block at q * 1024, lane l's 16 bytes (MX block
// 4 (l / 16) + q of row 16 rg + l % 16) at l * 16; then scales, the 256 B at
// nrg * nsc * 4096 + (rg * nsc + c) * 256 hold lane l's scale dword (blocks 4 (l / 16) .. + 3 of
// super-chunk c of row 16 rg + l % 16) at 4 l. Rows past R repeat row R - 1.
long long forward_layout_bytes(int R, int K);
hipError_t launch_forward_layout(const uint8_t* packed, const uint8_t* scales, uint8_t* out, int E, int R, int K,
                                 hipStream_t s);

// ---------------------------------------------------------------- transposed products
enum BwdMode : int {
  kBwdPlain = 0,   // y[row, c] (+)= sum_r A[row, r] W[r, c]
  kBwdDownT = 1,   // h = g . W2 -> grad_w partials, GLU backward -> bf16 d_gate | d_up
  kBwdGateUpT = 2, // y_pair[p, c] = [d_gate | d_up] . [W1 ; W3]
};

struct BwdArgs {
  const uint8_t* wp0;
  const uint8_t* ws0;
  const uint8_t* wp1;  // second row segment (W3), or null
  const uint8_t* ws1;
  long long wp_estride;
  long long ws_estride;
  int nseg;      // 1 or 2 row segments
  int R, C;      // each segment is [R, C]
  const uint16_t* a_hi;  // bf16 [rows, lda], contraction index in [0, nseg*R), zero padded
  const uint16_t* a_lo;
  long long lda;
  const int* a_row_map;
  const int4* tiles;
  const int* n_tiles;
  int M;
  int n_ct;  // column tiles of kBwdColsPerTile
  float* y;
  long long ldy;
  int accumulate;
  // kBwdDownT
  const float* row_w;
  const float* saved;  // [rows, 2C] gate | up
  int act_kind;
  uint16_t* d_hi;      // [rows, 2C]
  uint16_t* d_lo;
  float* gw_part;      // [rows, n_ct]
  // kBwdDownT with LoRA: h = g . W2 of row p gains lora_rq[a_row_map[p], 0:C) (the down
  // adapter's A^T q of the row's token), so both the GLU backward and grad_w see it
  const float* lora_rq;  // [tokens, C] fp32, or null
  // Bucket split, as in FwdArgs: small-bucket tiles take one-tile work-groups, large-bucket
  // groups work-groups that reuse each decoded weight slab for all of the group's tiles.
  const int* small_tiles;
  const int* n_small;
  const int4* groups;
  const int* n_groups;
  // Backward layout (launch_backward_layout) of each row segment (W; W1 and W3 for two), or
  // null: the work-groups of kBwdDownT / kBwdGateUpT then read it instead of wp / ws. Needs
  // backward_layout_ok(R, C).
  const uint8_t* bl0;
  const uint8_t* bl1;
  long long bl_estride;  // bytes per expert: backward_layout_bytes(R, C)
};

constexpr int kFwdRowsPerTile = 16;
constexpr int kGroupTiles = 4;     // row tiles of one large-bucket group
constexpr int kWideGroupTiles = 8;  // row tiles of one wide group (the forward-layout large-bucket forward)
constexpr int kGroupMinTiles = 4;  // experts with at least this many tiles take the large-bucket path
constexpr int kFwdColsPerTile = 64;  // kFwdPlain / kFwdDown; kFwdGateUp covers 32 features
constexpr int kBwdColsPerTile = 256;  // output columns of one transposed-product wave

// Whether launch_fwd splits a routed product over W [R, K] into small-bucket and large-bucket
// work-groups: the large-bucket shape needs the fast path (K a multiple of 512, one buffer
// resource addressing the whole matrix). Without the split every tile takes the one-tile
// work-groups, whose gate/up product reads the token-major (XT) rows of x for every tile.
bool fwd_bucket_split(int R, int K);
hipError_t launch_fwd(const FwdArgs& a, int mode, int max_tiles, hipStream_t s);
hipError_t launch_bwd(const BwdArgs& a, int mode, int max_tiles, hipStream_t s);

// Backward layout: a load-time copy of E stacked MXFP4 matrices [R, C] (codes [R, C/2], E8M0
// scales [R, C/32]) for the one-tile transposed products. Per expert, blocks (32-row step st,
// 256-column stripe c) in order st * (C / 256) + c: each block's 4 KiB of codes in the order the
// lanes of the stripe's wave load them (lane 16g + n, load u: bytes 8n .. 8n + 7 of rows 8g + 2u
// and 8g + 2u + 1), then, after every block's codes, 256 B of scales per block (8 bytes per lane
// pair: the scale bytes of rows 8g .. 8g + 7 for the pair's MX block). R % 32 == 0, C % 256 == 0.
bool backward_layout_ok(int R, int C);
long long backward_layout_bytes(int R, int C);  // per expert; 0 unless backward_layout_ok(R, C)
hipError_t launch_backward_layout(const uint8_t* packed, const uint8_t* scales, uint8_t* out, int E, int R, int C,
                                  hipStream_t s);

// ---------------------------------------------------------------- elementwise / routing
// Two-term quantisation of activation rows into the AT layout of the work tiles. Tile t slot i
// holds row tiles[t].y + i (through row_map when given: the token of a (token, slot) pair);
// with tiles == null the tiles are dense: tile t holds rows 16t.. of `rows`. Unused slots get
// zeros. max_tiles bounds the grid; the live tile count is read from n_tiles on the device.
// large_only: only the tiles of large buckets (tiles[t].w != 0); the others are left untouched.
// xt (with meta and row_map): the XT rows of x written by launch_quant_rows on the same stream;
// when that call wrote them (meta says some bucket is small) the tiles are copied from them
// instead of quantising x again (the same bytes). x3 (with row_map): where the tiles are quantised
// from x, also the X3 rows of their tokens (launch_quant_rows writes them otherwise). x3_any
// (with x3): set to non-zero when some block has a third term (it must be zero before the call).
// groups (with large_only; n_groups on the device): the large buckets' tiles are found through
// the routing's group list by a resident grid, instead of one work-group per tile and chunk.
hipError_t launch_quant_tiles(const void* x, int x_bf16, long long ldx, int rows, int K, const int4* tiles,
                              const int* n_tiles, int max_tiles, const int* row_map, int large_only, const uint8_t* xt,
                              const int* meta, uint8_t* out, uint8_t* x3, int* x3_any, hipStream_t s,
                              const int4* groups = nullptr, const int* n_groups = nullptr);
// Rows 0 .. rows - 1 of x into the XT layout (xt_row_bytes(K) per row), followed by zero rows
// up to xt_rows(rows): row `rows` is the all-zero row a tile's unused slots gather. x3 (or null):
// the third term of the flagged blocks in the X3 layout (x3_row_bytes(K) per row; rows < rows).
// With meta saying every bucket is large the call writes nothing (launch_quant_tiles writes X3).
inline long long xt_rows(int rows) { return ((long long)rows + 16) / 16 * 16; }
hipError_t launch_quant_rows(const void* x, int x_bf16, long long ldx, int rows, int K, const int* meta, uint8_t* out,
                             uint8_t* x3, int* x3_any, hipStream_t s);
hipError_t launch_split_bf16(const float* x, long long ldx, int rows, int K, int Kpad, uint16_t* hi,
                             uint16_t* lo, hipStream_t s);
hipError_t launch_dequant(void* out, int out_bf16, const uint8_t* packed, const uint8_t* scales, int K, int R,
                          hipStream_t s);
// Routing: per-expert counts, scan, the tile list (tiles[t] = {expert, first pair row, rows, large}),
// the small-bucket tile indices, the large-bucket groups ({expert, first tile, tiles, 0}) of up to
// kGroupTiles tiles and the same tiles again as wide groups of up to kWideGroupTiles (the full
// ones first), meta = {tiles, flags (bit 0: an id outside [0, E)), small tiles, groups, wide
// groups, full wide groups, third term present (set by the quantisers), -, then the work queues
// (2 ints each) of the wide-group launches of the forward gate/up and down products, ...} (16
// ints, all zeroed here), and the pair maps.
hipError_t launch_route(const void* topk_idx, int idx64, const float* topk_w, int N, int k, int E,
                        int* counts, int* offsets, int* cursor, int4* tiles, int* small_tiles, int4* groups,
                        int4* wgroups, int* meta, int* pair_token, float* pair_w, int* pair_of, hipStream_t s);
hipError_t launch_combine(float* out, const float* ypair, long long ldy, const int* pair_of, int N, int k,
                          int D, hipStream_t s);
// Top-1 routing (the down product writes token rows itself): zeros into the rows of tokens with no
// pair (pair_of[t] < 0, an id outside [0, E)).
hipError_t launch_zero_unrouted(float* out, long long ldo, int D, const int* pair_of, int N, hipStream_t s);
hipError_t launch_combine_bwd(float* grad_h, float* grad_w, const float* dxpair, long long ldy,
                              const float* gw_part, int n_ct, const int* pair_of, int N, int k, int D,
                              hipStream_t s);
hipError_t launch_zero(void* p, size_t bytes, hipStream_t s);
// ---------------------------------------------------------------- LoRA coupling
// Encodings of the row-major matrices the LoRA kernels read.
enum LoraSrc : int {
  kLoraF32 = 0,   // p0: fp32 [rows, ld]
  kLoraBF16 = 1,  // p0: bf16 [rows, ld]
  kLoraGLU = 2,   // p0: saved fp32 gate | up [rows, 2F]; element (row, c) = GLU(gate[c], up[c])
  kLoraHiLo = 3,  // p0 / p1: bf16 hi and lo [rows, ld]; element = hi + lo
};
struct LoraMat {
  int kind;
  const void* p0;
  const void* p1;
  long long ld;
  int F, act_kind;  // kLoraGLU
};
// Small dense factor M of a LoRA adapter, addressed as M(j, k) (j < rank): j-major means
// M[j * ld + k] (lora_A [r, in]), k-major means M[k * ld + j] (lora_B [out, r]).
struct LoraFactor {
  const float* m;
  long long ld;
  int kmajor;
  float scale;
};

constexpr int kLoraMaxRank = 32;

// Destination of an outer-product gradient: element (j, c) of segment s goes to
// p[s][kmajor[s] ? c * ld[s] + j : j * ld[s] + c] times scale[s].
struct LoraOuterDst {
  float* p[2];
  long long ld[2];
  int kmajor[2];
  float scale[2];
  int split_j;  // coefficients j >= split_j go to p[1] (index minus split_j), or 0
};

// One job of a LoRA pass (launch_lora_pass), over a source of `rows` rows (tokens, or pairs in
// bucket order; rows at or past *rows_dev, when given, are skipped) in nseg <= 2 segments of K
// columns (a multiple of 32), segment s starting at source column koff[s]:
//   kLoraRowDot: partial row dots of out[row, s*r + j] = sum_k src(row, koff_s + k) f_s(j, k)
//     (nseg 2), or of out[row, n*r + j] with factor f_n on the one segment (nseg 1, n < nfac <= 2);
//   kLoraOuter: partial column sums of G[j, s*K + c] = sum over q < rows of
//     row_w[q] * coef[crow(q), coff_s + j] * src(row(q), koff_s + c), j < m <= 64: with row_of,
//     q runs over (token, slot) pairs in token order, row(q) = row_of[q] (skipped when negative)
//     and crow(q) = q / k, so the sums do not depend on the bucket order; else row(q) = crow(q)
//     = q. row_w null: 1.
// Factor scales are not applied here (the finish applies them).
//   kLoraRowOuter: both, over one two-term (hi + lo) pair source with row_of (nseg segments, m = r <=
//     16 coefficients per segment, factor f_s on segment s): each element is read once.
enum LoraJobType : int { kLoraRowDot = 0, kLoraOuter = 1, kLoraRowOuter = 2 };
struct LoraPassJob {
  int type;
  LoraMat src;
  int rows;
  const int* rows_dev;
  int nseg, K;
  int koff[2];
  int r;
  int nfac;
  LoraFactor f[2];
  const float* coef;
  long long ldc;
  int coff[2];
  const int* row_of;
  int k;
  const float* row_w;
  int m;
};
// Partials a pass job leaves for its finish: `count` slices (row dots: [count, rows, m_out]) or
// row chunks (outer products: [count, m, nseg * K]); a fused job leaves its outer-product
// partials in p and its row-dot partials in p2 (count2 slices of [rows, nseg * r]).
struct LoraPartial {
  const float* p;
  int count;
  const float* p2;
  int count2;
};
size_t lora_pass_partial_floats(const LoraPassJob* jobs, int n);
// Up to 4 jobs in one launch; parts[i] receives job i's partials (inside `partial`, which holds
// lora_pass_partial_floats(jobs, n) floats).
hipError_t launch_lora_pass(const LoraPassJob* jobs, int n, float* partial, LoraPartial* parts, hipStream_t s);

// One job of launch_lora_finish: the partials added in a fixed order.
//   kLoraFinCoef: value (row, j) = scale[j / r] * sum over slices of the row-dot partials
//     ([count, prow, m]); with pair_of, rows are pairs and out[t, j] = sum over token t's slots, in
//     slot order, of (topk_w[t, s] or 1) * value(pair_of[t, s], j); else out[t, j] = value(t, j);
//     out is [ntok, m].
//   kLoraFinOuter: G[j, c] = sum over chunks of the outer partials ([count, om, Ctot]), written
//     through dst; segments by column (Kseg > 0: s = c / Kseg) or by j (dst.split_j).
enum LoraFinType : int { kLoraFinCoef = 0, kLoraFinOuter = 1 };
struct LoraFinishJob {
  int type;
  LoraPartial part;
  int prow, m, r;
  float scale[2];
  const int* pair_of;
  const float* topk_w;
  int k, ntok;
  float* out;
  int om, Ctot, Kseg;
  LoraOuterDst dst;
};
hipError_t launch_lora_finish(const LoraFinishJob* jobs, int n, hipStream_t s);

// out[t, c] = ef_s.scale * sum_{j < r} coef[t, ecoff_s + j] * ef_s(j, c - s*Cseg) for t < ntok,
// c < Cexp (multiples of 4), segment s = c / Cseg (Cseg 0 or >= Cexp: one segment; two segments
// share the factor layout); coef rows hold m floats, out rows are ldo apart. With part (row-dot
// partials [count, ntok, m] of tokens), the coefficient rows are first reduced from them
// (coef[t, j] = part_scale[j / r] * the slices' sum, added in slice order) and written to coef.
hipError_t launch_lora_expand(float* coef, int m, int ntok, int r, float* out, long long ldo, int Cexp,
                              int Cseg, const LoraFactor* ef, const int* ecoff, hipStream_t s,
                              const LoraPartial* part = nullptr, const float* part_scale = nullptr);

// out[t, c] = sum over token t's slots, in slot order, of rows[pair_of[t, s], c] (skipped when
// negative) + sum over segments s < nseg of f_s.scale * sum_{j < r} coef[t, s*r + j] f_s(j, c);
// with grad_w, also grad_w[t, s] = sum over ct < n_ct of gw_part[pair, ct] (the backward combine).
hipError_t launch_lora_combine(float* out, const float* rows, long long ldy, const int* pair_of, int N, int k, int D,
                               const float* coef, int r, int nseg, const LoraFactor* f, float* grad_w,
                               const float* gw_part, int n_ct, hipStream_t s);

// Router selection (sigmoid, bias, top-k, renormalise, scale), one wave per token.
hipError_t launch_router_topk(long long* topk_idx, float* topk_w, const float* logits, const float* bias, int N,
                              int E, int top_k, float scale, int renormalize, hipStream_t s);
hipError_t launch_router_topk_bwd(float* grad_logits, const long long* topk_idx, const float* grad_w,
                                  const float* logits, int N, int E, int top_k, float scale, int renormalize,
                                  hipStream_t s);


}  // namespace mx
