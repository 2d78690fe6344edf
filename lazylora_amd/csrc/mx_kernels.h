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
  // work: tiles[t] = {expert, first row, row count <= 16, 0}; null = dense, rows 16t.. of M
  const int4* tiles;
  const int* n_tiles;
  int M;
  int n_ct;  // column tiles per row tile
  // outputs
  float* y;
  long long ldy;
  const float* row_w;    // kFwdDown: combine weight per row
  uint8_t* q_tiles;      // kFwdGateUp: act in the AT layout with K = R (= F), same tiles
  float* save;           // kFwdGateUp: [rows, 2R] gate | up in fp32, or null
  int act_kind;
};

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
};

constexpr int kFwdRowsPerTile = 16;
constexpr int kFwdColsPerTile = 64;  // kFwdPlain / kFwdDown; kFwdGateUp covers 32 features
constexpr int kBwdColsPerTile = 512;

hipError_t launch_fwd(const FwdArgs& a, int mode, int max_tiles, hipStream_t s);
hipError_t launch_bwd(const BwdArgs& a, int mode, int max_tiles, hipStream_t s);

// ---------------------------------------------------------------- elementwise / routing
// Two-term quantisation of activation rows into the AT layout of the work tiles. Tile t slot i
// holds row tiles[t].y + i (through row_map when given: the token of a (token, slot) pair);
// with tiles == null the tiles are dense: tile t holds rows 16t.. of `rows`. Unused slots get
// zeros. max_tiles bounds the grid; the live tile count is read from n_tiles on the device.
hipError_t launch_quant_tiles(const void* x, int x_bf16, long long ldx, int rows, int K, const int4* tiles,
                              const int* n_tiles, int max_tiles, const int* row_map, uint8_t* out,
                              hipStream_t s);
hipError_t launch_split_bf16(const float* x, long long ldx, int rows, int K, int Kpad, uint16_t* hi,
                             uint16_t* lo, hipStream_t s);
hipError_t launch_dequant(float* out, const uint8_t* packed, const uint8_t* scales, int K, int R,
                          hipStream_t s);
hipError_t launch_route(const void* topk_idx, int idx64, const float* topk_w, int N, int k, int E,
                        int* counts, int* offsets, int* cursor, int4* tiles, int* meta, int* pair_token,
                        float* pair_w, int* pair_of, hipStream_t s);
hipError_t launch_combine(float* out, const float* ypair, long long ldy, const int* pair_of, int N, int k,
                          int D, hipStream_t s);
hipError_t launch_combine_bwd(float* grad_h, float* grad_w, const float* dxpair, long long ldy,
                              const float* gw_part, int n_ct, const int* pair_of, int N, int k, int D,
                              hipStream_t s);
hipError_t launch_zero(void* p, size_t bytes, hipStream_t s);
// Router selection (sigmoid, bias, top-k, renormalise, scale), one wave per token.
hipError_t launch_router_topk(long long* topk_idx, float* topk_w, const float* logits, const float* bias, int N,
                              int E, int top_k, float scale, int renormalize, hipStream_t s);
hipError_t launch_router_topk_bwd(float* grad_logits, const long long* topk_idx, const float* grad_w,
                                  const float* logits, int N, int E, int top_k, float scale, int renormalize,
                                  hipStream_t s);


}  // namespace mx
