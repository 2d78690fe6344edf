// C ABI entry points (declared in include/lazylora_mxfp4.h): argument checks, workspace
// carving and launch sequences. No device memory is allocated here; callers pass workspaces.
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "../../include/lazylora_mxfp4.h"
#include "mx_device.h"
#include "mx_kernels.h"

// Device scratch of mxfp4_gemm_noalloc (see scratch_on_current_device below).
constexpr size_t kScratchBytes = size_t(16) << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, const char* detail = "")
{
  snprintf(g_err, sizeof(g_err), fmt, detail);
  return code;
}

int hip_fail(hipError_t e, const char* where)
{
  snprintf(g_err, sizeof(g_err), "%s: %s", where, hipGetErrorString(e));
  return MXFP4_EHIP;
}

#define MX_TRY(expr, where)                          \
  do {                                               \
    hipError_t e__ = (expr);                         \
    if (e__ != hipSuccess) return hip_fail(e__, where); \
  } while (0)

// Optional phase timing of the routed-layer calls (the analogue of the reference's
// LAZYLORA_PROFILE per-phase timings, lazy_lora/trainer/lazy_trainer.py:192-194). While
// enabled, each call records a HIP event on its stream before its first launch and after each
// phase, into the next slot of a ring of kRing calls. Nothing synchronises until the times
// are read, so timing can stay on inside a timed loop.
struct PhaseTimer {
  static constexpr int kRing = 128;
  static constexpr int kMaxPhases = 16;
  bool on = false;
  int calls = 0;  // calls recorded since enabled
  int cur = -1;   // ring slot of the call in progress
  int n[kRing] = {};
  const char* names[kRing][kMaxPhases] = {};
  hipEvent_t ev[kRing][kMaxPhases + 1] = {};
  bool created = false;

  hipError_t enable(bool e)
  {
    on = e;
    calls = 0;
    cur = -1;
    if (e && !created) {
      for (int c = 0; c < kRing; ++c)
        for (int p = 0; p <= kMaxPhases; ++p) {
          hipError_t r = hipEventCreate(&ev[c][p]);
          if (r != hipSuccess) return r;
        }
      created = true;
    }
    return hipSuccess;
  }
  hipError_t begin(hipStream_t s)
  {
    if (!on) return hipSuccess;
    cur = calls % kRing;
    ++calls;
    n[cur] = 0;
    return hipEventRecord(ev[cur][0], s);
  }
  hipError_t mark(const char* name, hipStream_t s)
  {
    if (!on || cur < 0 || n[cur] >= kMaxPhases) return hipSuccess;
    names[cur][n[cur]] = name;
    ++n[cur];
    return hipEventRecord(ev[cur][n[cur]], s);
  }
};
thread_local PhaseTimer g_timer;

#define MX_PHASE(name, s) MX_TRY(g_timer.mark(name, s), "phase timer")

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Bytes of the two-term activation operand (AT layout) for `tiles` work tiles of row length K.
size_t at_bytes(long long tiles, int K) { return align_up((size_t)(tiles * mx::at_tile_bytes(K))); }

long long pad32(long long v) { return (v + 31) / 32 * 32; }

mx::LoraMat mat_f32(const void* p, long long ld) { return mx::LoraMat{mx::kLoraF32, p, nullptr, ld, 0, 0}; }
mx::LoraFactor jmajor(const float* m, long long ld, float scale) { return mx::LoraFactor{m, ld, 0, scale}; }
mx::LoraFactor kmajor(const float* m, long long ld, float scale) { return mx::LoraFactor{m, ld, 1, scale}; }

// Row-dot job over nseg segments of K columns (the second at source column koff1).
mx::LoraPassJob rowdot_job(const mx::LoraMat& src, int rows, const int* rows_dev, int nseg, int K, int koff1, int r,
                           int nfac, mx::LoraFactor f0, mx::LoraFactor f1)
{
  mx::LoraPassJob j = {};
  j.type = mx::kLoraRowDot; j.src = src; j.rows = rows; j.rows_dev = rows_dev;
  j.nseg = nseg; j.K = K; j.koff[1] = koff1; j.r = r; j.nfac = nfac; j.f[0] = f0; j.f[1] = f1;
  return j;
}

// Outer-product job: m coefficients per segment, from coef columns coff_s (the second at coff1).
// Pair sources (row_of = pair_of) are walked over the (token, slot) pairs, k slots per token.
mx::LoraPassJob outer_job(const mx::LoraMat& src, int rows, int nseg, int K, int koff1, int r, const float* coef,
                          long long ldc, int coff1, const int* row_of, int k, const float* row_w, int m)
{
  mx::LoraPassJob j = {};
  j.type = mx::kLoraOuter; j.src = src; j.rows = rows;
  j.nseg = nseg; j.K = K; j.koff[1] = koff1; j.r = r;
  j.coef = coef; j.ldc = ldc; j.coff[1] = coff1; j.row_of = row_of; j.k = k; j.row_w = row_w; j.m = m;
  return j;
}

// The passes of the LoRA stages (pointers may be null when only sizing the partials):
// adapter inputs U = [A_gate x | A_up x] (pass_in); v = A_down act per pair (pass_mid);
// q = B_down^T g per token (pass_q); dh = [B_gate^T d_gate | B_up^T d_up] per pair with the B_gate,
// B_up, A_down and B_down gradients (pass_dx); the A_gate / A_up gradients (pass_grads).
struct LoraPtrs {
  mx::LoraMat x, g, act, d;
  const float* m[6];
  const int* n_valid;
  const int* pair_of;
  const float* topk_w;
  int k;
  const float *u, *q, *vsum, *dsum;
};

int lora_pass_jobs(int stage, const LoraPtrs& p, int N, long long P, int D, int F, int r, mx::LoraPassJob* j)
{
  switch (stage) {
    case 0:
      j[0] = rowdot_job(p.x, N, nullptr, 1, D, 0, r, 2, jmajor(p.m[0], D, 1.f), jmajor(p.m[2], D, 1.f));
      return 1;
    case 1:
      j[0] = rowdot_job(p.act, (int)P, p.n_valid, 1, F, 0, r, 1, jmajor(p.m[4], F, 1.f), jmajor(p.m[4], F, 1.f));
      return 1;
    case 2:
      j[0] = rowdot_job(p.g, N, nullptr, 1, D, 0, r, 1, kmajor(p.m[5], r, 1.f), kmajor(p.m[5], r, 1.f));
      return 1;
    case 3: {
      int n = 0;
      j[n] = outer_job(p.d, (int)P, 2, F, F, r, p.u, 2 * r, r, p.pair_of, p.k, nullptr, r);
      j[n].f[0] = kmajor(p.m[1], r, 1.f);
      j[n].f[1] = kmajor(p.m[3], r, 1.f);
      if (r <= 16) {
        j[n++].type = mx::kLoraRowOuter;  // with the row dots dh = [B_gate^T d_gate | B_up^T d_up]
      } else {
        ++n;
        j[n++] = rowdot_job(p.d, (int)P, p.n_valid, 2, F, F, r, 1, kmajor(p.m[1], r, 1.f), kmajor(p.m[3], r, 1.f));
      }
      j[n++] = outer_job(p.act, (int)P, 1, F, 0, r, p.q, r, 0, p.pair_of, p.k, p.topk_w, r);
      j[n++] = outer_job(p.g, N, 1, D, 0, r, p.vsum, r, 0, nullptr, 1, nullptr, r);
      return n;
    }
    default:
      j[0] = outer_job(p.x, N, 1, D, 0, r, p.dsum, 2 * r, 0, nullptr, 1, nullptr, 2 * r);
      return 1;
  }
}
constexpr int kLoraStages = 5;

// Partial floats of the largest LoRA pass over every rank.
size_t lora_part_floats(int N, long long P, int D, int F)
{
  LoraPtrs p = {};
  p.x = mat_f32(nullptr, D); p.g = mat_f32(nullptr, D);
  p.act = mx::LoraMat{mx::kLoraGLU, nullptr, nullptr, 2LL * F, F, 0};
  p.d = mx::LoraMat{mx::kLoraHiLo, nullptr, nullptr, 2LL * F, 0, 0};
  size_t best = 0;
  for (int r = 1; r <= mx::kLoraMaxRank; ++r)
    for (int st = 0; st < kLoraStages; ++st) {
      mx::LoraPassJob j[4];
      const int n = lora_pass_jobs(st, p, N, P, D, F, r, j);
      best = std::max(best, mx::lora_pass_partial_floats(j, n));
    }
  return best;
}

// Routed-layer workspace: one layout for forward and backward so the backward can reuse
// what the forward left behind.
struct MoeLayout {
  size_t meta, counts, offsets, cursor, tiles, small_tiles, groups, wgroups, pair_token, pair_w, pair_of;
  size_t at_x, xt_x, x3_x, at_act;
  size_t saved, ypair, g_hi, g_lo, d_hi, d_lo, gw_part;
  size_t l_u, l_delta, l_vsum, l_q, l_rq, l_dsum, l_part;  // LoRA (rank <= kLoraMaxRank)
  size_t end;
  int max_tiles, n_ct_bwd;
};

MoeLayout moe_layout(int N, int k, int E, int D, int F)
{
  MoeLayout L;
  const long long P = (long long)N * k;
  L.max_tiles = (int)((P + mx::kFwdRowsPerTile - 1) / mx::kFwdRowsPerTile + E);
  L.n_ct_bwd = (F + mx::kBwdColsPerTile - 1) / mx::kBwdColsPerTile;
  size_t o = 0;
  L.meta = o; o = align_up(o + 16 * sizeof(int));
  L.counts = o; o = align_up(o + sizeof(int) * (size_t)E);
  L.offsets = o; o = align_up(o + sizeof(int) * (size_t)(E + 1));
  L.cursor = o; o = align_up(o + sizeof(int) * (size_t)E);
  L.tiles = o; o = align_up(o + sizeof(int4) * (size_t)L.max_tiles);
  L.small_tiles = o; o = align_up(o + sizeof(int) * (size_t)L.max_tiles);
  L.groups = o; o = align_up(o + sizeof(int4) * (size_t)L.max_tiles);
  L.wgroups = o; o = align_up(o + sizeof(int4) * (size_t)L.max_tiles);
  L.pair_token = o; o = align_up(o + sizeof(int) * (size_t)P);
  L.pair_w = o; o = align_up(o + sizeof(float) * (size_t)P);
  L.pair_of = o; o = align_up(o + sizeof(int) * (size_t)P);
  L.at_x = o; o += at_bytes(L.max_tiles, D);
  L.xt_x = o; o = align_up(o + (size_t)(mx::xt_rows(N) * mx::xt_row_bytes(D)));
  L.x3_x = o; o = align_up(o + (size_t)(mx::xt_rows(N) * mx::x3_row_bytes(D)));
  L.at_act = o; o += at_bytes(L.max_tiles, F);
  L.saved = o; o = align_up(o + sizeof(float) * (size_t)(P * 2 * F));
  L.ypair = o; o = align_up(o + sizeof(float) * (size_t)(P * D));
  L.g_hi = o; o = align_up(o + 2 * (size_t)(N * (long long)D));
  L.g_lo = o; o = align_up(o + 2 * (size_t)(N * (long long)D));
  L.d_hi = o; o = align_up(o + 2 * (size_t)(P * 2 * F));
  L.d_lo = o; o = align_up(o + 2 * (size_t)(P * 2 * F));
  L.gw_part = o; o = align_up(o + sizeof(float) * (size_t)(P * L.n_ct_bwd));
  const size_t R = mx::kLoraMaxRank;
  L.l_u = o; o = align_up(o + sizeof(float) * (size_t)N * 2 * R);
  L.l_delta = o; o = align_up(o + sizeof(float) * (size_t)N * 2 * F);
  L.l_vsum = o; o = align_up(o + sizeof(float) * (size_t)N * R);
  L.l_q = o; o = align_up(o + sizeof(float) * (size_t)N * R);
  L.l_rq = o; o = align_up(o + sizeof(float) * (size_t)N * F);
  L.l_dsum = o; o = align_up(o + sizeof(float) * (size_t)N * 2 * R);
  L.l_part = o; o = align_up(o + sizeof(float) * lora_part_floats(N, P, D, F));
  L.end = o;
  return L;
}

template <typename T>
T* at(void* ws, size_t off) { return reinterpret_cast<T*>(reinterpret_cast<char*>(ws) + off); }

int check_moe_args(const void* h, int h_dtype, const void* idx, int idx_dtype, const float* w, int N, int k,
                   const uint8_t* const* wts, int E, int D, int F, int act_kind)
{
  if (N < 0 || k <= 0 || E <= 0 || D <= 0 || F <= 0) return fail(MXFP4_EINVAL, "moe: N, k, E, D, F must be positive%s");
  if (D % 32 || F % 32) return fail(MXFP4_EINVAL, "moe: D and F must be multiples of 32%s");
  if (h_dtype != MXFP4_F32 && h_dtype != MXFP4_BF16) return fail(MXFP4_EINVAL, "moe: h must be fp32 or bf16%s");
  if (idx_dtype != MXFP4_I32 && idx_dtype != MXFP4_I64) return fail(MXFP4_EINVAL, "moe: topk_idx must be int32 or int64%s");
  if (act_kind != MXFP4_ACT_SWIGLU && act_kind != MXFP4_ACT_SITU) return fail(MXFP4_EINVAL, "moe: unknown act_kind%s");
  if (N > 0 && (!h || !idx || !w)) return fail(MXFP4_EINVAL, "moe: null input pointer%s");
  for (int i = 0; i < 6; ++i) {
    if (!wts[i]) return fail(MXFP4_EINVAL, "moe: null expert weight pointer%s");
    if (!aligned16(wts[i])) return fail(MXFP4_EINVAL, "moe: packed weights and scales must be 16-byte aligned%s");
  }
  // the activation quantisers read h two elements at a time
  if (N > 0 && ((uintptr_t)h & (h_dtype == MXFP4_BF16 ? 3 : 7)))
    return fail(MXFP4_EINVAL, "moe: h must be 8-byte (fp32) or 4-byte (bf16) aligned%s");
  if ((long long)N * k > (1ll << 30)) return fail(MXFP4_EINVAL, "moe: too many (token, slot) pairs%s");
  return MXFP4_OK;
}

// Small-bucket tile list and large-bucket groups of the routed layer (see launch_route).
template <typename Args>
void set_buckets(Args& a, void* ws, const MoeLayout& L)
{
  a.small_tiles = at<int>(ws, L.small_tiles);
  a.n_small = at<int>(ws, L.meta) + 2;
  a.groups = at<int4>(ws, L.groups);
  a.n_groups = at<int>(ws, L.meta) + 3;
  if constexpr (std::is_same<Args, mx::FwdArgs>::value) {
    a.wgroups = at<int4>(ws, L.wgroups);
    a.n_wgroups = at<int>(ws, L.meta) + 4;
  }
}

// The layer's LoRA adapters, shared by all its experts (lazy_trainer.py:130-134).
struct Lora {
  const float* m[6] = {};  // A_gate [r, D], B_gate [F, r], A_up [r, D], B_up [F, r], A_down [r, F], B_down [D, r]
  float sg = 0.f, su = 0.f, sd = 0.f;  // alpha / r of gate, up, down
  int r = 0;                           // 0: LoRA off
};

int check_lora(const float* const* lora, const float* scaling, int rank, Lora& lo)
{
  lo = Lora{};
  if (!lora) return MXFP4_OK;
  if (rank < 1 || rank > mx::kLoraMaxRank) return fail(MXFP4_EINVAL, "moe: LoRA rank must lie in [1, 32]%s");
  if (!scaling) return fail(MXFP4_EINVAL, "moe: null LoRA scaling%s");
  for (int i = 0; i < 6; ++i) {
    if (!lora[i]) return fail(MXFP4_EINVAL, "moe: null LoRA factor%s");
    if (!aligned16(lora[i])) return fail(MXFP4_EINVAL, "moe: LoRA factors must be 16-byte aligned%s");
    lo.m[i] = lora[i];
  }
  lo.sg = scaling[0]; lo.su = scaling[1]; lo.sd = scaling[2];
  lo.r = rank;
  return MXFP4_OK;
}

// Device pointers of the LoRA stages: sources, adapters, routing and coefficient buffers.
LoraPtrs lora_ptrs(const Lora& lo, const void* h, int h_dtype, const float* topk_w, int k, const float* grad_out,
                   void* ws, const MoeLayout& L, int E, int D, int F, int act_kind)
{
  LoraPtrs p = {};
  p.x = mx::LoraMat{h_dtype == MXFP4_BF16 ? mx::kLoraBF16 : mx::kLoraF32, h, nullptr, D, 0, 0};
  p.g = mat_f32(grad_out, D);
  p.act = mx::LoraMat{mx::kLoraGLU, at<float>(ws, L.saved), nullptr, 2LL * F, F, act_kind};
  p.d = mx::LoraMat{mx::kLoraHiLo, at<uint16_t>(ws, L.d_hi), at<uint16_t>(ws, L.d_lo), 2LL * F, 0, 0};
  for (int i = 0; i < 6; ++i) p.m[i] = lo.m[i];
  p.n_valid = at<int>(ws, L.offsets) + E;
  p.pair_of = at<int>(ws, L.pair_of);
  p.topk_w = topk_w;
  p.k = k;
  p.u = at<float>(ws, L.l_u);
  p.q = at<float>(ws, L.l_q);
  p.vsum = at<float>(ws, L.l_vsum);
  p.dsum = at<float>(ws, L.l_dsum);
  return p;
}

hipError_t run_lora_pass(int stage, const LoraPtrs& p, int N, long long P, int D, int F, int r, void* ws,
                         const MoeLayout& L, mx::LoraPartial* parts, hipStream_t s)
{
  mx::LoraPassJob j[4];
  const int n = lora_pass_jobs(stage, p, N, P, D, F, r, j);
  return mx::launch_lora_pass(j, n, at<float>(ws, L.l_part), parts, s);
}

// Finish job turning row-dot partials into coefficient rows (see launch_lora_finish).
mx::LoraFinishJob coef_job(const mx::LoraPartial& part, int prow, int m, int r, float s0, float s1, int ntok,
                           float* out)
{
  mx::LoraFinishJob f = {};
  f.type = mx::kLoraFinCoef; f.part = part; f.prow = prow; f.m = m; f.r = r;
  f.scale[0] = s0; f.scale[1] = s1; f.ntok = ntok; f.out = out;
  return f;
}

// Finish job writing an outer-product gradient.
mx::LoraFinishJob grad_job(const mx::LoraPartial& part, int om, int Ctot, int Kseg, const mx::LoraOuterDst& dst)
{
  mx::LoraFinishJob f = {};
  f.type = mx::kLoraFinOuter; f.part = part; f.om = om; f.Ctot = Ctot; f.Kseg = Kseg; f.dst = dst;
  return f;
}

mx::LoraOuterDst dst_of(float* p0, long long ld0, int km0, float s0, float* p1, long long ld1, int km1, float s1,
                        int split_j)
{
  mx::LoraOuterDst d = {};
  d.p[0] = p0; d.ld[0] = ld0; d.kmajor[0] = km0; d.scale[0] = s0;
  d.p[1] = p1 ? p1 : p0; d.ld[1] = p1 ? ld1 : ld0; d.kmajor[1] = p1 ? km1 : km0; d.scale[1] = p1 ? s1 : s0;
  d.split_j = split_j;
  return d;
}

// Forward-layout copies {W1, W3, W2} (null array or entries: that product reads the checkpoint
// layout). An entry needs its matrix's K (D for W1 and W3, F for W2) to be a multiple of 512.
// With MXFP4_MOE_BWD_LAYOUT, entries 3..5 are the backward-layout copies of W1, W3, W2.
int check_forward_layout(const uint8_t* const* fl, int D, int F, int flags)
{
  if (!fl) return MXFP4_OK;
  for (int i = 0; i < 3; ++i) {
    if (!fl[i]) continue;
    if ((i < 2 ? D : F) % 512) return fail(MXFP4_EINVAL, "moe: a forward layout needs its K to be a multiple of 512%s");
    if (!aligned16(fl[i])) return fail(MXFP4_EINVAL, "moe: forward layouts must be 16-byte aligned%s");
  }
  if (!fl[0] != !fl[1]) return fail(MXFP4_EINVAL, "moe: give the forward layouts of W1 and W3 together%s");
  if (!(flags & MXFP4_MOE_BWD_LAYOUT)) return MXFP4_OK;
  for (int i = 3; i < 6; ++i) {
    if (!fl[i]) continue;
    if (!(i < 5 ? mx::backward_layout_ok(F, D) : mx::backward_layout_ok(D, F)))
      return fail(MXFP4_EINVAL, "moe: a backward layout needs K a multiple of 256 (D for W1 and W3, F for W2)%s");
    if (!aligned16(fl[i])) return fail(MXFP4_EINVAL, "moe: backward layouts must be 16-byte aligned%s");
  }
  if (!fl[3] != !fl[4]) return fail(MXFP4_EINVAL, "moe: give the backward layouts of W1 and W3 together%s");
  return MXFP4_OK;
}

// Routing + quantised x + gate/up (+GLU) into the workspace. With LoRA also the per-token
// adapter inputs U = [A_gate x | A_up x], their gate/up deltas (added in the product's
// epilogue) and V = sum over a token's slots of w * A_down act; gate|up are then always saved,
// since V and the backward read them.
int moe_front(const void* h, int h_dtype, const void* idx, int idx_dtype, const float* w, int N, int k,
              const uint8_t* const* wts, const uint8_t* const* fl, int E, int D, int F, int act_kind, bool save,
              const Lora& lo, void* ws, const MoeLayout& L, hipStream_t s)
{
  const long long P = (long long)N * k;
  MX_TRY(mx::launch_route(idx, idx_dtype == MXFP4_I64, w, N, k, E, at<int>(ws, L.counts), at<int>(ws, L.offsets),
                          at<int>(ws, L.cursor), at<int4>(ws, L.tiles), at<int>(ws, L.small_tiles),
                          at<int4>(ws, L.groups), at<int4>(ws, L.wgroups), at<int>(ws, L.meta), at<int>(ws, L.pair_token),
                          at<float>(ws, L.pair_w), at<int>(ws, L.pair_of), s),
         "route");
  MX_PHASE("route", s);
  // h once per token in the XT layout (with a zero row N for the unused slots of a tile), which
  // the one-tile work-groups gather; when the gate/up product splits its buckets, the tiles of
  // large buckets also in the AT layout, which the grouped work-groups re-read for every column
  // tile, and the XT rows are skipped when no bucket is small (the routing's meta says so on
  // the device). Without the split every tile reads the XT rows, so they are always written.
  const bool gu_split = mx::fwd_bucket_split(F, D);
  MX_TRY(mx::launch_quant_rows(h, h_dtype == MXFP4_BF16, D, N, D, gu_split ? at<int>(ws, L.meta) : nullptr,
                               at<uint8_t>(ws, L.xt_x), at<uint8_t>(ws, L.x3_x), at<int>(ws, L.meta) + 6, s),
         "quantise h");
  if (gu_split) {
    MX_TRY(mx::launch_quant_tiles(h, h_dtype == MXFP4_BF16, D, N, D, at<int4>(ws, L.tiles), at<int>(ws, L.meta),
                                  L.max_tiles, at<int>(ws, L.pair_token), 1, at<uint8_t>(ws, L.xt_x),
                                  at<int>(ws, L.meta), at<uint8_t>(ws, L.at_x), at<uint8_t>(ws, L.x3_x),
                                  at<int>(ws, L.meta) + 6, s, at<int4>(ws, L.groups), at<int>(ws, L.meta) + 3),
           "quantise h tiles");
  }
  MX_PHASE("quant_h", s);
  if (F % mx::kChunk) {  // padding blocks of the act buffer are read by the down product
    MX_TRY(mx::launch_zero(at<void>(ws, L.at_act), at_bytes(L.max_tiles, F), s), "zero act");
  }
  mx::FwdArgs a = {};
  a.wp0 = wts[0]; a.ws0 = wts[1]; a.wp1 = wts[2]; a.ws1 = wts[3];
  a.wp_estride = (long long)F * D / 2;
  a.ws_estride = (long long)F * D / 32;
  a.R = F; a.K = D;
  a.a_tiles = at<uint8_t>(ws, L.at_x);
  a.a_rows = at<uint8_t>(ws, L.xt_x);
  a.a_row_bytes = mx::xt_row_bytes(D);
  a.a_zero_row = N;
  a.x3 = at<uint8_t>(ws, L.x3_x);
  a.x3_row_bytes = mx::x3_row_bytes(D);
  a.x3_any = at<int>(ws, L.meta) + 6;
  a.row_token = at<int>(ws, L.pair_token);
  a.tiles = at<int4>(ws, L.tiles); a.n_tiles = at<int>(ws, L.meta);
  a.n_ct = F / 32;
  a.q_tiles = at<uint8_t>(ws, L.at_act);
  set_buckets(a, ws, L);
  if (fl && fl[0] && fl[1]) {
    a.fl0 = fl[0]; a.fl1 = fl[1];
    a.fl_estride = mx::forward_layout_bytes(F, D);
  }
  a.wcounter = at<int>(ws, L.meta) + 8;
  a.save = (save || lo.r) ? at<float>(ws, L.saved) : nullptr;
  a.act_kind = act_kind;
  const int r = lo.r;
  LoraPtrs lp = {};
  mx::LoraPartial parts[4];
  if (r) {  // U = [A_gate x | A_up x] per token, expanded into the gate/up deltas s B U
    lp = lora_ptrs(lo, h, h_dtype, w, k, nullptr, ws, L, E, D, F, act_kind);
    MX_TRY(run_lora_pass(0, lp, N, P, D, F, r, ws, L, parts, s), "LoRA: A x");
    const mx::LoraFactor fb[2] = {kmajor(lo.m[1], r, lo.sg), kmajor(lo.m[3], r, lo.su)};
    const int coff[2] = {0, r};
    const float one[2] = {1.f, 1.f};
    MX_TRY(mx::launch_lora_expand(at<float>(ws, L.l_u), 2 * r, N, r, at<float>(ws, L.l_delta), 2LL * F, 2 * F, F, fb,
                                  coff, s, &parts[0], one),
           "LoRA: gate/up deltas");
    a.lora_delta = at<float>(ws, L.l_delta);
    MX_PHASE("lora_in", s);
  }
  MX_TRY(mx::launch_fwd(a, mx::kFwdGateUp, L.max_tiles, s), "gate/up product");
  MX_PHASE("fwd_gateup", s);
  if (r) {  // V = sum over a token's slots of w * A_down act
    MX_TRY(run_lora_pass(1, lp, N, P, D, F, r, ws, L, parts, s), "LoRA: A_down act");
    mx::LoraFinishJob f = coef_job(parts[0], (int)P, r, r, 1.f, 1.f, N, at<float>(ws, L.l_vsum));
    f.pair_of = at<int>(ws, L.pair_of); f.topk_w = w; f.k = k;
    MX_TRY(mx::launch_lora_finish(&f, 1, s), "LoRA: slot sum");
    MX_PHASE("lora_mid", s);
  }
  return MXFP4_OK;
}

// Argument checks of the single-expert forward product (mxfp4_gemm and mxfp4_gemm_noalloc).
int check_gemm_args(const float* y, const float* x, const uint8_t* packed, const uint8_t* scales, int M, int K,
                    int R)
{
  if (M < 0 || R < 0 || K <= 0 || K % 32) return fail(MXFP4_EINVAL, "gemm: K must be a positive multiple of 32%s");
  if (M == 0 || R == 0) return MXFP4_OK;
  if (!y || !x || !packed || !scales) return fail(MXFP4_EINVAL, "gemm: null pointer%s");
  if (!aligned16(packed) || !aligned16(scales)) return fail(MXFP4_EINVAL, "gemm: packed and scales must be 16-byte aligned%s");
  if (((uintptr_t)x & 7) != 0) return fail(MXFP4_EINVAL, "gemm: x must be 8-byte aligned%s");
  return MXFP4_OK;
}

// y[M, R] = x . W^T with x's two-term e4m3 tiles staged at `tiles` (at_bytes(ceil(M/16), K)
// bytes, fully rewritten by the quantiser: unused row slots and K positions past the row end are
// written as zeros, so the buffer needs no clearing between calls).
int gemm_into(float* y, const float* x, const uint8_t* packed, const uint8_t* scales, int M, int K, int R,
              uint8_t* tiles_dev, hipStream_t stream)
{
  const int tiles = (M + mx::kFwdRowsPerTile - 1) / mx::kFwdRowsPerTile;
  MX_TRY(mx::launch_quant_tiles(x, 0, K, M, K, nullptr, nullptr, tiles, nullptr, 0, nullptr, nullptr, tiles_dev,
                                nullptr, nullptr, stream),
         "gemm: quantise x");
  mx::FwdArgs a = {};
  a.wp0 = packed; a.ws0 = scales;
  a.R = R; a.K = K;
  a.a_tiles = tiles_dev;
  a.M = M;
  a.n_ct = (R + mx::kFwdColsPerTile - 1) / mx::kFwdColsPerTile;
  a.y = y; a.ldy = R;
  MX_TRY(mx::launch_fwd(a, mx::kFwdPlain, tiles, stream), "gemm: product");
  return MXFP4_OK;
}

// ---------------------------------------------------------------- allocation-free scratch
// mxfp4_gemm_noalloc stages its activation tiles in the file-scope device array `scratch` (top of
// this file) instead of a caller workspace. Every GPU that loads the library holds its own copy
// until the process ends.
// Host code never uses the array's name as an address (on the host it is only a stand-in
// symbol): the device address is looked up once per device with hipGetSymbolAddress, with that
// device current, and kept in g_scratch. All calls on one device share the array, so calls that
// overlap on one device (two streams, two host threads) race on it.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch[kMaxDevices] = {};

int scratch_on_current_device(uint8_t** out)
{
  int dev = 0;
  MX_TRY(hipGetDevice(&dev), "gemm_noalloc: hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(MXFP4_EINVAL, "gemm_noalloc: device index out of range%s");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    MX_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "gemm_noalloc: hipGetSymbolAddress(scratch)");
    if (!p) return fail(MXFP4_EHIP, "gemm_noalloc: no device address for the scratch array%s");
    g_scratch[dev] = static_cast<uint8_t*>(p);
  }
  *out = g_scratch[dev];
  return MXFP4_OK;
}

}  // namespace

extern "C" {

const char* mxfp4_last_error(void) { return g_err; }

int mxfp4_threads(void)
{
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 1;
  return cus > 0 ? cus : 1;
}

int mxfp4_dequant(float* out, const uint8_t* packed, const uint8_t* scales, int K, int R, hipStream_t stream)
{
  if (K <= 0 || R < 0 || K % 32) return fail(MXFP4_EINVAL, "dequant: K must be a positive multiple of 32%s");
  if (R > 0 && (!out || !packed || !scales)) return fail(MXFP4_EINVAL, "dequant: null pointer%s");
  MX_TRY(mx::launch_dequant(out, 0, packed, scales, K, R, stream), "dequant");
  return MXFP4_OK;
}

int mxfp4_dequant_bf16(uint16_t* out, const uint8_t* packed, const uint8_t* scales, int K, int R, hipStream_t stream)
{
  if (K <= 0 || R < 0 || K % 32) return fail(MXFP4_EINVAL, "dequant_bf16: K must be a positive multiple of 32%s");
  if (R > 0 && (!out || !packed || !scales)) return fail(MXFP4_EINVAL, "dequant_bf16: null pointer%s");
  if (R > 0 && ((uintptr_t)out & 3)) return fail(MXFP4_EINVAL, "dequant_bf16: out must be 4-byte aligned%s");
  MX_TRY(mx::launch_dequant(out, 1, packed, scales, K, R, stream), "dequant_bf16");
  return MXFP4_OK;
}

size_t mxfp4_gemm_workspace_size(int M, int K, int R)
{
  (void)R;
  if (M <= 0 || K <= 0) return 0;
  return at_bytes((M + mx::kFwdRowsPerTile - 1) / mx::kFwdRowsPerTile, K);
}

int mxfp4_gemm(float* y, const float* x, const uint8_t* packed, const uint8_t* scales, int M, int K, int R,
               void* workspace, size_t workspace_bytes, hipStream_t stream)
{
  const int rc = check_gemm_args(y, x, packed, scales, M, K, R);
  if (rc != MXFP4_OK || M == 0 || R == 0) return rc;
  const int tiles = (M + mx::kFwdRowsPerTile - 1) / mx::kFwdRowsPerTile;
  if (!workspace || workspace_bytes < at_bytes(tiles, K)) return fail(MXFP4_EWORKSPACE, "gemm: workspace too small%s");
  return gemm_into(y, x, packed, scales, M, K, R, at<uint8_t>(workspace, 0), stream);
}

int mxfp4_gemm_noalloc(float* y, const float* x, const uint8_t* packed, const uint8_t* scales, int M, int K, int R,
                       hipStream_t stream)
{
  const int rc = check_gemm_args(y, x, packed, scales, M, K, R);
  if (rc != MXFP4_OK || M == 0 || R == 0) return rc;
  const int tiles = (M + mx::kFwdRowsPerTile - 1) / mx::kFwdRowsPerTile;
  if (at_bytes(tiles, K) > kScratchBytes)
    return fail(MXFP4_EWORKSPACE,
                "gemm_noalloc: the activation tiles of this M x K exceed the library's 16 MiB device scratch "
                "(ceil(M/16) * ceil(K/512) * 16896 bytes); use mxfp4_gemm with a workspace%s");
  uint8_t* tiles_dev = nullptr;
  const int src = scratch_on_current_device(&tiles_dev);
  if (src != MXFP4_OK) return src;
  return gemm_into(y, x, packed, scales, M, K, R, tiles_dev, stream);
}

size_t mxfp4_gemm_t_workspace_size(int M, int K, int R)
{
  (void)K;
  if (M <= 0 || R <= 0) return 0;
  return 2 * align_up(2 * (size_t)M * (size_t)pad32(R));
}

int mxfp4_gemm_t(float* y, const float* dy, const uint8_t* packed, const uint8_t* scales, int M, int K, int R,
                 void* workspace, size_t workspace_bytes, hipStream_t stream)
{
  if (M < 0 || R < 0 || K <= 0 || K % 32) return fail(MXFP4_EINVAL, "gemm_t: K must be a positive multiple of 32%s");
  if (M == 0 || R == 0) return MXFP4_OK;
  if (!y || !dy || !packed || !scales) return fail(MXFP4_EINVAL, "gemm_t: null pointer%s");
  if (!aligned16(packed) || !aligned16(scales)) return fail(MXFP4_EINVAL, "gemm_t: packed and scales must be 16-byte aligned%s");
  if (((uintptr_t)dy & 3) != 0) return fail(MXFP4_EINVAL, "gemm_t: dy must be 4-byte aligned%s");
  if (!aligned16(y)) return fail(MXFP4_EINVAL, "gemm_t: y must be 16-byte aligned%s");
  const size_t need = mxfp4_gemm_t_workspace_size(M, K, R);
  if (!workspace || workspace_bytes < need) return fail(MXFP4_EWORKSPACE, "gemm_t: workspace too small%s");
  const long long rp = pad32(R);
  uint16_t* hi = at<uint16_t>(workspace, 0);
  uint16_t* lo = at<uint16_t>(workspace, need / 2);
  MX_TRY(mx::launch_split_bf16(dy, R, M, R, (int)rp, hi, lo, stream), "gemm_t: split dy");
  mx::BwdArgs a = {};
  a.wp0 = packed; a.ws0 = scales;
  a.nseg = 1; a.R = R; a.C = K;
  a.a_hi = hi; a.a_lo = lo; a.lda = rp;
  a.M = M;
  a.n_ct = (K + mx::kBwdColsPerTile - 1) / mx::kBwdColsPerTile;
  a.y = y; a.ldy = K; a.accumulate = 1;
  const int tiles = (M + mx::kFwdRowsPerTile - 1) / mx::kFwdRowsPerTile;
  MX_TRY(mx::launch_bwd(a, mx::kBwdPlain, tiles, stream), "gemm_t: product");
  return MXFP4_OK;
}

size_t mxfp4_moe_workspace_size(int N, int k, int E, int D, int F)
{
  if (N < 0 || k <= 0 || E <= 0 || D <= 0 || F <= 0) return 0;
  return moe_layout(N, k, E, D, F).end;
}

size_t mxfp4_forward_layout_bytes(int E, int R, int K)
{
  if (E <= 0 || R <= 0 || K <= 0 || K % 512) return 0;
  return (size_t)E * (size_t)mx::forward_layout_bytes(R, K);
}

int mxfp4_forward_layout(uint8_t* dst, const uint8_t* packed, const uint8_t* scales, int E, int R, int K,
                         hipStream_t stream)
{
  if (E < 0 || R < 0 || K <= 0 || K % 512)
    return fail(MXFP4_EINVAL, "forward_layout: K must be a positive multiple of 512%s");
  if (E == 0 || R == 0) return MXFP4_OK;
  if (!dst || !packed || !scales) return fail(MXFP4_EINVAL, "forward_layout: null pointer%s");
  if (!aligned16(dst) || !aligned16(packed) || !aligned16(scales))
    return fail(MXFP4_EINVAL, "forward_layout: dst, packed and scales must be 16-byte aligned%s");
  const uintptr_t d0 = (uintptr_t)dst, d1 = d0 + mxfp4_forward_layout_bytes(E, R, K);
  const uintptr_t p0 = (uintptr_t)packed, p1 = p0 + (size_t)E * R * (K / 2);
  const uintptr_t s0 = (uintptr_t)scales, s1 = s0 + (size_t)E * R * (K / 32);
  if ((d0 < p1 && p0 < d1) || (d0 < s1 && s0 < d1))
    return fail(MXFP4_EINVAL, "forward_layout: dst overlaps packed or scales%s");
  MX_TRY(mx::launch_forward_layout(packed, scales, dst, E, R, K, stream), "forward_layout");
  return MXFP4_OK;
}

size_t mxfp4_backward_layout_bytes(int E, int R, int K)
{
  if (E <= 0 || !mx::backward_layout_ok(R, K)) return 0;
  return (size_t)E * (size_t)mx::backward_layout_bytes(R, K);
}

int mxfp4_backward_layout(uint8_t* dst, const uint8_t* packed, const uint8_t* scales, int E, int R, int K,
                          hipStream_t stream)
{
  if (E < 0 || !mx::backward_layout_ok(R, K))
    return fail(MXFP4_EINVAL, "backward_layout: R must be a positive multiple of 32 and K of 256%s");
  if (E == 0) return MXFP4_OK;
  if (!dst || !packed || !scales) return fail(MXFP4_EINVAL, "backward_layout: null pointer%s");
  if (!aligned16(dst) || !aligned16(packed) || !aligned16(scales))
    return fail(MXFP4_EINVAL, "backward_layout: dst, packed and scales must be 16-byte aligned%s");
  const uintptr_t d0 = (uintptr_t)dst, d1 = d0 + mxfp4_backward_layout_bytes(E, R, K);
  const uintptr_t p0 = (uintptr_t)packed, p1 = p0 + (size_t)E * R * (K / 2);
  const uintptr_t s0 = (uintptr_t)scales, s1 = s0 + (size_t)E * R * (K / 32);
  if ((d0 < p1 && p0 < d1) || (d0 < s1 && s0 < d1))
    return fail(MXFP4_EINVAL, "backward_layout: dst overlaps packed or scales%s");
  MX_TRY(mx::launch_backward_layout(packed, scales, dst, E, R, K, stream), "backward_layout");
  return MXFP4_OK;
}

int mxfp4_moe_forward_fl(float* out, const void* h, int h_dtype, const void* topk_idx, int idx_dtype,
                         const float* topk_w, int N, int k, const uint8_t* w1p, const uint8_t* w1s, const uint8_t* w3p,
                         const uint8_t* w3s, const uint8_t* w2p, const uint8_t* w2s, const uint8_t* const* fwd_layout,
                         int E, int D, int F, int act_kind, const float* const* lora, const float* lora_scaling,
                         int lora_rank, int flags, void* workspace, size_t workspace_bytes, hipStream_t stream)
{
  const uint8_t* wts[6] = {w1p, w1s, w3p, w3s, w2p, w2s};
  int rc = check_moe_args(h, h_dtype, topk_idx, idx_dtype, topk_w, N, k, wts, E, D, F, act_kind);
  if (rc) return rc;
  rc = check_forward_layout(fwd_layout, D, F, flags);
  if (rc) return rc;
  Lora lo;
  rc = check_lora(lora, lora_scaling, lora_rank, lo);
  if (rc) return rc;
  if (lo.r && !aligned16(h)) return fail(MXFP4_EINVAL, "moe_forward: h must be 16-byte aligned with LoRA%s");
  if (N > 0 && !out) return fail(MXFP4_EINVAL, "moe_forward: null output%s");
  const MoeLayout L = moe_layout(N, k, E, D, F);
  if (!workspace || workspace_bytes < L.end) return fail(MXFP4_EWORKSPACE, "moe_forward: workspace too small%s");
  if (N == 0) return MXFP4_OK;
  MX_TRY(g_timer.begin(stream), "phase timer");
  rc = moe_front(h, h_dtype, topk_idx, idx_dtype, topk_w, N, k, wts, fwd_layout, E, D, F, act_kind,
                 (flags & MXFP4_MOE_SAVE) != 0, lo, workspace, L, stream);
  if (rc) return rc;
  mx::FwdArgs a = {};
  a.wp0 = w2p; a.ws0 = w2s;
  if (fwd_layout && fwd_layout[2]) {
    a.fl0 = fwd_layout[2];
    a.fl_estride = mx::forward_layout_bytes(D, F);
  }
  a.wp_estride = (long long)F * D / 2;
  a.ws_estride = (long long)F * D / 32;
  a.R = D; a.K = F;
  a.a_tiles = at<uint8_t>(workspace, L.at_act);
  a.tiles = at<int4>(workspace, L.tiles); a.n_tiles = at<int>(workspace, L.meta);
  a.n_ct = (D + mx::kFwdColsPerTile - 1) / mx::kFwdColsPerTile;
  a.y = at<float>(workspace, L.ypair); a.ldy = D;
  // top-1 routing without LoRA: each token has at most one row, which the down product writes
  // straight into out (already weighted); only tokens with no row need their zeros
  const bool direct = k == 1 && !lo.r;
  if (direct) {
    a.y = out;
    a.y_rows = at<int>(workspace, L.pair_token);
  }
  a.row_w = at<float>(workspace, L.pair_w);
  set_buckets(a, workspace, L);
  a.wcounter = at<int>(workspace, L.meta) + 10;
  MX_TRY(mx::launch_fwd(a, mx::kFwdDown, L.max_tiles, stream), "moe_forward: down product");
  MX_PHASE("fwd_down", stream);
  if (direct) {
    MX_TRY(mx::launch_zero_unrouted(out, D, D, at<int>(workspace, L.pair_of), N, stream), "moe_forward: unrouted rows");
  } else if (lo.r) {  // out = combine + s_down B_down V, V = sum over the token's slots of w A_down act
    const mx::LoraFactor fb = kmajor(lo.m[5], lo.r, lo.sd);
    MX_TRY(mx::launch_lora_combine(out, at<float>(workspace, L.ypair), D, at<int>(workspace, L.pair_of), N, k, D,
                                   at<float>(workspace, L.l_vsum), lo.r, 1, &fb, nullptr, nullptr, 0, stream),
           "moe_forward: combine");
  } else {
    MX_TRY(mx::launch_combine(out, at<float>(workspace, L.ypair), D, at<int>(workspace, L.pair_of), N, k, D, stream),
           "moe_forward: combine");
  }
  MX_PHASE("fwd_combine", stream);
  return MXFP4_OK;
}

int mxfp4_moe_forward_lora(float* out, const void* h, int h_dtype, const void* topk_idx, int idx_dtype,
                           const float* topk_w, int N, int k, const uint8_t* w1p, const uint8_t* w1s,
                           const uint8_t* w3p, const uint8_t* w3s, const uint8_t* w2p, const uint8_t* w2s, int E,
                           int D, int F, int act_kind, const float* const* lora, const float* lora_scaling,
                           int lora_rank, int flags, void* workspace, size_t workspace_bytes, hipStream_t stream)
{
  return mxfp4_moe_forward_fl(out, h, h_dtype, topk_idx, idx_dtype, topk_w, N, k, w1p, w1s, w3p, w3s, w2p, w2s,
                              nullptr, E, D, F, act_kind, lora, lora_scaling, lora_rank, flags, workspace,
                              workspace_bytes, stream);
}

int mxfp4_moe_forward(float* out, const void* h, int h_dtype, const void* topk_idx, int idx_dtype,
                      const float* topk_w, int N, int k, const uint8_t* w1p, const uint8_t* w1s, const uint8_t* w3p,
                      const uint8_t* w3s, const uint8_t* w2p, const uint8_t* w2s, int E, int D, int F, int act_kind,
                      int flags, void* workspace, size_t workspace_bytes, hipStream_t stream)
{
  return mxfp4_moe_forward_lora(out, h, h_dtype, topk_idx, idx_dtype, topk_w, N, k, w1p, w1s, w3p, w3s, w2p, w2s, E,
                                D, F, act_kind, nullptr, nullptr, 0, flags, workspace, workspace_bytes, stream);
}

int mxfp4_moe_backward_fl(float* grad_h, float* grad_w, const float* grad_out, const void* h, int h_dtype,
                          const void* topk_idx, int idx_dtype, const float* topk_w, int N, int k, const uint8_t* w1p,
                          const uint8_t* w1s, const uint8_t* w3p, const uint8_t* w3s, const uint8_t* w2p,
                          const uint8_t* w2s, const uint8_t* const* fwd_layout, int E, int D, int F, int act_kind,
                          const float* const* lora, const float* lora_scaling, int lora_rank,
                          float* const* lora_grads, int flags, void* workspace, size_t workspace_bytes,
                          hipStream_t stream)
{
  const uint8_t* wts[6] = {w1p, w1s, w3p, w3s, w2p, w2s};
  int rc = check_moe_args(h, h_dtype, topk_idx, idx_dtype, topk_w, N, k, wts, E, D, F, act_kind);
  if (rc) return rc;
  rc = check_forward_layout(fwd_layout, D, F, flags);
  if (rc) return rc;
  Lora lo;
  rc = check_lora(lora, lora_scaling, lora_rank, lo);
  if (rc) return rc;
  if (lo.r) {
    if (!aligned16(h) || !aligned16(grad_out))
      return fail(MXFP4_EINVAL, "moe_backward: h and grad_out must be 16-byte aligned with LoRA%s");
    if (!lora_grads) return fail(MXFP4_EINVAL, "moe_backward: null LoRA gradient array%s");
    for (int i = 0; i < 6; ++i)
      if (!lora_grads[i]) return fail(MXFP4_EINVAL, "moe_backward: null LoRA gradient%s");
  }
  if (N > 0 && (!grad_h || !grad_w || !grad_out)) return fail(MXFP4_EINVAL, "moe_backward: null pointer%s");
  const MoeLayout L = moe_layout(N, k, E, D, F);
  if (!workspace || workspace_bytes < L.end) return fail(MXFP4_EWORKSPACE, "moe_backward: workspace too small%s");
  if (N == 0) {
    if (lo.r) {  // no tokens: the adapter gradients are zero
      const size_t n[6] = {(size_t)lo.r * D, (size_t)F * lo.r, (size_t)lo.r * D, (size_t)F * lo.r, (size_t)lo.r * F,
                           (size_t)D * lo.r};
      for (int i = 0; i < 6; ++i) MX_TRY(mx::launch_zero(lora_grads[i], n[i] * sizeof(float), stream), "zero grads");
    }
    return MXFP4_OK;
  }
  MX_TRY(g_timer.begin(stream), "phase timer");
  if (!(flags & MXFP4_MOE_REUSE_FORWARD)) {
    rc = moe_front(h, h_dtype, topk_idx, idx_dtype, topk_w, N, k, wts, fwd_layout, E, D, F, act_kind, true, lo,
                   workspace, L, stream);
    if (rc) return rc;
  }
  // grad_out -> bf16 hi + lo, the A operand of the W2 transposed product
  MX_TRY(mx::launch_split_bf16(grad_out, D, N, D, D, at<uint16_t>(workspace, L.g_hi), at<uint16_t>(workspace, L.g_lo),
                               stream),
         "moe_backward: split grad_out");
  MX_PHASE("split_grad", stream);
  const int r = lo.r;
  const long long P = (long long)N * k;
  LoraPtrs lp = {};
  mx::LoraPartial parts[4];
  if (r) {  // q = s_down B_down^T g per token, and its expansion A_down^T q for the W2 epilogue
    lp = lora_ptrs(lo, h, h_dtype, topk_w, k, grad_out, workspace, L, E, D, F, act_kind);
    MX_TRY(run_lora_pass(2, lp, N, P, D, F, r, workspace, L, parts, stream), "moe_backward: LoRA B_down^T g");
    const mx::LoraFactor fa = jmajor(lo.m[4], F, 1.f);
    const int coff = 0;
    const float sd[2] = {lo.sd, lo.sd};
    MX_TRY(mx::launch_lora_expand(at<float>(workspace, L.l_q), r, N, r, at<float>(workspace, L.l_rq), F, F, 0, &fa,
                                  &coff, stream, &parts[0], sd),
           "moe_backward: LoRA A_down^T q");
    MX_PHASE("lora_q", stream);
  }
  mx::BwdArgs b = {};
  b.wp0 = w2p; b.ws0 = w2s;
  b.wp_estride = (long long)F * D / 2;
  b.ws_estride = (long long)F * D / 32;
  b.nseg = 1; b.R = D; b.C = F;
  b.a_hi = at<uint16_t>(workspace, L.g_hi); b.a_lo = at<uint16_t>(workspace, L.g_lo); b.lda = D;
  b.a_row_map = at<int>(workspace, L.pair_token);
  b.tiles = at<int4>(workspace, L.tiles); b.n_tiles = at<int>(workspace, L.meta);
  b.n_ct = L.n_ct_bwd;
  b.row_w = at<float>(workspace, L.pair_w);
  b.saved = at<float>(workspace, L.saved);
  b.act_kind = act_kind;
  b.d_hi = at<uint16_t>(workspace, L.d_hi); b.d_lo = at<uint16_t>(workspace, L.d_lo);
  b.gw_part = at<float>(workspace, L.gw_part);
  set_buckets(b, workspace, L);
  b.lora_rq = r ? at<float>(workspace, L.l_rq) : nullptr;
  const bool bl = fwd_layout && (flags & MXFP4_MOE_BWD_LAYOUT);
  if (bl && fwd_layout[5]) {
    b.bl0 = fwd_layout[5];
    b.bl_estride = mx::backward_layout_bytes(D, F);
  }
  MX_TRY(mx::launch_bwd(b, mx::kBwdDownT, L.max_tiles, stream), "moe_backward: W2 transposed product");
  MX_PHASE("bwd_down_t", stream);
  if (r) {
    // one pass over d = [d_gate | d_up], act and g: dh = [s_gate B_gate^T d_gate | s_up B_up^T d_up]
    // per pair, summed over each token's slots into Dsum, and the B_gate, B_up, A_down and B_down
    // gradients (lora_layer.py:178-226, summed over the experts)
    MX_TRY(run_lora_pass(3, lp, N, P, D, F, r, workspace, L, parts, stream), "moe_backward: LoRA pass over d");
    mx::LoraFinishJob f[4];
    const int o = r <= 16 ? 0 : 1;  // rank above 16: the row dots are a job of their own
    const mx::LoraPartial dh = r <= 16 ? mx::LoraPartial{parts[0].p2, parts[0].count2, nullptr, 0} : parts[1];
    f[0] = coef_job(dh, (int)P, 2 * r, r, lo.sg, lo.su, N, at<float>(workspace, L.l_dsum));
    f[0].pair_of = at<int>(workspace, L.pair_of); f[0].k = k;
    // B_gate, B_up: s * sum over pairs of d_gate (d_up) (x) A_gate x (A_up x) of the pair's token
    f[1] = grad_job(parts[0], r, 2 * F, F, dst_of(lora_grads[1], r, 1, lo.sg, lora_grads[3], r, 1, lo.su, 0));
    // A_down: sum over pairs of w q(token) (x) act
    f[2] = grad_job(parts[1 + o], r, F, 0, dst_of(lora_grads[4], F, 0, 1.f, nullptr, 0, 0, 0.f, 0));
    // B_down: s * sum over tokens of g (x) V
    f[3] = grad_job(parts[2 + o], r, D, 0, dst_of(lora_grads[5], r, 1, lo.sd, nullptr, 0, 0, 0.f, 0));
    MX_TRY(mx::launch_lora_finish(f, 4, stream), "moe_backward: LoRA slot sums and B/A_down gradients");
    MX_PHASE("lora_dx", stream);
  }

  mx::BwdArgs c = {};
  c.wp0 = w1p; c.ws0 = w1s; c.wp1 = w3p; c.ws1 = w3s;
  c.wp_estride = (long long)F * D / 2;
  c.ws_estride = (long long)F * D / 32;
  c.nseg = 2; c.R = F; c.C = D;
  c.a_hi = at<uint16_t>(workspace, L.d_hi); c.a_lo = at<uint16_t>(workspace, L.d_lo); c.lda = 2LL * F;
  c.tiles = at<int4>(workspace, L.tiles); c.n_tiles = at<int>(workspace, L.meta);
  c.n_ct = (D + mx::kBwdColsPerTile - 1) / mx::kBwdColsPerTile;
  c.y = at<float>(workspace, L.ypair); c.ldy = D;
  set_buckets(c, workspace, L);
  if (bl && fwd_layout[3] && fwd_layout[4]) {
    c.bl0 = fwd_layout[3]; c.bl1 = fwd_layout[4];
    c.bl_estride = mx::backward_layout_bytes(F, D);
  }
  MX_TRY(mx::launch_bwd(c, mx::kBwdGateUpT, L.max_tiles, stream), "moe_backward: W1|W3 transposed product");
  MX_PHASE("bwd_gateup_t", stream);
  if (r) {  // grad_h = combine + A_gate^T Dsum_gate + A_up^T Dsum_up
    const mx::LoraFactor fa[2] = {jmajor(lo.m[0], D, 1.f), jmajor(lo.m[2], D, 1.f)};
    MX_TRY(mx::launch_lora_combine(grad_h, at<float>(workspace, L.ypair), D, at<int>(workspace, L.pair_of), N, k, D,
                                   at<float>(workspace, L.l_dsum), r, 2, fa, grad_w, at<float>(workspace, L.gw_part),
                                   L.n_ct_bwd, stream),
           "moe_backward: combine");
  } else {
    MX_TRY(mx::launch_combine_bwd(grad_h, grad_w, at<float>(workspace, L.ypair), D, at<float>(workspace, L.gw_part),
                                  L.n_ct_bwd, at<int>(workspace, L.pair_of), N, k, D, stream),
           "moe_backward: combine");
  }
  MX_PHASE("bwd_combine", stream);
  if (r) {  // A_gate / A_up: sum over tokens of [Dsum_gate | Dsum_up] (x) x
    MX_TRY(run_lora_pass(4, lp, N, P, D, F, r, workspace, L, parts, stream), "moe_backward: LoRA pass over x");
    const mx::LoraFinishJob f =
        grad_job(parts[0], 2 * r, D, 0, dst_of(lora_grads[0], D, 0, 1.f, lora_grads[2], D, 0, 1.f, r));
    MX_TRY(mx::launch_lora_finish(&f, 1, stream), "moe_backward: LoRA grad A_gate/A_up");
    MX_PHASE("lora_grads", stream);
  }
  return MXFP4_OK;
}

int mxfp4_moe_backward_lora(float* grad_h, float* grad_w, const float* grad_out, const void* h, int h_dtype,
                            const void* topk_idx, int idx_dtype, const float* topk_w, int N, int k,
                            const uint8_t* w1p, const uint8_t* w1s, const uint8_t* w3p, const uint8_t* w3s,
                            const uint8_t* w2p, const uint8_t* w2s, int E, int D, int F, int act_kind,
                            const float* const* lora, const float* lora_scaling, int lora_rank,
                            float* const* lora_grads, int flags, void* workspace, size_t workspace_bytes,
                            hipStream_t stream)
{
  return mxfp4_moe_backward_fl(grad_h, grad_w, grad_out, h, h_dtype, topk_idx, idx_dtype, topk_w, N, k, w1p, w1s,
                               w3p, w3s, w2p, w2s, nullptr, E, D, F, act_kind, lora, lora_scaling, lora_rank,
                               lora_grads, flags, workspace, workspace_bytes, stream);
}

int mxfp4_moe_backward(float* grad_h, float* grad_w, const float* grad_out, const void* h, int h_dtype,
                       const void* topk_idx, int idx_dtype, const float* topk_w, int N, int k, const uint8_t* w1p,
                       const uint8_t* w1s, const uint8_t* w3p, const uint8_t* w3s, const uint8_t* w2p,
                       const uint8_t* w2s, int E, int D, int F, int act_kind, int flags, void* workspace,
                       size_t workspace_bytes, hipStream_t stream)
{
  return mxfp4_moe_backward_lora(grad_h, grad_w, grad_out, h, h_dtype, topk_idx, idx_dtype, topk_w, N, k, w1p, w1s,
                                 w3p, w3s, w2p, w2s, E, D, F, act_kind, nullptr, nullptr, 0, nullptr, flags, workspace,
                                 workspace_bytes, stream);
}

int mxfp4_moe_timing(int enable)
{
  MX_TRY(g_timer.enable(enable != 0), "moe_timing: create events");
  return MXFP4_OK;
}

int mxfp4_moe_timed_calls(void) { return g_timer.calls; }

int mxfp4_moe_phase_times(int call, float* ms, const char** names, int max_phases)
{
  if (call < 0 || call >= g_timer.calls || call < g_timer.calls - PhaseTimer::kRing)
    return fail(MXFP4_EINVAL, "moe_phase_times: call not in the timing ring%s");
  const int slot = call % PhaseTimer::kRing;
  const int n = g_timer.n[slot];
  if (n > 0) MX_TRY(hipEventSynchronize(g_timer.ev[slot][n]), "moe_phase_times: sync");
  for (int p = 0; p < n && p < max_phases; ++p) {
    float t = 0.f;
    MX_TRY(hipEventElapsedTime(&t, g_timer.ev[slot][p], g_timer.ev[slot][p + 1]), "moe_phase_times: elapsed");
    if (ms) ms[p] = t;
    if (names) names[p] = g_timer.names[slot][p];
  }
  return n;
}

int mxfp4_router_topk(int64_t* topk_idx, float* topk_w, const float* logits, const float* bias, int N, int E,
                      int top_k, float routed_scaling_factor, int renormalize, hipStream_t stream)
{
  if (N < 0 || E <= 0 || E > 4096) return fail(MXFP4_EINVAL, "router_topk: need 0 < E <= 4096 and N >= 0%s");
  if (top_k < 1 || top_k > E || top_k > 64) return fail(MXFP4_EINVAL, "router_topk: need 1 <= top_k <= min(E, 64)%s");
  if (N == 0) return MXFP4_OK;
  if (!topk_idx || !topk_w || !logits) return fail(MXFP4_EINVAL, "router_topk: null pointer%s");
  MX_TRY(mx::launch_router_topk(reinterpret_cast<long long*>(topk_idx), topk_w, logits, bias, N, E, top_k,
                                routed_scaling_factor, renormalize, stream),
         "router_topk");
  return MXFP4_OK;
}

int mxfp4_router_topk_backward(float* grad_logits, const int64_t* topk_idx, const float* grad_w, const float* logits,
                               int N, int E, int top_k, float routed_scaling_factor, int renormalize,
                               hipStream_t stream)
{
  if (N < 0 || E <= 0 || E > 4096) return fail(MXFP4_EINVAL, "router_topk_backward: need 0 < E <= 4096 and N >= 0%s");
  if (top_k < 1 || top_k > E || top_k > 64)
    return fail(MXFP4_EINVAL, "router_topk_backward: need 1 <= top_k <= min(E, 64)%s");
  if (N == 0) return MXFP4_OK;
  if (!grad_logits || !topk_idx || !grad_w || !logits) return fail(MXFP4_EINVAL, "router_topk_backward: null pointer%s");
  MX_TRY(mx::launch_router_topk_bwd(grad_logits, reinterpret_cast<const long long*>(topk_idx), grad_w, logits, N, E,
                                    top_k, routed_scaling_factor, renormalize, stream),
         "router_topk_backward");
  return MXFP4_OK;
}

int mxfp4_moe_route_status(const void* workspace, int* host_flags, hipStream_t stream)
{
  if (!workspace || !host_flags) return fail(MXFP4_EINVAL, "route_status: null pointer%s");
  MX_TRY(hipStreamSynchronize(stream), "route_status: sync");
  int meta[2] = {0, 0};
  MX_TRY(hipMemcpy(meta, workspace, sizeof(meta), hipMemcpyDeviceToHost), "route_status: copy");
  *host_flags = meta[1];
  return MXFP4_OK;
}

}  // extern "C"
