/*
 * CPU restatement of LazyLoRA's MXFP4 routed-expert path. TEST INFRASTRUCTURE ONLY.
 *
 * This file is the checker and the CPU baseline. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it. The product (lazylora_amd) never calls it.
 *
 * Format (lazy_lora/native/mxfp4_gemm.c:12-18): W is [R, K] row-major; packed is [R, K/2]
 * bytes with the low nibble holding the even element; scales is [R, K/32] E8M0 bytes. A code
 * is sign (bit 3) plus a magnitude index into {0, .5, 1, 1.5, 2, 3, 4, 6}; code 8 is -0.0.
 * The group multiplier is 2^(s-127), and any scale byte >= 253 contributes zero
 * (mxfp4_gemm.c:16-18, :40-42; lazy_lora/streaming/expert_streamer.py:55-63).
 *
 * The products follow the reference's accumulation schedule so that, compiled with the same
 * flags (-O3 -mavx2 -mfma -fopenmp, lazy_lora/native/build.sh:5), they produce the same fp32
 * bits wherever the reference itself can run (K <= 4096 for the forward product):
 *   forward   (mxfp4_gemm.c:64-94)  rows of W decoded 8 at a time; each dot product uses 8
 *             interleaved fp32 partial sums folded as ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)).
 *   transpose (mxfp4_gemm.c:96-129) threads own 32-column groups of y; rows are accumulated
 *             in ascending order, 8 at a time, so the result is deterministic.
 * The one deliberate difference: the decoded tile here is sized by K (heap, per thread), so
 * the K = 7168 gate/up products of the BASELINE shapes run; the reference's fixed stack tile
 * holds at most K = 4096 (mxfp4_gemm.c:72).
 *
 * Above the products, oracle_moe_forward / oracle_moe_backward compose one routed-expert
 * layer the way lazy_lora/trainer/lazy_trainer.py:806-880 does with LoRA off: per active
 * expert, gather its rows, gate/up products, GLU, down product, weighted index_add; and in
 * backward the recompute, grad_w = <g, down_e>, d_down = g * tw, three transposed products,
 * the GLU derivative and the index_add of the input gradient.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define MX_GROUP 32
#define ROW_BLOCK 8

/* E2M1 magnitudes by code, sign in bit 3 (mxfp4_gemm.c:33-34; expert_streamer.py:57-58). */
static const float kE2M1[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                                -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

/* 2^(s-127) for s < 253, else 0 (mxfp4_gemm.c:38-43). Built with exact integer bit patterns:
 * s >= 1 is the normal float with exponent field s; s = 0 is the subnormal 2^-127. */
static float e8m0_value(int s)
{
    if (s >= 253) return 0.0f;
    uint32_t bits = s >= 1 ? ((uint32_t)s << 23) : 0x00400000u;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static float g_e8m0[256];
static int g_e8m0_built = 0;

static void build_e8m0(void)
{
    for (int s = 0; s < 256; s++) g_e8m0[s] = e8m0_value(s);
    g_e8m0_built = 1;
}

/* One row of W [K] decoded to fp32 (mxfp4_gemm.c:45-62). */
static void decode_one_row(float *dst, const uint8_t *row_packed, const uint8_t *row_scales, int K)
{
    const int groups = K / MX_GROUP;
    for (int g = 0; g < groups; g++) {
        const float mult = g_e8m0[row_scales[g]];
        const uint8_t *src = row_packed + g * (MX_GROUP / 2);
        float *out = dst + g * MX_GROUP;
        for (int b = 0; b < MX_GROUP / 2; b++) {
            out[2 * b] = kE2M1[src[b] & 0xF] * mult;
            out[2 * b + 1] = kE2M1[src[b] >> 4] * mult;
        }
    }
}

int oracle_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* out[R, K] = decoded W (mxfp4_gemm.c:142-150). Bit-exact by construction. */
void oracle_dequant(float *out, const uint8_t *packed, const uint8_t *scales, int K, int R)
{
    if (!g_e8m0_built) build_e8m0();
#pragma omp parallel for schedule(static)
    for (int r = 0; r < R; r++)
        decode_one_row(out + (size_t)r * K, packed + (size_t)r * (K / 2),
                       scales + (size_t)r * (K / MX_GROUP), K);
}

/* y[M, R] = x[M, K] . W^T (mxfp4_gemm.c:64-94), tile sized by K. */
void oracle_gemm(float *y, const float *x, const uint8_t *packed, const uint8_t *scales,
                 int M, int K, int R)
{
    if (!g_e8m0_built) build_e8m0();
#pragma omp parallel
    {
        float *tile = (float *)malloc(sizeof(float) * ROW_BLOCK * (size_t)K);
#pragma omp for schedule(dynamic, 4)
        for (int r0 = 0; r0 < R; r0 += ROW_BLOCK) {
            const int nrows = (r0 + ROW_BLOCK <= R) ? ROW_BLOCK : R - r0;
            for (int i = 0; i < nrows; i++)
                decode_one_row(tile + (size_t)i * K, packed + (size_t)(r0 + i) * (K / 2),
                               scales + (size_t)(r0 + i) * (K / MX_GROUP), K);
            for (int m = 0; m < M; m++) {
                const float *xr = x + (size_t)m * K;
                for (int i = 0; i < nrows; i++) {
                    const float *w = tile + (size_t)i * K;
                    float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f, p4 = 0.f, p5 = 0.f, p6 = 0.f, p7 = 0.f;
                    int k = 0;
                    for (; k + 7 < K; k += 8) {
                        p0 += xr[k] * w[k];
                        p1 += xr[k + 1] * w[k + 1];
                        p2 += xr[k + 2] * w[k + 2];
                        p3 += xr[k + 3] * w[k + 3];
                        p4 += xr[k + 4] * w[k + 4];
                        p5 += xr[k + 5] * w[k + 5];
                        p6 += xr[k + 6] * w[k + 6];
                        p7 += xr[k + 7] * w[k + 7];
                    }
                    float acc = ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7));
                    for (; k < K; k++) acc += xr[k] * w[k];
                    y[(size_t)m * R + r0 + i] = acc;
                }
            }
        }
        free(tile);
    }
}

/* y[M, K] += dy[M, R] . W (mxfp4_gemm.c:96-129). */
void oracle_gemm_t(float *y, const float *dy, const uint8_t *packed, const uint8_t *scales,
                   int M, int K, int R)
{
    if (!g_e8m0_built) build_e8m0();
    const int groups = K / MX_GROUP;
#pragma omp parallel for schedule(static)
    for (int g = 0; g < groups; g++) {
        float wtile[ROW_BLOCK][MX_GROUP];
        for (int r0 = 0; r0 < R; r0 += ROW_BLOCK) {
            const int nrows = (r0 + ROW_BLOCK <= R) ? ROW_BLOCK : R - r0;
            for (int i = 0; i < nrows; i++) {
                const int r = r0 + i;
                const float mult = g_e8m0[scales[(size_t)r * groups + g]];
                const uint8_t *src = packed + (size_t)r * (K / 2) + g * (MX_GROUP / 2);
                for (int b = 0; b < MX_GROUP / 2; b++) {
                    wtile[i][2 * b] = kE2M1[src[b] & 0xF] * mult;
                    wtile[i][2 * b + 1] = kE2M1[src[b] >> 4] * mult;
                }
            }
            for (int m = 0; m < M; m++) {
                const float *d = dy + (size_t)m * R + r0;
                float *o = y + (size_t)m * K + g * MX_GROUP;
                for (int i = 0; i < nrows; i++) {
                    const float coef = d[i];
                    for (int c = 0; c < MX_GROUP; c++) o[c] += coef * wtile[i][c];
                }
            }
        }
    }
}

/* ------------------------------------------------------------------ GLU epilogues
 * act_kind 0 = SwiGLU: silu(g) * u.
 * act_kind 1 = SiTU-GLU (lazy_lora/core/situ_activation.py:47-75, constants :22-23):
 *   beta * tanh(g / beta) * sigmoid(g) * lbeta * tanh(u / lbeta), beta = 4, lbeta = 25.
 * Backward of SiTU-GLU follows situ_activation.py:78-134. Computed in fp32 like the reference. */
#define SITU_BETA 4.0f
#define SITU_LBETA 25.0f

static float sigmoidf_(float v) { return 1.0f / (1.0f + expf(-v)); }

static void glu_forward(float *act, const float *gate, const float *up, size_t n, int kind)
{
    for (size_t i = 0; i < n; i++) {
        const float g = gate[i], u = up[i];
        if (kind == 0) {
            act[i] = g * sigmoidf_(g) * u;
        } else {
            const float a = SITU_BETA * tanhf(g / SITU_BETA) * sigmoidf_(g);
            act[i] = a * (SITU_LBETA * tanhf(u / SITU_LBETA));
        }
    }
}

static void glu_backward(float *dgate, float *dup, const float *dact, const float *gate,
                         const float *up, size_t n, int kind)
{
    for (size_t i = 0; i < n; i++) {
        const float go = dact[i], g = gate[i], u = up[i];
        const float s = sigmoidf_(g);
        if (kind == 0) {
            const float silu = g * s;
            dgate[i] = go * u * (s * (1.0f + g * (1.0f - s)));
            dup[i] = go * silu;
        } else {
            const float t = tanhf(g / SITU_BETA);
            const float a = SITU_BETA * t * s;
            const float da = (1.0f - t * t) * s + SITU_BETA * t * s * (1.0f - s);
            const float tu = tanhf(u / SITU_LBETA);
            dgate[i] = go * (SITU_LBETA * tu) * da;
            dup[i] = go * a * (1.0f - tu * tu);
        }
    }
}

/* ------------------------------------------------------------------ routed layer
 * Expert e's matrices: w1 (gate) and w3 (up) are [F, D] -> packed [F, D/2], scales [F, D/32];
 * w2 (down) is [D, F] -> packed [D, F/2], scales [D, F/32]. They are passed as stacked
 * arrays, expert-major, with these per-expert strides. */
typedef struct {
    const uint8_t *w1p, *w1s, *w3p, *w3s, *w2p, *w2s;
} oracle_expert_set;

static void expert_ptrs(const oracle_expert_set *es, int e, int D, int F, const uint8_t **p)
{
    const size_t gp = (size_t)F * D / 2, gs = (size_t)F * D / 32;
    p[0] = es->w1p + e * gp;
    p[1] = es->w1s + e * gs;
    p[2] = es->w3p + e * gp;
    p[3] = es->w3s + e * gs;
    p[4] = es->w2p + e * gp;
    p[5] = es->w2s + e * gs;
}

/* Rows of expert e: tokens whose top-k list holds e (lazy_trainer.py:823-826). Returns the
 * count; rows[] gets token ids ascending, tw[] the summed combine weight of e per row. */
static int expert_rows(int e, const int64_t *topk_idx, const float *topk_w, int N, int k,
                       int *rows, float *tw)
{
    int n = 0;
    for (int t = 0; t < N; t++) {
        float w = 0.f;
        int hit = 0;
        for (int s = 0; s < k; s++)
            if (topk_idx[(size_t)t * k + s] == e) {
                w += topk_w[(size_t)t * k + s];
                hit = 1;
            }
        if (hit) {
            rows[n] = t;
            tw[n] = w;
            n++;
        }
    }
    return n;
}

/* out[N, D] fp32 = sum over experts of tw * expert(h) (lazy_trainer.py:806-834), with experts
 * visited in the order given by expert_order[0..n_active). */
void oracle_moe_forward(float *out, const float *h, const int64_t *topk_idx, const float *topk_w,
                        int N, int k, const uint8_t *w1p, const uint8_t *w1s, const uint8_t *w3p,
                        const uint8_t *w3s, const uint8_t *w2p, const uint8_t *w2s, int D, int F,
                        const int *expert_order, int n_active, int act_kind)
{
    oracle_expert_set es = {w1p, w1s, w3p, w3s, w2p, w2s};
    memset(out, 0, sizeof(float) * (size_t)N * D);
    int *rows = (int *)malloc(sizeof(int) * N);
    float *tw = (float *)malloc(sizeof(float) * N);
    float *x = (float *)malloc(sizeof(float) * (size_t)N * D);
    float *gate = (float *)malloc(sizeof(float) * (size_t)N * F);
    float *up = (float *)malloc(sizeof(float) * (size_t)N * F);
    float *act = (float *)malloc(sizeof(float) * (size_t)N * F);
    float *down = (float *)malloc(sizeof(float) * (size_t)N * D);
    for (int a = 0; a < n_active; a++) {
        const int e = expert_order[a];
        const int n = expert_rows(e, topk_idx, topk_w, N, k, rows, tw);
        if (n == 0) continue;
        const uint8_t *p[6];
        expert_ptrs(&es, e, D, F, p);
        for (int i = 0; i < n; i++) memcpy(x + (size_t)i * D, h + (size_t)rows[i] * D, sizeof(float) * D);
        oracle_gemm(gate, x, p[0], p[1], n, D, F);
        oracle_gemm(up, x, p[2], p[3], n, D, F);
        glu_forward(act, gate, up, (size_t)n * F, act_kind);
        oracle_gemm(down, act, p[4], p[5], n, F, D);
        for (int i = 0; i < n; i++) {
            float *o = out + (size_t)rows[i] * D;
            const float *dn = down + (size_t)i * D;
            for (int d = 0; d < D; d++) o[d] += dn[d] * tw[i];
        }
    }
    free(rows); free(tw); free(x); free(gate); free(up); free(act); free(down);
}

/* (grad_h [N, D], grad_w [N, k]) of oracle_moe_forward for upstream grad_out [N, D]
 * (lazy_trainer.py:836-880, LoRA off). */
void oracle_moe_backward(float *grad_h, float *grad_w, const float *grad_out, const float *h,
                         const int64_t *topk_idx, const float *topk_w, int N, int k,
                         const uint8_t *w1p, const uint8_t *w1s, const uint8_t *w3p,
                         const uint8_t *w3s, const uint8_t *w2p, const uint8_t *w2s, int D, int F,
                         const int *expert_order, int n_active, int act_kind)
{
    oracle_expert_set es = {w1p, w1s, w3p, w3s, w2p, w2s};
    memset(grad_h, 0, sizeof(float) * (size_t)N * D);
    memset(grad_w, 0, sizeof(float) * (size_t)N * k);
    int *rows = (int *)malloc(sizeof(int) * N);
    float *tw = (float *)malloc(sizeof(float) * N);
    float *x = (float *)malloc(sizeof(float) * (size_t)N * D);
    float *g = (float *)malloc(sizeof(float) * (size_t)N * D);
    float *gate = (float *)malloc(sizeof(float) * (size_t)N * F);
    float *up = (float *)malloc(sizeof(float) * (size_t)N * F);
    float *act = (float *)malloc(sizeof(float) * (size_t)N * F);
    float *down = (float *)malloc(sizeof(float) * (size_t)N * D);
    float *dact = (float *)malloc(sizeof(float) * (size_t)N * F);
    float *dgate = (float *)malloc(sizeof(float) * (size_t)N * F);
    float *dup = (float *)malloc(sizeof(float) * (size_t)N * F);
    float *dx = (float *)malloc(sizeof(float) * (size_t)N * D);
    for (int a = 0; a < n_active; a++) {
        const int e = expert_order[a];
        const int n = expert_rows(e, topk_idx, topk_w, N, k, rows, tw);
        if (n == 0) continue;
        const uint8_t *p[6];
        expert_ptrs(&es, e, D, F, p);
        for (int i = 0; i < n; i++) {
            memcpy(x + (size_t)i * D, h + (size_t)rows[i] * D, sizeof(float) * D);
            memcpy(g + (size_t)i * D, grad_out + (size_t)rows[i] * D, sizeof(float) * D);
        }
        oracle_gemm(gate, x, p[0], p[1], n, D, F);
        oracle_gemm(up, x, p[2], p[3], n, D, F);
        glu_forward(act, gate, up, (size_t)n * F, act_kind);
        oracle_gemm(down, act, p[4], p[5], n, F, D);
        /* grad_w[t, slot] += <g_t, down_e,t> for the slot that chose e (:861-862) */
        for (int i = 0; i < n; i++) {
            float dot = 0.f;
            for (int d = 0; d < D; d++) dot += g[(size_t)i * D + d] * down[(size_t)i * D + d];
            for (int s = 0; s < k; s++)
                if (topk_idx[(size_t)rows[i] * k + s] == e) grad_w[(size_t)rows[i] * k + s] += dot;
        }
        /* d_down = g * tw (:864-865), then three transposed products and the GLU derivative */
        for (int i = 0; i < n; i++)
            for (int d = 0; d < D; d++) g[(size_t)i * D + d] *= tw[i];
        memset(dact, 0, sizeof(float) * (size_t)n * F);
        oracle_gemm_t(dact, g, p[4], p[5], n, F, D);
        glu_backward(dgate, dup, dact, gate, up, (size_t)n * F, act_kind);
        memset(dx, 0, sizeof(float) * (size_t)n * D);
        oracle_gemm_t(dx, dgate, p[0], p[1], n, D, F);
        float *dx2 = down; /* reuse: [n, D] */
        memset(dx2, 0, sizeof(float) * (size_t)n * D);
        oracle_gemm_t(dx2, dup, p[2], p[3], n, D, F);
        for (int i = 0; i < n; i++) {
            float *o = grad_h + (size_t)rows[i] * D;
            for (int d = 0; d < D; d++) o[d] += dx[(size_t)i * D + d] + dx2[(size_t)i * D + d];
        }
    }
    free(rows); free(tw); free(x); free(g); free(gate); free(up); free(act); free(down);
    free(dact); free(dgate); free(dup); free(dx);
}
