/* knx_oracle.c — CPU oracle for the KERNIX forward hot path.  TEST INFRASTRUCTURE ONLY (see knx_oracle.h).
 * Build: oracle/build_oracle.sh (gcc -O3 -ffp-contract=off).  Not linked into the product library. */
#include "knx_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

/* ---- parallel-for: chunks handed out from an atomic counter to T threads (the calling thread included), the work
 * distribution of the reference pool, src/kernix_runtime.c:34-40, :107-138. ---- */
static int g_threads = 8;

void ko_set_threads(int n) { g_threads = n < 1 ? 1 : n > 256 ? 256 : n; }
int ko_get_threads(void) { return g_threads; }

typedef void (*ko_chunk_fn)(void* ctx, size_t chunk);
typedef struct { ko_chunk_fn fn; void* ctx; size_t n; atomic_size_t next; } ko_job;

static void* ko_drain(void* p)
{
    ko_job* j = (ko_job*)p;
    size_t c;
    while ((c = atomic_fetch_add_explicit(&j->next, 1, memory_order_relaxed)) < j->n) j->fn(j->ctx, c);
    return NULL;
}

static void ko_par(size_t n, ko_chunk_fn fn, void* ctx)
{
    ko_job j = { fn, ctx, n, 0 };
    int t = g_threads;
    if ((size_t)t > n) t = (int)n;
    if (t <= 1) { ko_drain(&j); return; }
    pthread_t th[256];
    int started = 0;
    for (int i = 0; i < t - 1; i++)
        if (pthread_create(&th[started], NULL, ko_drain, &j) == 0) started++;
    ko_drain(&j);
    for (int i = 0; i < started; i++) pthread_join(th[i], NULL);
}

/* ---- a16: tools/knx_quant.py:18-25 (float64 arithmetic, numpy rint = round half to even) ---- */
void ko_quantize_cols(const double* w, int k, int n, float* scale, int8_t* q)
{
    for (int c = 0; c < n; c++) {
        double m = 0.0;
        for (int i = 0; i < k; i++) { double a = fabs(w[(size_t)i * n + c]); if (a > m) m = a; }
        scale[c] = m > 0.0 ? (float)(m / 127.0) : 1.0f;
        const double s = (double)scale[c];
        for (int i = 0; i < k; i++) {
            double v = nearbyint(w[(size_t)i * n + c] / s);
            v = v > 127.0 ? 127.0 : v < -127.0 ? -127.0 : v;
            q[(size_t)i * n + c] = (int8_t)v;
        }
    }
}

/* ---- a1 input side: include/kernix_model.h:115-142 ---- */
static void ko_quant_row(const float* xr, int k, int8_t* xq, float* sx, int* bad)
{
    float m = 0.0f;
    for (int j = 0; j < k; j++) { const float a = fabsf(xr[j]); m = (a > m || a != a) ? a : m; }
    if (!(m <= FLT_MAX)) { *bad = 1; *sx = NAN; memset(xq, 0, (size_t)k); return; }
    *bad = 0;
    const float s = m > 0.0f ? m / 127.0f : 1.0f, inv = 1.0f / s;
    for (int j = 0; j < k; j++) {
        const float v = rintf(xr[j] * inv);
        xq[j] = (int8_t)(v > 127.0f ? 127.0f : v < -127.0f ? -127.0f : v);
    }
    *sx = s;
}

void ko_quantize_rows(const float* x, int rows, int k, int8_t* xq, float* sx, int* bad)
{
    for (int r = 0; r < rows; r++) ko_quant_row(x + (size_t)r * k, k, xq + (size_t)r * k, &sx[r], &bad[r]);
}

/* ---- a1: include/kernix_model.h:99-182, scalar fallback :158-177 ---- */
void ko_qmatmul(const float* x, int rows, int k, int n, const int8_t* q, const float* scale, const float* bias,
                int accumulate, float* y, int32_t* acc_out)
{
    int8_t* xq = malloc((size_t)(k > 0 ? k : 1));
    int32_t* acc = malloc(sizeof(int32_t) * (size_t)(n > 0 ? n : 1));
    for (int r = 0; r < rows; r++) {
        float* yr = y + (size_t)r * n;
        float sx;
        int bad;
        ko_quant_row(x + (size_t)r * k, k, xq, &sx, &bad);
        for (int c = 0; c < n; c++) acc[c] = 0;
        for (int t = 0; t < k; t++) {
            const int32_t a = xq[t];
            const int8_t* qr = q + (size_t)t * n;
            for (int c = 0; c < n; c++) acc[c] += a * (int32_t)qr[c];
        }
        if (acc_out) memcpy(acc_out + (size_t)r * n, acc, sizeof(int32_t) * (size_t)n);
        if (bad) { for (int c = 0; c < n; c++) yr[c] = NAN; continue; }
        for (int c = 0; c < n; c++) {
            float v = (float)acc[c] * sx;
            v = v * scale[c];
            if (bias) v = v + bias[c];
            yr[c] = accumulate ? yr[c] + v : v;
        }
    }
    free(xq);
    free(acc);
}

/* ---- activations: include/kernix_model.h:463-517 ---- */
static float ko_relu6(float v) { return v < 0.0f ? 0.0f : v > 6.0f ? 6.0f : v; }
static float ko_softplus(float v) { return v > 20.0f ? v : log1pf(expf(v)); }

static float ko_act1(float x, int act, float alpha)
{
    switch (act) {
    case 0: return x >= 0.0f ? x : 0.0f; /* vDSP_vthr(x, 0): x >= 0 ? x : 0 (NaN → 0) */
    case 1: {
        const float zz = x * 0.70710678f, t = expf(-zz * zz);
        const float z = fabsf(x) * 0.70710678f;
        const float kk = 1.0f / (1.0f + 0.3275911f * z);
        const float p = kk * (0.254829592f + kk * (-0.284496736f + kk * (1.421413741f + kk * (-1.453152027f + kk * 1.061405429f))));
        const float e = 1.0f - p * t;
        return 0.5f * x * (1.0f + (x < 0.0f ? -e : e));
    }
    case 2: { const float s = 1.0f / (1.0f + expf(-x)); return x * s; }
    case 3: return 1.0f / (1.0f + expf(-x));
    case 4: return tanhf(x);
    case 5: return x < 0.0f ? alpha * x : x;
    case 6: return x < 0.0f ? alpha * expm1f(x) : x;
    case 7: return 1.0507009873554805f * (x < 0.0f ? 1.6732632423543772f * expm1f(x) : x);
    case 8: return ko_softplus(x);
    case 9: return ko_relu6(x);
    case 10: return ko_relu6(x + 3.0f) / 6.0f;
    case 11: return x * ko_relu6(x + 3.0f) / 6.0f;
    case 12: return 0.5f * x * (1.0f + tanhf(0.7978845608028654f * (x + 0.044715f * x * x * x)));
    case 13: return expf(x);
    case 14: return x * tanhf(ko_softplus(x));
    case 15: return x / (1.0f + fabsf(x));
    default: return x;
    }
}

void ko_act(float* o, size_t n, int act, float alpha)
{
    if (act < 0) return;
    for (size_t i = 0; i < n; i++) o[i] = ko_act1(o[i], act, alpha);
}

/* ---- standalone int8 GEMM (benchmark configuration) ---- */
typedef struct {
    int M, N, K;
    const int8_t* A; const float* sa; const int8_t* W; const float* sw; const float* bias;
    int act; float alpha; float* Y; int32_t* acc;
} ko_i8_ctx;

static void ko_i8_rows(void* p, size_t ch)
{
    const ko_i8_ctx* c = (const ko_i8_ctx*)p;
    const int m = (int)ch;
    const int8_t* a = c->A + (size_t)m * c->K;
    for (int n = 0; n < c->N; n++) {
        const int8_t* w = c->W + (size_t)n * c->K;
        int32_t s = 0;
        for (int k = 0; k < c->K; k++) s += (int32_t)a[k] * (int32_t)w[k];
        if (c->acc) c->acc[(size_t)m * c->N + n] = s;
        if (c->Y) {
            float v = (float)s * c->sa[m];
            v = v * c->sw[n];
            if (c->bias) v = v + c->bias[n];
            c->Y[(size_t)m * c->N + n] = ko_act1(v, c->act, c->alpha);
        }
    }
}

void ko_i8gemm(int M, int N, int K, const int8_t* A, const float* sa, const int8_t* W, const float* sw,
               const float* bias, int act, float alpha, float* Y, int32_t* acc)
{
    ko_i8_ctx c = { M, N, K, A, sa, W, sw, bias, act, alpha, Y, acc };
    ko_par((size_t)M, ko_i8_rows, &c);
}

/* ---- native float GEMM, include/kernix.h:108-124 (i-k-j, float accumulation) + bias_act ---- */
typedef struct {
    int M, N, K; const float* A; const float* W; const float* bias; int act; float alpha; float* C; int f64; int per;
} ko_mm_ctx;

static void ko_mm_rows(void* p, size_t ch)
{
    const ko_mm_ctx* c = (const ko_mm_ctx*)p;
    const int r0 = (int)ch * c->per, r1 = r0 + c->per < c->M ? r0 + c->per : c->M;
    double* d = c->f64 ? malloc(sizeof(double) * (size_t)c->N) : NULL;
    for (int i = r0; i < r1; i++) {
        float* cr = c->C + (size_t)i * c->N;
        if (c->f64) {
            for (int j = 0; j < c->N; j++) d[j] = 0.0;
            for (int k = 0; k < c->K; k++) {
                const double a = c->A[(size_t)i * c->K + k];
                const float* wr = c->W + (size_t)k * c->N;
                for (int j = 0; j < c->N; j++) d[j] += a * (double)wr[j];
            }
            for (int j = 0; j < c->N; j++) cr[j] = (float)d[j];
        } else {
            for (int j = 0; j < c->N; j++) cr[j] = 0.0f;
            for (int k = 0; k < c->K; k++) {
                const float a = c->A[(size_t)i * c->K + k];
                const float* wr = c->W + (size_t)k * c->N;
                for (int j = 0; j < c->N; j++) cr[j] += a * wr[j];
            }
        }
        if (c->bias) for (int j = 0; j < c->N; j++) cr[j] = cr[j] + c->bias[j];
        ko_act(cr, (size_t)c->N, c->act, c->alpha);
    }
    free(d);
}

static void ko_mm(int M, int N, int K, const float* A, const float* W, const float* bias, int act, float alpha, float* C, int f64)
{
    if (M <= 0 || N <= 0) return;
    ko_mm_ctx c = { M, N, K, A, W, bias, act, alpha, C, f64, 0 };
    c.per = M >= 64 ? (M + 63) / 64 : 1; /* ~64 row pieces, include/kernix.h:95-104 */
    ko_par((size_t)((M + c.per - 1) / c.per), ko_mm_rows, &c);
}

void ko_dense(int M, int N, int K, const float* A, const float* W, const float* bias, int act, float alpha, float* C)
{
    ko_mm(M, N, K, A, W, bias, act, alpha, C, 0);
}

void ko_dense_f64(int M, int N, int K, const float* A, const float* W, const float* bias, int act, float alpha, float* C)
{
    ko_mm(M, N, K, A, W, bias, act, alpha, C, 1);
}

/* ---- rows: include/kernix.h:652-677 ---- */
void ko_layernorm(const float* x, float* y, int rows, int cols, const float* gamma, const float* beta, float eps)
{
    for (int r = 0; r < rows; r++) {
        const float* xr = x + (size_t)r * cols;
        float* o = y + (size_t)r * cols;
        float s = 0.0f;
        for (int c = 0; c < cols; c++) s += xr[c];
        const float mean = s / (float)cols;
        float ss = 0.0f;
        for (int c = 0; c < cols; c++) { const float d = xr[c] - mean; o[c] = d; ss += d * d; }
        const float rstd = 1.0f / sqrtf(ss / (float)cols + eps);
        for (int c = 0; c < cols; c++) {
            float v = o[c] * rstd;
            if (gamma && beta) v = v * gamma[c] + beta[c];
            else if (gamma) v = v * gamma[c];
            else if (beta) v = v + beta[c];
            o[c] = v;
        }
    }
}

void ko_softmax(const float* x, float* y, int rows, int cols)
{
    for (int r = 0; r < rows; r++) {
        const float* xr = x + (size_t)r * cols;
        float* o = y + (size_t)r * cols;
        float m = -INFINITY;
        for (int c = 0; c < cols; c++) m = xr[c] > m ? xr[c] : m;
        float s = 0.0f;
        for (int c = 0; c < cols; c++) { o[c] = expf(xr[c] - m); s += o[c]; }
        const float inv = 1.0f / s;
        for (int c = 0; c < cols; c++) o[c] = o[c] * inv;
    }
}

/* ---- convolution: im2col rows (ky,kx,ci) per group, then the native GEMM, include/kernix_model.h:677-693, :754-768 ---- */
void ko_conv(int B, int H, int W, int C, int Ho, int Wo, int Co, int kh, int kw, int sh, int sw, int dh, int dw,
             int pt, int pl, int groups, const float* x, const float* w, const float* bias, int act, float alpha, float* y)
{
    const int cg = C / groups, cog = Co / groups, K = kh * kw * cg;
    const size_t rows = (size_t)B * Ho * Wo;
    const size_t tile = 4096;
    float* col = malloc(sizeof(float) * tile * (size_t)K);
    float* part = malloc(sizeof(float) * tile * (size_t)cog);
    float* wg = malloc(sizeof(float) * (size_t)K * cog);
    for (int g = 0; g < groups; g++) {
        for (int k = 0; k < K; k++)
            for (int j = 0; j < cog; j++) wg[(size_t)k * cog + j] = w[(size_t)k * Co + g * cog + j];
        for (size_t r0 = 0; r0 < rows; r0 += tile) {
            const size_t r1 = r0 + tile < rows ? r0 + tile : rows;
            for (size_t r = r0; r < r1; r++) {
                const size_t b = r / ((size_t)Ho * Wo), oy = (r / Wo) % Ho, ox = r % Wo;
                float* o = col + (r - r0) * K;
                for (int ky = 0; ky < kh; ky++) {
                    const long iy = (long)oy * sh - pt + (long)ky * dh;
                    for (int kx = 0; kx < kw; kx++, o += cg) {
                        const long ix = (long)ox * sw - pl + (long)kx * dw;
                        if (iy < 0 || iy >= H || ix < 0 || ix >= W) memset(o, 0, sizeof(float) * cg);
                        else memcpy(o, x + (((size_t)b * H + iy) * W + ix) * C + (size_t)g * cg, sizeof(float) * cg);
                    }
                }
            }
            ko_dense((int)(r1 - r0), cog, K, col, wg, NULL, -1, 0.0f, part);
            for (size_t r = r0; r < r1; r++)
                memcpy(y + r * Co + (size_t)g * cog, part + (r - r0) * cog, sizeof(float) * cog);
        }
    }
    for (size_t r = 0; r < rows; r++) {
        float* o = y + r * Co;
        if (bias) for (int j = 0; j < Co; j++) o[j] = o[j] + bias[j];
        ko_act(o, (size_t)Co, act, alpha);
    }
    free(col);
    free(part);
    free(wg);
}

/* ---- attention core: include/kernix_model.h:1021-1046 ---- */
void ko_attention_core(const float* Q, const float* K, const float* V, float* ctx, int B, int H, int Rq, int S, int dk,
                       int dv, float scale, int causal)
{
    float* p = malloc(sizeof(float) * (size_t)S);
    for (int b = 0; b < B; b++)
        for (int h = 0; h < H; h++)
            for (int i = 0; i < Rq; i++) {
                const float* q = Q + ((size_t)b * Rq + i) * H * dk + (size_t)h * dk;
                for (int j = 0; j < S; j++) {
                    const float* kr = K + ((size_t)b * S + j) * H * dk + (size_t)h * dk;
                    float s = 0.0f;
                    for (int t = 0; t < dk; t++) s += q[t] * kr[t];
                    p[j] = scale * s;
                    if (causal && j > i) p[j] = -INFINITY;
                }
                ko_softmax(p, p, 1, S);
                float* o = ctx + ((size_t)b * Rq + i) * H * dv + (size_t)h * dv;
                for (int t = 0; t < dv; t++) o[t] = 0.0f;
                for (int j = 0; j < S; j++) {
                    const float* vr = V + ((size_t)b * S + j) * H * dv + (size_t)h * dv;
                    for (int t = 0; t < dv; t++) o[t] += p[j] * vr[t];
                }
            }
    free(p);
}

/* ---- binary / global pool: include/kernix_model.h:864-906, :810-830 ---- */
static float ko_bin1(int op, float a, float b)
{
    switch (op) {
    case 0: return a + b;
    case 1: return a - b;
    case 2: return a * b;
    case 3: return a / b;
    case 4: return a > b ? a : b;
    default: return a < b ? a : b;
    }
}

void ko_binary(int op, const float* a, int ra, int ca, const float* b, int rb, int cb, float* y, int B, int R, int C)
{
    for (size_t i = 0; i < (size_t)B * R; i++) {
        const size_t bi = i / R, ri = i % R;
        const float* ar = a + (bi * ra + (ra == 1 ? 0 : ri)) * ca;
        const float* br = b + (bi * rb + (rb == 1 ? 0 : ri)) * cb;
        for (int j = 0; j < C; j++) y[i * C + j] = ko_bin1(op, ar[ca == 1 ? 0 : j], br[cb == 1 ? 0 : j]);
    }
}

void ko_global_pool(int type, const float* x, int B, int R, int C, float* y)
{
    for (int b = 0; b < B; b++) {
        float* o = y + (size_t)b * C;
        memcpy(o, x + (size_t)b * R * C, sizeof(float) * C);
        for (int i = 1; i < R; i++) {
            const float* xp = x + ((size_t)b * R + i) * C;
            for (int j = 0; j < C; j++) o[j] = type == 0 ? (o[j] > xp[j] ? o[j] : xp[j]) : o[j] + xp[j];
        }
        if (type == 1) {
            const float inv = 1.0f / (float)R;
            for (int j = 0; j < C; j++) o[j] = o[j] * inv;
        }
    }
}
