/* knx_decode.c — turns the bytes of a .knx file into op records (kernix_step with host weights), nothing more.
 *
 * The file is untrusted.  It is mapped read-only and consumed through a cursor whose every read is bounded by the
 * end of the mapping; the first failure is kept (later reads return zeros) and the decoder checks it at the points
 * where a bad value could otherwise steer an allocation.  Each op kind is described by a row of a schema table —
 * how many KNX3 inputs it takes and the allowed range of each u32 field of its record — and a small function for
 * what follows the fixed fields (floats, weight blocks, cross-field rules).  Sizes are always checked against the
 * bytes left before anything is allocated, so a forged size cannot make the loader allocate.
 *
 * The accepted files are the reference's (format: reference docs/mlp-runtime-design.md §4, docs/int8-quantization-
 * design.md §4, docs/graph-runtime-design.md §3; loader behaviour: include/kernix_model.h:387-460 for weight blocks,
 * :1082-1243 for op records).  Shapes, activation folding and storage planning are in knx_graph.c.
 */
#include <fcntl.h>
#include <float.h>
#include <limits.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "knx_internal.h"

/* ---------------------------------------------------------------- host tensors (reference include/kernix.h:146-227) */
float_tensor* kernix_float_new(int rows, int cols, int zero)
{
    if (rows < 0 || cols < 0) return NULL;
    const size_t count = (size_t)rows * (size_t)cols;
    size_t bytes = (count * sizeof(float) + 63) & ~(size_t)63; /* whole 64-byte lines, at least one */
    if (bytes == 0) bytes = 64;
    float_tensor* t = malloc(sizeof *t);
    void* mem = NULL;
    if (t == NULL || posix_memalign(&mem, 64, bytes) != 0) {
        free(t);
        return NULL;
    }
    if (zero) memset(mem, 0, count * sizeof(float));
    *t = (float_tensor){ rows, cols, mem };
    return t;
}

float_tensor* float_zeros(int rows, int cols) { return kernix_float_new(rows, cols, 1); }

void float_free(float_tensor* t)
{
    if (t != NULL) free(t->tensor);
    free(t);
}

/* ---------------------------------------------------------------- int8 weights (reference include/kernix_model.h:52-95)
 * The file holds q as k×n (input-major); this build keeps it as np×kp, one output channel per row with its k values
 * contiguous and zero padded — the operand layout of the int8 MFMA GEMM — plus np scales (0 past n). */
kernix_qweight* kernix_qweight_pack(const int8_t* q, const float* scale, int k, int n)
{
    if (q == NULL || scale == NULL || k < 1 || n < 1 || k > KERNIX_INT8_MAX_K || n > INT_MAX - 16) return NULL;
    kernix_qweight* w = calloc(1, sizeof *w);
    if (w == NULL) return NULL;
    w->k = k;
    w->n = n;
    w->kp = (k + 63) & ~63;
    w->np = (n + 15) & ~15;
    w->q = calloc((size_t)w->np * (size_t)w->kp, 1);
    w->scale = calloc((size_t)w->np, sizeof(float));
    if (w->q == NULL || w->scale == NULL) {
        kernix_qweight_free(w);
        return NULL;
    }
    memcpy(w->scale, scale, (size_t)n * sizeof(float));
    for (int c = 0; c < n; c++) {
        int8_t* row = w->q + (size_t)c * (size_t)w->kp;
        const int8_t* src = q + c;
        for (int r = 0; r < k; r++, src += n) row[r] = *src;
    }
    return w;
}

void kernix_qweight_unpack(const kernix_qweight* w, float* dst)
{
    for (int c = 0; c < w->n; c++) {
        const int8_t* row = w->q + (size_t)c * (size_t)w->kp;
        const float s = w->scale[c];
        for (int r = 0; r < w->k; r++) dst[(size_t)r * (size_t)w->n + c] = (float)row[r] * s;
    }
}

void kernix_qweight_free(kernix_qweight* w)
{
    if (w == NULL) return;
    free(w->q);
    free(w->scale);
    free(w);
}

/* ---------------------------------------------------------------- cursor */
typedef struct {
    const unsigned char* at;
    const unsigned char* end;
    const char* why; /* first failure, NULL while every read succeeded */
} cursor;

static const char* const SHORT = "file shorter than declared";

static void fail(cursor* c, const char* why)
{
    if (c->why == NULL) c->why = why;
}

static size_t left(const cursor* c) { return c->why ? 0 : (size_t)(c->end - c->at); }

/* n bytes at the cursor (advanced past them), or NULL (and the cursor failed) if the file ends first */
static const unsigned char* take(cursor* c, size_t n)
{
    if (c->why != NULL) return NULL;
    if (n > (size_t)(c->end - c->at)) {
        fail(c, SHORT);
        return NULL;
    }
    const unsigned char* p = c->at;
    c->at += n;
    return p;
}

static uint32_t get_u32(cursor* c)
{
    const unsigned char* p = take(c, 4);
    return p ? (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24 : 0;
}

static float get_f32(cursor* c)
{
    const uint32_t u = get_u32(c);
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* n little-endian floats into dst (the mapping may be unaligned) */
static int get_floats(cursor* c, float* dst, size_t n)
{
    if (n > left(c) / 4) {
        fail(c, SHORT);
        return -1;
    }
    const unsigned char* p = take(c, 4 * n);
    if (p == NULL) return -1;
    memcpy(dst, p, 4 * n);
    return 0;
}

/* a new array of n floats read from the file; NULL (nothing allocated) when the file does not hold them */
static float* new_floats(cursor* c, size_t n)
{
    if (n > left(c) / 4) {
        fail(c, SHORT);
        return NULL;
    }
    float* p = malloc(n ? 4 * n : 4);
    if (p == NULL) fail(c, "out of memory");
    else if (get_floats(c, p, n) != 0) { free(p); p = NULL; }
    return p;
}

/* ---------------------------------------------------------------- weight blocks
 * A k×n weight: KNX1 bare floats; KNX2/3 a u32 dtype then F32 f32[k·n] | I8_COL f32 scale[n] i8[k·n] |
 * I8_ROW f32 scale[k] i8[k·n].  Scales must be finite and positive.  Where the op keeps int8 weights (`to_q` given)
 * an I8_COL block becomes a packed kernix_qweight (k ≤ KERNIX_INT8_MAX_K); every other block becomes fp32,
 * w = q·scale exactly, into a new host tensor (`to_t`) or a plain array (`to_a`). */
static int read_block(cursor* c, int ver, uint64_t k, uint64_t n, float_tensor** to_t, float** to_a,
                      kernix_qweight** to_q)
{
    if (k < 1 || n < 1 || k > INT_MAX || n > INT_MAX || k * n > INT_MAX) {
        fail(c, "weight size out of range");
        return -1;
    }
    const uint32_t dt = ver >= 2 ? get_u32(c) : KERNIX_DT_F32;
    if (c->why) return -1;
    if (dt > KERNIX_DT_I8_ROW) {
        fail(c, "unknown weight dtype");
        return -1;
    }
    const size_t count = (size_t)(k * n);
    const size_t nscale = dt == KERNIX_DT_I8_COL ? (size_t)n : dt == KERNIX_DT_I8_ROW ? (size_t)k : 0;
    const size_t body = dt == KERNIX_DT_F32 ? 4 * count : 4 * nscale + count;
    if (body > left(c)) { /* before any allocation */
        fail(c, SHORT);
        return -1;
    }
    const int keep_q = to_q != NULL && dt == KERNIX_DT_I8_COL;
    if (keep_q && k > KERNIX_INT8_MAX_K) {
        fail(c, "int8 weight input size out of range");
        return -1;
    }
    float* scales = NULL;
    if (nscale) {
        if ((scales = malloc(4 * nscale)) == NULL) {
            fail(c, "out of memory");
            return -1;
        }
        get_floats(c, scales, nscale);
        for (size_t i = 0; c->why == NULL && i < nscale; i++)
            if (!(scales[i] > 0.0f && scales[i] <= FLT_MAX)) fail(c, "int8 scale not finite and positive");
    }
    const unsigned char* raw = take(c, dt == KERNIX_DT_F32 ? 4 * count : count);
    if (raw == NULL) {
        free(scales);
        return -1;
    }
    if (keep_q) {
        *to_q = kernix_qweight_pack((const int8_t*)raw, scales, (int)k, (int)n);
        free(scales);
        if (*to_q == NULL) fail(c, "out of memory");
        return *to_q ? 0 : -1;
    }
    float* dst;
    if (to_t != NULL) {
        *to_t = kernix_float_new((int)k, (int)n, 0);
        dst = *to_t ? (*to_t)->tensor : NULL;
    } else {
        dst = *to_a = malloc(4 * count);
    }
    if (dst == NULL) {
        free(scales);
        fail(c, "out of memory");
        return -1;
    }
    if (dt == KERNIX_DT_F32) {
        memcpy(dst, raw, 4 * count);
    } else {
        const int8_t* q = (const int8_t*)raw;
        for (size_t r = 0; r < (size_t)k; r++)
            for (size_t j = 0; j < (size_t)n; j++) {
                const size_t at = r * (size_t)n + j;
                dst[at] = (float)q[at] * scales[dt == KERNIX_DT_I8_COL ? j : r];
            }
    }
    free(scales);
    return 0;
}

/* ---------------------------------------------------------------- op schema */
#define IMAX ((uint32_t)INT_MAX)
#define GMAX ((uint32_t)KERNIX_MAX_GEOM)
#define UMAX UINT32_MAX

typedef struct {
    uint32_t lo, hi;
} span;

typedef int (*tail_fn)(cursor* c, int ver, const uint32_t* a, kernix_step* s);

typedef struct {
    const char* name;
    unsigned char in_lo, in_hi; /* KNX3 input count */
    unsigned char nf;           /* fixed u32 fields */
    span f[14];
    tail_fn tail;               /* what follows the fixed fields */
} opdef;

static uint64_t gate_count(int kind) { return kind == KERNIX_OP_LSTM ? 4 : kind == KERNIX_OP_GRU ? 3 : 1; }

static int t_linear(cursor* c, int ver, const uint32_t* a, kernix_step* s)
{
    s->in = (int)a[0];
    s->out = (int)a[1];
    if (read_block(c, ver, a[0], a[1], &s->w, NULL, &s->q) != 0) return -1;
    if (a[2]) s->bias = new_floats(c, a[1]);
    return c->why ? -1 : 0;
}

static int t_act(cursor* c, int ver, const uint32_t* a, kernix_step* s)
{
    if (ver >= 3) s->alpha = get_f32(c);
    if (c->why) return -1;
    if (!isfinite(s->alpha)) {
        fail(c, "activation parameter not finite");
        return -1;
    }
    s->act = (int)a[0];
    return 0;
}

static int t_layernorm(cursor* c, int ver, const uint32_t* a, kernix_step* s)
{
    (void)ver;
    s->eps = get_f32(c);
    if (c->why) return -1;
    if (!(s->eps >= 0.0f && s->eps <= FLT_MAX)) {
        fail(c, "LayerNorm epsilon not finite and non-negative");
        return -1;
    }
    s->in = s->out = (int)a[0];
    if (a[1]) {
        s->gamma = new_floats(c, a[0]);
        s->beta = new_floats(c, a[0]);
    }
    return c->why ? -1 : 0;
}

static int t_none(cursor* c, int ver, const uint32_t* a, kernix_step* s)
{
    (void)ver; (void)a; (void)s;
    return c->why ? -1 : 0;
}

/* recurrent layer: per direction W (in × G·u, fp32), U (u × G·u, int8 kept), bias (G·u, GRU 2·G·u) */
static int rnn_weights(cursor* c, int ver, kernix_step* s)
{
    const uint64_t gu = gate_count(s->kind) * (uint64_t)s->out;
    const uint64_t nb = s->kind == KERNIX_OP_GRU ? 2 * gu : gu;
    for (int d = 0; d < s->dirs; d++) {
        if (read_block(c, ver, (uint64_t)s->in, gu, d ? &s->w_b : &s->w, NULL, NULL) != 0 ||
            read_block(c, ver, (uint64_t)s->out, gu, NULL, d ? &s->rec_b : &s->rec, d ? &s->q_b : &s->q) != 0)
            return -1;
        float** b = d ? &s->bias_b : &s->bias;
        if ((*b = new_floats(c, nb)) == NULL) return -1;
    }
    return 0;
}

/* KNX3 recurrent record: in units act ret_seq dirs merge */
static int t_rnn(cursor* c, int ver, const uint32_t* a, kernix_step* s)
{
    s->in = (int)a[0];
    s->out = (int)a[1];
    s->act = (int)a[2];
    s->ret_seq = (int)a[3];
    s->dirs = (int)a[4];
    s->merge = (int)a[5];
    return rnn_weights(c, ver, s);
}

/* KNX1/2 LSTM record: in units act ret_seq seq (one direction; ReLU or tanh) */
static int t_lstm_v12(cursor* c, int ver, const uint32_t* a, kernix_step* s)
{
    if (a[2] != KERNIX_ACT_RELU && a[2] != KERNIX_ACT_TANH) {
        fail(c, "LSTM activation must be ReLU or tanh");
        return -1;
    }
    s->in = (int)a[0];
    s->out = (int)a[1];
    s->act = (int)a[2];
    s->ret_seq = (int)a[3];
    s->seq = (int)a[4];
    s->dirs = 1;
    s->merge = KERNIX_MERGE_CONCAT;
    return rnn_weights(c, ver, s);
}

static int t_conv(cursor* c, int ver, const uint32_t* a, kernix_step* s)
{
    if (a[0] % a[12] != 0 || a[1] % a[12] != 0) {
        fail(c, "convolution channels not divisible by the groups");
        return -1;
    }
    int* dst[12] = { &s->in, &s->out, &s->kh, &s->kw, &s->sh, &s->sw, &s->dh, &s->dw, &s->pt, &s->pb, &s->pl, &s->pr };
    for (int i = 0; i < 12; i++) *dst[i] = (int)a[i];
    s->groups = (int)a[12];
    const uint64_t rows = (uint64_t)a[2] * a[3] * (a[0] / a[12]);
    if (read_block(c, ver, rows, a[1], &s->w, NULL, NULL) != 0) return -1;
    if (a[13]) s->bias = new_floats(c, a[1]);
    return c->why ? -1 : 0;
}

static int t_pool(cursor* c, int ver, const uint32_t* a, kernix_step* s)
{
    (void)ver;
    if (a[5] >= a[1] || a[6] >= a[1] || a[7] >= a[2] || a[8] >= a[2]) { /* an all-padding window */
        fail(c, "pooling padding not smaller than the window");
        return -1;
    }
    s->ptype = (int)a[0];
    int* dst[8] = { &s->kh, &s->kw, &s->sh, &s->sw, &s->pt, &s->pb, &s->pl, &s->pr };
    for (int i = 0; i < 8; i++) *dst[i] = (int)a[1 + i];
    s->count_pad = (int)a[9];
    return c->why ? -1 : 0;
}

static int t_global_pool(cursor* c, int ver, const uint32_t* a, kernix_step* s)
{
    (void)ver;
    s->ptype = (int)a[0];
    return c->why ? -1 : 0;
}

/* RESHAPE / PERMUTE: nd, then nd values (a shape of positive sizes / a permutation of 0..nd-1) */
static int t_axes(cursor* c, int ver, const uint32_t* a, kernix_step* s)
{
    (void)ver;
    s->nd = (int)a[0];
    unsigned used = 0;
    for (int k = 0; k < s->nd; k++) {
        const uint32_t v = get_u32(c);
        if (c->why) return -1;
        if (s->kind == KERNIX_OP_RESHAPE) {
            if (v < 1 || v > IMAX) { fail(c, "Reshape size out of range"); return -1; }
            s->d[k] = (int)v;
        } else {
            if (v >= (uint32_t)s->nd || (used & (1u << v))) { fail(c, "Permute order is not a permutation"); return -1; }
            used |= 1u << v;
            s->perm[k] = (int)v;
        }
    }
    return 0;
}

static int t_binary(cursor* c, int ver, const uint32_t* a, kernix_step* s) { (void)ver; s->bop = (int)a[0]; return c->why ? -1 : 0; }
static int t_concat(cursor* c, int ver, const uint32_t* a, kernix_step* s) { (void)ver; s->axis = (int)a[0]; return c->why ? -1 : 0; }

static int t_embedding(cursor* c, int ver, const uint32_t* a, kernix_step* s)
{
    if (read_block(c, ver, a[0], a[1], &s->w, NULL, NULL) != 0) return -1; /* checks the sizes */
    s->in = (int)a[0];
    s->out = (int)a[1];
    return 0;
}

static int t_affine(cursor* c, int ver, const uint32_t* a, kernix_step* s)
{
    (void)ver;
    s->in = s->out = (int)a[0];
    s->gamma = new_floats(c, a[0]);
    s->beta = new_floats(c, a[0]);
    return c->why ? -1 : 0;
}

static int t_add_const(cursor* c, int ver, const uint32_t* a, kernix_step* s)
{
    (void)ver;
    s->in = (int)a[0];
    s->cst = new_floats(c, a[0]);
    return c->why ? -1 : 0;
}

/* heads dk dv causal cq cv ck cout has_bias, then Wq [bq] Wk [bk] Wv [bv] Wo [bo] (all fp32 on the host) */
static int t_attention(cursor* c, int ver, const uint32_t* a, kernix_step* s)
{
    s->heads = (int)a[0];
    s->dk = (int)a[1];
    s->dv = (int)a[2];
    s->causal = (int)a[3];
    s->in = (int)a[4];
    s->out = (int)a[7];
    const uint64_t hk = (uint64_t)a[0] * a[1], hv = (uint64_t)a[0] * a[2];
    struct { uint64_t rows, cols; float_tensor** w; float** b; } part[4] = {
        { a[4], hk, &s->w, &s->bias }, { a[6], hk, &s->wk, &s->bk }, { a[5], hv, &s->wv, &s->bv }, { hv, a[7], &s->wo, &s->bo },
    };
    for (int i = 0; i < 4; i++) {
        if (read_block(c, ver, part[i].rows, part[i].cols, part[i].w, NULL, NULL) != 0) return -1;
        if (a[8] && (*part[i].b = new_floats(c, part[i].cols)) == NULL) return -1;
    }
    return 0;
}

static int t_select(cursor* c, int ver, const uint32_t* a, kernix_step* s)
{
    (void)ver;
    s->axis = (int)a[0];
    s->start = (int)a[1];
    s->len = (int)a[2];
    s->squeeze = (int)a[3];
    return c->why ? -1 : 0;
}

static int t_pad(cursor* c, int ver, const uint32_t* a, kernix_step* s)
{
    (void)ver;
    s->pt = (int)a[0]; s->pb = (int)a[1]; s->pl = (int)a[2]; s->pr = (int)a[3];
    return c->why ? -1 : 0;
}

static int t_upsample(cursor* c, int ver, const uint32_t* a, kernix_step* s)
{
    (void)ver;
    s->sh = (int)a[0];
    s->sw = (int)a[1];
    return c->why ? -1 : 0;
}

#define POS { 1, IMAX }
#define FLAG { 0, 1 }
#define G1 { 1, GMAX }
#define G0 { 0, GMAX }
#define ANY { 0, UMAX }

/* KNX3 records, indexed by op id */
static const opdef OPS[KERNIX_OP_LAST + 1] = {
    [KERNIX_OP_LINEAR] = { "Linear", 1, 1, 3, { POS, POS, FLAG }, t_linear },
    [KERNIX_OP_ACT] = { "activation", 1, 1, 1, { { 0, KERNIX_ACT_LAST } }, t_act },
    [KERNIX_OP_LAYERNORM] = { "LayerNorm", 1, 1, 2, { POS, FLAG }, t_layernorm },
    [KERNIX_OP_SOFTMAX] = { "Softmax", 1, 1, 0, { { 0, 0 } }, t_none },
    [KERNIX_OP_LSTM] = { "LSTM", 1, 1, 6, { POS, { 1, KERNIX_CHUNK / 2 }, { 0, KERNIX_ACT_LAST }, FLAG, { 1, 2 }, { 0, KERNIX_MERGE_AVE } }, t_rnn },
    [KERNIX_OP_GRU] = { "GRU", 1, 1, 6, { POS, { 1, KERNIX_CHUNK / 2 }, { 0, KERNIX_ACT_LAST }, FLAG, { 1, 2 }, { 0, KERNIX_MERGE_AVE } }, t_rnn },
    [KERNIX_OP_RNN] = { "RNN", 1, 1, 6, { POS, { 1, KERNIX_CHUNK / 2 }, { 0, KERNIX_ACT_LAST }, FLAG, { 1, 2 }, { 0, KERNIX_MERGE_AVE } }, t_rnn },
    [KERNIX_OP_CONV] = { "convolution", 1, 1, 14, { POS, POS, G1, G1, G1, G1, G1, G1, G0, G0, G0, G0, { 1, UMAX }, FLAG }, t_conv },
    [KERNIX_OP_POOL] = { "pooling", 1, 1, 10, { { 0, KERNIX_POOL_AVG }, G1, G1, G1, G1, ANY, ANY, ANY, ANY, FLAG }, t_pool },
    [KERNIX_OP_GLOBAL_POOL] = { "global pooling", 1, 1, 1, { { 0, KERNIX_POOL_AVG } }, t_global_pool },
    [KERNIX_OP_RESHAPE] = { "Reshape", 1, 1, 1, { { 1, KERNIX_MAX_DIMS } }, t_axes },
    [KERNIX_OP_PERMUTE] = { "Permute", 1, 1, 1, { { 1, KERNIX_MAX_DIMS } }, t_axes },
    [KERNIX_OP_BINARY] = { "binary op", 2, 2, 1, { { 0, KERNIX_BIN_MIN } }, t_binary },
    [KERNIX_OP_CONCAT] = { "Concatenate", 2, KERNIX_MAX_INPUTS, 1, { { 0, KERNIX_AXIS_LAST } }, t_concat },
    [KERNIX_OP_EMBEDDING] = { "Embedding", 1, 1, 2, { ANY, ANY }, t_embedding },
    [KERNIX_OP_AFFINE] = { "Affine", 1, 1, 1, { POS }, t_affine },
    [KERNIX_OP_ADD_CONST] = { "constant add", 1, 1, 1, { POS }, t_add_const },
    [KERNIX_OP_ATTENTION] = { "attention", 1, 3, 9, { { 1, 4096 }, { 1, 65536 }, { 1, 65536 }, FLAG, POS, POS, POS, POS, FLAG }, t_attention },
    [KERNIX_OP_SELECT] = { "Select", 1, 1, 4, { { 0, KERNIX_AXIS_LAST }, { 0, IMAX }, POS, FLAG }, t_select },
    [KERNIX_OP_PAD] = { "padding", 1, 1, 4, { G0, G0, G0, G0 }, t_pad },
    [KERNIX_OP_UPSAMPLE] = { "UpSampling", 1, 1, 2, { G1, G1 }, t_upsample },
};

/* KNX1/KNX2 records (sequential files: LINEAR, ACT with ids up to tanh, LAYERNORM, SOFTMAX, LSTM) */
static const opdef OPS_V12[KERNIX_OP_LSTM + 1] = {
    [KERNIX_OP_LINEAR] = { "Linear", 1, 1, 3, { POS, POS, FLAG }, t_linear },
    [KERNIX_OP_ACT] = { "activation", 1, 1, 1, { { 0, KERNIX_ACT_TANH } }, t_act },
    [KERNIX_OP_LAYERNORM] = { "LayerNorm", 1, 1, 2, { POS, FLAG }, t_layernorm },
    [KERNIX_OP_SOFTMAX] = { "Softmax", 1, 1, 0, { { 0, 0 } }, t_none },
    [KERNIX_OP_LSTM] = { "LSTM", 1, 1, 5, { POS, { 1, KERNIX_CHUNK / 2 }, { 0, KERNIX_ACT_TANH }, FLAG, POS }, t_lstm_v12 },
};

/* one op record at the cursor into s (s->kind already set); index i is the op's position (KNX3 input ids ≤ i) */
static int decode_op(cursor* c, int ver, int i, kernix_step* s)
{
    const opdef* d = ver >= 3 ? &OPS[s->kind] : &OPS_V12[s->kind];
    s->act = KERNIX_ACT_NONE;
    s->dirs = 1;
    s->groups = 1;
    s->kh = s->kw = s->sh = s->sw = s->dh = s->dw = 1;
    if (ver >= 3) {
        const uint32_t n_in = get_u32(c);
        if (c->why) return -1;
        if (n_in < d->in_lo || n_in > d->in_hi) {
            fail(c, "op input count out of range");
            return -1;
        }
        s->n_in = (int)n_in;
        for (uint32_t k = 0; k < n_in; k++) {
            const uint32_t id = get_u32(c);
            if (c->why) return -1;
            if (id > (uint32_t)i) {
                fail(c, "op input refers to a later op");
                return -1;
            }
            s->inp[k] = (int)id;
        }
    } else {
        s->n_in = 1;
        s->inp[0] = i; /* the previous op's output (0 = the model input) */
    }
    uint32_t a[14] = { 0 };
    for (int k = 0; k < d->nf; k++) {
        a[k] = get_u32(c);
        if (c->why) return -1;
        if (a[k] < d->f[k].lo || a[k] > d->f[k].hi) {
            static _Thread_local char msg[96];
            snprintf(msg, sizeof msg, "%s field %d out of range", d->name, k);
            fail(c, msg);
            return -1;
        }
    }
    return d->tail(c, ver, a, s);
}

/* ---------------------------------------------------------------- file */
void knx_file_release(knx_file* f)
{
    if (f == NULL) return;
    for (int i = 0; f->ops != NULL && i < f->n_ops; i++) knx_step_host_free(&f->ops[i]);
    free(f->ops);
    memset(f, 0, sizeof *f);
}

int knx_decode(const char* path, knx_file* f, const char** why)
{
    memset(f, 0, sizeof *f);
    *why = "cannot open the file";
    const int fd = path ? open(path, O_RDONLY | O_CLOEXEC) : -1;
    if (fd < 0) return -1;
    struct stat st;
    if (fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        close(fd);
        return -1;
    }
    const size_t size = (size_t)st.st_size;
    void* map = size ? mmap(NULL, size, PROT_READ, MAP_PRIVATE, fd, 0) : NULL;
    close(fd);
    if (size && map == MAP_FAILED) {
        *why = "cannot map the file";
        return -1;
    }
    cursor c = { map, (const unsigned char*)map + size, NULL };

    const unsigned char* magic = take(&c, 4);
    const uint32_t n_ops = get_u32(&c);
    if (c.why == NULL) {
        f->version = memcmp(magic, "KNX1", 4) == 0 ? 1 : memcmp(magic, "KNX2", 4) == 0 ? 2 : memcmp(magic, "KNX3", 4) == 0 ? 3 : 0;
        if (f->version == 0) fail(&c, "not a KNX1/KNX2/KNX3 file");
        else if (n_ops < 1 || n_ops > KERNIX_MODEL_MAX_OPS) fail(&c, "op count out of range");
    }
    if (c.why == NULL && f->version == 3) { /* layout, input rank, per-sample input shape */
        const uint32_t layout = get_u32(&c), nd = get_u32(&c);
        if (c.why == NULL && (layout > 1 || nd < 1 || nd > KERNIX_MAX_DIMS)) fail(&c, "input shape out of range");
        for (uint32_t k = 0; c.why == NULL && k < nd; k++) {
            const uint32_t v = get_u32(&c);
            f->in_d[k] = v > IMAX ? 0 : (int)v; /* 0 is rejected with the shape */
        }
        f->layout = (int)layout;
        f->in_nd = (int)nd;
    }
    if (c.why == NULL && (f->ops = calloc(n_ops, sizeof(kernix_step))) == NULL) fail(&c, "out of memory");
    for (uint32_t i = 0; c.why == NULL && i < n_ops; i++) {
        kernix_step* s = &f->ops[i];
        const uint32_t kind = get_u32(&c);
        if (c.why) break;
        if (kind > (uint32_t)(f->version == 3 ? KERNIX_OP_LAST : KERNIX_OP_LSTM)) {
            fail(&c, "unknown op");
            break;
        }
        s->kind = (int)kind;
        f->n_ops = (int)i + 1; /* release() frees what this op allocated, even if it fails half way */
        decode_op(&c, f->version, (int)i, s);
    }
    if (c.why == NULL && c.at != c.end) fail(&c, "trailing data after the last op");
    if (map != NULL) munmap(map, size);
    if (c.why != NULL) {
        *why = c.why;
        knx_file_release(f);
        return -1;
    }
    *why = NULL;
    return 0;
}
