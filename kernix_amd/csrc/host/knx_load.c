/* knx_load.c — .knx loader of the KERNIX MI355X runtime: parse (KNX1/KNX2/KNX3), validate, infer shapes, fuse
 * activations, plan storage buffers.  Pure host code: nothing here touches the device (weights are uploaded by the
 * first forward), so a model can be loaded and inspected without a GPU.
 *
 * The file is untrusted input.  Every read is checked against the bytes left; sizes are checked before anything is
 * allocated; the same files are rejected as by the reference loader (reference include/kernix_model.h:387-460,
 * :1050-1601, format docs/mlp-runtime-design.md §4, docs/int8-quantization-design.md §4, docs/graph-runtime-design.md §3).
 */
#include <float.h>
#include <limits.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "knx_internal.h"

/* ---------------------------------------------------------------- host tensors (reference include/kernix.h:146-227) */
float_tensor* kernix_float_new(int rows, int cols, int zero)
{
    if (rows < 0 || cols < 0) return NULL;
    float_tensor* t = malloc(sizeof *t);
    if (t == NULL) return NULL;
    const size_t n = (size_t)rows * (size_t)cols;
    const size_t bytes = (n * sizeof(float) + 63) / 64 * 64;
    void* mem = NULL;
    if (posix_memalign(&mem, 64, bytes ? bytes : 64) != 0) { free(t); return NULL; }
    t->row = rows;
    t->col = cols;
    t->tensor = mem;
    if (zero) memset(mem, 0, n * sizeof(float));
    return t;
}

float_tensor* float_zeros(int rows, int cols) { return kernix_float_new(rows, cols, 1); }

void float_free(float_tensor* t)
{
    if (t == NULL) return;
    free(t->tensor);
    free(t);
}

/* ---------------------------------------------------------------- int8 weights (reference include/kernix_model.h:52-95) */
static int round_up(int v, int m) { return (v + m - 1) / m * m; }

kernix_qweight* kernix_qweight_pack(const int8_t* q, const float* scale, int k, int n)
{
    if (q == NULL || scale == NULL || k < 1 || n < 1 || k > KERNIX_INT8_MAX_K || n > INT_MAX - 16) return NULL;
    kernix_qweight* w = calloc(1, sizeof *w);
    if (w == NULL) return NULL;
    w->k = k;
    w->n = n;
    w->kp = round_up(k, 64);
    w->np = round_up(n, 16);
    w->q = calloc((size_t)w->kp * (size_t)w->np, 1);
    w->scale = calloc((size_t)w->np, sizeof(float));
    if (w->q == NULL || w->scale == NULL) { kernix_qweight_free(w); return NULL; }
    memcpy(w->scale, scale, sizeof(float) * (size_t)n);
    /* file order k×n (in×out) → device order n×kp (one output channel per row, k contiguous) */
    for (int i = 0; i < k; i++) {
        const int8_t* src = q + (size_t)i * n;
        for (int j = 0; j < n; j++) w->q[(size_t)j * w->kp + i] = src[j];
    }
    return w;
}

void kernix_qweight_unpack(const kernix_qweight* w, float* dst)
{
    for (int i = 0; i < w->k; i++)
        for (int j = 0; j < w->n; j++) dst[(size_t)i * w->n + j] = (float)w->q[(size_t)j * w->kp + i] * w->scale[j];
}

void kernix_qweight_free(kernix_qweight* w)
{
    if (w == NULL) return;
    free(w->q);
    free(w->scale);
    free(w);
}

/* ---------------------------------------------------------------- bounded reader */
typedef struct {
    FILE* f;
    size_t left;
} knx_rd;

static int rd_u32(knx_rd* r, uint32_t* v)
{
    if (r->left < 4 || fread(v, 4, 1, r->f) != 1) return -1;
    r->left -= 4;
    return 0;
}

static int rd_u32s(knx_rd* r, uint32_t* v, int n)
{
    for (int i = 0; i < n; i++)
        if (rd_u32(r, &v[i]) != 0) return -1;
    return 0;
}

static int rd_f32s(knx_rd* r, float* dst, size_t n)
{
    if (dst == NULL || n > r->left / 4 || fread(dst, 4, n, r->f) != n) return -1;
    r->left -= n * 4;
    return 0;
}

/* n floats into a new array, or NULL (nothing allocated) when the file does not hold them */
static float* rd_new_f32s(knx_rd* r, size_t n)
{
    if (n > r->left / 4) return NULL;
    float* p = malloc((n ? n : 1) * sizeof(float));
    if (p != NULL && rd_f32s(r, p, n) != 0) { free(p); p = NULL; }
    return p;
}

/* ---------------------------------------------------------------- weight blocks */
static uint64_t block_bytes(uint32_t dt, uint64_t k, uint64_t n)
{
    return dt == KERNIX_DT_F32 ? 4 * k * n : dt == KERNIX_DT_I8_COL ? 4 * n + k * n : 4 * k + k * n;
}

/* Reads a k×n weight block.  With keep_int8 and an I8_COL block the weight stays int8 (*wq); otherwise it becomes
 * fp32 in *wt (a new host tensor) or *wr (a new array). */
static int rd_weight(knx_rd* r, int ver, uint64_t k, uint64_t n, int keep_int8, float_tensor** wt, float** wr,
                     kernix_qweight** wq, const char** err)
{
    if (k < 1 || n < 1 || k > INT_MAX || n > INT_MAX || k * n > (uint64_t)INT_MAX) { *err = "weight size out of range"; return -1; }
    uint32_t dt = KERNIX_DT_F32;
    if (ver >= 2 && rd_u32(r, &dt) != 0) return -1;
    if (dt > KERNIX_DT_I8_ROW) { *err = "unknown weight dtype"; return -1; }
    if (block_bytes(dt, k, n) > r->left) return -1; /* before any allocation: a forged size must not allocate */
    const size_t cnt = (size_t)k * (size_t)n;
    const int as_int8 = keep_int8 && dt == KERNIX_DT_I8_COL;
    float* dst = NULL;
    if (!as_int8) {
        if (wt != NULL) {
            if ((*wt = kernix_float_new((int)k, (int)n, 0)) == NULL) { *err = "out of memory"; return -1; }
            dst = (*wt)->tensor;
        } else if ((dst = *wr = malloc(sizeof(float) * cnt)) == NULL) {
            *err = "out of memory";
            return -1;
        }
    }
    if (dt == KERNIX_DT_F32) return rd_f32s(r, dst, cnt);
    if (as_int8 && k > KERNIX_INT8_MAX_K) { *err = "int8 weight input size out of range"; return -1; }
    const size_t ns = dt == KERNIX_DT_I8_COL ? (size_t)n : (size_t)k;
    float* sc = malloc(sizeof(float) * ns);
    int8_t* q = malloc(cnt);
    int rc = -1;
    if (sc == NULL || q == NULL) { *err = "out of memory"; goto done; }
    if (rd_f32s(r, sc, ns) != 0 || cnt > r->left || fread(q, 1, cnt, r->f) != cnt) goto done;
    r->left -= cnt;
    for (size_t i = 0; i < ns; i++)
        if (!(sc[i] > 0.0f && sc[i] <= FLT_MAX)) { *err = "int8 scale not finite and positive"; goto done; }
    if (as_int8) {
        if ((*wq = kernix_qweight_pack(q, sc, (int)k, (int)n)) == NULL) { *err = "out of memory"; goto done; }
    } else {
        const int col = dt == KERNIX_DT_I8_COL;
        for (size_t i = 0; i < (size_t)k; i++)
            for (size_t j = 0; j < (size_t)n; j++) dst[i * n + j] = (float)q[i * n + j] * sc[col ? j : i];
    }
    rc = 0;
done:
    free(sc);
    free(q);
    return rc;
}

/* ---------------------------------------------------------------- op records */
static int geom_ok(uint32_t v, uint32_t lo) { return v >= lo && v <= KERNIX_MAX_GEOM; }
static uint64_t gates_of(int kind) { return kind == KERNIX_OP_LSTM ? 4 : kind == KERNIX_OP_GRU ? 3 : 1; }

static int parse_op(knx_rd* r, int ver, kernix_step* s, const char** err)
{
    uint32_t a[16];
    s->act = KERNIX_ACT_NONE;
    s->dirs = 1;
    s->groups = 1;
    s->kh = s->kw = s->sh = s->sw = s->dh = s->dw = 1;
    switch (s->kind) {
    case KERNIX_OP_LINEAR: /* in, out, has_bias · W(in×out) [· b] */
        if (rd_u32s(r, a, 3) != 0) return -1;
        if (a[0] < 1 || a[1] < 1 || a[0] > INT_MAX || a[1] > INT_MAX || a[2] > 1) { *err = "Linear size out of range"; return -1; }
        s->in = (int)a[0];
        s->out = (int)a[1];
        if (rd_weight(r, ver, a[0], a[1], 1, &s->w, NULL, &s->q, err) != 0) return -1;
        return a[2] && (s->bias = rd_new_f32s(r, a[1])) == NULL ? -1 : 0;
    case KERNIX_OP_ACT: /* act [· f32 alpha in KNX3] */
        if (rd_u32(r, &a[0]) != 0 || (ver >= 3 && rd_f32s(r, &s->alpha, 1) != 0)) return -1;
        if (a[0] > (uint32_t)(ver >= 3 ? KERNIX_ACT_LAST : KERNIX_ACT_TANH) || !isfinite(s->alpha)) { *err = "unknown activation"; return -1; }
        s->act = (int)a[0];
        return 0;
    case KERNIX_OP_LAYERNORM: /* cols, affine, f32 eps [· γ · β] */
        if (rd_u32s(r, a, 2) != 0 || rd_f32s(r, &s->eps, 1) != 0) return -1;
        if (a[0] < 1 || a[0] > INT_MAX || a[1] > 1 || !(s->eps >= 0.0f) || isinf(s->eps)) { *err = "LayerNorm value out of range"; return -1; }
        s->in = s->out = (int)a[0];
        return a[1] && ((s->gamma = rd_new_f32s(r, a[0])) == NULL || (s->beta = rd_new_f32s(r, a[0])) == NULL) ? -1 : 0;
    case KERNIX_OP_SOFTMAX:
        return 0;
    case KERNIX_OP_LSTM:
    case KERNIX_OP_GRU:
    case KERNIX_OP_RNN: {
        if (ver < 3) { /* KNX1/2 LSTM: in, units, act (relu/tanh), ret_seq, seq */
            if (rd_u32s(r, a, 5) != 0) return -1;
            if (a[0] < 1 || a[0] > INT_MAX || a[1] < 1 || a[1] > KERNIX_CHUNK / 2 || a[3] > 1 || a[4] < 1 || a[4] > INT_MAX ||
                (a[2] != KERNIX_ACT_RELU && a[2] != KERNIX_ACT_TANH)) { *err = "LSTM value out of range"; return -1; }
            s->seq = (int)a[4];
            a[4] = 1;
            a[5] = KERNIX_MERGE_CONCAT;
        } else { /* KNX3: in, units, act, ret_seq, dirs, merge */
            if (rd_u32s(r, a, 6) != 0) return -1;
            if (a[0] < 1 || a[0] > INT_MAX || a[1] < 1 || a[1] > KERNIX_CHUNK / 2 || a[2] > KERNIX_ACT_LAST || a[3] > 1 ||
                a[4] < 1 || a[4] > 2 || a[5] > KERNIX_MERGE_AVE) { *err = "RNN value out of range"; return -1; }
        }
        s->in = (int)a[0];
        s->out = (int)a[1];
        s->act = (int)a[2];
        s->ret_seq = (int)a[3];
        s->dirs = (int)a[4];
        s->merge = (int)a[5];
        const uint64_t gu = gates_of(s->kind) * (uint64_t)a[1], nb = s->kind == KERNIX_OP_GRU ? 2 * gu : gu;
        for (int d = 0; d < s->dirs; d++) { /* input weight always fp32; recurrent weight may stay int8 */
            if (rd_weight(r, ver, a[0], gu, 0, d ? &s->w_b : &s->w, NULL, NULL, err) != 0 ||
                rd_weight(r, ver, a[1], gu, 1, NULL, d ? &s->rec_b : &s->rec, d ? &s->q_b : &s->q, err) != 0) return -1;
            if ((*(d ? &s->bias_b : &s->bias) = rd_new_f32s(r, nb)) == NULL) return -1;
        }
        return 0;
    }
    case KERNIX_OP_CONV: /* cin cout kh kw sh sw dh dw pt pb pl pr groups has_bias · W((kh·kw·cin/g)×cout) [· b] */
        if (rd_u32s(r, a, 14) != 0) return -1;
        if (a[0] < 1 || a[0] > INT_MAX || a[1] < 1 || a[1] > INT_MAX || !geom_ok(a[2], 1) || !geom_ok(a[3], 1) ||
            !geom_ok(a[4], 1) || !geom_ok(a[5], 1) || !geom_ok(a[6], 1) || !geom_ok(a[7], 1) || !geom_ok(a[8], 0) ||
            !geom_ok(a[9], 0) || !geom_ok(a[10], 0) || !geom_ok(a[11], 0) || a[12] < 1 || a[0] % a[12] != 0 ||
            a[1] % a[12] != 0 || a[13] > 1) { *err = "convolution value out of range"; return -1; }
        s->in = (int)a[0]; s->out = (int)a[1];
        s->kh = (int)a[2]; s->kw = (int)a[3]; s->sh = (int)a[4]; s->sw = (int)a[5]; s->dh = (int)a[6]; s->dw = (int)a[7];
        s->pt = (int)a[8]; s->pb = (int)a[9]; s->pl = (int)a[10]; s->pr = (int)a[11]; s->groups = (int)a[12];
        if (rd_weight(r, ver, (uint64_t)a[2] * a[3] * (a[0] / a[12]), a[1], 0, &s->w, NULL, NULL, err) != 0) return -1;
        return a[13] && (s->bias = rd_new_f32s(r, a[1])) == NULL ? -1 : 0;
    case KERNIX_OP_POOL: /* type kh kw sh sw pt pb pl pr count_pad */
        if (rd_u32s(r, a, 10) != 0) return -1;
        if (a[0] > KERNIX_POOL_AVG || !geom_ok(a[1], 1) || !geom_ok(a[2], 1) || !geom_ok(a[3], 1) || !geom_ok(a[4], 1) ||
            a[5] >= a[1] || a[6] >= a[1] || a[7] >= a[2] || a[8] >= a[2] || a[9] > 1) {
            *err = "pooling value out of range"; /* padding ≥ window would leave empty windows */
            return -1;
        }
        s->ptype = (int)a[0]; s->kh = (int)a[1]; s->kw = (int)a[2]; s->sh = (int)a[3]; s->sw = (int)a[4];
        s->pt = (int)a[5]; s->pb = (int)a[6]; s->pl = (int)a[7]; s->pr = (int)a[8]; s->count_pad = (int)a[9];
        return 0;
    case KERNIX_OP_GLOBAL_POOL:
        if (rd_u32(r, &a[0]) != 0) return -1;
        if (a[0] > KERNIX_POOL_AVG) { *err = "pooling value out of range"; return -1; }
        s->ptype = (int)a[0];
        return 0;
    case KERNIX_OP_RESHAPE:
    case KERNIX_OP_PERMUTE: {
        if (rd_u32(r, &a[0]) != 0) return -1;
        if (a[0] < 1 || a[0] > KERNIX_MAX_DIMS) { *err = "number of axes out of range"; return -1; }
        s->nd = (int)a[0];
        if (rd_u32s(r, a + 1, s->nd) != 0) return -1;
        unsigned seen = 0;
        for (int k = 0; k < s->nd; k++) {
            const uint32_t v = a[1 + k];
            if (s->kind == KERNIX_OP_RESHAPE) {
                if (v < 1 || v > INT_MAX) { *err = "Reshape shape out of range"; return -1; }
                s->d[k] = (int)v;
            } else {
                if (v >= (uint32_t)s->nd || ((seen >> v) & 1u)) { *err = "Permute axis order invalid"; return -1; }
                s->perm[k] = (int)v;
                seen |= 1u << v;
            }
        }
        return 0;
    }
    case KERNIX_OP_BINARY:
        if (rd_u32(r, &a[0]) != 0) return -1;
        if (a[0] > KERNIX_BIN_MIN) { *err = "unknown binary op"; return -1; }
        s->bop = (int)a[0];
        return 0;
    case KERNIX_OP_CONCAT:
        if (rd_u32(r, &a[0]) != 0) return -1;
        if (a[0] > KERNIX_AXIS_LAST) { *err = "Concatenate axis out of range"; return -1; }
        s->axis = (int)a[0];
        return 0;
    case KERNIX_OP_EMBEDDING: /* vocab, dim · table */
        if (rd_u32s(r, a, 2) != 0) return -1;
        s->in = (int)(a[0] > INT_MAX ? 0 : a[0]);
        s->out = (int)(a[1] > INT_MAX ? 0 : a[1]);
        return rd_weight(r, ver, a[0], a[1], 0, &s->w, NULL, NULL, err);
    case KERNIX_OP_AFFINE: /* c · scale · shift */
        if (rd_u32(r, &a[0]) != 0) return -1;
        if (a[0] < 1 || a[0] > INT_MAX) { *err = "Affine size out of range"; return -1; }
        s->in = s->out = (int)a[0];
        return (s->gamma = rd_new_f32s(r, a[0])) == NULL || (s->beta = rd_new_f32s(r, a[0])) == NULL ? -1 : 0;
    case KERNIX_OP_ADD_CONST:
        if (rd_u32(r, &a[0]) != 0) return -1;
        if (a[0] < 1 || a[0] > INT_MAX) { *err = "constant size out of range"; return -1; }
        s->in = (int)a[0];
        return (s->cst = rd_new_f32s(r, a[0])) == NULL ? -1 : 0;
    case KERNIX_OP_ATTENTION: { /* heads dk dv causal cq cv ck cout has_bias · Wq [bq] Wk [bk] Wv [bv] Wo [bo] */
        if (rd_u32s(r, a, 9) != 0) return -1;
        if (a[0] < 1 || a[0] > 4096 || a[1] < 1 || a[1] > 65536 || a[2] < 1 || a[2] > 65536 || a[3] > 1 || a[8] > 1 ||
            a[4] < 1 || a[4] > INT_MAX || a[5] < 1 || a[5] > INT_MAX || a[6] < 1 || a[6] > INT_MAX || a[7] < 1 || a[7] > INT_MAX) {
            *err = "attention value out of range";
            return -1;
        }
        s->heads = (int)a[0]; s->dk = (int)a[1]; s->dv = (int)a[2]; s->causal = (int)a[3];
        s->in = (int)a[4]; s->out = (int)a[7];
        const uint64_t hk = (uint64_t)a[0] * a[1], hv = (uint64_t)a[0] * a[2];
        if (rd_weight(r, ver, a[4], hk, 0, &s->w, NULL, NULL, err) != 0 || (a[8] && (s->bias = rd_new_f32s(r, hk)) == NULL) ||
            rd_weight(r, ver, a[6], hk, 0, &s->wk, NULL, NULL, err) != 0 || (a[8] && (s->bk = rd_new_f32s(r, hk)) == NULL) ||
            rd_weight(r, ver, a[5], hv, 0, &s->wv, NULL, NULL, err) != 0 || (a[8] && (s->bv = rd_new_f32s(r, hv)) == NULL) ||
            rd_weight(r, ver, hv, a[7], 0, &s->wo, NULL, NULL, err) != 0 || (a[8] && (s->bo = rd_new_f32s(r, a[7])) == NULL))
            return -1;
        return 0;
    }
    case KERNIX_OP_SELECT: /* axis start len squeeze */
        if (rd_u32s(r, a, 4) != 0) return -1;
        if (a[0] > KERNIX_AXIS_LAST || a[1] > INT_MAX || a[2] < 1 || a[2] > INT_MAX || a[3] > 1) { *err = "Select value out of range"; return -1; }
        s->axis = (int)a[0]; s->start = (int)a[1]; s->len = (int)a[2]; s->squeeze = (int)a[3];
        return 0;
    case KERNIX_OP_PAD:
        if (rd_u32s(r, a, 4) != 0) return -1;
        if (!geom_ok(a[0], 0) || !geom_ok(a[1], 0) || !geom_ok(a[2], 0) || !geom_ok(a[3], 0)) { *err = "padding value out of range"; return -1; }
        s->pt = (int)a[0]; s->pb = (int)a[1]; s->pl = (int)a[2]; s->pr = (int)a[3];
        return 0;
    case KERNIX_OP_UPSAMPLE:
        if (rd_u32s(r, a, 2) != 0) return -1;
        if (!geom_ok(a[0], 1) || !geom_ok(a[1], 1)) { *err = "UpSampling value out of range"; return -1; }
        s->sh = (int)a[0]; s->sw = (int)a[1];
        return 0;
    default:
        *err = "unknown op";
        return -1;
    }
}

/* ---------------------------------------------------------------- shapes (reference include/kernix_model.h:1246-1394) */
static int val_set(kernix_val* v, int nd, const int* d)
{
    if (nd < 1 || nd > KERNIX_MAX_DIMS) return -1;
    uint64_t r = 1;
    for (int k = 0; k < nd; k++) {
        if (d[k] < 1) return -1;
        if (k < nd - 1 && (r *= (uint64_t)d[k]) > INT_MAX) return -1;
    }
    if (r * (uint64_t)d[nd - 1] > INT_MAX) return -1;
    memset(v, 0, sizeof *v);
    v->nd = nd;
    memcpy(v->d, d, sizeof(int) * (size_t)nd);
    v->r = (int)r;
    v->c = d[nd - 1];
    v->st = -1;
    v->last = -1;
    return 0;
}

static int infer(kernix_step* s, int ver, const kernix_val* fv, kernix_val* out, const char** err)
{
    const kernix_val* x = &fv[s->inp[0]];
    int nd = x->nd, d[KERNIX_MAX_DIMS];
    memcpy(d, x->d, sizeof d);
    switch (s->kind) {
    case KERNIX_OP_LINEAR:
        if (x->c != s->in) { *err = "Linear input size differs from the previous output"; return -1; }
        d[nd - 1] = s->out;
        break;
    case KERNIX_OP_ACT:
    case KERNIX_OP_SOFTMAX:
        break;
    case KERNIX_OP_LAYERNORM:
        if (x->c != s->in) { *err = "LayerNorm size differs from the previous output"; return -1; }
        break;
    case KERNIX_OP_LSTM:
    case KERNIX_OP_GRU:
    case KERNIX_OP_RNN: {
        if (x->c != s->in) { *err = "RNN input size differs from the previous output"; return -1; }
        if (ver < 3 && s->seq != x->r) { *err = "LSTM sequence length differs from the previous step"; return -1; }
        s->seq = x->r;
        const int uo = s->dirs == 2 && s->merge == KERNIX_MERGE_CONCAT ? 2 * s->out : s->out;
        if (s->ret_seq) { nd = 2; d[0] = x->r; d[1] = uo; }
        else { nd = 1; d[0] = uo; }
        break;
    }
    case KERNIX_OP_CONV:
    case KERNIX_OP_POOL:
    case KERNIX_OP_PAD:
    case KERNIX_OP_UPSAMPLE: {
        if (nd != 2 && nd != 3) { *err = "convolution/pooling input must be T×C or H×W×C"; return -1; }
        if (nd == 2 && (s->kw != 1 || s->sw != 1 || s->dw != 1 || s->pl != 0 || s->pr != 0)) { *err = "2-D kernel on a 1-D (T×C) input"; return -1; }
        if (s->kind == KERNIX_OP_CONV && x->c != s->in) { *err = "convolution input channels differ from the previous output"; return -1; }
        const int64_t H = d[0], W = nd == 3 ? d[1] : 1;
        int64_t Ho, Wo;
        if (s->kind == KERNIX_OP_PAD) { Ho = H + s->pt + s->pb; Wo = W + s->pl + s->pr; }
        else if (s->kind == KERNIX_OP_UPSAMPLE) { Ho = H * s->sh; Wo = W * s->sw; }
        else {
            const int64_t nh = H + s->pt + s->pb - ((int64_t)s->dh * (s->kh - 1) + 1);
            const int64_t nw = W + s->pl + s->pr - ((int64_t)s->dw * (s->kw - 1) + 1);
            if (nh < 0 || nw < 0) { *err = "convolution/pooling output size ≤ 0"; return -1; }
            Ho = nh / s->sh + 1;
            Wo = nw / s->sw + 1;
        }
        if (Ho > INT_MAX || Wo > INT_MAX) { *err = "shape out of range"; return -1; }
        d[0] = (int)Ho;
        if (nd == 3) d[1] = (int)Wo;
        if (s->kind == KERNIX_OP_CONV) d[nd - 1] = s->out;
        break;
    }
    case KERNIX_OP_GLOBAL_POOL:
        nd = 1;
        d[0] = x->c;
        break;
    case KERNIX_OP_RESHAPE: {
        uint64_t n = 1;
        for (int k = 0; k < s->nd; k++) n *= (uint64_t)s->d[k];
        if (n != (uint64_t)x->r * (uint64_t)x->c) { *err = "Reshape size differs from the input"; return -1; }
        nd = s->nd;
        memcpy(d, s->d, sizeof d);
        break;
    }
    case KERNIX_OP_PERMUTE:
        if (s->nd != nd) { *err = "Permute axis count differs from the input"; return -1; }
        for (int k = 0; k < nd; k++) d[k] = x->d[s->perm[k]];
        break;
    case KERNIX_OP_BINARY: {
        const kernix_val* y = &fv[s->inp[1]];
        const int R = x->r > y->r ? x->r : y->r, C = x->c > y->c ? x->c : y->c;
        const kernix_val* big = (int64_t)x->r * x->c >= (int64_t)y->r * y->c ? x : y;
        if ((x->r != R && x->r != 1) || (y->r != R && y->r != 1) || (x->c != C && x->c != 1) || (y->c != C && y->c != 1) || big->r != R) {
            *err = "binary op input shapes do not broadcast";
            return -1;
        }
        nd = big->nd;
        memcpy(d, big->d, sizeof d);
        d[nd - 1] = C;
        break;
    }
    case KERNIX_OP_CONCAT: {
        const int ax = s->axis == KERNIX_AXIS_FIRST ? 0 : nd - 1;
        int64_t sum = 0;
        for (int k = 0; k < s->n_in; k++) {
            const kernix_val* v = &fv[s->inp[k]];
            int same = v->nd == nd;
            for (int j = 0; same && j < nd; j++)
                if (j != ax) same = v->d[j] == x->d[j];
            if (!same) { *err = "Concatenate input shapes do not match"; return -1; }
            sum += v->d[ax];
        }
        if (sum > INT_MAX) { *err = "shape out of range"; return -1; }
        d[ax] = (int)sum;
        break;
    }
    case KERNIX_OP_EMBEDDING:
        if (nd >= KERNIX_MAX_DIMS) { *err = "number of axes out of range"; return -1; }
        d[nd++] = s->out;
        break;
    case KERNIX_OP_AFFINE:
        if (x->c != s->in) { *err = "Affine size differs from the previous output"; return -1; }
        break;
    case KERNIX_OP_ADD_CONST:
        if ((int64_t)x->r * x->c != s->in) { *err = "constant size differs from the previous output"; return -1; }
        break;
    case KERNIX_OP_ATTENTION: {
        const kernix_val* v = &fv[s->inp[s->n_in > 1 ? 1 : 0]];
        const kernix_val* k = &fv[s->inp[s->n_in > 2 ? 2 : s->n_in > 1 ? 1 : 0]];
        if (x->c != s->w->row || v->c != s->wv->row || k->c != s->wk->row || k->r != v->r) {
            *err = "attention input sizes differ from the weights";
            return -1;
        }
        d[nd - 1] = s->out;
        break;
    }
    case KERNIX_OP_SELECT: {
        const int ax = s->axis == KERNIX_AXIS_FIRST ? 0 : nd - 1;
        if ((int64_t)s->start + s->len > d[ax]) { *err = "Select range outside the input"; return -1; }
        d[ax] = s->len;
        if (s->squeeze && s->len == 1 && nd > 1) {
            memmove(d + ax, d + ax + 1, sizeof(int) * (size_t)(nd - 1 - ax));
            nd--;
        }
        break;
    }
    default:
        break;
    }
    if (val_set(out, nd, d) != 0) { *err = "shape out of range"; return -1; }
    return 0;
}

/* ---------------------------------------------------------------- storage plan
 * Each value gets a storage buffer.  Ops that read and write the same positions (elementwise and row-wise) write
 * into their input's buffer when that input is dead afterwards and has the same size; RESHAPE aliases its input;
 * otherwise the smallest free buffer that is large enough is reused (or the largest free one grows, or a new one
 * is opened).  A buffer is free at step i when every value stored in it was last read before step i. */
static int writes_in_place(int kind)
{
    return kind == KERNIX_OP_ACT || kind == KERNIX_OP_LAYERNORM || kind == KERNIX_OP_SOFTMAX || kind == KERNIX_OP_AFFINE ||
           kind == KERNIX_OP_ADD_CONST || kind == KERNIX_OP_BINARY;
}

static int plan(kernix_model* m)
{
    const int n = m->n_steps;
    size_t* cap = calloc((size_t)n + 1, sizeof(size_t));
    int* busy_until = calloc((size_t)n + 1, sizeof(int));
    if (cap == NULL || busy_until == NULL) { free(cap); free(busy_until); return -1; }
    int nbuf = 0;
    for (int i = 0; i < n; i++) {
        const kernix_step* s = &m->steps[i];
        kernix_val* v = &m->vals[i + 1];
        const size_t need = (size_t)v->r * (size_t)v->c;
        int st = -2;
        if (s->kind == KERNIX_OP_RESHAPE) {
            st = m->vals[s->inp[0]].st;
        } else if (writes_in_place(s->kind)) {
            const int n_try = s->kind == KERNIX_OP_BINARY ? 2 : 1;
            /* a binary op reuses the buffer of the previous step's output first: the runtime can then fold the op
             * into that step's epilogue (the folded step must not write where it still reads its own inputs) */
            const int first = n_try == 2 && s->inp[1] == i ? 1 : 0;
            for (int t = 0; t < n_try && st == -2; t++) {
                const int k = (first + t) % n_try;
                const kernix_val* u = &m->vals[s->inp[k]];
                if (u->st >= 0 && busy_until[u->st] <= i && (size_t)u->r * (size_t)u->c == need) st = u->st;
            }
        }
        if (st == -2) {
            int best = -1;
            for (int k = 0; k < nbuf; k++) {
                if (busy_until[k] >= i) continue;
                if (best < 0) { best = k; continue; }
                const int fits = cap[k] >= need, best_fits = cap[best] >= need;
                if (fits ? (!best_fits || cap[k] < cap[best]) : (!best_fits && cap[k] > cap[best])) best = k;
            }
            if (best < 0) best = nbuf++;
            if (cap[best] < need) cap[best] = need;
            st = best;
        }
        v->st = st;
        if (st >= 0) {
            if (busy_until[st] < v->last) busy_until[st] = v->last;
            if (busy_until[st] < i) busy_until[st] = i;
        }
    }
    free(busy_until);
    m->n_st = nbuf;
    m->st_cap = cap;
    m->st = calloc((size_t)(nbuf ? nbuf : 1), sizeof(float_tensor*));
    return m->st == NULL ? -1 : 0;
}

/* ---------------------------------------------------------------- model */
void knx_step_host_free(kernix_step* s)
{
    float_free(s->w); float_free(s->w_b); float_free(s->wk); float_free(s->wv); float_free(s->wo);
    kernix_qweight_free(s->q); kernix_qweight_free(s->q_b);
    free(s->rec); free(s->rec_b); free(s->bias); free(s->bias_b); free(s->bk); free(s->bv); free(s->bo);
    free(s->gamma); free(s->beta); free(s->cst);
}

/* 0 when CONV runs as a plain GEMM on its input (1×1, stride 1, no padding, one group), else its GEMM depth. */
size_t knx_conv_is_gemm(const kernix_step* s)
{
    const int pointwise = s->kh == 1 && s->kw == 1 && s->sh == 1 && s->sw == 1 && s->pt == 0 && s->pb == 0 && s->pl == 0 && s->pr == 0;
    if (s->groups == 1 && pointwise) return 0;
    return (size_t)s->kh * s->kw * (size_t)(s->in / s->groups);
}

static void compute_ws_fixed(kernix_model* m)
{
    m->ws_fixed = 0;
    if (m->int8_mode != KERNIX_INT8_REF) return; /* the fp32 copies exist only in the reference dispatch */
    for (int i = 0; i < m->n_steps; i++) {
        if (m->steps[i].q != NULL) m->ws_fixed += (size_t)m->steps[i].q->k * (size_t)m->steps[i].q->n;
        if (m->steps[i].q_b != NULL) m->ws_fixed += (size_t)m->steps[i].q_b->k * (size_t)m->steps[i].q_b->n;
    }
}

int kernix_model_set_int8_mode(kernix_model* m, int mode)
{
    if (m == NULL || (mode != KERNIX_INT8_REF && mode != KERNIX_INT8_I8)) return -1;
    if (m->int8_mode == mode) return 0;
    knx_model_release_device_ws(m);
    m->int8_mode = mode;
    compute_ws_fixed(m);
    return 0;
}

kernix_model* kernix_model_load(const char* path)
{
    FILE* f = path ? fopen(path, "rb") : NULL;
    if (f == NULL) {
        KNX_LOG("model load failed (%s): cannot open the file\n", path ? path : "NULL");
        return NULL;
    }
    kernix_model* m = NULL;
    kernix_val* fv = NULL;
    int* cons = NULL;
    int* map = NULL;
    const char* err = "file shorter than declared";
    knx_rd r = { f, 0 };
    long size;
    uint32_t magic, n_ops, hdr[2 + KERNIX_MAX_DIMS];
    if (fseek(f, 0, SEEK_END) != 0 || (size = ftell(f)) < 0 || fseek(f, 0, SEEK_SET) != 0) goto fail;
    r.left = (size_t)size;

    if (rd_u32(&r, &magic) != 0 || rd_u32(&r, &n_ops) != 0) goto fail;
    const int ver = memcmp(&magic, "KNX1", 4) == 0 ? 1 : memcmp(&magic, "KNX2", 4) == 0 ? 2 : memcmp(&magic, "KNX3", 4) == 0 ? 3 : 0;
    if (ver == 0) { err = "not a KNX1/KNX2/KNX3 file"; goto fail; }
    if (n_ops < 1 || n_ops > KERNIX_MODEL_MAX_OPS) { err = "op count out of range"; goto fail; }

    m = calloc(1, sizeof *m);
    if (m != NULL) m->steps = calloc(n_ops, sizeof(kernix_step));
    fv = calloc((size_t)n_ops + 1, sizeof(kernix_val));
    cons = calloc((size_t)n_ops + 1, sizeof(int));
    map = calloc((size_t)n_ops + 1, sizeof(int));
    if (m == NULL || m->steps == NULL || fv == NULL || cons == NULL || map == NULL) { err = "out of memory"; goto fail; }
    m->batch = -1;

    if (ver == 3) { /* layout, in_nd, per-sample input shape (channels-last) */
        if (rd_u32s(&r, hdr, 2) != 0) goto fail;
        if (hdr[0] > 1 || hdr[1] < 1 || hdr[1] > KERNIX_MAX_DIMS) { err = "input shape out of range"; goto fail; }
        int d[KERNIX_MAX_DIMS];
        if (rd_u32s(&r, hdr + 2, (int)hdr[1]) != 0) goto fail;
        for (uint32_t k = 0; k < hdr[1]; k++) d[k] = hdr[2 + k] > INT_MAX ? 0 : (int)hdr[2 + k];
        if (val_set(&fv[0], (int)hdr[1], d) != 0) { err = "input shape out of range"; goto fail; }
        m->layout = (int)hdr[0];
    }
    for (uint32_t i = 0; i < n_ops; i++) {
        kernix_step* s = &m->steps[i];
        uint32_t kind;
        if (rd_u32(&r, &kind) != 0) goto fail;
        if (kind > (uint32_t)(ver == 3 ? KERNIX_OP_LAST : KERNIX_OP_LSTM)) { err = "unknown op"; goto fail; }
        s->kind = (int)kind;
        if (ver == 3) { /* input value ids: 0 = model input, k+1 = output of op k (earlier ops only) */
            uint32_t n_in;
            if (rd_u32(&r, &n_in) != 0) goto fail;
            const uint32_t lo = kind == KERNIX_OP_BINARY || kind == KERNIX_OP_CONCAT ? 2 : 1;
            const uint32_t hi = kind == KERNIX_OP_BINARY ? 2 : kind == KERNIX_OP_CONCAT ? KERNIX_MAX_INPUTS : kind == KERNIX_OP_ATTENTION ? 3 : 1;
            if (n_in < lo || n_in > hi) { err = "op input count out of range"; goto fail; }
            s->n_in = (int)n_in;
            for (uint32_t k = 0; k < n_in; k++) {
                uint32_t id;
                if (rd_u32(&r, &id) != 0) goto fail;
                if (id > i) { err = "op input refers to a later op"; goto fail; }
                s->inp[k] = (int)id;
            }
        } else {
            s->n_in = 1;
            s->inp[0] = (int)i;
        }
        m->n_steps = (int)i + 1; /* free() releases up to this step if parsing fails below */
        if (parse_op(&r, ver, s, &err) != 0) goto fail;
    }
    if (r.left != 0) { err = "trailing data after the last op"; goto fail; }

    if (ver < 3) { /* input shape: in size of the first sized op, × the first LSTM's sequence length */
        int in_dim = 0, seq = 0;
        for (uint32_t i = 0; i < n_ops; i++) {
            const kernix_step* s = &m->steps[i];
            if (in_dim == 0 && (s->kind == KERNIX_OP_LINEAR || s->kind == KERNIX_OP_LAYERNORM || s->kind == KERNIX_OP_LSTM)) in_dim = s->in;
            if (seq == 0 && s->kind == KERNIX_OP_LSTM) seq = s->seq;
        }
        if (in_dim == 0) { err = "no Linear or LayerNorm: input size unknown"; goto fail; }
        const int d[2] = { seq ? seq : in_dim, in_dim };
        if (val_set(&fv[0], seq ? 2 : 1, d) != 0) { err = "input shape out of range"; goto fail; }
    }
    for (uint32_t i = 0; i < n_ops; i++)
        if (infer(&m->steps[i], ver, fv, &fv[i + 1], &err) != 0) goto fail;

    /* Fuse an ACT into the LINEAR/CONV that produces its only input (the activation then runs in the GEMM epilogue). */
    for (uint32_t i = 0; i < n_ops; i++)
        for (int k = 0; k < m->steps[i].n_in; k++) cons[m->steps[i].inp[k]]++;
    cons[n_ops]++; /* the model output */
    int n = 0;
    for (uint32_t i = 0; i < n_ops; i++) {
        kernix_step s = m->steps[i];
        for (int k = 0; k < s.n_in; k++) s.inp[k] = map[s.inp[k]];
        if (s.kind == KERNIX_OP_ACT && s.inp[0] > 0 && cons[m->steps[i].inp[0]] == 1) {
            kernix_step* p = &m->steps[s.inp[0] - 1]; /* already compacted */
            if ((p->kind == KERNIX_OP_LINEAR || p->kind == KERNIX_OP_CONV) && p->act == KERNIX_ACT_NONE) {
                p->act = s.act;
                p->alpha = s.alpha;
                map[i + 1] = s.inp[0];
                continue;
            }
        }
        m->steps[n] = s;
        fv[n + 1] = fv[i + 1];
        map[i + 1] = n + 1;
        n++;
    }
    if (n < (int)n_ops) memset(&m->steps[n], 0, sizeof(kernix_step) * (n_ops - (uint32_t)n));
    m->n_steps = n;
    m->n_vals = n + 1;
    m->out_v = map[n_ops];
    m->vals = fv;
    fv = NULL;
    m->views = calloc((size_t)m->n_vals, sizeof(float_tensor));
    if (m->views == NULL) { err = "out of memory"; goto fail; }
    for (int i = 0; i < n; i++)
        for (int k = 0; k < m->steps[i].n_in; k++) m->vals[m->steps[i].inp[k]].last = i;
    m->vals[m->out_v].last = n;
    if (plan(m) != 0) { err = "out of memory"; goto fail; }

    const kernix_val* vin = &m->vals[0];
    const kernix_val* vout = &m->vals[m->out_v];
    m->in_dim = vin->c;
    m->seq_len = vin->r;
    m->out_dim = vout->r * vout->c;
    m->in_nd = vin->nd;
    memcpy(m->in_shape, vin->d, sizeof m->in_shape);
    m->out_nd = vout->nd;
    memcpy(m->out_shape, vout->d, sizeof m->out_shape);
    m->ws_limit = KERNIX_WORKSPACE_LIMIT;
    {
        const char* mode = getenv("KERNIX_INT8_MODE");
        m->int8_mode = (mode != NULL && strcmp(mode, "i8") == 0) ? KERNIX_INT8_I8 : KERNIX_INT8_REF;
    }
    if (knx_model_count_ws(m, &m->ws_per_sample) != 0) { err = "workspace size out of range"; goto fail; }
    compute_ws_fixed(m);
    free(cons);
    free(map);
    fclose(f);
    return m;

fail:
    KNX_LOG("model load failed (%s): %s\n", path, err);
    kernix_model_free(m);
    free(fv);
    free(cons);
    free(map);
    fclose(f);
    return NULL;
}

void kernix_model_free(kernix_model* m)
{
    if (m == NULL) return;
    knx_model_release_device_all(m);
    for (int i = 0; m->steps != NULL && i < m->n_steps; i++) knx_step_host_free(&m->steps[i]);
    free(m->steps);
    free(m->vals);
    free(m->views);
    free(m->st_cap);
    free(m->st);
    free(m);
}

void kernix_model_set_workspace_limit(kernix_model* m, size_t bytes)
{
    if (m != NULL) m->ws_limit = bytes;
}

int kernix_model_set_ane(kernix_model* m, int on)
{
    if (m == NULL) return -1;
    if (!on) { m->ane = 0; return 0; }
    return -1; /* no Neural Engine on this platform */
}

void kernix_model_ane_info(const kernix_model* m, kernix_ane_info* out)
{
    (void)m;
    if (out != NULL) memset(out, 0, sizeof *out);
}
