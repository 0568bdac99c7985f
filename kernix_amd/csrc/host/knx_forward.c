/* knx_forward.c — device residency, workspace and forward of the KERNIX MI355X runtime.
 *
 * Replaces the reference's host-memory workspace, chunked execution and per-op CPU/Metal dispatch
 * (reference include/kernix_model.h:1603-1694 workspace, :1844-1905 step dispatch, :1995-2064 forward) with:
 *   - weights uploaded once, on the first forward, and kept on the device until kernix_model_free;
 *   - one device arena per chunk size holding every storage buffer, per-step scratch, the dequantized int8 copies
 *     and the staged input (allocated only when the chunk size changes, released by trim);
 *   - every step enqueued on the model's stream; the host waits once per forward, after the device→host copy.
 * Chunking under ws_limit and its results are the reference's: a batch larger than the limit allows runs in
 * chunks of equal size (the last one smaller) and returns the concatenated output.
 */
#include <limits.h>
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "knx_internal.h"

#define KNX_ALIGN 256

static int hip_ok(int rc, const char* what)
{
    if (rc == KNX_OK) return 0;
    KNX_LOG("KERNIX: %s failed: %s\n", what, knx_hip_last_error());
    return -1;
}

/* ---------------------------------------------------------------- device weights */
static int up(void** dst, const void* src, size_t bytes, void* stream)
{
    *dst = NULL;
    if (src == NULL) return 0;
    if (knx_hip_malloc(dst, bytes) != KNX_OK) return -1;
    return knx_hip_memcpy_h2d(*dst, src, bytes, stream) == KNX_OK ? 0 : -1;
}

static int up_f(float** dst, const float* src, size_t n, void* stream) { return up((void**)dst, src, n * sizeof(float), stream); }
static int up_t(float** dst, const float_tensor* t, void* stream)
{
    return t == NULL ? (*dst = NULL, 0) : up_f(dst, t->tensor, (size_t)t->row * (size_t)t->col, stream);
}
/* K×N host weight → N×K device copy (both GEMM operands K-contiguous, see knx_hip_sgemm_nt_ep) */
static int up_tT(float** dst, const float_tensor* t, void* stream)
{
    *dst = NULL;
    if (t == NULL) return 0;
    const size_t k = (size_t)t->row, n = (size_t)t->col;
    float* h = malloc(sizeof(float) * k * n);
    if (h == NULL) return -1;
    for (size_t i = 0; i < k; i++)
        for (size_t j = 0; j < n; j++) h[j * k + i] = t->tensor[i * n + j];
    int rc = up_f(dst, h, k * n, stream);
    if (rc == 0) rc = knx_hip_stream_sync(stream) != KNX_OK; /* the copy reads h: wait before freeing it */
    free(h);
    return rc;
}
static int up_q(int8_t** dq, float** ds, const kernix_qweight* q, void* stream)
{
    *dq = NULL;
    *ds = NULL;
    if (q == NULL) return 0;
    if (up((void**)dq, q->q, (size_t)q->np * (size_t)q->kp, stream) != 0) return -1;
    return up_f(ds, q->scale, (size_t)q->np, stream);
}

static size_t gates(int kind) { return kind == KERNIX_OP_LSTM ? 4 : kind == KERNIX_OP_GRU ? 3 : 1; }

/* ATTENTION whose queries, keys and values all come from one input: Q|K|V are one GEMM against the stacked weights */
static int attn_self(const kernix_step* s)
{
    const int iv = s->inp[s->n_in > 1 ? 1 : 0], ik = s->inp[s->n_in > 2 ? 2 : s->n_in > 1 ? 1 : 0];
    return iv == s->inp[0] && ik == s->inp[0];
}

/* [Wqᵀ; Wkᵀ; Wvᵀ] ((2·H·dk + H·dv) × in) and [bq | bk | bv] (zeros for absent biases, NULL if all are absent) */
static int up_qkv(struct knx_dstep* d, const kernix_step* s, void* stream)
{
    const float_tensor* w[3] = { s->w, s->wk, s->wv };
    const float* b[3] = { s->bias, s->bk, s->bv };
    const size_t in = (size_t)s->w->row;
    size_t n = 0;
    for (int t = 0; t < 3; t++) n += (size_t)w[t]->col;
    float* h = malloc(sizeof(float) * n * in);
    float* hb = (b[0] || b[1] || b[2]) ? calloc(n, sizeof(float)) : NULL;
    int rc = h == NULL || ((b[0] || b[1] || b[2]) && hb == NULL);
    for (size_t t = 0, off = 0; !rc && t < 3; off += (size_t)w[t]->col, t++) {
        const size_t c = (size_t)w[t]->col;
        for (size_t i = 0; i < in; i++)
            for (size_t j = 0; j < c; j++) h[(off + j) * in + i] = w[t]->tensor[i * c + j];
        if (b[t]) memcpy(hb + off, b[t], sizeof(float) * c);
    }
    if (!rc) rc = up_f(&d->wqkv, h, n * in, stream) || (hb && up_f(&d->bqkv, hb, n, stream));
    if (!rc) rc = knx_hip_stream_sync(stream) != KNX_OK; /* the copies read h and hb: wait before freeing them */
    free(h);
    free(hb);
    return rc;
}

static int upload_step(kernix_step* s, void* stream)
{
    struct knx_dstep* d = calloc(1, sizeof *d);
    if (d == NULL) return -1;
    s->dev = d;
    const size_t gu = gates(s->kind) * (size_t)s->out;
    const size_t nb = s->kind == KERNIX_OP_GRU ? 2 * gu : gu;
    switch (s->kind) {
    case KERNIX_OP_LINEAR:
        if (up_tT(&d->w, s->w, stream) || up_q(&d->q, &d->qscale, s->q, stream) || up_f(&d->bias, s->bias, (size_t)s->out, stream)) return -1;
        break;
    case KERNIX_OP_LAYERNORM:
        if (up_f(&d->gamma, s->gamma, (size_t)s->in, stream) || up_f(&d->beta, s->beta, (size_t)s->in, stream)) return -1;
        break;
    case KERNIX_OP_AFFINE:
        if (up_f(&d->gamma, s->gamma, (size_t)s->in, stream) || up_f(&d->beta, s->beta, (size_t)s->in, stream)) return -1;
        break;
    case KERNIX_OP_ADD_CONST:
        if (up_f(&d->cst, s->cst, (size_t)s->in, stream)) return -1;
        break;
    case KERNIX_OP_CONV:
        if (up_tT(&d->w, s->w, stream) || up_f(&d->bias, s->bias, (size_t)s->out, stream)) return -1;
        break;
    case KERNIX_OP_EMBEDDING:
        if (up_t(&d->w, s->w, stream) || up_f(&d->bias, s->bias, (size_t)s->out, stream)) return -1;
        break;
    case KERNIX_OP_LSTM:
    case KERNIX_OP_GRU:
    case KERNIX_OP_RNN:
        /* the input weight as gates·u × in (K-contiguous: the input projection runs on the NT GEMM kernels); a float U
         * stays u × gates·u as in the file, the layout whose columns the single-workgroup recurrence loads coalesced
         * (its transposed copy made every lane read a row of its own: LSTM batch 1 71 → 91 µs) */
        if (up_tT(&d->w, s->w, stream) || up_f(&d->bias, s->bias, nb, stream) || up_q(&d->q, &d->qscale, s->q, stream) ||
            up_f(&d->rec, s->rec, (size_t)s->out * gu, stream))
            return -1;
        if (s->dirs == 2 && (up_tT(&d->w_b, s->w_b, stream) || up_f(&d->bias_b, s->bias_b, nb, stream) ||
                             up_q(&d->q_b, &d->qscale_b, s->q_b, stream) || up_f(&d->rec_b, s->rec_b, (size_t)s->out * gu, stream)))
            return -1;
        if (s->dirs == 2 && s->merge == KERNIX_MERGE_AVE) {
            float* h = malloc(sizeof(float) * (size_t)s->out);
            float* z = calloc((size_t)s->out, sizeof(float));
            int rc = h == NULL || z == NULL;
            for (int i = 0; !rc && i < s->out; i++) h[i] = 0.5f;
            if (!rc) rc = up_f(&d->half, h, (size_t)s->out, stream) || up_f(&d->zero, z, (size_t)s->out, stream);
            /* the copies read h and z: wait before freeing them */
            if (!rc) rc = knx_hip_stream_sync(stream) != KNX_OK;
            free(h);
            free(z);
            if (rc) return -1;
        }
        break;
    case KERNIX_OP_ATTENTION: {
        const size_t hk = (size_t)s->heads * s->dk, hv = (size_t)s->heads * s->dv;
        if (attn_self(s) ? up_qkv(d, s, stream) != 0
                         : (up_tT(&d->w, s->w, stream) || up_f(&d->bias, s->bias, hk, stream) || up_tT(&d->wk, s->wk, stream) ||
                            up_f(&d->bk, s->bk, hk, stream) || up_tT(&d->wv, s->wv, stream) || up_f(&d->bv, s->bv, hv, stream)))
            return -1;
        if (up_tT(&d->wo, s->wo, stream) || up_f(&d->bo, s->bo, (size_t)s->out, stream)) return -1;
        break;
    }
    default:
        break;
    }
    return 0;
}

static void free_dstep(kernix_step* s)
{
    struct knx_dstep* d = s->dev;
    if (d == NULL) return;
    void* p[] = { d->w, d->bias, d->gamma, d->beta, d->cst, d->q, d->qscale, d->rec, d->w_b, d->bias_b, d->q_b,
                  d->qscale_b, d->rec_b, d->wk, d->wv, d->wo, d->bk, d->bv, d->bo, d->half, d->zero, d->wqkv, d->bqkv };
    for (size_t i = 0; i < sizeof p / sizeof p[0]; i++) knx_hip_free(p[i]);
    free(d);
    s->dev = NULL;
}

/* Creates the device state and uploads every weight (first forward only). */
static int ensure_device(kernix_model* m)
{
    if (m->dev != NULL && m->dev->uploaded) return 0;
    if (knx_hip_init() != KNX_OK) {
        KNX_LOG("KERNIX: no usable MI355X (gfx950) device: %s\n", knx_hip_last_error());
        return -1;
    }
    if (m->dev == NULL) {
        m->dev = calloc(1, sizeof *m->dev);
        if (m->dev == NULL) return -1;
        if (hip_ok(knx_hip_get_device(&m->dev->device), "device query") != 0) return -1;
        if (hip_ok(knx_hip_stream_create(&m->dev->stream), "stream creation") != 0 ||
            hip_ok(knx_hip_event_create_ordering(&m->dev->done), "event creation") != 0 ||
            hip_ok(knx_hip_host_malloc((void**)&m->dev->chain_status, sizeof(int)), "status word allocation") != 0)
            return -1;
        *m->dev->chain_status = 0;
    }
    for (int i = 0; i < m->n_steps; i++) {
        if (m->steps[i].dev != NULL) continue;
        if (upload_step(&m->steps[i], m->dev->stream) != 0) {
            KNX_LOG("KERNIX: weight upload failed: %s\n", knx_hip_last_error());
            return -1;
        }
    }
    if (hip_ok(knx_hip_stream_sync(m->dev->stream), "weight upload") != 0) return -1;
    m->dev->uploaded = 1;
    return 0;
}

/* ---------------------------------------------------------------- workspace */
/* COUNT: floats per sample; SIZE: arena bytes only; ALLOC: place every view in the arena; VIEW: shrink row counts */
enum { WS_COUNT, WS_SIZE, WS_ALLOC, WS_VIEW };

typedef struct {
    int mode;
    size_t off;      /* arena bytes used so far (ALLOC / sizing) */
    char* base;      /* arena (ALLOC) */
    size_t floats;   /* floats counted (COUNT) */
} ws_ctx;

static void* ws_take(ws_ctx* c, size_t bytes)
{
    const size_t at = c->off;
    c->off += (bytes + KNX_ALIGN - 1) / KNX_ALIGN * KNX_ALIGN;
    return c->base ? c->base + at : NULL;
}

/* One device tensor of rows × cols floats in the arena: COUNT adds its floats, ALLOC places a new view,
 * VIEW shrinks the rows of the existing one. */
static int ws_tensor(ws_ctx* c, float_tensor** t, size_t rows, size_t cols)
{
    if (rows > INT_MAX || cols > INT_MAX) return -1;
    c->floats += rows * cols;
    if (c->mode == WS_VIEW) { if (*t) (*t)->row = (int)rows; return 0; }
    if (c->mode == WS_COUNT) return 0;
    float* p = ws_take(c, rows * cols * sizeof(float));
    if (c->mode == WS_ALLOC) {
        if ((*t = malloc(sizeof(float_tensor))) == NULL) return -1;
        **t = (float_tensor){ (int)rows, (int)cols, p };
    }
    return 0;
}

static int int8_rows(const kernix_model* m, size_t rows)
{
    if (m->int8_mode == KERNIX_INT8_I8) return (int)rows;
    return (int)(rows < KERNIX_INT8_MAX_ROWS ? rows : KERNIX_INT8_MAX_ROWS);
}

/* Scratch for the grid-barrier launches (knx_hip_linear_chain, knx_hip_rnn_recurrence: their barrier words): one
 * block when the model has two LINEAR steps or more, or a recurrent step, else none. */
static size_t chain_scratch_bound(const kernix_model* m)
{
    int n = 0, rnn = 0;
    for (int i = 0; i < m->n_steps; i++) {
        const int k = m->steps[i].kind;
        n += k == KERNIX_OP_LINEAR;
        rnn |= k == KERNIX_OP_LSTM || k == KERNIX_OP_GRU || k == KERNIX_OP_RNN;
    }
    return n >= 2 || rnn ? KNX_ALIGN : 0;
}

/* Walks every workspace tensor for chunks of B samples.  ALLOC also places the dequantized int8 copies (the
 * reference allocates them only when the chunk has more than KERNIX_INT8_MAX_ROWS rows, and so does this). */
static int ws_walk(kernix_model* m, size_t B, ws_ctx* c)
{
    /* the value region: B × st_span floats, storage buffer k at float offset st_off[k]·B */
    if (m->st_span > SIZE_MAX / 8 / (B ? B : 1)) return -1;
    c->floats += B * m->st_span;
    if (c->mode == WS_SIZE || c->mode == WS_ALLOC) {
        float* region = ws_take(c, B * m->st_span * sizeof(float));
        for (int k = 0; c->mode == WS_ALLOC && k < m->n_st; k++) {
            if ((m->st[k] = malloc(sizeof(float_tensor))) == NULL) return -1;
            *m->st[k] = (float_tensor){ (int)B, (int)m->st_cap[k], region + m->st_off[k] * B };
        }
    } else if (c->mode == WS_VIEW) {
        for (int k = 0; k < m->n_st; k++)
            if (m->st[k]) m->st[k]->row = (int)B;
    }
    for (int i = 0; i < m->n_steps; i++) {
        kernix_step* s = &m->steps[i];
        const kernix_val* vi = &m->vals[s->inp[0]];
        const size_t rin = B * (size_t)vi->r;
        if (c->mode != WS_COUNT) s->buf = &m->views[i + 1];
        switch (s->kind) {
        case KERNIX_OP_LINEAR:
        case KERNIX_OP_LSTM:
        case KERNIX_OP_GRU:
        case KERNIX_OP_RNN: {
            const int rnn = s->kind != KERNIX_OP_LINEAR;
            const size_t qrows = rnn ? B : rin; /* rows of the int8 product: batch for the recurrence */
            if (rnn) {
                /* h and the recurrent terms double as the one-launch recurrence's two h buffers: rows of u4 */
                const size_t u = (size_t)s->out, gu = gates(s->kind) * u, u4 = (u + 3) / 4 * 4;
                if (ws_tensor(c, &s->tmp[0], rin, gu) || ws_tensor(c, &s->tmp[1], B, gu) ||
                    (s->kind == KERNIX_OP_LSTM && ws_tensor(c, &s->tmp[2], B, u)) || ws_tensor(c, &s->tmp[3], B, u4) ||
                    ws_tensor(c, &s->tmp[4], B, gu > u4 ? gu : u4) ||
                    (s->dirs == 2 && s->merge != KERNIX_MERGE_CONCAT && ws_tensor(c, &s->tmp[5], s->ret_seq ? rin : B, u)))
                    return -1;
            }
            if (s->q == NULL) break;
            /* int8 input rows and their scales, used only by the int8 path (both RNN directions run one after the
             * other and share it: their recurrent weights have the same shape) */
            const size_t xr = (size_t)int8_rows(m, qrows);
            const size_t kp = (size_t)s->q->kp;
            if (m->int8_mode == KERNIX_INT8_I8) c->floats += xr * (kp / 4 + 1);
            if (c->mode == WS_SIZE || c->mode == WS_ALLOC) {
                int8_t* xq = ws_take(c, xr * kp);
                float* sx = ws_take(c, xr * sizeof(float));
                if (c->mode == WS_ALLOC) { s->dev->xq = xq; s->dev->sx = sx; s->dev->xq_rows = (int)xr; }
            }
            /* fp32 copies of the int8 weights (counted in ws_fixed): reference dispatch with more rows than the
             * int8 threshold */
            if ((c->mode == WS_SIZE || c->mode == WS_ALLOC) && m->int8_mode == KERNIX_INT8_REF && qrows > KERNIX_INT8_MAX_ROWS) {
                float* p = ws_take(c, (size_t)s->q->k * (size_t)s->q->n * sizeof(float));
                float* pb = s->q_b ? ws_take(c, (size_t)s->q_b->k * (size_t)s->q_b->n * sizeof(float)) : NULL;
                if (c->mode == WS_ALLOC) {
                    if ((s->deq = malloc(sizeof(float_tensor))) == NULL) return -1;
                    *s->deq = (float_tensor){ s->q->n, s->q->k, p }; /* N×K: the transposed weight */
                    if (s->q_b) {
                        if ((s->deq_b = malloc(sizeof(float_tensor))) == NULL) return -1;
                        *s->deq_b = (float_tensor){ s->q_b->n, s->q_b->k, pb };
                    }
                }
            }
            break;
        }
        case KERNIX_OP_ATTENTION: {
            const kernix_val* vv = &m->vals[s->inp[s->n_in > 1 ? 1 : 0]];
            const size_t S = (size_t)vv->r, SR = B * S, H = (size_t)s->heads;
            /* Q, K, V (one rin × (2·H·dk + H·dv) block for self-attention), scores, context, Vᵀ */
            if (attn_self(s) ? ws_tensor(c, &s->tmp[0], rin, 2 * H * s->dk + H * s->dv)
                             : (ws_tensor(c, &s->tmp[0], rin, H * s->dk) || ws_tensor(c, &s->tmp[1], SR, H * s->dk) ||
                                ws_tensor(c, &s->tmp[2], SR, H * s->dv)))
                return -1;
            if (ws_tensor(c, &s->tmp[3], rin * H, S) || ws_tensor(c, &s->tmp[4], rin, H * s->dv) ||
                ws_tensor(c, &s->tmp[5], H * s->dv, SR))
                return -1;
            break;
        }
        default:
            break;
        }
    }
    /* Linear chains (a fixed size, outside the per-sample count) */
    if (c->mode == WS_SIZE || c->mode == WS_ALLOC) {
        const size_t cb = chain_scratch_bound(m);
        void* p = cb ? ws_take(c, cb) : NULL;
        if (c->mode == WS_ALLOC) { m->dev->chain = p; m->dev->chain_bytes = cb; }
    }
    /* staged model input */
    c->floats += B * (size_t)m->seq_len * (size_t)m->in_dim;
    if (c->mode == WS_SIZE || c->mode == WS_ALLOC) {
        float* din = ws_take(c, B * (size_t)m->seq_len * (size_t)m->in_dim * sizeof(float));
        if (c->mode == WS_ALLOC) m->dev->d_in = din;
    }
    return 0;
}

int knx_model_count_ws(kernix_model* m, size_t* per_sample)
{
    ws_ctx c = { WS_COUNT, 0, NULL, 0 };
    if (ws_walk(m, 1, &c) != 0) return -1;
    *per_sample = c.floats;
    return 0;
}

static void free_views(kernix_model* m)
{
    for (int k = 0; m->st != NULL && k < m->n_st; k++) { free(m->st[k]); m->st[k] = NULL; }
    for (int i = 0; m->steps != NULL && i < m->n_steps; i++) {
        kernix_step* s = &m->steps[i];
        s->buf = NULL;
        for (int k = 0; k < 6; k++) { free(s->tmp[k]); s->tmp[k] = NULL; }
        free(s->deq);
        s->deq = NULL;
        free(s->deq_b);
        s->deq_b = NULL;
        if (s->dev) { s->dev->xq = NULL; s->dev->sx = NULL; s->dev->xq_rows = 0; }
    }
}

static void free_out_all(kernix_model* m)
{
    if (m->out_all == NULL) return;
    if (m->dev && m->dev->out_all_pinned) knx_hip_host_free(m->out_all->tensor);
    else free(m->out_all->tensor);
    free(m->out_all);
    m->out_all = NULL;
    if (m->dev) m->dev->out_all_pinned = 0;
}

/* Every call on a model runs on the model's device (the one current at its first forward), whatever device the
 * calling thread has current; the thread's own device is restored on return.  prev: the device to restore, or -1. */
static int enter_device(const kernix_model* m, int* prev)
{
    *prev = -1;
    int cur = -1;
    if (m == NULL || m->dev == NULL) return 0;
    if (knx_hip_get_device(&cur) != KNX_OK) return -1;
    if (cur == m->dev->device) return 0;
    if (knx_hip_set_device(m->dev->device) != KNX_OK) return -1;
    *prev = cur;
    return 0;
}

static void leave_device(int prev)
{
    if (prev >= 0) knx_hip_set_device(prev);
}

static void release_ws(kernix_model* m);

/* Releases the workspace (arena, views, host output buffers); weights stay on the device. */
void knx_model_release_device_ws(kernix_model* m)
{
    int prev;
    if (m == NULL || enter_device(m, &prev) != 0) return;
    release_ws(m);
    leave_device(prev);
}

static void release_ws(kernix_model* m)
{
    if (m == NULL) return;
    m->batch = -1;
    if (m->dev != NULL) {
        if (m->dev->stream) knx_hip_stream_sync(m->dev->stream);
        if (m->dev->done_recorded) knx_hip_event_sync(m->dev->done); /* a forward on a caller's stream */
        knx_hip_free(m->dev->arena);
        m->dev->arena = NULL;
        m->dev->arena_bytes = 0;
        m->dev->d_in = NULL;
        m->dev->chain = NULL;
        m->dev->chain_bytes = 0;
        knx_hip_host_free(m->dev->h_out);
        m->dev->h_out = NULL;
        m->dev->h_out_floats = 0;
        knx_hip_free(m->dev->cf_in);
        m->dev->cf_in = NULL;
        m->dev->cf_in_floats = 0;
    }
    free_out_all(m);
    free_views(m);
    m->out_view = (float_tensor){ 0, m->out_dim, NULL };
}

void knx_model_release_device_all(kernix_model* m)
{
    int prev;
    if (m == NULL || enter_device(m, &prev) != 0) return;
    release_ws(m);
    for (int i = 0; m->steps != NULL && i < m->n_steps; i++) free_dstep(&m->steps[i]);
    if (m->dev != NULL) {
        knx_hip_stream_destroy(m->dev->stream);
        knx_hip_event_destroy(m->dev->done);
        knx_hip_stream_destroy(m->dev->copy_stream);
        for (int h = 0; h < 2; h++) {
            knx_hip_event_destroy(m->dev->ev_in[h]);
            knx_hip_event_destroy(m->dev->ev_used[h]);
        }
        for (int k = 0; k < KNX_RING_SLOTS; k++) {
            if (m->dev->ring_ev[k]) knx_hip_event_sync(m->dev->ring_ev[k]);
            knx_hip_event_destroy(m->dev->ring_ev[k]);
            knx_hip_host_free(m->dev->ring[k]);
        }
        knx_hip_host_free(m->dev->stage); /* release_ws has synchronized the model's stream */
        knx_hip_host_free(m->dev->chain_status);
        free(m->dev);
        m->dev = NULL;
    }
    leave_device(prev);
}

void kernix_model_trim(kernix_model* m) { knx_model_release_device_ws(m); }

/* Allocates the workspace for chunks of `rows` input rows (the old one is released first). */
static int alloc_ws(kernix_model* m, int rows)
{
    release_ws(m);
    const size_t B = (size_t)rows / (size_t)m->seq_len;
    ws_ctx c = { WS_SIZE, 0, NULL, 0 };
    if (ws_walk(m, B, &c) != 0) return -1;
    const size_t bytes = c.off;
    void* arena = NULL;
    if (hip_ok(knx_hip_malloc(&arena, bytes), "workspace allocation") != 0) return -1;
    m->dev->arena = arena;
    m->dev->arena_bytes = bytes;
    ws_ctx a = { WS_ALLOC, 0, arena, 0 };
    if (ws_walk(m, B, &a) != 0) { knx_model_release_device_ws(m); return -1; }
    /* the chain's barrier words start at zero (every launch leaves them so) */
    if (m->dev->chain && hip_ok(knx_hip_memset(m->dev->chain, 0, KNX_ALIGN, m->dev->stream), "workspace set-up") != 0) {
        knx_model_release_device_ws(m);
        return -1;
    }
    /* the fp32 copies of the int8 weights, computed on the device from the uploaded int8 weights */
    for (int i = 0; i < m->n_steps; i++) {
        kernix_step* s = &m->steps[i];
        if (s->deq && hip_ok(knx_hip_dequant_t(s->dev->q, s->q->kp, s->dev->qscale, s->q->k, s->q->n, s->deq->tensor, m->dev->stream), "dequantization") != 0) {
            knx_model_release_device_ws(m);
            return -1;
        }
        if (s->deq_b && hip_ok(knx_hip_dequant_t(s->dev->q_b, s->q_b->kp, s->dev->qscale_b, s->q_b->k, s->q_b->n, s->deq_b->tensor, m->dev->stream), "dequantization") != 0) {
            knx_model_release_device_ws(m);
            return -1;
        }
    }
    m->batch = rows;
    return 0;
}

static void ws_view(kernix_model* m, int rows)
{
    ws_ctx c = { WS_VIEW, 0, NULL, 0 };
    ws_walk(m, (size_t)rows / (size_t)m->seq_len, &c);
}

/* ---------------------------------------------------------------- steps */
static void hw(const kernix_val* v, int* H, int* W)
{
    *H = v->d[0];
    *W = v->nd == 3 ? v->d[1] : 1;
}

/* y (rows × n) = act(x·Wtᵀ + bias) [+ res]: the fp32 Linear, with a following elementwise add fused when res is set. */
static int fp32_linear(int rows, int n, int k, const float* x, const float* wt, const float* bias, int act, float alpha,
                       const float* res, float* y, void* st)
{
    if (res != NULL)
        return hip_ok(knx_hip_sgemm_nt_ep_res(rows, n, k, x, k, wt, k, bias, act, alpha, res, n, y, n, st), "fp32 GEMM + add");
    return hip_ok(knx_hip_sgemm_nt_ep(rows, n, k, x, k, wt, k, bias, act, alpha, y, n, st), "fp32 GEMM");
}

/* y (rows × n) = act(x·W + bias) with int8 weights: int8 arithmetic (per-row int8 input, int32 accumulation) or
 * the fp32 copy, per the model's int8 mode; accumulate adds into y (RNN recurrence). */
static int run_qlinear(const kernix_model* m, const kernix_qweight* q, const int8_t* dq, const float* dscale,
                       const float_tensor* deq, int8_t* xq, float* sx, int xq_rows, const float* x, int rows,
                       const float* bias, int act, float alpha, int accumulate, const float* res, float* y, void* st)
{
    const int use_i8 = m->int8_mode == KERNIX_INT8_I8 || rows <= KERNIX_INT8_MAX_ROWS;
    if (use_i8) {
        if (rows > xq_rows || xq == NULL) { KNX_LOG("KERNIX: int8 scratch too small (%d > %d rows)\n", rows, xq_rows); return -1; }
        return hip_ok(knx_hip_qlinear(x, q->k, rows, q->k, q->kp, xq, sx, dq, q->kp, q->n, dscale, bias, act, alpha,
                                      accumulate, res, q->n, y, q->n, st), res ? "int8 GEMM + add" : "int8 GEMM");
    }
    if (deq == NULL) { KNX_LOG("KERNIX: missing fp32 copy of an int8 weight\n"); return -1; }
    if (accumulate) return -1; /* the recurrence adds through a separate buffer on this path */
    return fp32_linear(rows, q->n, q->k, x, deq->tensor, bias, act, alpha, res, y, st);
}

/* KNX_RNN_PERSISTENT=0: every timestep as its own launches (tests); also off while a host forward recomputes one
 * whose grid-barrier launch gave up */
static int rnn_persistent(const kernix_model* m)
{
    const char* e = getenv("KNX_RNN_PERSISTENT");
    return m->dev->chain != NULL && !m->dev->no_chain && (e == NULL || *e != '0');
}

/* The LINEAR step that reads only an RNN's last state, run at the end of the recurrence's launch (rnn_dense_fusable):
 * its weight in the form its own step would use (int8 q with its scales, or fp32 w: n rows of k floats). */
struct rnn_dense {
    const float* w;
    const int8_t* q;
    int kp;
    const float* qscale;
    const float* bias;
    int n, act;
    float alpha;
    float* y;
};

/* One direction of an RNN, reference include/kernix_model.h:563-632: the input projection of all timesteps is one
 * GEMM; then the timesteps in one launch (knx_hip_rnn_recurrence) where the shape fits it, else per timestep h·U
 * (int8 or fp32) and the gates as launches of their own.  With `dense` the LINEAR after it runs in the same launch
 * (knx_hip_rnn_recurrence_dense; rnn_dense_fusable has checked that it fits). */
static int run_rnn_dir(const kernix_model* m, kernix_step* s, int dir, const float_tensor* x, float* dst, int stride, void* st,
                       const struct rnn_dense* dense)
{
    struct knx_dstep* d = s->dev;
    const int kind = s->kind, T = s->seq, u = s->out, gu = (int)gates(kind) * u;
    const int B = x->row / T;
    if (B == 0) return 0;
    const float* W = dir ? d->w_b : d->w;
    const float* bias = dir ? d->bias_b : d->bias;
    const float* brec = kind == KERNIX_OP_GRU ? bias + gu : NULL;
    const kernix_qweight* q = dir ? s->q_b : s->q;
    const int8_t* dq = dir ? d->q_b : d->q;
    const float* dsc = dir ? d->qscale_b : d->qscale;
    const float_tensor* deq = dir ? s->deq_b : s->deq;
    const float* U = q != NULL ? (deq ? deq->tensor : NULL) : (dir ? d->rec_b : d->rec);
    float* zx = s->tmp[0]->tensor;
    float* z = s->tmp[1]->tensor;
    float* c = kind == KERNIX_OP_LSTM ? s->tmp[2]->tensor : NULL;
    float* h = s->tmp[3]->tensor;
    float* hu = s->tmp[4]->tensor;
    /* both directions use the step's one int8 scratch (xq_rows rows): they run one after the other on one stream */
    int8_t* xq = d->xq;
    float* sx = d->sx;
    if (hip_ok(knx_hip_sgemm_nt_ep(x->row, gu, s->in, x->tensor, s->in, W, s->in, bias, -1, 0.0f, zx, gu, st), "RNN input projection"))
        return -1;
    const int i8 = q != NULL && (m->int8_mode == KERNIX_INT8_I8 || B <= KERNIX_INT8_MAX_ROWS);
    if (dense != NULL) {
        if (!i8 && U == NULL) return -1;
        return hip_ok(knx_hip_rnn_recurrence_dense(kind, s->act, s->alpha, B, T, u, dir, zx, i8 ? NULL : U, q != NULL,
                                                   i8 ? dq : NULL, q != NULL ? q->kp : 0, dsc, brec, dst, stride, dense->w,
                                                   dense->q, dense->kp, dense->qscale, dense->bias, dense->n, dense->act,
                                                   dense->alpha, dense->y, st),
                      "RNN recurrence + Linear");
    }
    if (rnn_persistent(m) && knx_hip_rnn_recurrence_fits(kind, B, u, i8)) {
        /* every timestep in one launch; h alternates between h and the recurrent-term buffer (B rows of u4 each) */
        if (!i8 && U == NULL) return -1;
        return hip_ok(knx_hip_rnn_recurrence(kind, s->act, s->alpha, B, T, u, dir, zx, i8 ? NULL : U, q != NULL,
                                             i8 ? dq : NULL, q != NULL ? q->kp : 0, dsc, brec, h, hu, dst, stride,
                                             s->ret_seq, m->dev->chain, m->dev->chain_bytes, m->dev->chain_status, st),
                      "RNN recurrence");
    }
    for (int step = 0; step < T; step++) {
        const int t = dir ? T - 1 - step : step;
        if (hip_ok(knx_hip_copy_cols(zx + (size_t)t * gu, T * gu, 0, z, gu, 0, B, gu, st), "RNN gate copy")) return -1;
        const float* rec_term = NULL;
        if (step == 0) {
            if (kind == KERNIX_OP_GRU) { /* h = 0: the recurrent term is the recurrent bias */
                if (hip_ok(knx_hip_sgemm_ep(B, gu, 0, NULL, 0, NULL, gu, brec, -1, 0.0f, hu, gu, st), "RNN bias")) return -1;
                rec_term = hu;
            }
        } else if (i8) {
            float* target = kind == KERNIX_OP_GRU ? hu : z;
            if (run_qlinear(m, q, dq, dsc, NULL, xq, sx, d->xq_rows, h, B, brec, -1, 0.0f, kind != KERNIX_OP_GRU, NULL, target, st)) return -1;
            rec_term = kind == KERNIX_OP_GRU ? hu : NULL;
        } else {
            if (U == NULL) return -1;
            /* the fp32 copy of an int8 U is stored transposed (gu × u); a float U is u × gu as in the file */
            const int rc = q != NULL ? knx_hip_sgemm_nt_ep(B, gu, u, h, u, U, u, brec, -1, 0.0f, hu, gu, st)
                                     : knx_hip_sgemm_ep(B, gu, u, h, u, U, gu, brec, -1, 0.0f, hu, gu, st);
            if (hip_ok(rc, "RNN recurrence")) return -1;
            rec_term = hu;
        }
        float* out_t = s->ret_seq ? dst + (size_t)t * stride : NULL;
        if (hip_ok(knx_hip_rnn_gates(kind, s->act, s->alpha, B, u, step == 0, z, rec_term, c, h, out_t, T * stride, st), "RNN gates")) return -1;
    }
    if (!s->ret_seq && hip_ok(knx_hip_copy_cols(h, u, 0, dst, stride, 0, B, u, st), "RNN output")) return -1;
    return 0;
}

static int run_rnn(const kernix_model* m, kernix_step* s, const float_tensor* x, float_tensor* y, void* st)
{
    const int u = s->out;
    if (s->dirs == 1) return run_rnn_dir(m, s, 0, x, y->tensor, u, st, NULL);
    if (s->merge == KERNIX_MERGE_CONCAT)
        return run_rnn_dir(m, s, 0, x, y->tensor, 2 * u, st, NULL) || run_rnn_dir(m, s, 1, x, y->tensor + u, 2 * u, st, NULL)
                   ? -1 : 0;
    float* bw = s->tmp[5]->tensor;
    if (run_rnn_dir(m, s, 0, x, y->tensor, u, st, NULL) || run_rnn_dir(m, s, 1, x, bw, u, st, NULL)) return -1;
    const int rows = y->row;
    if (hip_ok(knx_hip_binary(s->merge == KERNIX_MERGE_MUL ? KERNIX_BIN_MUL : KERNIX_BIN_ADD, y->tensor, rows, u, bw, rows, u,
                              y->tensor, 1, rows, u, st), "RNN merge")) return -1;
    if (s->merge == KERNIX_MERGE_AVE && hip_ok(knx_hip_affine(y->tensor, y->tensor, rows, u, s->dev->half, s->dev->zero, st), "RNN merge"))
        return -1;
    return 0;
}

/* Step i into y (its own output value, or with `res` set the output of the BINARY add that follows it: then the
 * step's epilogue adds res, see fusable_add). */
static int run_step(kernix_model* m, int i, int B, void* st, float_tensor* y_into, const float* res)
{
    kernix_step* s = &m->steps[i];
    struct knx_dstep* d = s->dev;
    const float_tensor* a = &m->views[s->inp[0]];
    float_tensor* y = y_into != NULL ? y_into : &m->views[i + 1];
    const kernix_val* vi = &m->vals[s->inp[0]];
    const kernix_val* vo = &m->vals[i + 1];
    const int rows = y->row, cols = y->col;
    switch (s->kind) {
    case KERNIX_OP_LINEAR:
        if (s->q != NULL)
            return run_qlinear(m, s->q, d->q, d->qscale, s->deq, d->xq, d->sx, d->xq_rows, a->tensor, a->row, d->bias,
                               s->act, s->alpha, 0, res, y->tensor, st);
        return fp32_linear(a->row, s->out, s->in, a->tensor, d->w, d->bias, s->act, s->alpha, res, y->tensor, st);
    case KERNIX_OP_ACT:
        return hip_ok(knx_hip_bias_act(a->tensor, y->tensor, rows, cols, NULL, s->act, s->alpha, st), "activation");
    case KERNIX_OP_LAYERNORM:
        return hip_ok(knx_hip_layernorm(a->tensor, y->tensor, rows, cols, d->gamma, d->beta, s->eps, st), "layer_norm");
    case KERNIX_OP_SOFTMAX:
        return hip_ok(knx_hip_softmax(a->tensor, y->tensor, rows, cols, st), "softmax");
    case KERNIX_OP_LSTM:
    case KERNIX_OP_GRU:
    case KERNIX_OP_RNN:
        return run_rnn(m, s, a, y, st);
    case KERNIX_OP_CONV: {
        if (knx_conv_is_gemm(s) == 0) /* 1×1 stride 1: a GEMM on the NHWC rows */
            return fp32_linear(a->row, s->out, s->in, a->tensor, d->w, d->bias, s->act, s->alpha, res, y->tensor, st);
        knx_conv_geom g;
        hw(vi, &g.H, &g.W);
        hw(vo, &g.Ho, &g.Wo);
        g.B = a->row / (g.H * g.W);
        g.C = vi->c; g.Co = vo->c;
        g.kh = s->kh; g.kw = s->kw; g.sh = s->sh; g.sw = s->sw; g.dh = s->dh; g.dw = s->dw; g.pt = s->pt; g.pl = s->pl;
        g.groups = s->groups;
        if (res != NULL)
            return hip_ok(knx_hip_conv_t_res(&g, a->tensor, d->w, d->bias, s->act, s->alpha, res, y->tensor, st),
                          "convolution + add");
        return hip_ok(knx_hip_conv_t(&g, a->tensor, d->w, d->bias, s->act, s->alpha, y->tensor, st), "convolution");
    }
    case KERNIX_OP_POOL: {
        knx_conv_geom g;
        memset(&g, 0, sizeof g);
        hw(vi, &g.H, &g.W);
        hw(vo, &g.Ho, &g.Wo);
        g.C = vi->c; g.Co = vi->c;
        g.B = a->row / (g.H * g.W);
        g.kh = s->kh; g.kw = s->kw; g.sh = s->sh; g.sw = s->sw; g.pt = s->pt; g.pl = s->pl; g.dh = g.dw = 1; g.groups = 1;
        return hip_ok(knx_hip_pool(s->ptype, &g, s->count_pad, a->tensor, y->tensor, st), "pooling");
    }
    case KERNIX_OP_GLOBAL_POOL:
        return hip_ok(knx_hip_global_pool(s->ptype, a->tensor, a->row / vi->r, vi->r, vi->c, y->tensor, st), "global pooling");
    case KERNIX_OP_RESHAPE:
        return 0;
    case KERNIX_OP_PERMUTE:
        return hip_ok(knx_hip_permute(a->tensor, y->tensor, B, vi->nd, vi->d, s->perm, st), "permute");
    case KERNIX_OP_BINARY: {
        const kernix_val* vb = &m->vals[s->inp[1]];
        return hip_ok(knx_hip_binary(s->bop, a->tensor, vi->r, vi->c, m->views[s->inp[1]].tensor, vb->r, vb->c, y->tensor,
                                     B, vo->r, vo->c, st), "binary op");
    }
    case KERNIX_OP_CONCAT: {
        const size_t R = (size_t)vo->r, C = (size_t)vo->c, per = R * C;
        int off = 0;
        for (int k = 0; k < s->n_in; k++) {
            const kernix_val* v = &m->vals[s->inp[k]];
            const float* src = m->views[s->inp[k]].tensor;
            if (s->axis == KERNIX_AXIS_LAST) {
                if (hip_ok(knx_hip_copy_cols(src, v->c, 0, y->tensor, (int)C, off, B * (int)R, v->c, st), "concatenate")) return -1;
                off += v->c;
            } else {
                const int pk = v->r * v->c;
                if (hip_ok(knx_hip_copy_cols(src, pk, 0, y->tensor, (int)per, off, B, pk, st), "concatenate")) return -1;
                off += pk;
            }
        }
        return 0;
    }
    case KERNIX_OP_EMBEDDING:
        return hip_ok(knx_hip_embedding(a->tensor, a->row * a->col, d->w, s->in, s->out, y->tensor, st), "embedding");
    case KERNIX_OP_AFFINE:
        return hip_ok(knx_hip_affine(a->tensor, y->tensor, rows, cols, d->gamma, d->beta, st), "affine");
    case KERNIX_OP_ADD_CONST:
        return hip_ok(knx_hip_add_const(a->tensor, y->tensor, B, s->in, d->cst, st), "add_const");
    case KERNIX_OP_ATTENTION: {
        const int iv = s->inp[s->n_in > 1 ? 1 : 0], ik = s->inp[s->n_in > 2 ? 2 : s->n_in > 1 ? 1 : 0];
        const float_tensor* vq = a;
        const float_tensor* vv = &m->views[iv];
        const float_tensor* vk = &m->views[ik];
        const int Rq = vi->r, S = m->vals[iv].r, H = s->heads, hk = H * s->dk, hv = H * s->dv;
        if (B == 0) return 0;
        float* ctx = s->tmp[4]->tensor;
        float *Q, *K, *V;
        int ldq = hk, ldk = hk, ldv = hv;
        if (d->wqkv) {
            const int n = 2 * hk + hv;
            Q = s->tmp[0]->tensor;
            K = Q + hk;
            V = Q + 2 * hk;
            ldq = ldk = ldv = n;
            if (hip_ok(knx_hip_sgemm_nt_ep(vq->row, n, vq->col, vq->tensor, vq->col, d->wqkv, vq->col, d->bqkv, -1, 0.0f, Q, n, st), "attention QKV"))
                return -1;
        } else {
            Q = s->tmp[0]->tensor;
            K = s->tmp[1]->tensor;
            V = s->tmp[2]->tensor;
            if (hip_ok(knx_hip_sgemm_nt_ep(vq->row, hk, vq->col, vq->tensor, vq->col, d->w, vq->col, d->bias, -1, 0.0f, Q, hk, st), "attention Q") ||
                hip_ok(knx_hip_sgemm_nt_ep(vk->row, hk, vk->col, vk->tensor, vk->col, d->wk, vk->col, d->bk, -1, 0.0f, K, hk, st), "attention K") ||
                hip_ok(knx_hip_sgemm_nt_ep(vv->row, hv, vv->col, vv->tensor, vv->col, d->wv, vv->col, d->bv, -1, 0.0f, V, hv, st), "attention V"))
                return -1;
        }
        if (hip_ok(knx_hip_attention_core_ex(Q, ldq, K, ldk, V, ldv, s->tmp[5]->tensor, ctx, s->tmp[3]->tensor, B, H, Rq, S,
                                             s->dk, s->dv, 1.0f / sqrtf((float)s->dk), s->causal, st), "attention"))
            return -1;
        return fp32_linear(vq->row, s->out, hv, ctx, d->wo, d->bo, -1, 0.0f, res, y->tensor, st);
    }
    case KERNIX_OP_SELECT: {
        const int per = vi->r * vi->c;
        if (s->axis == KERNIX_AXIS_FIRST) {
            const int blk = per / vi->d[0], n = blk * s->len;
            return hip_ok(knx_hip_copy_cols(a->tensor, per, s->start * blk, y->tensor, n, 0, B, n, st), "select");
        }
        return hip_ok(knx_hip_copy_cols(a->tensor, vi->c, s->start, y->tensor, s->len, 0, B * vi->r, s->len, st), "select");
    }
    case KERNIX_OP_PAD: {
        int H, W, Ho, Wo;
        hw(vi, &H, &W);
        hw(vo, &Ho, &Wo);
        return hip_ok(knx_hip_pad(a->tensor, y->tensor, a->row / (H * W), H, W, vi->c, Ho, Wo, s->pt, s->pl, st), "pad");
    }
    case KERNIX_OP_UPSAMPLE: {
        int H, W;
        hw(vi, &H, &W);
        return hip_ok(knx_hip_upsample(a->tensor, y->tensor, a->row / (H * W), H, W, vi->c, s->sh, s->sw, st), "upsample");
    }
    default:
        return -1;
    }
}

/* The value the BINARY add after step i adds to step i's output, when the two can run as one pass (else −1): step i
 * is a Linear, a convolution or an attention (whose last operation is the output projection), step i+1 adds its
 * output and one other value of the same shape (no broadcast), nothing else reads step i's output, and the add's
 * output storage is not one that step i reads (the fused epilogue writes it while step i still reads its inputs).
 * The fused epilogue computes act(step i) and then adds the other value, the two fp32 roundings of the separate
 * steps (reference include/kernix_model.h:1853-1860 then :877-906), so the result is the same bit for bit. */
static int fusable_add(const kernix_model* m, int i)
{
    if (i + 1 >= m->n_steps) return -1;
    const kernix_step* s = &m->steps[i];
    const kernix_step* n = &m->steps[i + 1];
    if (s->kind != KERNIX_OP_LINEAR && s->kind != KERNIX_OP_CONV && s->kind != KERNIX_OP_ATTENTION) return -1;
    /* the GEMM epilogues load the residual ahead of their stores only after no activation or ReLU (the producers of
     * residual adds in practice); after another activation the add stays a step of its own */
    if (s->kind != KERNIX_OP_ATTENTION && s->act != KERNIX_ACT_NONE && s->act != KERNIX_ACT_RELU) return -1;
    if (n->kind != KERNIX_OP_BINARY || n->bop != KERNIX_BIN_ADD || n->n_in != 2) return -1;
    const int own = i + 1; /* value index of step i's output */
    if ((n->inp[0] == own) == (n->inp[1] == own)) return -1;
    const int other = n->inp[0] == own ? n->inp[1] : n->inp[0];
    const kernix_val* vo = &m->vals[own];
    const kernix_val* vr = &m->vals[other];
    const kernix_val* vy = &m->vals[i + 2];
    if (vo->last != i + 1 || m->out_v == own) return -1;
    if (vr->r != vo->r || vr->c != vo->c || vy->r != vo->r || vy->c != vo->c) return -1;
    for (int k = 0; k < s->n_in; k++)
        if (knx_storage_overlaps(m, s->inp[k], i + 2)) return -1;
    return other;
}

/* An RNN step i (one direction, its last state only) whose output is read only by step i + 1, a LINEAR (and not by a
 * fused add after it): the LINEAR runs at the end of the recurrence's launch on the last state still in LDS, with the
 * arithmetic its own step would have (run_qlinear: int8 in i8 mode or at <= KERNIX_INT8_MAX_ROWS rows, the same bits;
 * else fp32 on the fp32 or dequantized weight) — one launch and one round trip through memory less. */
static int rnn_dense_fusable(const kernix_model* m, int i)
{
    if (i + 1 >= m->n_steps) return 0;
    const kernix_step* s = &m->steps[i];
    const kernix_step* n = &m->steps[i + 1];
    if (s->kind != KERNIX_OP_LSTM && s->kind != KERNIX_OP_GRU && s->kind != KERNIX_OP_RNN) return 0;
    if (s->dirs != 1 || s->ret_seq || n->kind != KERNIX_OP_LINEAR || n->n_in != 1 || n->inp[0] != i + 1) return 0;
    const kernix_val* v = &m->vals[i + 1];
    if (v->last != i + 1 || m->out_v == i + 1 || fusable_add(m, i + 1) >= 0) return 0;
    /* the launch writes both outputs (the step temporaries it reads are outside the value storage) */
    if (!rnn_persistent(m) || n->in != s->out || knx_storage_overlaps(m, i + 1, i + 2)) return 0;
    const int B = m->views[s->inp[0]].row / s->seq;
    if (B <= 0) return 0;
    const int rec_i8 = s->q != NULL && (m->int8_mode == KERNIX_INT8_I8 || B <= KERNIX_INT8_MAX_ROWS);
    const int lin_i8 = n->q != NULL && (m->int8_mode == KERNIX_INT8_I8 || B <= KERNIX_INT8_MAX_ROWS);
    if (n->q != NULL && !lin_i8 && n->deq == NULL) return 0;
    return knx_hip_rnn_recurrence_dense_fits(s->kind, B, s->out, rec_i8, n->out);
}

/* Runs RNN step i with the LINEAR step i + 1 (see rnn_dense_fusable). */
static int run_rnn_dense(kernix_model* m, int i, void* st)
{
    kernix_step* s = &m->steps[i];
    const kernix_step* n = &m->steps[i + 1];
    const struct knx_dstep* d = n->dev;
    const float_tensor* x = &m->views[s->inp[0]];
    const int B = x->row / s->seq;
    const int lin_i8 = n->q != NULL && (m->int8_mode == KERNIX_INT8_I8 || B <= KERNIX_INT8_MAX_ROWS);
    struct rnn_dense dn;
    dn.w = lin_i8 ? NULL : n->q != NULL ? n->deq->tensor : d->w;
    dn.q = lin_i8 ? d->q : NULL;
    dn.kp = lin_i8 ? n->q->kp : 0;
    dn.qscale = lin_i8 ? d->qscale : NULL;
    dn.bias = d->bias;
    dn.n = n->out;
    dn.act = n->act;
    dn.alpha = n->alpha;
    dn.y = m->views[i + 2].tensor;
    return run_rnn_dir(m, s, 0, x, m->views[i + 1].tensor, s->out, st, &dn);
}

/* LAYERNORM step i whose output is read only by step i + 1, an int8 LINEAR that runs int8 arithmetic at more than 4
 * rows (i8 mode) and so quantizes its input rows anyway: both run as knx_hip_layernorm_quantize into the LINEAR's
 * int8 scratch and the int8 GEMM, and the fp32 LAYERNORM output is never written.  The normalized rows are computed
 * by the same vector kernel as the separate layer_norm (cols % 4 == 0, ≤ 2048, 16-byte aligned), so the int8 rows,
 * their scales and the outputs are the same bits. */
static int ln_quant_fusable(const kernix_model* m, int i)
{
    if (i + 1 >= m->n_steps) return 0;
    const kernix_step* s = &m->steps[i];
    const kernix_step* n = &m->steps[i + 1];
    if (s->kind != KERNIX_OP_LAYERNORM || n->kind != KERNIX_OP_LINEAR || n->q == NULL) return 0;
    if (n->n_in != 1 || n->inp[0] != i + 1) return 0;
    const kernix_val* v = &m->vals[i + 1];
    if (v->last != i + 1 || m->out_v == i + 1) return 0;
    const float_tensor* a = &m->views[s->inp[0]];
    const struct knx_dstep* dl = s->dev;
    const struct knx_dstep* d = n->dev;
    if (m->int8_mode != KERNIX_INT8_I8 || a->row <= 4 || d->xq == NULL || a->row > d->xq_rows) return 0;
    if (a->col % 4 != 0 || a->col > 2048 || a->col != n->q->k) return 0;
    return (((uintptr_t)a->tensor | (uintptr_t)dl->gamma | (uintptr_t)dl->beta) & 15) == 0;
}

/* Runs LAYERNORM step i with the int8 LINEAR step i + 1 (see ln_quant_fusable), and the BINARY add after the LINEAR
 * when fusable_add allows.  Returns the number of steps run, or -1. */
static int run_ln_quant(kernix_model* m, int i, int fuse, void* st)
{
    const kernix_step* ln = &m->steps[i];
    const kernix_step* s = &m->steps[i + 1];
    const struct knx_dstep* dl = ln->dev;
    const struct knx_dstep* d = s->dev;
    const kernix_qweight* q = s->q;
    const float_tensor* a = &m->views[ln->inp[0]];
    if (hip_ok(knx_hip_layernorm_quantize(a->tensor, a->row, a->col, dl->gamma, dl->beta, ln->eps, q->kp, d->xq, d->sx,
                                          st), "layer_norm + quantize"))
        return -1;
    const int r = fuse ? fusable_add(m, i + 1) : -1;
    if (r >= 0) {
        if (hip_ok(knx_hip_i8gemm_res(a->row, q->n, q->kp, d->xq, q->kp, d->sx, d->q, q->kp, d->qscale, d->bias, s->act,
                                      s->alpha, m->views[r].tensor, q->n, m->views[i + 3].tensor, q->n, st),
                   "int8 GEMM + add"))
            return -1;
        return 3;
    }
    if (hip_ok(knx_hip_i8gemm(a->row, q->n, q->kp, d->xq, q->kp, d->sx, d->q, q->kp, d->qscale, d->bias, s->act, s->alpha,
                              0, m->views[i + 2].tensor, q->n, NULL, 0, st), "int8 GEMM"))
        return -1;
    return 2;
}

/* ---------------------------------------------------------------- Linear chains
 * Consecutive LINEAR steps over at most 64 rows run as one knx_hip_linear_chain launch instead of one or two
 * launches each (reference include/kernix_model.h:1843-1860 step after step): step j > i reads only step j − 1's
 * output, which no other step reads and which is not the model's output.  Each step keeps the arithmetic its own
 * launch would have: int8 (knx_hip_qlinear's bits) where run_qlinear would use int8, else fp32 on the fp32 or
 * dequantized weight.  A step whose output feeds a fused add (fusable_add) ends the run before it. */
static int chain_enabled(void)
{
    const char* e = getenv("KNX_CHAIN");
    return e == NULL || *e != '0';
}

static int chain_layer(const kernix_model* m, int j, int rows, knx_chain_layer* c)
{
    const kernix_step* s = &m->steps[j];
    const struct knx_dstep* d = s->dev;
    if (s->kind != KERNIX_OP_LINEAR || s->n_in != 1 || s->in % 4 != 0) return -1;
    memset(c, 0, sizeof *c);
    c->bias = d->bias;
    c->y = m->views[j + 1].tensor;
    c->k = s->in;
    c->n = s->out;
    c->ldy = s->out;
    c->act = s->act;
    c->alpha = s->alpha;
    if (s->q != NULL && (m->int8_mode == KERNIX_INT8_I8 || rows <= KERNIX_INT8_MAX_ROWS)) {
        if (s->q->kp > 2048) return -1; /* an int8 layer's rows must fit one pass of the chain's loads */
        c->i8 = 1;
        c->w = d->q;
        c->sw = d->qscale;
        c->kp = s->q->kp;
        c->ldw = s->q->kp;
        return 0;
    }
    c->w = s->q != NULL ? (s->deq != NULL ? s->deq->tensor : NULL) : d->w;
    c->kp = c->ldw = s->in;
    return c->w != NULL ? 0 : -1;
}

/* Number of steps from i that run as one chain (≥ 2), their layers in c; 0 if none. */
static int chain_len(const kernix_model* m, int i, int fuse, knx_chain_layer* c)
{
    const kernix_step* s0 = &m->steps[i];
    if (s0->kind != KERNIX_OP_LINEAR || s0->n_in != 1 || m->dev->chain == NULL) return 0;
    const float_tensor* x = &m->views[s0->inp[0]];
    const int rows = x->row;
    if (rows < 1 || rows > 64 || ((uintptr_t)x->tensor & 15) != 0) return 0;
    int n = 0;
    for (int j = i; j < m->n_steps && n < KNX_CHAIN_MAX_LAYERS; j++) {
        const kernix_step* s = &m->steps[j];
        const int v = s->inp[0]; /* value read by step j */
        if (j > i && (s->kind != KERNIX_OP_LINEAR || s->n_in != 1 || v != j || m->vals[v].last != j || m->out_v == v ||
                      ((uintptr_t)m->views[v].tensor & 15) != 0))
            break;
        if (knx_storage_overlaps(m, v, j + 1) || (fuse && fusable_add(m, j) >= 0)) break;
        if (chain_layer(m, j, rows, &c[n]) != 0) break;
        /* the output may be the caller's buffer (direct_output): it must not overlap the layer's input either */
        const char* a = (const char*)m->views[v].tensor;
        const char* b = (const char*)c[n].y;
        const size_t na = (size_t)rows * (size_t)c[n].k * sizeof(float), nb = (size_t)rows * (size_t)c[n].n * sizeof(float);
        if (a < b + nb && b < a + na) break;
        n++;
    }
    if (n < 2) return 0;
    /* one launch beats one launch per layer where the layers run int8 arithmetic or the rows are few; fp32 layers
     * over more rows each fill the GPU better on their own (int8 MLP at 64 rows: 15.6 µs as three fp32 launches
     * against 22 µs as a chain; int8: 22.7 against 24.2 µs; one row: 18.6 against 20.2 µs) */
    if (rows > 16)
        for (int l = 0; l < n; l++)
            if (!c[l].i8) return 0;
    const size_t need = knx_hip_linear_chain_scratch(c, n, rows);
    return need != 0 && need <= m->dev->chain_bytes ? n : 0;
}

static int fuse_enabled(void)
{
    const char* nf = getenv("KNX_NO_FUSE");
    return nf == NULL || *nf == '\0' || *nf == '0';
}

/* Enqueues every step for one chunk whose input starts at `in` (device); the output value goes to `out` instead of
 * its storage buffer when out is not NULL (see direct_output). */
static int run_chunk(kernix_model* m, const float* in, int B, float* out, void* st)
{
    for (int v = 0; v < m->n_vals; v++) {
        const kernix_val* val = &m->vals[v];
        m->views[v] = (float_tensor){ B * val->r, val->c, val->st < 0 ? (float*)in : m->st[val->st]->tensor };
    }
    if (out != NULL) m->views[m->out_v].tensor = out;
    if (B == 0) return 0;
    const int fuse = fuse_enabled(), chains = chain_enabled() && !m->dev->no_chain;
    knx_chain_layer cl[KNX_CHAIN_MAX_LAYERS];
    for (int i = 0; i < m->n_steps; i++) {
        const int nc = chains ? chain_len(m, i, fuse, cl) : 0;
        if (nc >= 2) {
            const float_tensor* x = &m->views[m->steps[i].inp[0]];
            if (hip_ok(knx_hip_linear_chain(x->tensor, x->col, x->row, cl, nc, m->dev->chain, m->dev->chain_bytes,
                                            m->dev->chain_status, st),
                       "Linear chain"))
                return -1;
            i += nc - 1;
            continue;
        }
        if (fuse && rnn_dense_fusable(m, i)) {
            if (run_rnn_dense(m, i, st) != 0) return -1;
            i++;
            continue;
        }
        if (fuse && ln_quant_fusable(m, i)) {
            const int c = run_ln_quant(m, i, fuse, st);
            if (c < 0) return -1;
            i += c - 1;
            continue;
        }
        const int r = fuse ? fusable_add(m, i) : -1;
        if (r >= 0) { /* step i and the add that follows it, in one pass */
            if (run_step(m, i, B, st, &m->views[i + 2], m->views[r].tensor) != 0) return -1;
            i++;
        } else if (run_step(m, i, B, st, NULL, NULL) != 0) {
            return -1;
        }
    }
    return 0;
}

/* ---------------------------------------------------------------- ordering between forwards
 * Every forward (host or device buffers, on the model's stream or a caller's) uses the model's one workspace, so
 * forwards run one after the other on the device, in the order they were called.  The model remembers the stream of
 * the last forward.  A forward on the same stream is ordered by the stream itself.  A forward on another stream first
 * makes its stream wait for the event `done`: recorded right after every forward that ran on a caller's stream, and,
 * when the previous forward ran on the model's own stream, recorded on that stream at the switch.  Freeing the
 * workspace waits for the model's stream and for `done` on the host. */
static int order_after_previous(kernix_model* m, void* st)
{
    struct knx_dmodel* d = m->dev;
    if (!d->have_last || d->last_stream == st) return 0;
    if (!d->done_recorded) { /* the previous forward ran on the model's stream (which is still alive: it is ours) */
        if (hip_ok(knx_hip_event_record(d->done, d->last_stream), "event record")) return -1;
        d->done_recorded = 1;
    }
    return hip_ok(knx_hip_stream_wait_event(st, d->done), "stream wait");
}

/* after the last operation of a forward (or of the workspace set-up) enqueued on st */
static int mark_done(kernix_model* m, void* st)
{
    struct knx_dmodel* d = m->dev;
    d->have_last = 1;
    d->last_stream = st;
    d->done_recorded = 0;
    if (st == d->stream) return 0; /* recorded lazily, when another stream comes next */
    if (hip_ok(knx_hip_event_record(d->done, st), "event record")) return -1;
    d->done_recorded = 1;
    return 0;
}

/* ---------------------------------------------------------------- forward
 * A batch of `samples` runs as consecutive pieces of at most `per` samples each, `per` the most the workspace limit
 * holds (ws_fixed + per·ws_per_sample floats ≤ ws_limit bytes; at least one sample; the whole batch when there is no
 * limit).  The workspace is sized for `per` samples and the last, shorter piece uses a prefix of it — the reference's
 * chunking rule (include/kernix_model.h:2036-2062), so m->batch reads the same. */
static int piece_samples(const kernix_model* m, int samples)
{
    if (m->ws_limit == 0 || m->ws_per_sample == 0) return samples;
    const size_t fixed = m->ws_fixed * sizeof(float), each = m->ws_per_sample * sizeof(float);
    const size_t fit = m->ws_limit > fixed ? (m->ws_limit - fixed) / each : 0;
    if (fit >= (size_t)samples) return samples;
    return fit ? (int)fit : 1;
}

/* Device state, weights and a workspace for pieces of `per` samples (reallocated only when `per` changes); the
 * workspace's own setup (dequantized copies) is ordered before the next forward through `done`. */
static int prepare(kernix_model* m, int per)
{
    if (ensure_device(m) != 0) return -1;
    const int rows = per * m->seq_len;
    if (rows == m->batch) return 0;
    if (alloc_ws(m, rows) != 0) return -1;
    return mark_done(m, m->dev->stream);
}

/* The forward's output value can be written by its producing step straight into the caller's device buffer `out`
 * (no copy afterwards): it is not the input or a view of another value (RESHAPE), no RESHAPE makes a view of it, and
 * out does not overlap the input rows x.  Every other step reads and writes the workspace as planned; the producing
 * step then runs out of place where the plan had it in place. */
static int direct_output(const kernix_model* m, const float* x, size_t x_bytes, const float* out, size_t out_bytes)
{
    const int ov = m->out_v;
    if (ov < 1 || m->vals[ov].st < 0 || m->steps[ov - 1].kind == KERNIX_OP_RESHAPE) return 0;
    for (int i = ov; i < m->n_steps; i++)
        if (m->steps[i].kind == KERNIX_OP_RESHAPE && m->steps[i].inp[0] == ov) return 0;
    const char* a = (const char*)x;
    const char* b = (const char*)out;
    return b + out_bytes <= a || a + x_bytes <= b;
}

/* One piece: samples [s0, s0 + n) of the batch, whose input rows start at x (device memory); the output goes to dst
 * (device or pinned host memory, `to_host` says which, holding the whole batch's output) at the piece's rows:
 * written there directly by the last step when direct_output allows, else copied from the workspace. */
static int run_piece(kernix_model* m, const float* x, int s0, int n, float* dst, int to_host, void* st)
{
    const size_t out_row = (size_t)m->out_dim;
    const size_t bytes = (size_t)n * out_row * sizeof(float);
    float* at = dst + (size_t)s0 * out_row;
    const size_t x_bytes = (size_t)n * (size_t)m->seq_len * (size_t)m->in_dim * sizeof(float);
    const int direct = !to_host && direct_output(m, x, x_bytes, at, bytes);
    ws_view(m, n * m->seq_len);
    if (run_chunk(m, x, n, direct ? at : NULL, st) != 0) return -1;
    if (direct) return 0;
    const float* y = m->views[m->out_v].tensor;
    return hip_ok(to_host ? knx_hip_memcpy_d2h(at, y, bytes, st) : knx_hip_memcpy_d2d(at, y, bytes, st), "output copy");
}

/* Pinned host memory for `samples` outputs.  An unchunked forward returns a view of h_out (kept, grown when a
 * larger batch needs more); a chunked one returns out_all, a host tensor of exactly the batch's rows. */
static float* host_output(kernix_model* m, int samples, int chunked)
{
    const size_t floats = (size_t)samples * (size_t)m->out_dim;
    void* p = NULL;
    if (!chunked) {
        if (m->dev->h_out == NULL || m->dev->h_out_floats < floats) {
            knx_hip_host_free(m->dev->h_out);
            m->dev->h_out = NULL;
            m->dev->h_out_floats = 0;
            if (hip_ok(knx_hip_host_malloc(&p, floats * sizeof(float)), "pinned output allocation")) return NULL;
            m->dev->h_out = p;
            m->dev->h_out_floats = floats;
        }
        return m->dev->h_out;
    }
    if (m->out_all != NULL && m->out_all->row == samples) return m->out_all->tensor;
    free_out_all(m);
    float_tensor* t = malloc(sizeof *t);
    if (t == NULL || hip_ok(knx_hip_host_malloc(&p, floats * sizeof(float)), "pinned output allocation")) {
        free(t);
        return NULL;
    }
    *t = (float_tensor){ samples, m->out_dim, p };
    m->out_all = t;
    m->dev->out_all_pinned = 1;
    return p;
}

/* ---------------------------------------------------------------- host-buffer forward: overlapped input copies
 * A batch whose input is large (≥ 32 MB: its copy then takes about as long as the compute) overlaps its input copies
 * with compute.  It runs as sub-pieces of about a quarter of the batch, each at most half a workspace piece, so that
 * the staged device input holds two of them; while piece i computes on the model's stream, piece i + 1 is copied
 * into the other half on a copy stream.  Events order each half: its copy before the compute that reads it, and that
 * compute before the copy two pieces later that overwrites it.  The workspace stays sized for the reference's pieces
 * (m->batch as without overlap); the outputs go to the pinned host buffer piece by piece on the model's stream.
 *
 * The caller's input is pageable memory, which the runtime copies through one staging buffer, host copy and DMA one
 * after the other (≈ 20 GB/s measured for 128 MB), and such a copy did not overlap the compute of the previous piece.
 * These copies go through the model's own ring of four pinned 4 MB buffers instead: the host copies chunk j + 1
 * (split over four threads) into the next slot while the DMA of chunk j runs; a slot is reused once the event
 * recorded after its DMA has completed.  fp32 MLP 8192 × 4096 forward from host buffers: 11.2 ms without overlap,
 * 8.2 ms overlapped with one copying thread, 7.4 ms with four.  Inputs from 1 MB to 32 MB keep the runtime's copy
 * (through the ring they were 0-3% faster, not worth 16 MB of pinned memory per model); smaller ones go through the
 * staging buffer (stage_in). */
#define KNX_RING_BYTES ((size_t)4 << 20)
#define KNX_OVERLAP_MIN_BYTES ((size_t)32 << 20)

/* Host copies into the staging ring: one thread reaches 19–31 GB/s into pinned memory on the MI355X host, four
 * 40–46 GB/s.  A process-wide pool of KNX_COPY_HELPERS threads (started on first use, kept until the process ends)
 * takes equal parts of a copy while the calling thread copies the first part; one copy at a time (a mutex), so
 * concurrent forwards of different models take turns. */
#define KNX_COPY_HELPERS 3

static struct {
    pthread_once_t once;
    int ok;
    pthread_mutex_t run;      /* one copy at a time */
    pthread_mutex_t mu;
    pthread_cond_t go, done;
    char* dst;
    const char* src;
    size_t part, last;        /* bytes per helper part; total bytes */
    unsigned gen;             /* incremented per copy */
    int pending;              /* helper parts not yet finished */
} g_copy = { PTHREAD_ONCE_INIT, 0, PTHREAD_MUTEX_INITIALIZER, PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER,
             PTHREAD_COND_INITIALIZER, NULL, NULL, 0, 0, 0, 0 };

static void* copy_helper(void* arg)
{
    const size_t idx = (size_t)(uintptr_t)arg; /* part idx + 1 of the copy (part 0 is the caller's) */
    unsigned seen = 0;
    for (;;) {
        pthread_mutex_lock(&g_copy.mu);
        while (g_copy.gen == seen) pthread_cond_wait(&g_copy.go, &g_copy.mu);
        seen = g_copy.gen;
        char* dst = g_copy.dst;
        const char* src = g_copy.src;
        const size_t part = g_copy.part, total = g_copy.last;
        pthread_mutex_unlock(&g_copy.mu);
        const size_t off = (idx + 1) * part;
        if (off < total) memcpy(dst + off, src + off, total - off < part ? total - off : part);
        pthread_mutex_lock(&g_copy.mu);
        if (--g_copy.pending == 0) pthread_cond_signal(&g_copy.done);
        pthread_mutex_unlock(&g_copy.mu);
    }
    return NULL;
}

static void copy_pool_start(void)
{
    pthread_attr_t a;
    if (pthread_attr_init(&a) != 0) return;
    pthread_attr_setdetachstate(&a, PTHREAD_CREATE_DETACHED);
    int n = 0;
    for (size_t i = 0; i < KNX_COPY_HELPERS; i++) {
        pthread_t t;
        if (pthread_create(&t, &a, copy_helper, (void*)(uintptr_t)i) == 0) n++;
    }
    pthread_attr_destroy(&a);
    g_copy.ok = n == KNX_COPY_HELPERS;
}

/* memcpy of n bytes split over the caller and the helpers (a plain memcpy if the pool could not start, or for fewer
 * than 256 KB); also the C ABI's copy of a forward's output into the caller's buffer */
void knx_copy_parallel(void* dst, const void* src, size_t n)
{
    pthread_once(&g_copy.once, copy_pool_start);
    if (!g_copy.ok || n < ((size_t)256 << 10)) {
        memcpy(dst, src, n);
        return;
    }
    pthread_mutex_lock(&g_copy.run);
    const size_t part = (n / (KNX_COPY_HELPERS + 1) + 63) & ~(size_t)63;
    pthread_mutex_lock(&g_copy.mu);
    g_copy.dst = dst;
    g_copy.src = src;
    g_copy.part = part;
    g_copy.last = n;
    g_copy.pending = KNX_COPY_HELPERS;
    g_copy.gen++;
    pthread_cond_broadcast(&g_copy.go);
    pthread_mutex_unlock(&g_copy.mu);
    memcpy(dst, src, part < n ? part : n);
    pthread_mutex_lock(&g_copy.mu);
    while (g_copy.pending > 0) pthread_cond_wait(&g_copy.done, &g_copy.mu);
    pthread_mutex_unlock(&g_copy.mu);
    pthread_mutex_unlock(&g_copy.run);
}

static int ring_ready(kernix_model* m)
{
    struct knx_dmodel* d = m->dev;
    for (int k = 0; k < KNX_RING_SLOTS; k++) {
        if (d->ring[k] != NULL) continue;
        if (hip_ok(knx_hip_host_malloc(&d->ring[k], KNX_RING_BYTES), "pinned staging allocation") ||
            hip_ok(knx_hip_event_create(&d->ring_ev[k]), "event creation"))
            return -1;
    }
    return 0;
}

/* bytes from pageable host memory src to device memory dst through the staging ring, enqueued on stream st (returns
 * when the last chunk has been handed to the DMA; the copy is complete in stream order) */
static int copy_in(kernix_model* m, float* dst, const float* src, size_t bytes, void* st)
{
    struct knx_dmodel* d = m->dev;
    if (ring_ready(m) != 0) return -1;
    for (size_t off = 0; off < bytes; off += KNX_RING_BYTES) {
        const size_t n = bytes - off < KNX_RING_BYTES ? bytes - off : KNX_RING_BYTES;
        const int k = d->ring_next;
        d->ring_next = (k + 1) % KNX_RING_SLOTS;
        if (hip_ok(knx_hip_event_sync(d->ring_ev[k]), "staging wait")) return -1; /* slot k's previous DMA is done */
        knx_copy_parallel(d->ring[k], (const char*)src + off, n);
        if (hip_ok(knx_hip_memcpy_h2d((char*)dst + off, d->ring[k], n, st), "input copy") ||
            hip_ok(knx_hip_event_record(d->ring_ev[k], st), "event record"))
            return -1;
    }
    return 0;
}

/* A piece of at most KNX_STAGE_MAX bytes without overlap: the host copies it into the model's pinned staging buffer
 * and a copy kernel on the model's stream reads it from there (pinned host memory is mapped into the device's address
 * space).  The runtime's pageable copy would stage the bytes through its own buffer and hand the transfer to the copy
 * engine, whose completion the first kernel then waits for (larger inputs keep the copy engine, which moves bulk data
 * faster than a kernel reading over PCIe).  A host forward ends with a synchronization of the model's stream, so the
 * buffer is free when the next one starts; only a later piece of the same forward (or a forward that failed after
 * the copy was enqueued) finds stage_pending set and waits for the stream first. */
#define KNX_STAGE_MAX ((size_t)1 << 20)

static int stage_in(kernix_model* m, float* dst, const float* src, size_t bytes, void* st)
{
    struct knx_dmodel* d = m->dev;
    if (d->stage_pending && hip_ok(knx_hip_stream_sync(st), "staging wait")) return -1;
    d->stage_pending = 0;
    if (d->stage_bytes < bytes) {
        knx_hip_host_free(d->stage);
        d->stage = NULL;
        d->stage_bytes = 0;
        const size_t want = (bytes + 65535) / 65536 * 65536;
        if (hip_ok(knx_hip_host_malloc(&d->stage, want), "pinned staging allocation")) return -1;
        d->stage_bytes = want;
    }
    knx_copy_parallel(d->stage, src, bytes);
    const int n = (int)(bytes / sizeof(float));
    if (hip_ok(knx_hip_copy_cols(d->stage, n, 0, dst, n, 0, 1, n, st), "input copy")) return -1;
    d->stage_pending = 1;
    return 0;
}

static int overlap_ready(kernix_model* m)
{
    struct knx_dmodel* d = m->dev;
    if (d->copy_stream != NULL) return 0;
    if (hip_ok(knx_hip_stream_create(&d->copy_stream), "stream creation")) return -1;
    for (int h = 0; h < 2; h++)
        if (hip_ok(knx_hip_event_create(&d->ev_in[h]), "event creation") ||
            hip_ok(knx_hip_event_create(&d->ev_used[h]), "event creation"))
            return -1;
    return 0;
}

/* sub-piece size for an overlapped forward of `samples` in workspace pieces of `per`, or 0 for none */
static int overlap_piece(const kernix_model* m, int samples, int per)
{
    const size_t in_bytes = (size_t)samples * (size_t)m->seq_len * (size_t)m->in_dim * sizeof(float);
    const char* e = getenv("KNX_OVERLAP");
    if ((e != NULL && *e == '0') || in_bytes < KNX_OVERLAP_MIN_BYTES || per < 2 || samples < 4) return 0;
    const int quarter = (samples + 3) / 4;
    return quarter < per / 2 ? quarter : per / 2;
}

static int forward_overlapped(kernix_model* m, const float* x, int samples, int pp, float* out, void* st)
{
    struct knx_dmodel* d = m->dev;
    const size_t in_row = (size_t)m->seq_len * (size_t)m->in_dim;
    if (overlap_ready(m) != 0) return -1;
    /* the copy stream must not start overwriting the staged input before the previous forward is done with it */
    if (hip_ok(knx_hip_event_record(d->ev_used[0], st), "event record") ||
        hip_ok(knx_hip_event_record(d->ev_used[1], st), "event record"))
        return -1;
    for (int s0 = 0, i = 0; s0 < samples; s0 += pp, i++) {
        const int n = samples - s0 < pp ? samples - s0 : pp, h = i & 1;
        float* buf = d->d_in + (size_t)h * (size_t)pp * in_row;
        if (hip_ok(knx_hip_stream_wait_event(d->copy_stream, d->ev_used[h]), "stream wait") ||
            copy_in(m, buf, x + (size_t)s0 * in_row, (size_t)n * in_row * sizeof(float), d->copy_stream) != 0 ||
            hip_ok(knx_hip_event_record(d->ev_in[h], d->copy_stream), "event record") ||
            hip_ok(knx_hip_stream_wait_event(st, d->ev_in[h]), "stream wait") ||
            run_piece(m, buf, s0, n, out, 1, st) != 0 ||
            hip_ok(knx_hip_event_record(d->ev_used[h], st), "event record"))
            return -1;
    }
    return 0;
}

/* A piece of n samples at src (device memory) in channels-first order (per sample C × S: C = in_dim, S = seq_len),
 * transposed into the staged input's channels-last rows (S × C), the order the steps read. */
static int transpose_in(kernix_model* m, const float* src, int n, void* st)
{
    const int d[2] = { m->in_dim, m->seq_len }, perm[2] = { 1, 0 };
    return hip_ok(knx_hip_permute(src, m->dev->d_in, n, 2, d, perm, st), "input transpose");
}

/* cf: the input holds each sample channels-first (the PyTorch layout of a model whose file records layout 1); it is
 * copied as it is and transposed on the device, instead of by the caller on the host. */
static const float_tensor* forward_host(kernix_model* m, const float_tensor* x, int cf)
{
    if (m == NULL || x == NULL || x->tensor == NULL || x->row < 0 || x->col != m->in_dim || x->row % m->seq_len != 0)
        return NULL;
    const int mine = (m->out_all != NULL && x->tensor == m->out_all->tensor) ||
                     (m->dev != NULL && m->dev->h_out != NULL && x->tensor == m->dev->h_out);
    if (mine) {
        KNX_LOG("forward: this model's output buffer cannot be its own input (pass a copy)\n");
        return NULL;
    }
    const int samples = x->row / m->seq_len;
    const int per = piece_samples(m, samples);
    if (prepare(m, per) != 0) return NULL;
    void* st = m->dev->stream;
    const int chunked = per < samples;
    float* out = host_output(m, samples, chunked);
    if (out == NULL || order_after_previous(m, st) != 0) return NULL;
    const size_t in_row = (size_t)m->seq_len * (size_t)m->in_dim;
    cf = cf && m->seq_len > 1; /* one row per sample: both orders are the same */
    if (cf && m->dev->cf_in_floats < (size_t)per * in_row) {
        knx_hip_free(m->dev->cf_in);
        m->dev->cf_in = NULL;
        m->dev->cf_in_floats = 0;
        if (hip_ok(knx_hip_malloc((void**)&m->dev->cf_in, (size_t)per * in_row * sizeof(float)), "input allocation"))
            return NULL;
        m->dev->cf_in_floats = (size_t)per * in_row;
    }
    const int pp = cf ? 0 : overlap_piece(m, samples, per);
    if (pp > 0) {
        if (forward_overlapped(m, x->tensor, samples, pp, out, st) != 0) return NULL;
    } else {
        for (int s0 = 0; s0 < samples; s0 += per) {
            const int n = samples - s0 < per ? samples - s0 : per;
            const float* src = x->tensor + (size_t)s0 * in_row;
            const size_t bytes = (size_t)n * in_row * sizeof(float);
            float* to = cf ? m->dev->cf_in : m->dev->d_in;
            /* the staged input holds one piece: piece s0 is copied to its start (channels-first: transposed there) */
            if ((bytes <= KNX_STAGE_MAX ? stage_in(m, to, src, bytes, st)
                                         : hip_ok(knx_hip_memcpy_h2d(to, src, bytes, st), "input copy")) ||
                (cf && transpose_in(m, to, n, st) != 0) || run_piece(m, m->dev->d_in, s0, n, out, 1, st) != 0)
                return NULL;
        }
    }
    if (mark_done(m, st) != 0 || hip_ok(knx_hip_stream_sync(st), "forward")) return NULL;
    m->dev->stage_pending = 0; /* every copy out of the staging buffer has completed */
    if (chunked) return m->out_all;
    m->out_view = (float_tensor){ samples, m->out_dim, out };
    return &m->out_view;
}

/* A chain launch whose workgroups could not all be resident (its barrier stopped waiting, so its outputs are wrong)
 * is recomputed in the same call: the whole forward again, every Linear its own launch. */
static const float_tensor* forward_host_checked(kernix_model* m, const float_tensor* x, int cf)
{
    int prev;
    if (enter_device(m, &prev) != 0) return NULL;
    const float_tensor* y = forward_host(m, x, cf);
    if (y != NULL && __atomic_exchange_n(m->dev->chain_status, 0, __ATOMIC_SEQ_CST)) {
        KNX_LOG("KERNIX: a Linear chain's workgroups were not all resident; forward recomputed one launch per layer\n");
        m->dev->no_chain = 1;
        y = forward_host(m, x, cf);
        m->dev->no_chain = 0;
        if (y != NULL && __atomic_exchange_n(m->dev->chain_status, 0, __ATOMIC_SEQ_CST)) y = NULL; /* cannot happen */
    }
    leave_device(prev);
    return y;
}

const float_tensor* kernix_model_forward(kernix_model* m, const float_tensor* x)
{
    return forward_host_checked(m, x, 0);
}

const float_tensor* kernix_model_forward_cf(kernix_model* m, const float_tensor* x)
{
    return forward_host_checked(m, x, m != NULL && m->layout == 1);
}

static int forward_device(kernix_model* m, const float* d_x, int rows, float* d_out, void* stream);

int kernix_model_forward_device(kernix_model* m, const float* d_x, int rows, float* d_out, void* stream)
{
    int prev;
    if (enter_device(m, &prev) != 0) return -1;
    const int rc = forward_device(m, d_x, rows, d_out, stream);
    leave_device(prev);
    return rc;
}

static int forward_device(kernix_model* m, const float* d_x, int rows, float* d_out, void* stream)
{
    if (m == NULL || d_x == NULL || d_out == NULL || rows < 0 || rows % m->seq_len != 0) return -1;
    const int samples = rows / m->seq_len;
    const int per = piece_samples(m, samples);
    if (prepare(m, per) != 0) return -1;
    void* st = stream ? stream : m->dev->stream;
    if (order_after_previous(m, st) != 0) return -1;
    const size_t in_row = (size_t)m->seq_len * (size_t)m->in_dim;
    for (int s0 = 0; s0 < samples; s0 += per) {
        const int n = samples - s0 < per ? samples - s0 : per;
        if (run_piece(m, d_x + (size_t)s0 * in_row, s0, n, d_out, 0, st) != 0) return -1;
    }
    return mark_done(m, st);
}

/* Waits for the model's last forward; -1 if a Linear chain launch of a device forward since the previous call could
 * not have all of its workgroups resident (the outputs of that forward are wrong: run it again), else 0. */
int kernix_model_device_status(kernix_model* m)
{
    if (m == NULL || m->dev == NULL || m->dev->chain_status == NULL) return 0;
    int prev;
    if (enter_device(m, &prev) != 0) return -1;
    struct knx_dmodel* d = m->dev;
    int rc = 0;
    if (d->have_last) {
        const int e = d->done_recorded ? knx_hip_event_sync(d->done) : knx_hip_stream_sync(d->last_stream);
        if (hip_ok(e, "device forward")) rc = -1;
    }
    if (__atomic_exchange_n(d->chain_status, 0, __ATOMIC_SEQ_CST)) rc = -1;
    leave_device(prev);
    return rc;
}

/* ---------------------------------------------------------------- kernel-level int8 contract
 * kernix_qmatmul on host pointers.  Like the reference, every call reads the weight (w->q, w->scale) as it is at that
 * call: the packed weight, the input, output, bias and int8 scratch are copied into one growable device buffer shared
 * by all calls (kept until the process ends), used on one stream under a lock, so a call allocates only when it needs
 * more device memory than any call before it.  Nothing is attached to the weight. */
static struct {
    pthread_mutex_t lock;
    void* stream;
    char* buf;
    size_t bytes;
} g_qm = { PTHREAD_MUTEX_INITIALIZER, NULL, NULL, 0 };

static size_t qm_round(size_t b) { return (b + KNX_ALIGN - 1) / KNX_ALIGN * KNX_ALIGN; }

static int qm_call(const float* x, int rows, const kernix_qweight* w, const float* bias, int accumulate, float* y)
{
    const size_t k = (size_t)w->k, n = (size_t)w->n, kp = (size_t)w->kp, np = (size_t)w->np, R = (size_t)rows;
    if (g_qm.stream == NULL && knx_hip_stream_create(&g_qm.stream) != KNX_OK) return -1;
    const size_t sz_w = qm_round(np * kp), sz_s = qm_round(np * 4);
    const size_t sz_x = qm_round(R * k * 4), sz_y = qm_round(R * n * 4), sz_b = qm_round(n * 4), sz_q = qm_round(R * kp);
    const size_t need = sz_w + sz_s + sz_x + sz_y + sz_b + sz_q + qm_round(R * 4);
    if (need > g_qm.bytes) {
        knx_hip_stream_sync(g_qm.stream);
        knx_hip_free(g_qm.buf);
        g_qm.buf = NULL;
        g_qm.bytes = 0;
        if (knx_hip_malloc((void**)&g_qm.buf, need) != KNX_OK) return -1;
        g_qm.bytes = need;
    }
    char* at = g_qm.buf;
    int8_t* dw = (int8_t*)at;                 at += sz_w;
    float* dscale = (float*)at;               at += sz_s;
    float* dx = (float*)at;                   at += sz_x;
    float* dy = (float*)at;                   at += sz_y;
    float* db = bias ? (float*)at : NULL;     at += sz_b;
    int8_t* dxq = (int8_t*)at;                at += sz_q;
    float* dsx = (float*)at;
    void* st = g_qm.stream;
    if (knx_hip_memcpy_h2d(dw, w->q, np * kp, st) || knx_hip_memcpy_h2d(dscale, w->scale, np * 4, st) ||
        knx_hip_memcpy_h2d(dx, x, R * k * 4, st) || (db && knx_hip_memcpy_h2d(db, bias, n * 4, st)) ||
        (accumulate && knx_hip_memcpy_h2d(dy, y, R * n * 4, st)))
        return -1;
    if (knx_hip_qlinear(dx, (int)k, rows, (int)k, (int)kp, dxq, dsx, dw, (int)kp, (int)n, dscale, db, -1,
                        0.0f, accumulate, NULL, 0, dy, (int)n, st) != KNX_OK)
        return -1;
    return knx_hip_memcpy_d2h(y, dy, R * n * 4, st) == KNX_OK && knx_hip_stream_sync(st) == KNX_OK ? 0 : -1;
}

int kernix_qmatmul(const float* x, int rows, const kernix_qweight* w, const float* bias, int accumulate, float* y)
{
    if (w == NULL || rows < 0 || (rows > 0 && (x == NULL || y == NULL))) return -1;
    if (rows == 0) return 0;
    if (knx_hip_init() != KNX_OK) {
        KNX_LOG("KERNIX: no usable MI355X (gfx950) device: %s\n", knx_hip_last_error());
        return -1;
    }
    pthread_mutex_lock(&g_qm.lock);
    const int rc = qm_call(x, rows, w, bias, accumulate, y);
    pthread_mutex_unlock(&g_qm.lock);
    if (rc != 0) KNX_LOG("KERNIX: kernix_qmatmul failed: %s\n", knx_hip_last_error());
    return rc;
}
