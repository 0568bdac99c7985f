/* knx_graph.c — from decoded op records to a runnable model: value shapes, activation folding, liveness and the
 * storage plan, plus the model-level API that needs no device (load, free, limits, int8 mode).
 *
 * Shapes follow the reference's rules (include/kernix_model.h:1246-1394; the file formats' docs/graph-runtime-design
 * .md §3): every value is per sample channels-last with 1-4 axes, rows = product of the leading axes.
 *
 * Storage plan (this build's own).  Every value written by a step lives in a slot; ops that rewrite their input in
 * place (activation, layer_norm, softmax, affine, constant add, binary) take over their input's slot when that input
 * dies at the step and has the same size, and RESHAPE is a view of its input's slot.  Each slot has a live interval
 * [first writing step, last reading step] and a size in floats per sample (rounded up to 64, so every slot of a
 * chunk of B samples starts on a 256-byte boundary).  Slots are then packed into one region with a greedy-by-size
 * offset assignment: largest first, each at the lowest offset where it overlaps no already placed slot whose interval
 * intersects its own.  A chunk of B samples holds slot k at float offset off[k]·B of the region.
 */
#include <limits.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "knx_internal.h"

/* ---------------------------------------------------------------- values */
static int value_init(kernix_val* v, int nd, const int* d)
{
    if (nd < 1 || nd > KERNIX_MAX_DIMS) return -1;
    uint64_t rows = 1;
    for (int k = 0; k < nd; k++) {
        if (d[k] < 1) return -1;
        if (k + 1 < nd && (rows *= (uint64_t)d[k]) > INT_MAX) return -1;
    }
    if (rows * (uint64_t)d[nd - 1] > INT_MAX) return -1;
    memset(v, 0, sizeof *v);
    v->nd = nd;
    memcpy(v->d, d, sizeof(int) * (size_t)nd);
    v->r = (int)rows;
    v->c = d[nd - 1];
    v->st = -1;
    v->last = -1;
    return 0;
}

static size_t value_floats(const kernix_val* v) { return (size_t)v->r * (size_t)v->c; }

/* ---------------------------------------------------------------- shapes */
typedef struct {
    int nd, d[KERNIX_MAX_DIMS];
} shape;

/* output spatial extent of a window op along one axis (n ≥ 0 required) */
static int64_t window_out(int64_t in, int pad_a, int pad_b, int k, int dil, int stride)
{
    const int64_t n = in + pad_a + pad_b - ((int64_t)dil * (k - 1) + 1);
    return n < 0 ? -1 : n / stride + 1;
}

/* CONV, POOL, PAD, UPSAMPLE over T×C or H×W×C */
static const char* spatial_shape(const kernix_step* s, const kernix_val* x, shape* o)
{
    if (x->nd != 2 && x->nd != 3) return "convolution/pooling input must be T×C or H×W×C";
    const int two_d = x->nd == 3;
    if (!two_d && (s->kw != 1 || s->sw != 1 || s->dw != 1 || s->pl != 0 || s->pr != 0))
        return "2-D kernel on a 1-D (T×C) input";
    if (s->kind == KERNIX_OP_CONV && x->c != s->in) return "convolution input channels differ from the previous output";
    const int64_t H = x->d[0], W = two_d ? x->d[1] : 1;
    int64_t Ho, Wo;
    switch (s->kind) {
    case KERNIX_OP_PAD: Ho = H + s->pt + s->pb; Wo = W + s->pl + s->pr; break;
    case KERNIX_OP_UPSAMPLE: Ho = H * s->sh; Wo = W * s->sw; break;
    default:
        Ho = window_out(H, s->pt, s->pb, s->kh, s->dh, s->sh);
        Wo = window_out(W, s->pl, s->pr, s->kw, s->dw, s->sw);
        if (Ho < 0 || Wo < 0) return "convolution/pooling output size ≤ 0";
    }
    if (Ho > INT_MAX || Wo > INT_MAX) return "shape out of range";
    o->d[0] = (int)Ho;
    if (two_d) o->d[1] = (int)Wo;
    if (s->kind == KERNIX_OP_CONV) o->d[o->nd - 1] = s->out;
    return NULL;
}

/* Elementwise broadcasting within a sample: the rows of both operands are the larger operand's rows (or 1), the
 * channels the wider channel count (or 1); the output takes the larger operand's shape (the first on a tie). */
static const char* binary_shape(const kernix_val* x, const kernix_val* y, shape* o)
{
    const kernix_val* big = (int64_t)x->r * x->c >= (int64_t)y->r * y->c ? x : y;
    const int R = x->r > y->r ? x->r : y->r, C = x->c > y->c ? x->c : y->c;
    const int ok = big->r == R && (x->r == R || x->r == 1) && (y->r == R || y->r == 1) && (x->c == C || x->c == 1) &&
                   (y->c == C || y->c == 1);
    if (!ok) return "binary op input shapes do not broadcast";
    o->nd = big->nd;
    memcpy(o->d, big->d, sizeof o->d);
    o->d[o->nd - 1] = C;
    return NULL;
}

/* The shape of step s's output from its inputs (vals), or an error.  KNX1/2 LSTMs take their sequence length from
 * the previous value (and must agree with the length in the file). */
static const char* step_shape(kernix_step* s, int ver, const kernix_val* vals, shape* o)
{
    const kernix_val* x = &vals[s->inp[0]];
    o->nd = x->nd;
    memcpy(o->d, x->d, sizeof o->d);
    int* last = &o->d[o->nd - 1];
    switch (s->kind) {
    case KERNIX_OP_LINEAR:
        if (x->c != s->in) return "Linear input size differs from the previous output";
        *last = s->out;
        return NULL;
    case KERNIX_OP_ACT:
    case KERNIX_OP_SOFTMAX:
        return NULL;
    case KERNIX_OP_LAYERNORM:
    case KERNIX_OP_AFFINE:
        return x->c == s->in ? NULL : "normalization size differs from the previous output";
    case KERNIX_OP_ADD_CONST:
        return (int64_t)x->r * x->c == s->in ? NULL : "constant size differs from the previous output";
    case KERNIX_OP_LSTM:
    case KERNIX_OP_GRU:
    case KERNIX_OP_RNN: {
        if (x->c != s->in) return "RNN input size differs from the previous output";
        if (ver < 3 && s->seq != x->r) return "LSTM sequence length differs from the previous step";
        s->seq = x->r;
        const int width = s->dirs == 2 && s->merge == KERNIX_MERGE_CONCAT ? 2 * s->out : s->out;
        *o = s->ret_seq ? (shape){ 2, { x->r, width } } : (shape){ 1, { width } };
        return NULL;
    }
    case KERNIX_OP_CONV:
    case KERNIX_OP_POOL:
    case KERNIX_OP_PAD:
    case KERNIX_OP_UPSAMPLE:
        return spatial_shape(s, x, o);
    case KERNIX_OP_GLOBAL_POOL:
        *o = (shape){ 1, { x->c } };
        return NULL;
    case KERNIX_OP_RESHAPE: {
        uint64_t n = 1;
        for (int k = 0; k < s->nd; k++) n *= (uint64_t)s->d[k];
        if (n != (uint64_t)value_floats(x)) return "Reshape size differs from the input";
        o->nd = s->nd;
        memcpy(o->d, s->d, sizeof o->d);
        return NULL;
    }
    case KERNIX_OP_PERMUTE:
        if (s->nd != x->nd) return "Permute axis count differs from the input";
        for (int k = 0; k < x->nd; k++) o->d[k] = x->d[s->perm[k]];
        return NULL;
    case KERNIX_OP_BINARY:
        return binary_shape(x, &vals[s->inp[1]], o);
    case KERNIX_OP_CONCAT: {
        const int ax = s->axis == KERNIX_AXIS_FIRST ? 0 : x->nd - 1;
        int64_t total = 0;
        for (int k = 0; k < s->n_in; k++) {
            const kernix_val* v = &vals[s->inp[k]];
            if (v->nd != x->nd) return "Concatenate input shapes do not match";
            for (int j = 0; j < x->nd; j++)
                if (j != ax && v->d[j] != x->d[j]) return "Concatenate input shapes do not match";
            total += v->d[ax];
        }
        if (total > INT_MAX) return "shape out of range";
        o->d[ax] = (int)total;
        return NULL;
    }
    case KERNIX_OP_EMBEDDING:
        if (x->nd >= KERNIX_MAX_DIMS) return "number of axes out of range";
        o->d[o->nd++] = s->out;
        return NULL;
    case KERNIX_OP_ATTENTION: {
        /* inputs (q[, v[, k]]): v defaults to q, k to v */
        const kernix_val* v = &vals[s->inp[s->n_in > 1 ? 1 : 0]];
        const kernix_val* k = &vals[s->inp[s->n_in > 2 ? 2 : s->n_in > 1 ? 1 : 0]];
        if (x->c != s->w->row || v->c != s->wv->row || k->c != s->wk->row || k->r != v->r)
            return "attention input sizes differ from the weights";
        *last = s->out;
        return NULL;
    }
    case KERNIX_OP_SELECT: {
        const int ax = s->axis == KERNIX_AXIS_FIRST ? 0 : x->nd - 1;
        if ((int64_t)s->start + s->len > x->d[ax]) return "Select range outside the input";
        o->d[ax] = s->len;
        if (s->squeeze && s->len == 1 && o->nd > 1) {
            for (int j = ax; j + 1 < o->nd; j++) o->d[j] = o->d[j + 1];
            o->nd--;
        }
        return NULL;
    }
    default:
        return "unknown op";
    }
}

/* KNX1/2 files carry no input shape: in_dim is the size of the first LINEAR / LAYERNORM / LSTM, and a file with an
 * LSTM feeds it sequences of that LSTM's length */
static const char* legacy_input(const knx_file* f, kernix_val* v0)
{
    int in_dim = 0, seq = 0;
    for (int i = 0; i < f->n_ops; i++) {
        const kernix_step* s = &f->ops[i];
        const int sized = s->kind == KERNIX_OP_LINEAR || s->kind == KERNIX_OP_LAYERNORM || s->kind == KERNIX_OP_LSTM;
        if (in_dim == 0 && sized) in_dim = s->in;
        if (seq == 0 && s->kind == KERNIX_OP_LSTM) seq = s->seq;
    }
    if (in_dim == 0) return "no Linear or LayerNorm: input size unknown";
    const int d[2] = { seq ? seq : in_dim, in_dim };
    return value_init(v0, seq ? 2 : 1, d) == 0 ? NULL : "input shape out of range";
}

/* ---------------------------------------------------------------- activation folding
 * An ACT step whose input is written by a LINEAR or CONV step without an activation, and read by nothing else,
 * becomes that step's epilogue activation (the reference's step count, include/kernix_model.h:1519-1540).
 * ops/vals are rewritten in place; returns the new step count and fills out_v (the model output's value id). */
static int fold_activations(kernix_step* ops, kernix_val* vals, int n, int* out_v)
{
    int* readers = calloc((size_t)n + 1, sizeof(int));
    int* renum = calloc((size_t)n + 1, sizeof(int)); /* old value id → new value id */
    if (readers == NULL || renum == NULL) {
        free(readers);
        free(renum);
        return -1;
    }
    for (int i = 0; i < n; i++)
        for (int k = 0; k < ops[i].n_in; k++) readers[ops[i].inp[k]]++;
    readers[n]++; /* the model output */
    int kept = 0;
    for (int i = 0; i < n; i++) {
        kernix_step s = ops[i];
        const int src = s.inp[0];
        for (int k = 0; k < s.n_in; k++) s.inp[k] = renum[s.inp[k]];
        kernix_step* producer = src > 0 ? &ops[s.inp[0] - 1] : NULL; /* already at its new index */
        const int foldable = s.kind == KERNIX_OP_ACT && producer != NULL && readers[src] == 1 &&
                             (producer->kind == KERNIX_OP_LINEAR || producer->kind == KERNIX_OP_CONV) &&
                             producer->act == KERNIX_ACT_NONE;
        if (foldable) {
            producer->act = s.act;
            producer->alpha = s.alpha;
            renum[i + 1] = s.inp[0];
            continue;
        }
        ops[kept] = s;
        vals[kept + 1] = vals[i + 1];
        renum[i + 1] = ++kept;
    }
    if (kept < n) memset(&ops[kept], 0, sizeof(kernix_step) * (size_t)(n - kept));
    *out_v = renum[n];
    free(readers);
    free(renum);
    return kept;
}

/* ---------------------------------------------------------------- storage plan */
static int rewrites_input(int kind)
{
    switch (kind) {
    case KERNIX_OP_ACT:
    case KERNIX_OP_LAYERNORM:
    case KERNIX_OP_SOFTMAX:
    case KERNIX_OP_AFFINE:
    case KERNIX_OP_ADD_CONST:
    case KERNIX_OP_BINARY:
        return 1;
    default:
        return 0;
    }
}

typedef struct {
    size_t cap;      /* floats per sample, multiple of 64 */
    int first, end;  /* live interval in steps, inclusive */
    size_t off;      /* per-sample float offset in the value region */
} slot;

static int by_size_desc(const void* a, const void* b)
{
    const slot* x = *(const slot* const*)a;
    const slot* y = *(const slot* const*)b;
    if (x->cap != y->cap) return x->cap > y->cap ? -1 : 1;
    return x->first - y->first;
}

static int by_offset(const void* a, const void* b)
{
    const slot* x = *(const slot* const*)a;
    const slot* y = *(const slot* const*)b;
    return x->off < y->off ? -1 : x->off > y->off;
}

static int plan_storage(kernix_model* m)
{
    const int n = m->n_steps;
    slot* sl = calloc((size_t)n + 1, sizeof(slot));
    slot** order = calloc((size_t)n + 1, sizeof(slot*));
    if (sl == NULL || order == NULL) {
        free(sl);
        free(order);
        return -1;
    }
    int ns = 0;
    for (int i = 0; i < n; i++) {
        const kernix_step* s = &m->steps[i];
        kernix_val* v = &m->vals[i + 1];
        const size_t need = value_floats(v);
        const int live_to = v->last > i ? v->last : i;
        int k = -1;
        if (s->kind == KERNIX_OP_RESHAPE) { /* a view: the input's slot (or the caller's input) */
            v->st = m->vals[s->inp[0]].st;
            if (v->st >= 0 && sl[v->st].end < live_to) sl[v->st].end = live_to;
            continue;
        }
        if (rewrites_input(s->kind)) {
            /* a binary op tries the previous step's output first, so that the runtime can fold the add into the
             * epilogue of the step that wrote it */
            int cand[2] = { s->inp[0], s->n_in > 1 ? s->inp[1] : -1 };
            if (s->kind == KERNIX_OP_BINARY && s->inp[1] == i) { cand[0] = s->inp[1]; cand[1] = s->inp[0]; }
            for (int t = 0; t < 2 && k < 0; t++) {
                if (cand[t] < 0) continue;
                const kernix_val* u = &m->vals[cand[t]];
                if (u->st >= 0 && sl[u->st].end <= i && value_floats(u) == need) k = u->st;
            }
        }
        if (k < 0) {
            k = ns++;
            sl[k].cap = (need + 63) / 64 * 64;
            sl[k].first = i;
            sl[k].end = live_to;
        } else if (sl[k].end < live_to) {
            sl[k].end = live_to;
        }
        v->st = k;
    }
    /* greedy by size: each slot at the lowest offset clear of every placed slot live at the same time */
    for (int k = 0; k < ns; k++) order[k] = &sl[k];
    qsort(order, (size_t)ns, sizeof(slot*), by_size_desc);
    const slot** clash = calloc((size_t)ns + 1, sizeof(slot*));
    if (clash == NULL) {
        free(sl);
        free(order);
        return -1;
    }
    size_t span = 0;
    for (int a = 0; a < ns; a++) {
        slot* s = order[a];
        int nc = 0;
        for (int b = 0; b < a; b++)
            if (order[b]->first <= s->end && s->first <= order[b]->end) clash[nc++] = order[b];
        qsort(clash, (size_t)nc, sizeof(slot*), by_offset);
        size_t off = 0;
        for (int j = 0; j < nc && off + s->cap > clash[j]->off; j++) /* stop at the first gap that fits */
            if (clash[j]->off + clash[j]->cap > off) off = clash[j]->off + clash[j]->cap;
        s->off = off;
        if (off + s->cap > span) span = off + s->cap;
    }
    free(clash);
    free(order);
    m->n_st = ns;
    m->st_cap = calloc((size_t)(ns ? ns : 1), sizeof(size_t));
    m->st_off = calloc((size_t)(ns ? ns : 1), sizeof(size_t));
    m->st = calloc((size_t)(ns ? ns : 1), sizeof(float_tensor*));
    if (m->st_cap == NULL || m->st_off == NULL || m->st == NULL) {
        free(sl);
        return -1;
    }
    for (int k = 0; k < ns; k++) {
        m->st_cap[k] = sl[k].cap;
        m->st_off[k] = sl[k].off;
    }
    m->st_span = span;
    free(sl);
    return 0;
}

/* 1 when values a and b (of one chunk) occupy overlapping storage; the model input is the caller's buffer */
int knx_storage_overlaps(const kernix_model* m, int a, int b)
{
    const int sa = m->vals[a].st, sb = m->vals[b].st;
    if (sa < 0 || sb < 0) return 0;
    return m->st_off[sa] < m->st_off[sb] + m->st_cap[sb] && m->st_off[sb] < m->st_off[sa] + m->st_cap[sa];
}

/* ---------------------------------------------------------------- model */
void knx_step_host_free(kernix_step* s)
{
    float_tensor* t[] = { s->w, s->w_b, s->wk, s->wv, s->wo };
    for (size_t i = 0; i < sizeof t / sizeof t[0]; i++) float_free(t[i]);
    float* f[] = { s->rec, s->rec_b, s->bias, s->bias_b, s->bk, s->bv, s->bo, s->gamma, s->beta, s->cst };
    for (size_t i = 0; i < sizeof f / sizeof f[0]; i++) free(f[i]);
    kernix_qweight_free(s->q);
    kernix_qweight_free(s->q_b);
}

size_t knx_conv_is_gemm(const kernix_step* s)
{
    const int pointwise = s->kh == 1 && s->kw == 1 && s->sh == 1 && s->sw == 1 && (s->pt | s->pb | s->pl | s->pr) == 0;
    return s->groups == 1 && pointwise ? 0 : (size_t)s->kh * (size_t)s->kw * (size_t)(s->in / s->groups);
}

/* floats of the dequantized int8 weight copies: they exist only under the reference dispatch */
static void count_fixed(kernix_model* m)
{
    size_t fixed = 0;
    for (int i = 0; m->int8_mode == KERNIX_INT8_REF && i < m->n_steps; i++) {
        const kernix_qweight* q[2] = { m->steps[i].q, m->steps[i].q_b };
        for (int d = 0; d < 2; d++)
            if (q[d] != NULL) fixed += (size_t)q[d]->k * (size_t)q[d]->n;
    }
    m->ws_fixed = fixed;
}

int kernix_model_set_int8_mode(kernix_model* m, int mode)
{
    if (m == NULL || (mode != KERNIX_INT8_REF && mode != KERNIX_INT8_I8)) return -1;
    if (m->int8_mode != mode) {
        knx_model_release_device_ws(m);
        m->int8_mode = mode;
        count_fixed(m);
    }
    return 0;
}

static const char* build_model(kernix_model* m, knx_file* f)
{
    const int n = f->n_ops;
    kernix_val* vals = calloc((size_t)n + 1, sizeof(kernix_val));
    if (vals == NULL) return "out of memory";
    m->vals = vals;
    const char* err = NULL;
    if (f->version == 3) err = value_init(&vals[0], f->in_nd, f->in_d) == 0 ? NULL : "input shape out of range";
    else err = legacy_input(f, &vals[0]);
    for (int i = 0; err == NULL && i < n; i++) {
        shape o;
        err = step_shape(&f->ops[i], f->version, vals, &o);
        if (err == NULL && value_init(&vals[i + 1], o.nd, o.d) != 0) err = "shape out of range";
    }
    if (err != NULL) return err;
    /* the steps take over the decoded records (and their weights) */
    m->steps = f->ops;
    f->ops = NULL;
    f->n_ops = 0;
    const int kept = fold_activations(m->steps, vals, n, &m->out_v);
    m->n_steps = kept < 0 ? n : kept;
    if (kept < 0) return "out of memory";
    m->n_vals = kept + 1;
    for (int i = 0; i < kept; i++)
        for (int k = 0; k < m->steps[i].n_in; k++) vals[m->steps[i].inp[k]].last = i;
    vals[m->out_v].last = kept;
    if ((m->views = calloc((size_t)m->n_vals, sizeof(float_tensor))) == NULL || plan_storage(m) != 0) return "out of memory";

    const kernix_val* in = &vals[0];
    const kernix_val* out = &vals[m->out_v];
    m->in_dim = in->c;
    m->seq_len = in->r;
    m->out_dim = out->r * out->c;
    m->in_nd = in->nd;
    m->out_nd = out->nd;
    memcpy(m->in_shape, in->d, sizeof m->in_shape);
    memcpy(m->out_shape, out->d, sizeof m->out_shape);
    m->layout = f->layout;
    m->ws_limit = KERNIX_WORKSPACE_LIMIT;
    const char* mode = getenv("KERNIX_INT8_MODE");
    m->int8_mode = mode != NULL && strcmp(mode, "i8") == 0 ? KERNIX_INT8_I8 : KERNIX_INT8_REF;
    if (knx_model_count_ws(m, &m->ws_per_sample) != 0) return "workspace size out of range";
    count_fixed(m);
    return NULL;
}

kernix_model* kernix_model_load(const char* path)
{
    knx_file f;
    const char* why = NULL;
    if (knx_decode(path, &f, &why) != 0) {
        KNX_LOG("model load failed (%s): %s\n", path ? path : "NULL", why);
        return NULL;
    }
    kernix_model* m = calloc(1, sizeof *m);
    why = m == NULL ? "out of memory" : NULL;
    if (m != NULL) {
        m->batch = -1;
        why = build_model(m, &f);
    }
    knx_file_release(&f); /* whatever build_model did not take over */
    if (why != NULL) {
        KNX_LOG("model load failed (%s): %s\n", path, why);
        kernix_model_free(m);
        return NULL;
    }
    return m;
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
    free(m->st_off);
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
    m->ane = 0;
    return on ? -1 : 0; /* there is no Neural Engine on this platform */
}

void kernix_model_ane_info(const kernix_model* m, kernix_ane_info* out)
{
    (void)m;
    if (out != NULL) *out = (kernix_ane_info){ 0, 0, 0, 0 };
}
