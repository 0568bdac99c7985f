/* capi_driver.c — runs a manifest of checks against libkernix.so through the public C API (kernix_model.h).
 *
 *   capi_driver <manifest>
 *
 * Each manifest line is a command and its arguments; file arguments are paths written by tests/test_c_api.py, which
 * also computes every expected value (with the CPU oracle).  The driver only calls the library and compares, so the
 * same C API a C application uses is what is tested.  Tensor files: u32 rows, u32 cols, then rows·cols values (f32,
 * or int8 for q files).  Prints one line per failed check and "<n> commands, <k> failed"; exit status 1 on failure.
 *
 * Commands (— GPU ones need the MI355X):
 *   reject F                         kernix_model_load(F) is NULL
 *   load F nsteps in out seq         loads; fields equal (−1: not checked)
 *   fixed F floats                   ws_fixed
 *   int8 F step q w rec              which host weights of a step exist (1/0)
 *   weight F step w|rec W            host fp32 weight of a step equals W bit for bit
 *   qpack Q S                        kernix_qweight_pack / _unpack round trip is exact; K above the bound is refused
 *   ane F                            set_ane(1) == -1, set_ane(0) == 0, ane_info all zero
 *   plan F                           values live at the same step never share storage (except an in-place hand-over)
 *   forward F X Y tol                — forward twice (no state kept between calls); max|y − Y| ≤ tol; X unchanged
 *   reuse F X                        — same batch again: the same output buffer
 *   edges F                          — 0 rows → 0 × out_dim; wrong width, NULL input, NULL model → NULL
 *   own F X                          — the model's own output as input is refused
 *   badrows F rows                   — rows not a multiple of seq_len is refused
 *   chunks F X tol                   — workspace limits of 1, 3 and S−1 samples: same output, batch = chunk rows;
 *                                      a smaller batch after chunks; trim empties the workspace; forward after trim
 *   deq F X samples expect           — after a forward of `samples` samples, int8 steps have an fp32 copy iff expect
 *   limit_deq F X samples            — under a limit of 3 samples' workspace a forward of `samples` runs in chunks of 3
 *                                      and every int8 step has its fp32 copy
 *   same F G X                       — F and G give the same bits
 *   qmatmul P                        — kernix_qmatmul on P_{q,scale,bias,x,yold,y,yacc}.bin: y and y+yold bit-exact
 *   qspecial P                       — the case with row 1 NaN-poisoned and row 2 zeroed: NaN row, bias row, row 0
 *   qbound                           — K = 131072, q = −128, x = 1: the int32-exact bound of the int8 product
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "kernix_model.h"

static int n_failed, n_cmds;
static char where[512];

#define EXPECT(cond)                                                                     \
    do {                                                                                 \
        if (!(cond)) {                                                                   \
            printf("FAIL [%s] line %d: %s\n", where, __LINE__, #cond);                  \
            n_failed++;                                                                  \
        }                                                                                \
    } while (0)

/* ---------------------------------------------------------------- files */
typedef struct {
    int rows, cols;
    void* data;
} blob;

static blob read_blob(const char* path, size_t elem)
{
    blob b = { 0, 0, NULL };
    FILE* f = fopen(path, "rb");
    uint32_t rc[2];
    if (f == NULL || fread(rc, 4, 2, f) != 2) {
        printf("cannot read %s\n", path);
        exit(2);
    }
    const size_t n = (size_t)rc[0] * rc[1];
    b.rows = (int)rc[0];
    b.cols = (int)rc[1];
    b.data = malloc(n * elem + 64);
    if (b.data == NULL || fread(b.data, elem, n, f) != n) {
        printf("short file %s\n", path);
        exit(2);
    }
    fclose(f);
    return b;
}

static float_tensor* read_tensor(const char* path)
{
    blob b = read_blob(path, 4);
    float_tensor* t = kernix_float_new(b.rows, b.cols, 0);
    memcpy(t->tensor, b.data, 4 * (size_t)b.rows * b.cols);
    free(b.data);
    return t;
}

static float max_diff(const float* a, const float* b, size_t n)
{
    float worst = 0.0f;
    for (size_t i = 0; i < n; i++) {
        const float d = fabsf(a[i] - b[i]);
        if (!(d <= worst)) worst = isnan(d) ? INFINITY : d;
    }
    return worst;
}

static int same_bits(const float* a, const float* b, size_t n) { return memcmp(a, b, n * sizeof(float)) == 0; }

static kernix_model* must_load(const char* path)
{
    kernix_model* m = kernix_model_load(path);
    EXPECT(m != NULL);
    return m;
}

/* ---------------------------------------------------------------- host-side commands */
static void cmd_load(const char* f, int nsteps, int in, int out, int seq)
{
    kernix_model* m = must_load(f);
    if (m == NULL) return;
    EXPECT(nsteps < 0 || m->n_steps == nsteps);
    EXPECT(in < 0 || m->in_dim == in);
    EXPECT(out < 0 || m->out_dim == out);
    EXPECT(seq < 0 || m->seq_len == seq);
    EXPECT(m->batch == -1);
    kernix_model_free(m);
}

static void cmd_int8(const char* f, int i, int q, int w, int rec)
{
    kernix_model* m = must_load(f);
    if (m == NULL) return;
    EXPECT(i < m->n_steps);
    if (i < m->n_steps) {
        EXPECT((m->steps[i].q != NULL) == q);
        EXPECT((m->steps[i].w != NULL) == w);
        EXPECT((m->steps[i].rec != NULL) == rec);
    }
    kernix_model_free(m);
}

static void cmd_weight(const char* f, int i, const char* which, const char* wpath)
{
    kernix_model* m = must_load(f);
    float_tensor* want = read_tensor(wpath);
    if (m != NULL && i < m->n_steps) {
        const kernix_step* s = &m->steps[i];
        const float* got = strcmp(which, "rec") == 0 ? s->rec : s->w ? s->w->tensor : NULL;
        EXPECT(got != NULL);
        if (got != NULL) EXPECT(same_bits(got, want->tensor, (size_t)want->row * want->col));
    }
    float_free(want);
    kernix_model_free(m);
}

static void cmd_qpack(const char* qpath, const char* spath)
{
    blob q = read_blob(qpath, 1), s = read_blob(spath, 4);
    const int k = q.rows, n = q.cols;
    kernix_qweight* w = kernix_qweight_pack(q.data, s.data, k, n);
    EXPECT(w != NULL);
    if (w != NULL) {
        EXPECT(w->k == k && w->n == n && w->kp >= k && w->np >= n && w->kp % 16 == 0 && w->np % 16 == 0);
        float* back = malloc(sizeof(float) * (size_t)k * n);
        kernix_qweight_unpack(w, back);
        int exact = 1;
        for (int r = 0; r < k; r++)
            for (int c = 0; c < n; c++)
                exact &= back[(size_t)r * n + c] == (float)((int8_t*)q.data)[(size_t)r * n + c] * ((float*)s.data)[c];
        EXPECT(exact);
        free(back);
    }
    kernix_qweight_free(w);
    EXPECT(kernix_qweight_pack(q.data, s.data, KERNIX_INT8_MAX_K + 1, 1) == NULL);
    EXPECT(kernix_qweight_pack(NULL, s.data, k, n) == NULL);
    free(q.data);
    free(s.data);
}

static void cmd_ane(const char* f)
{
    kernix_model* m = must_load(f);
    if (m == NULL) return;
    EXPECT(kernix_model_set_ane(m, 1) == -1);
    EXPECT(kernix_model_set_ane(m, 0) == 0);
    kernix_ane_info info = { 1, 1, 1, 1 };
    kernix_model_ane_info(m, &info);
    EXPECT(info.segments == 0 && info.compiles == 0 && info.ane_runs == 0 && info.failures == 0);
    kernix_model_free(m);
}

static int rewrites_input(int kind)
{
    return kind == KERNIX_OP_ACT || kind == KERNIX_OP_LAYERNORM || kind == KERNIX_OP_SOFTMAX || kind == KERNIX_OP_AFFINE ||
           kind == KERNIX_OP_ADD_CONST || kind == KERNIX_OP_BINARY;
}

/* Storage plan: two values live at the same step (intervals [written, last read]) never overlap in storage, except
 * a RESHAPE view and the value it views, and an in-place hand-over (value a last read by the step that rewrites it
 * into value b). */
static void cmd_plan(const char* f)
{
    kernix_model* m = must_load(f);
    if (m == NULL) return;
    int bad = 0;
    for (int a = 1; a < m->n_vals; a++) {
        const kernix_val* va = &m->vals[a];
        if (va->st < 0) continue;
        const int da = a - 1, la = va->last > da ? va->last : da;
        for (int b = a + 1; b < m->n_vals; b++) {
            const kernix_val* vb = &m->vals[b];
            if (vb->st < 0) continue;
            const int db = b - 1, lb = vb->last > db ? vb->last : db;
            if (la < db || lb < da) continue; /* never live together */
            const size_t oa = m->st_off[va->st], ob = m->st_off[vb->st];
            const size_t ea = oa + (size_t)va->r * va->c, eb = ob + (size_t)vb->r * vb->c;
            if (!(oa < eb && ob < ea)) continue;
            const int view = va->st == vb->st && (m->steps[da].kind == KERNIX_OP_RESHAPE || m->steps[db].kind == KERNIX_OP_RESHAPE);
            const int handover = va->st == vb->st && la == db && rewrites_input(m->steps[db].kind);
            if (!view && !handover) {
                printf("  %s: values %d and %d share storage while both live\n", f, a, b);
                bad++;
            }
        }
    }
    EXPECT(bad == 0);
    kernix_model_free(m);
}

/* ---------------------------------------------------------------- GPU commands */
static void cmd_forward(const char* f, const char* xp, const char* yp, float tol)
{
    kernix_model* m = must_load(f);
    float_tensor* x = read_tensor(xp);
    float_tensor* want = read_tensor(yp);
    const size_t nx = (size_t)x->row * x->col, ny = (size_t)want->row * want->col;
    float* before = malloc(nx * sizeof(float) + 4);
    memcpy(before, x->tensor, nx * sizeof(float));
    for (int rep = 0; m != NULL && rep < 2; rep++) {
        const float_tensor* y = kernix_model_forward(m, x);
        EXPECT(y != NULL && y->row * y->col == (int)ny);
        if (y == NULL) break;
        const float d = max_diff(y->tensor, want->tensor, ny);
        if (!(d <= tol)) printf("  %s: max abs diff %.3e > %.1e\n", f, d, tol);
        EXPECT(d <= tol);
    }
    EXPECT(same_bits(before, x->tensor, nx));
    free(before);
    float_free(x);
    float_free(want);
    kernix_model_free(m);
}

static void cmd_reuse(const char* f, const char* xp)
{
    kernix_model* m = must_load(f);
    float_tensor* x = read_tensor(xp);
    if (m != NULL) {
        const float_tensor* y1 = kernix_model_forward(m, x);
        const float* p1 = y1 ? y1->tensor : NULL;
        const float_tensor* y2 = kernix_model_forward(m, x);
        EXPECT(y1 != NULL && y2 == y1 && y2->tensor == p1);
    }
    float_free(x);
    kernix_model_free(m);
}

static void cmd_edges(const char* f)
{
    kernix_model* m = must_load(f);
    if (m == NULL) return;
    float_tensor* none = float_zeros(0, m->in_dim);
    const float_tensor* y = kernix_model_forward(m, none);
    EXPECT(y != NULL && y->row == 0 && y->col == m->out_dim);
    float_tensor* wrong = float_zeros(m->seq_len, m->in_dim + 1);
    EXPECT(kernix_model_forward(m, wrong) == NULL);
    EXPECT(kernix_model_forward(m, NULL) == NULL);
    EXPECT(kernix_model_forward(NULL, none) == NULL);
    float_free(none);
    float_free(wrong);
    kernix_model_free(m);
}

static void cmd_own(const char* f, const char* xp)
{
    kernix_model* m = must_load(f);
    float_tensor* x = read_tensor(xp);
    const float_tensor* y = m ? kernix_model_forward(m, x) : NULL;
    EXPECT(y != NULL);
    if (y != NULL) EXPECT(kernix_model_forward(m, y) == NULL);
    float_free(x);
    kernix_model_free(m);
}

static void cmd_badrows(const char* f, int rows)
{
    kernix_model* m = must_load(f);
    if (m == NULL) return;
    float_tensor* x = float_zeros(rows, m->in_dim);
    EXPECT(kernix_model_forward(m, x) == NULL);
    float_free(x);
    kernix_model_free(m);
}

static void cmd_chunks(const char* f, const char* xp, float tol)
{
    kernix_model* m = must_load(f);
    float_tensor* x = read_tensor(xp);
    if (m == NULL) { float_free(x); return; }
    const int T = m->seq_len, S = x->row / T;
    const size_t each = m->ws_per_sample * sizeof(float), fixed = m->ws_fixed * sizeof(float);
    kernix_model_set_workspace_limit(m, 0);
    const float_tensor* y = kernix_model_forward(m, x);
    EXPECT(y != NULL && m->batch == x->row);
    if (y == NULL) { float_free(x); kernix_model_free(m); return; }
    const size_t ny = (size_t)y->row * y->col;
    float* whole = malloc(ny * sizeof(float));
    memcpy(whole, y->tensor, ny * sizeof(float));
    const int per[3] = { 1, 3, S - 1 };
    for (int i = 0; i < 3; i++) {
        kernix_model_set_workspace_limit(m, fixed + each * (size_t)per[i] + (i == 0 ? 1 : 0));
        y = kernix_model_forward(m, x);
        EXPECT(y != NULL && y->row == S && y->col == m->out_dim && m->batch == per[i] * T);
        if (y != NULL) EXPECT(max_diff(y->tensor, whole, ny) <= tol);
    }
    /* a batch of 3 after the chunked runs reuses the workspace of 3-sample pieces */
    kernix_model_set_workspace_limit(m, fixed + each * 3);
    kernix_model_forward(m, x);
    const float_tensor x3 = { 3 * T, x->col, x->tensor };
    y = kernix_model_forward(m, &x3);
    EXPECT(y != NULL && m->batch == 3 * T);
    if (y != NULL) EXPECT(max_diff(y->tensor, whole, 3 * (size_t)m->out_dim) <= tol);
    kernix_model_trim(m);
    int empty = m->batch == -1 && m->in_copy == NULL && m->out_all == NULL;
    for (int i = 0; i < m->n_steps; i++) empty &= m->steps[i].buf == NULL && m->steps[i].tmp[0] == NULL && m->steps[i].deq == NULL;
    EXPECT(empty);
    y = kernix_model_forward(m, x);
    EXPECT(y != NULL);
    if (y != NULL) EXPECT(max_diff(y->tensor, whole, ny) <= tol);
    free(whole);
    float_free(x);
    kernix_model_free(m);
}

static void cmd_deq(const char* f, const char* xp, int samples, int expect)
{
    kernix_model* m = must_load(f);
    float_tensor* x = read_tensor(xp);
    if (m != NULL) {
        const float_tensor xs = { samples * m->seq_len, x->col, x->tensor };
        EXPECT(kernix_model_forward(m, &xs) != NULL);
        for (int i = 0; i < m->n_steps; i++)
            if (m->steps[i].q != NULL) EXPECT((m->steps[i].deq != NULL) == expect);
    }
    float_free(x);
    kernix_model_free(m);
}

static void cmd_limit_deq(const char* f, const char* xp, int samples)
{
    kernix_model* m = must_load(f);
    float_tensor* x = read_tensor(xp);
    if (m != NULL) {
        kernix_model_set_workspace_limit(m, (m->ws_fixed + m->ws_per_sample * 3) * sizeof(float));
        const float_tensor xs = { samples * m->seq_len, x->col, x->tensor };
        EXPECT(kernix_model_forward(m, &xs) != NULL && m->batch == 3 * m->seq_len);
        for (int i = 0; i < m->n_steps; i++)
            if (m->steps[i].q != NULL) EXPECT(m->steps[i].deq != NULL);
    }
    float_free(x);
    kernix_model_free(m);
}

static void cmd_same(const char* f, const char* g, const char* xp)
{
    kernix_model* a = must_load(f);
    kernix_model* b = must_load(g);
    float_tensor* x = read_tensor(xp);
    if (a != NULL && b != NULL) {
        const float_tensor* ya = kernix_model_forward(a, x);
        const float_tensor* yb = kernix_model_forward(b, x);
        EXPECT(ya != NULL && yb != NULL && ya->row == yb->row && ya->col == yb->col);
        if (ya != NULL && yb != NULL) EXPECT(same_bits(ya->tensor, yb->tensor, (size_t)ya->row * ya->col));
    }
    float_free(x);
    kernix_model_free(a);
    kernix_model_free(b);
}

static blob part(const char* prefix, const char* name, size_t elem)
{
    char path[1100];
    snprintf(path, sizeof path, "%s_%s.bin", prefix, name);
    return read_blob(path, elem);
}

static void cmd_qmatmul(const char* p, int special)
{
    blob q = part(p, "q", 1), s = part(p, "scale", 4), b = part(p, "bias", 4), x = part(p, "x", 4);
    blob yold = part(p, "yold", 4), y = part(p, "y", 4), yacc = part(p, "yacc", 4);
    const int k = q.rows, n = q.cols, rows = x.rows;
    kernix_qweight* w = kernix_qweight_pack(q.data, s.data, k, n);
    float* got = malloc(sizeof(float) * (size_t)rows * n + 4);
    EXPECT(w != NULL);
    if (w != NULL && !special) {
        EXPECT(kernix_qmatmul(x.data, rows, w, b.data, 0, got) == 0);
        EXPECT(same_bits(got, y.data, (size_t)rows * n));
        memcpy(got, yold.data, sizeof(float) * (size_t)rows * n);
        EXPECT(kernix_qmatmul(x.data, rows, w, b.data, 1, got) == 0);
        EXPECT(same_bits(got, yacc.data, (size_t)rows * n));
        EXPECT(kernix_qmatmul(x.data, 0, w, b.data, 0, got) == 0);
    } else if (w != NULL && rows >= 3) {
        float* xs = x.data;
        xs[k] = NAN;                                   /* row 1 */
        for (int j = 0; j < k; j++) xs[2 * k + j] = 0.0f; /* row 2 */
        EXPECT(kernix_qmatmul(xs, rows, w, b.data, 0, got) == 0);
        int nan_row = 1, bias_row = 1;
        for (int j = 0; j < n; j++) {
            nan_row &= isnan(got[n + j]);
            bias_row &= got[2 * n + j] == ((float*)b.data)[j];
        }
        EXPECT(nan_row && bias_row);
        EXPECT(same_bits(got, y.data, (size_t)n)); /* row 0 is untouched by the other rows */
    }
    kernix_qweight_free(w);
    free(got);
    free(q.data); free(s.data); free(b.data); free(x.data); free(yold.data); free(y.data); free(yacc.data);
}

static void cmd_qbound(void)
{
    const int k = KERNIX_INT8_MAX_K;
    int8_t* q = malloc((size_t)k);
    float* x = malloc(sizeof(float) * (size_t)k);
    for (int i = 0; i < k; i++) { q[i] = -128; x[i] = 1.0f; }
    const float one = 1.0f;
    kernix_qweight* w = kernix_qweight_pack(q, &one, k, 1);
    float y = 0.0f;
    EXPECT(w != NULL && kernix_qmatmul(x, 1, w, NULL, 0, &y) == 0);
    EXPECT(y == (float)(-128.0 * 127.0 * k) * (1.0f / 127.0f));
    kernix_qweight_free(w);
    free(q);
    free(x);
}

/* ---------------------------------------------------------------- manifest */
int main(int argc, char** argv)
{
    if (argc != 2) {
        printf("usage: %s <manifest>\n", argv[0]);
        return 2;
    }
    FILE* mf = fopen(argv[1], "r");
    if (mf == NULL) {
        printf("cannot open %s\n", argv[1]);
        return 2;
    }
    char line[4096];
    while (fgets(line, sizeof line, mf) != NULL) {
        line[strcspn(line, "\r\n")] = '\0';
        char c[32], a[1024], b[1024], d[1024];
        int i1 = 0, i2 = 0, i3 = 0, i4 = 0;
        float tol = 0.0f;
        if (line[0] == '\0' || line[0] == '#' || sscanf(line, "%31s", c) != 1) continue;
        snprintf(where, sizeof where, "%.500s", line);
        n_cmds++;
        const char* args = line + strlen(c);
        if (!strcmp(c, "reject") && sscanf(args, "%1023s", a) == 1) {
            kernix_model* m = kernix_model_load(a);
            EXPECT(m == NULL);
            kernix_model_free(m);
        } else if (!strcmp(c, "load") && sscanf(args, "%1023s %d %d %d %d", a, &i1, &i2, &i3, &i4) == 5) {
            cmd_load(a, i1, i2, i3, i4);
        } else if (!strcmp(c, "fixed") && sscanf(args, "%1023s %d", a, &i1) == 2) {
            kernix_model* m = must_load(a);
            if (m != NULL) EXPECT(m->ws_fixed == (size_t)i1);
            kernix_model_free(m);
        } else if (!strcmp(c, "int8") && sscanf(args, "%1023s %d %d %d %d", a, &i1, &i2, &i3, &i4) == 5) {
            cmd_int8(a, i1, i2, i3, i4);
        } else if (!strcmp(c, "weight") && sscanf(args, "%1023s %d %1023s %1023s", a, &i1, b, d) == 4) {
            cmd_weight(a, i1, b, d);
        } else if (!strcmp(c, "qpack") && sscanf(args, "%1023s %1023s", a, b) == 2) {
            cmd_qpack(a, b);
        } else if (!strcmp(c, "ane") && sscanf(args, "%1023s", a) == 1) {
            cmd_ane(a);
        } else if (!strcmp(c, "plan") && sscanf(args, "%1023s", a) == 1) {
            cmd_plan(a);
        } else if (!strcmp(c, "forward") && sscanf(args, "%1023s %1023s %1023s %f", a, b, d, &tol) == 4) {
            cmd_forward(a, b, d, tol);
        } else if (!strcmp(c, "reuse") && sscanf(args, "%1023s %1023s", a, b) == 2) {
            cmd_reuse(a, b);
        } else if (!strcmp(c, "edges") && sscanf(args, "%1023s", a) == 1) {
            cmd_edges(a);
        } else if (!strcmp(c, "own") && sscanf(args, "%1023s %1023s", a, b) == 2) {
            cmd_own(a, b);
        } else if (!strcmp(c, "badrows") && sscanf(args, "%1023s %d", a, &i1) == 2) {
            cmd_badrows(a, i1);
        } else if (!strcmp(c, "chunks") && sscanf(args, "%1023s %1023s %f", a, b, &tol) == 3) {
            cmd_chunks(a, b, tol);
        } else if (!strcmp(c, "deq") && sscanf(args, "%1023s %1023s %d %d", a, b, &i1, &i2) == 4) {
            cmd_deq(a, b, i1, i2);
        } else if (!strcmp(c, "limit_deq") && sscanf(args, "%1023s %1023s %d", a, b, &i1) == 3) {
            cmd_limit_deq(a, b, i1);
        } else if (!strcmp(c, "same") && sscanf(args, "%1023s %1023s %1023s", a, b, d) == 3) {
            cmd_same(a, b, d);
        } else if (!strcmp(c, "qmatmul") && sscanf(args, "%1023s", a) == 1) {
            cmd_qmatmul(a, 0);
        } else if (!strcmp(c, "qspecial") && sscanf(args, "%1023s", a) == 1) {
            cmd_qmatmul(a, 1);
        } else if (!strcmp(c, "qbound")) {
            cmd_qbound();
        } else {
            printf("FAIL [%s]: unknown or malformed command\n", where);
            n_failed++;
        }
    }
    fclose(mf);
    printf("%d commands, %d failed\n", n_cmds, n_failed);
    return n_failed ? 1 : 0;
}
