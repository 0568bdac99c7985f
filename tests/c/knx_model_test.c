/* knx_model_test.c — runtime checks of libkernix.so in C, following the reference's test/model_test.c
 * (loader rejection, forward accuracy and buffer reuse, LSTM, chunked execution, int8 kernel, KNX2 loader/forward).
 *
 *   knx_model_test cpu <dir>   loader and host-side checks (no GPU needed)
 *   knx_model_test gpu <dir>   forward checks on the MI355X
 *
 * <dir> holds fixtures written by tests/test_c_runtime.py: small.knx / wide.knx / inplace_first.knx and their
 * <name>_x_<batch>.bin / <name>_y_<batch>.bin pairs (u32 rows, u32 cols, f32 data; expected outputs from the oracle).
 * Prints one line per failed check and exits 1 if any failed. */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "kernix_model.h"

#define MAGIC1 0x31584E4Bu /* "KNX1" */
#define MAGIC2 0x32584E4Bu /* "KNX2" */
#define ONE 0x3F800000u

static int fails;
static char dir[1024];
#define CHECK(c) do { if (!(c)) { printf("  FAIL %s:%d  %s\n", __FILE__, __LINE__, #c); fails++; } } while (0)

static const char* path_of(const char* name)
{
    static char p[2][1200];
    static int k;
    k ^= 1;
    snprintf(p[k], sizeof p[k], "%s/%s", dir, name);
    return p[k];
}

static void write_file(const char* name, const void* data, size_t n)
{
    FILE* f = fopen(path_of(name), "wb");
    if (f == NULL || fwrite(data, 1, n, f) != n) { printf("cannot write %s\n", name); exit(2); }
    fclose(f);
}

static unsigned char* read_file(const char* name, size_t* n)
{
    FILE* f = fopen(path_of(name), "rb");
    if (f == NULL) { printf("missing fixture %s\n", name); exit(2); }
    fseek(f, 0, SEEK_END);
    *n = (size_t)ftell(f);
    rewind(f);
    unsigned char* p = malloc(*n + 4);
    if (p == NULL || fread(p, 1, *n, f) != *n) exit(2);
    fclose(f);
    return p;
}

static int rejected(const void* data, size_t n)
{
    write_file("bad.knx", data, n);
    kernix_model* m = kernix_model_load(path_of("bad.knx"));
    kernix_model_free(m);
    return m == NULL;
}

static float_tensor* load_tensor(const char* name)
{
    size_t n;
    unsigned char* p = read_file(name, &n);
    uint32_t rc[2];
    memcpy(rc, p, 8);
    float_tensor* t = kernix_float_new((int)rc[0], (int)rc[1], 0);
    if (t == NULL || n != 8 + 4 * (size_t)rc[0] * rc[1]) exit(2);
    memcpy(t->tensor, p + 8, n - 8);
    free(p);
    return t;
}

static float max_abs(const float_tensor* got, const float_tensor* want)
{
    if (got == NULL || got->row != want->row || got->col != want->col) return INFINITY;
    float worst = 0.0f;
    for (size_t i = 0; i < (size_t)want->row * want->col; i++) {
        const float d = fabsf(got->tensor[i] - want->tensor[i]);
        if (!(d <= worst)) worst = d;
    }
    return worst == worst ? worst : INFINITY;
}

/* ---------------------------------------------------------------- byte writers and the reference's LCG */
static uint32_t fw[8192];
static size_t fwn;
static uint32_t lcg = 12345;
static uint32_t lcg_next(void) { lcg = lcg * 1664525u + 1013904223u; return lcg >> 8; }
static void put(uint32_t v) { fw[fwn++] = v; }
static void put_floats(size_t n)
{
    for (size_t i = 0; i < n; i++) {
        float v = (float)lcg_next() / 16777216.0f - 0.5f;
        memcpy(&fw[fwn++], &v, 4);
    }
}
static void put_lstm(uint32_t in, uint32_t units, uint32_t act, uint32_t ret_seq, uint32_t seq)
{
    put(KERNIX_OP_LSTM); put(in); put(units); put(act); put(ret_seq); put(seq);
    put_floats((size_t)in * 4 * units + (size_t)units * 4 * units + 4 * units);
}

static unsigned char vb[1 << 21];
static size_t vbn;
static void vput(uint32_t v) { memcpy(vb + vbn, &v, 4); vbn += 4; }
static void vputf(float v) { memcpy(vb + vbn, &v, 4); vbn += 4; }
static void vput8(int8_t v) { vb[vbn++] = (unsigned char)v; }
static float vrandf(void) { return (float)(lcg_next() % 2001) * 0.0005f - 0.5f; }
static void vput_f32(int k, int n, float* keep)
{
    vput(KERNIX_DT_F32);
    for (int i = 0; i < k * n; i++) { float v = vrandf(); if (keep) keep[i] = v; vputf(v); }
}
static void vput_i8(int dt, int k, int n, int8_t* q, float* scale)
{
    const int ns = dt == KERNIX_DT_I8_COL ? n : k;
    vput((uint32_t)dt);
    for (int i = 0; i < ns; i++) { scale[i] = 0.01f + (float)(lcg_next() % 100) * 1e-4f; vputf(scale[i]); }
    for (int i = 0; i < k * n; i++) { q[i] = (int8_t)((int)(lcg_next() % 255) - 127); vput8(q[i]); }
}
static void vlinear_head(uint32_t in, uint32_t out, uint32_t bias) { vput(KERNIX_OP_LINEAR); vput(in); vput(out); vput(bias); }

/* LSTM(7→5, tanh, sequences, T=4) → LSTM(5→6, relu, last) → Linear(6→3), KNX1 */
static void write_lstm_model(const char* name)
{
    fwn = 0;
    lcg = 12345;
    put(MAGIC1); put(3);
    put_lstm(7, 5, KERNIX_ACT_TANH, 1, 4);
    put_lstm(5, 6, KERNIX_ACT_RELU, 0, 4);
    put(KERNIX_OP_LINEAR); put(6); put(3); put(0); put_floats(18);
    write_file(name, fw, fwn * 4);
}

/* ---------------------------------------------------------------- CPU checks */
static void check_load(void)
{
    kernix_model* m = kernix_model_load(path_of("small.knx"));
    CHECK(m != NULL && m->in_dim == 64 && m->out_dim == 10);
    CHECK(m != NULL && m->n_steps == 9); /* 14 ops, 5 activations fused into the Linear before them */
    kernix_model_free(m);
    kernix_model_free(NULL);
    CHECK(kernix_model_load(path_of("no_such_file.knx")) == NULL);
    size_t n;
    unsigned char* small = read_file("small.knx", &n);
    CHECK(rejected(small, n / 2));   /* truncated */
    CHECK(rejected(small, n + 4));   /* trailing bytes */
    small[3] = '2';
    CHECK(rejected(small, n));       /* KNX1 bytes read as KNX2 */
    free(small);
    uint32_t zero_ops[] = { MAGIC1, 0 };
    uint32_t many_ops[] = { MAGIC1, 1025 };
    uint32_t huge[] = { MAGIC1, 1, 0, 0xFFFFFFFFu, 0xFFFFFFFFu, 1 };
    uint32_t big[] = { MAGIC1, 1, 0, 30000, 30000, 0 };       /* valid ints, no data: rejected before allocating */
    uint32_t zero_dim[] = { MAGIC1, 1, 0, 0, 4, 0 };
    uint32_t chain[2 + 4 + 32 + 4 + 18] = { MAGIC1, 2, 0, 4, 8, 0 }; /* Linear(4,8) then Linear(9,2) */
    chain[38] = 0; chain[39] = 9; chain[40] = 2; chain[41] = 0;
    uint32_t ln[2 + 4 + 32 + 4] = { MAGIC1, 2, 0, 4, 8, 0 };         /* Linear(4,8) then LayerNorm(7) */
    ln[38] = 2; ln[39] = 7; ln[40] = 0; ln[41] = 0x3727C5ACu;
    uint32_t bad_kind[] = { MAGIC1, 1, 9 };
    uint32_t bad_act[] = { MAGIC1, 1, 1, 9 };
    uint32_t act_only[] = { MAGIC1, 1, 1, 0 };
    CHECK(rejected(zero_ops, sizeof zero_ops));
    CHECK(rejected(many_ops, sizeof many_ops));
    CHECK(rejected(huge, sizeof huge));
    CHECK(rejected(big, sizeof big));
    CHECK(rejected(zero_dim, sizeof zero_dim));
    CHECK(rejected(chain, sizeof chain));
    CHECK(rejected(ln, sizeof ln));
    CHECK(rejected(bad_kind, sizeof bad_kind));
    CHECK(rejected(bad_act, sizeof bad_act));
    CHECK(rejected(act_only, sizeof act_only));
    chain[39] = 8; /* Linear(8,2): now consistent */
    write_file("bad.knx", chain, sizeof chain - 2 * 4);
    m = kernix_model_load(path_of("bad.knx"));
    CHECK(m != NULL && m->in_dim == 4 && m->out_dim == 2 && m->n_steps == 2);
    kernix_model_free(m);
}

static void check_lstm_load(void)
{
    write_lstm_model("lstm.knx");
    kernix_model* m = kernix_model_load(path_of("lstm.knx"));
    CHECK(m != NULL && m->n_steps == 3 && m->in_dim == 7 && m->out_dim == 3 && m->seq_len == 4);
    kernix_model_free(m);
    fwn = 0; put(MAGIC1); put(1); put_lstm(7, 5, KERNIX_ACT_TANH, 0, 0);      /* seq_len 0 */
    CHECK(rejected(fw, fwn * 4));
    fwn = 0; put(MAGIC1); put(1); put_lstm(7, 5, KERNIX_ACT_GELU, 0, 4);      /* relu/tanh only */
    CHECK(rejected(fw, fwn * 4));
    fwn = 0; put(MAGIC1); put(1); put_lstm(7, 5, KERNIX_ACT_TANH, 2, 4);      /* ret_seq 0/1 */
    CHECK(rejected(fw, fwn * 4));
    fwn = 0; put(MAGIC1); put(2); put_lstm(7, 5, KERNIX_ACT_TANH, 0, 4); put_lstm(5, 6, KERNIX_ACT_RELU, 0, 4);
    CHECK(rejected(fw, fwn * 4));                                              /* LSTM after the sequence ended */
    fwn = 0; put(MAGIC1); put(1); put(KERNIX_OP_LSTM); put(7); put(100000); put(KERNIX_ACT_RELU); put(0); put(4);
    CHECK(rejected(fw, fwn * 4));                                              /* units too large, no data */
    fwn = 0; put(MAGIC1); put(1); put_lstm(7, 5, KERNIX_ACT_TANH, 0, 4);
    CHECK(rejected(fw, fwn * 4 - 4));                                          /* truncated */
}

static void check_v2_load(void)
{
    int8_t q[4096];
    float sc[4096];
    vbn = 0; vput(0x33584E4Bu); vput(1); vlinear_head(4, 2, 0); vput_f32(4, 2, NULL);
    CHECK(rejected(vb, vbn));                                      /* KNX3 header missing */
    vbn = 0; vput(MAGIC2); vput(1); vlinear_head(4, 2, 0); vput(3); for (int i = 0; i < 8; i++) vputf(0.1f);
    CHECK(rejected(vb, vbn));                                      /* dtype 3 */
    vbn = 0; vput(MAGIC2); vput(1); vlinear_head(4, 2, 0); vput(KERNIX_DT_I8_COL); vputf(0.1f);
    CHECK(rejected(vb, vbn));                                      /* truncated scales */
    vbn = 0; vput(MAGIC2); vput(1); vlinear_head(4, 2, 0); vput_i8(KERNIX_DT_I8_COL, 4, 2, q, sc);
    CHECK(rejected(vb, vbn - 1));                                  /* truncated int8 */
    const float bad[4] = { 0.0f, -1.0f, NAN, INFINITY };
    for (int b = 0; b < 4; b++) {
        vbn = 0; vput(MAGIC2); vput(1); vlinear_head(4, 2, 0); vput_i8(KERNIX_DT_I8_COL, 4, 2, q, sc);
        memcpy(vb + 8 + 16 + 4 + 4, &bad[b], 4);
        CHECK(rejected(vb, vbn));                                  /* scale 0 / −1 / NaN / inf */
    }
    vbn = 0; vput(MAGIC2); vput(1); vlinear_head(KERNIX_INT8_MAX_K + 1, 1, 0); vput(KERNIX_DT_I8_COL); vputf(0.01f);
    for (int i = 0; i < KERNIX_INT8_MAX_K + 1; i++) vput8(1);
    CHECK(rejected(vb, vbn));                                      /* K above the int32-exact bound */
    vbn = 0; vput(MAGIC2); vput(1); vlinear_head(KERNIX_INT8_MAX_K, 1, 0); vput(KERNIX_DT_I8_COL); vputf(0.01f);
    for (int i = 0; i < KERNIX_INT8_MAX_K; i++) vput8(1);
    write_file("v2.knx", vb, vbn);
    kernix_model* m = kernix_model_load(path_of("v2.knx"));
    CHECK(m != NULL && m->steps[0].q != NULL);                     /* exactly the bound: accepted */
    kernix_model_free(m);

    /* I8_ROW Linear is dequantized at load: w[k][n] = q·scale[k] exactly */
    vbn = 0; vput(MAGIC2); vput(1); vlinear_head(3, 5, 0); vput_i8(KERNIX_DT_I8_ROW, 3, 5, q, sc);
    write_file("v2.knx", vb, vbn);
    m = kernix_model_load(path_of("v2.knx"));
    int row_ok = m != NULL && m->steps[0].q == NULL && m->steps[0].w != NULL;
    for (int i = 0; row_ok && i < 15; i++) row_ok = m->steps[0].w->tensor[i] == (float)q[i] * sc[i / 5];
    CHECK(row_ok);
    kernix_model_free(m);

    /* LSTM input weight I8_COL becomes fp32; the fp32 recurrent weight stays fp32 */
    vbn = 0; vput(MAGIC2); vput(1); vput(KERNIX_OP_LSTM); vput(3); vput(2); vput(KERNIX_ACT_TANH); vput(0); vput(2);
    vput_i8(KERNIX_DT_I8_COL, 3, 8, q, sc); vput_f32(2, 8, NULL); for (int i = 0; i < 8; i++) vputf(0.0f);
    write_file("v2.knx", vb, vbn);
    m = kernix_model_load(path_of("v2.knx"));
    int lstm_ok = m != NULL && m->steps[0].q == NULL && m->steps[0].rec != NULL && m->steps[0].w != NULL;
    for (int i = 0; lstm_ok && i < 24; i++) lstm_ok = m->steps[0].w->tensor[i] == (float)q[i] * sc[i % 8];
    CHECK(lstm_ok);
    kernix_model_free(m);
}

static void check_qweight_pack(void)
{
    lcg = 12345;
    const int k = 55, n = 31;
    int8_t* q = malloc((size_t)k * n);
    float scale[31], deq[55 * 31];
    for (int i = 0; i < k * n; i++) q[i] = (int8_t)((int)(lcg_next() % 255) - 127);
    for (int i = 0; i < n; i++) scale[i] = 0.001f + (float)(lcg_next() % 1000) * 1e-5f;
    kernix_qweight* w = kernix_qweight_pack(q, scale, k, n);
    CHECK(w != NULL && w->k == k && w->n == n && w->kp % 16 == 0 && w->np % 16 == 0 && w->kp >= k && w->np >= n);
    if (w != NULL) {
        kernix_qweight_unpack(w, deq);
        int ok = 1;
        for (int i = 0; i < k * n; i++) ok &= deq[i] == (float)q[i] * scale[i % n];
        CHECK(ok);
    }
    kernix_qweight_free(w);
    CHECK(kernix_qweight_pack(q, scale, KERNIX_INT8_MAX_K + 1, 1) == NULL);
    free(q);
}

/* qLSTM: LSTM(7→5, tanh, seq, T=4) → LSTM(5→6, relu) → Linear(6→3), recurrences and Linear I8_COL */
typedef struct { float w1[7 * 20], b1[20], w2[5 * 24], b2[24], bd[3]; int8_t u1[5 * 20], u2[6 * 24], d[6 * 3]; float s1[20], s2[24], sd[3]; } qlstm_ref;
static void write_qlstm_model(const char* name, qlstm_ref* r)
{
    lcg = 777;
    vbn = 0; vput(MAGIC2); vput(3);
    vput(KERNIX_OP_LSTM); vput(7); vput(5); vput(KERNIX_ACT_TANH); vput(1); vput(4);
    vput_f32(7, 20, r->w1); vput_i8(KERNIX_DT_I8_COL, 5, 20, r->u1, r->s1); for (int i = 0; i < 20; i++) vputf(r->b1[i] = vrandf());
    vput(KERNIX_OP_LSTM); vput(5); vput(6); vput(KERNIX_ACT_RELU); vput(0); vput(4);
    vput_f32(5, 24, r->w2); vput_i8(KERNIX_DT_I8_COL, 6, 24, r->u2, r->s2); for (int i = 0; i < 24; i++) vputf(r->b2[i] = vrandf());
    vlinear_head(6, 3, 1); vput_i8(KERNIX_DT_I8_COL, 6, 3, r->d, r->sd); for (int i = 0; i < 3; i++) vputf(r->bd[i] = vrandf());
    write_file(name, vb, vbn);
}

static void check_ws_fixed(void)
{
    static qlstm_ref r;
    write_qlstm_model("qlstm.knx", &r);
    kernix_model* m = kernix_model_load(path_of("qlstm.knx"));
    CHECK(m != NULL && m->steps[0].q != NULL && m->steps[1].q != NULL && m->steps[2].q != NULL &&
          m->ws_fixed == 5 * 20 + 6 * 24 + 6 * 3);
    CHECK(m != NULL && kernix_model_set_ane(m, 1) == -1 && kernix_model_set_ane(m, 0) == 0);
    kernix_ane_info ai;
    kernix_model_ane_info(m, &ai);
    CHECK(ai.segments == 0 && ai.compiles == 0 && ai.ane_runs == 0 && ai.failures == 0);
    kernix_model_free(m);
}

/* ---------------------------------------------------------------- GPU checks */
static void check_model(kernix_model* m, const char* name, int batch)
{
    char px[128], py[128];
    snprintf(px, sizeof px, "%s_x_%d.bin", name, batch);
    snprintf(py, sizeof py, "%s_y_%d.bin", name, batch);
    float_tensor* x = load_tensor(px);
    float_tensor* want = load_tensor(py);
    const size_t bytes = sizeof(float) * (size_t)x->row * x->col;
    float* before = malloc(bytes);
    memcpy(before, x->tensor, bytes);
    const float d = max_abs(kernix_model_forward(m, x), want);
    printf("  %-14s batch %-5d max abs err %.2e\n", name, batch, d);
    CHECK(d <= 1e-4f);
    CHECK(memcmp(before, x->tensor, bytes) == 0); /* the input is not modified */
    free(before);
    float_free(x);
    float_free(want);
}

static void check_forward(void)
{
    kernix_model* m = kernix_model_load(path_of("small.knx"));
    if (m == NULL) { fails++; return; }
    check_model(m, "small", 1);
    check_model(m, "small", 37);
    check_model(m, "small", 4096);
    check_model(m, "small", 37);
    float_tensor* x37 = load_tensor("small_x_37.bin");
    const float_tensor* y1 = kernix_model_forward(m, x37);
    const float* p1 = y1 ? y1->tensor : NULL;
    const float_tensor* y2 = kernix_model_forward(m, x37);
    CHECK(y1 != NULL && y1 == y2 && y2->tensor == p1); /* same batch: same buffers, no allocation */
    float_free(x37);
    float_tensor* x0 = float_zeros(0, 64);
    const float_tensor* y0 = kernix_model_forward(m, x0);
    CHECK(y0 != NULL && y0->row == 0 && y0->col == 10);
    float_free(x0);
    float_tensor* xbad = float_zeros(2, 63);
    CHECK(kernix_model_forward(m, xbad) == NULL);
    CHECK(kernix_model_forward(m, NULL) == NULL);
    CHECK(kernix_model_forward(NULL, xbad) == NULL);
    float_free(xbad);
    kernix_model_free(m);

    m = kernix_model_load(path_of("wide.knx")); /* 9000 columns */
    if (m != NULL) check_model(m, "wide", 5); else fails++;
    kernix_model_free(m);
    m = kernix_model_load(path_of("inplace_first.knx")); /* first step in place: the caller's input is kept */
    if (m != NULL) check_model(m, "inplace_first", 3); else fails++;
    kernix_model_free(m);

    /* identity Linear(4,4): exact; its own output as input is rejected */
    uint32_t sq[6 + 16] = { MAGIC1, 1, 0, 4, 4, 0 };
    for (int i = 0; i < 4; i++) sq[6 + i * 5] = ONE;
    write_file("id.knx", sq, sizeof sq);
    m = kernix_model_load(path_of("id.knx"));
    float_tensor* x4 = float_zeros(2, 4);
    for (int i = 0; i < 8; i++) x4->tensor[i] = (float)i;
    const float_tensor* y = m ? kernix_model_forward(m, x4) : NULL;
    CHECK(y != NULL && max_abs(y, x4) == 0.0f);
    CHECK(y != NULL && kernix_model_forward(m, y) == NULL);
    float_free(x4);
    kernix_model_free(m);
}

static float r_sig(float v) { return 1.0f / (1.0f + expf(-v)); }
static float r_act(int act, float v) { return act == KERNIX_ACT_TANH ? tanhf(v) : v > 0.0f ? v : 0.0f; }

/* Keras LSTM (gates i f g o) with double accumulation, reading the host weights of the loaded step */
static void ref_lstm(const kernix_step* s, const float* x, int B, float* out)
{
    const int T = s->seq, u = s->out, in = s->in;
    for (int b = 0; b < B; b++) {
        float h[64] = { 0 }, c[64] = { 0 }, z[256];
        for (int t = 0; t < T; t++) {
            for (int j = 0; j < 4 * u; j++) {
                double acc = s->bias[j];
                for (int k = 0; k < in; k++) acc += (double)x[(b * T + t) * in + k] * s->w->tensor[k * 4 * u + j];
                for (int k = 0; k < u; k++) acc += (double)h[k] * s->rec[k * 4 * u + j];
                z[j] = (float)acc;
            }
            for (int k = 0; k < u; k++) {
                c[k] = r_sig(z[u + k]) * c[k] + r_sig(z[k]) * r_act(s->act, z[2 * u + k]);
                h[k] = r_sig(z[3 * u + k]) * r_act(s->act, c[k]);
                if (s->ret_seq) out[(b * T + t) * u + k] = h[k];
            }
        }
        if (!s->ret_seq) memcpy(out + b * u, h, sizeof(float) * (size_t)u);
    }
}

static void check_lstm(void)
{
    write_lstm_model("lstm.knx");
    kernix_model* m = kernix_model_load(path_of("lstm.knx"));
    if (m == NULL) { fails++; return; }
    const int B = 3;
    float_tensor* x = float_zeros(B * 4, 7);
    for (int i = 0; i < B * 4 * 7; i++) x->tensor[i] = (float)((i * 37) % 23 - 11) * 0.1f;
    float h1[3 * 4 * 5], h2[3 * 6];
    float wt[9] = { 0 };
    float_tensor want = { B, 3, wt };
    ref_lstm(&m->steps[0], x->tensor, B, h1);
    ref_lstm(&m->steps[1], h1, B, h2);
    for (int b = 0; b < B; b++)
        for (int j = 0; j < 3; j++)
            for (int k = 0; k < 6; k++) want.tensor[b * 3 + j] += h2[b * 6 + k] * m->steps[2].w->tensor[k * 3 + j];
    for (int rep = 0; rep < 2; rep++) { /* second call: no state (h, c) leaks through the reused buffers */
        const float d = max_abs(kernix_model_forward(m, x), &want);
        printf("  LSTM x2 + Linear     max abs err %.2e\n", d);
        CHECK(d <= 1e-5f);
    }
    float_tensor* x7 = float_zeros(7, 7); /* rows not a multiple of T */
    CHECK(kernix_model_forward(m, x7) == NULL);
    float_free(x7);
    float_free(x);
    kernix_model_free(m);
}

/* chunked == unchunked; reuse after the last chunk; trim empties the workspace (reference test/model_test.c:296-360) */
static void check_chunk_model(kernix_model* m, const float_tensor* x, const char* name, float tol)
{
    const int samples = x->row / m->seq_len, T = m->seq_len;
    const size_t per = m->ws_per_sample * sizeof(float), fixed = m->ws_fixed * sizeof(float);
    kernix_model_set_workspace_limit(m, 0);
    const float_tensor* y = kernix_model_forward(m, x);
    CHECK(y != NULL && m->batch == x->row);
    if (y == NULL) return;
    float_tensor* want = float_zeros(y->row, y->col);
    memcpy(want->tensor, y->tensor, sizeof(float) * (size_t)y->row * y->col);
    const size_t limits[] = { fixed + 1, fixed + per * 3, fixed + per * (size_t)(samples - 1) };
    const int chunks[] = { 1, 3, samples - 1 };
    float worst = 0.0f;
    for (int i = 0; i < 3; i++) {
        kernix_model_set_workspace_limit(m, limits[i]);
        y = kernix_model_forward(m, x);
        CHECK(y != NULL && y->row == samples && y->col == m->out_dim && m->batch == chunks[i] * T);
        const float d = y != NULL ? max_abs(y, want) : 1.0f;
        worst = d > worst ? d : worst;
    }
    kernix_model_set_workspace_limit(m, fixed + per * 3);
    kernix_model_forward(m, x);
    const float_tensor x3 = { 3 * T, x->col, x->tensor }, want3 = { 3, want->col, want->tensor };
    y = kernix_model_forward(m, &x3);
    CHECK(y != NULL && m->batch == 3 * T);
    const float d3 = y != NULL ? max_abs(y, &want3) : 1.0f;
    kernix_model_trim(m);
    int empty = m->batch == -1 && m->in_copy == NULL && m->out_all == NULL;
    for (int i = 0; i < m->n_steps; i++) empty &= m->steps[i].buf == NULL && m->steps[i].tmp[0] == NULL && m->steps[i].deq == NULL;
    CHECK(empty);
    y = kernix_model_forward(m, x);
    const float dt = y != NULL ? max_abs(y, want) : 1.0f;
    printf("  %-18s chunked %.1e, reuse after chunks %.1e, after trim %.1e\n", name, worst, d3, dt);
    CHECK(worst <= tol && d3 <= tol && dt <= tol);
    float_free(want);
}

static void check_chunk(void)
{
    float_tensor* x = float_zeros(10, 8);
    for (int i = 0; i < 80; i++) x->tensor[i] = (float)((i * 29) % 17 - 8) * 0.2f;
    kernix_model* m = kernix_model_load(path_of("inplace_first.knx"));
    if (m != NULL) check_chunk_model(m, x, "inplace_first", 1e-5f); else fails++;
    kernix_model_free(m);
    float_free(x);
    float_tensor* xs = load_tensor("small_x_37.bin");
    m = kernix_model_load(path_of("small.knx"));
    if (m != NULL) check_chunk_model(m, xs, "small (MLP)", 1e-5f); else fails++;
    kernix_model_free(m);
    float_free(xs);
    write_lstm_model("chunk_lstm.knx");
    x = float_zeros(10 * 4, 7);
    for (int i = 0; i < 10 * 4 * 7; i++) x->tensor[i] = (float)((i * 37) % 23 - 11) * 0.1f;
    m = kernix_model_load(path_of("chunk_lstm.knx"));
    if (m != NULL) check_chunk_model(m, x, "LSTM x2", 1e-5f); else fails++;
    kernix_model_free(m);
    float_free(x);
}

/* int8 kernel vs the reference definition (int64 accumulation of the same int8 values) */
static void ref_qmatmul(const float* x, int rows, int k, int n, const int8_t* q, const float* scale, const float* bias,
                        int accumulate, float* y)
{
    for (int i = 0; i < rows; i++) {
        const float* xr = x + (size_t)i * k;
        float m = 0.0f;
        for (int j = 0; j < k; j++) m = fmaxf(m, fabsf(xr[j]));
        const float sx = m > 0.0f ? m / 127.0f : 1.0f, inv = 1.0f / sx;
        for (int c = 0; c < n; c++) {
            int64_t s = 0;
            for (int j = 0; j < k; j++) {
                float v = rintf(xr[j] * inv);
                v = v > 127.0f ? 127.0f : v < -127.0f ? -127.0f : v;
                s += (int64_t)v * q[(size_t)j * n + c];
            }
            float r = (float)s * sx;
            r = r * scale[c];
            r = r + (bias ? bias[c] : 0.0f);
            y[(size_t)i * n + c] = accumulate ? y[(size_t)i * n + c] + r : r;
        }
    }
}

static void check_qmatmul(void)
{
    const int cases[][3] = { { 55, 31, 1 }, { 64, 256, 1 }, { 128, 512, 3 }, { 114, 512, 32 }, { 16, 16, 1 }, { 1, 1, 1 } };
    float worst = 0.0f;
    lcg = 12345;
    for (int c = 0; c < 6; c++) {
        const int k = cases[c][0], n = cases[c][1], rows = cases[c][2];
        int8_t* q = malloc((size_t)k * n);
        float *scale = malloc(sizeof(float) * n), *bias = malloc(sizeof(float) * n), *x = malloc(sizeof(float) * rows * k);
        float *y = malloc(sizeof(float) * rows * n), *want = malloc(sizeof(float) * rows * n);
        for (size_t i = 0; i < (size_t)k * n; i++) q[i] = (int8_t)((int)(lcg_next() % 255) - 127);
        for (int i = 0; i < n; i++) { scale[i] = 0.001f + (float)(lcg_next() % 1000) * 1e-5f; bias[i] = (float)(lcg_next() % 200) * 0.01f - 1.0f; }
        for (int i = 0; i < rows * k; i++) x[i] = (float)(lcg_next() % 2001) * 0.003f - 3.0f;
        kernix_qweight* w = kernix_qweight_pack(q, scale, k, n);
        CHECK(w != NULL);
        if (w == NULL) continue;
        for (int acc = 0; acc < 2; acc++) {
            for (int i = 0; i < rows * n; i++) y[i] = want[i] = (float)(i % 7) * 0.5f;
            CHECK(kernix_qmatmul(x, rows, w, bias, acc, y) == 0);
            ref_qmatmul(x, rows, k, n, q, scale, bias, acc, want);
            float mx = 1e-30f, d = 0.0f;
            for (int i = 0; i < rows * n; i++) { mx = fmaxf(mx, fabsf(want[i])); d = fmaxf(d, fabsf(y[i] - want[i])); }
            worst = fmaxf(worst, d / mx);
        }
        if (rows >= 3) { /* NaN row → all NaN; zero row → exactly bias */
            x[k] = NAN;
            for (int j = 0; j < k; j++) x[2 * k + j] = 0.0f;
            CHECK(kernix_qmatmul(x, rows, w, bias, 0, y) == 0);
            int nan_ok = 1, other_ok = 1, zero_ok = 1;
            ref_qmatmul(x, 1, k, n, q, scale, bias, 0, want);
            for (int j = 0; j < n; j++) {
                nan_ok &= isnan(y[n + j]);
                other_ok &= fabsf(y[j] - want[j]) <= 1e-5f * fmaxf(1.0f, fabsf(want[j]));
                zero_ok &= y[2 * n + j] == bias[j];
            }
            CHECK(nan_ok && other_ok && zero_ok);
        }
        kernix_qweight_free(w);
        free(q); free(scale); free(bias); free(x); free(y); free(want);
    }
    const int bk = KERNIX_INT8_MAX_K; /* −128 boundary: 128·127·K < 2³¹ */
    int8_t* q = malloc(bk);
    float* x = malloc(sizeof(float) * bk);
    for (int i = 0; i < bk; i++) { q[i] = -128; x[i] = 1.0f; }
    const float one = 1.0f;
    kernix_qweight* w = kernix_qweight_pack(q, &one, bk, 1);
    float y = 0.0f;
    CHECK(w != NULL && kernix_qmatmul(x, 1, w, NULL, 0, &y) == 0);
    CHECK(y == (float)(-128.0 * 127.0 * bk) * (1.0f / 127.0f));
    kernix_qweight_free(w);
    free(q);
    free(x);
    printf("  int8 kernel max rel err vs reference %.1e\n", worst);
    CHECK(worst <= 1e-5f);
}

static void ref_qlstm_layer(const float* x, int B, int in, int u, int ret, const float* w, const float* b, const int8_t* q,
                            const float* sc, int deq, float* out)
{
    const int T = 4, g = 4 * u;
    for (int s = 0; s < B; s++) {
        float h[8] = { 0 }, c[8] = { 0 }, z[32], hu[32];
        for (int t = 0; t < T; t++) {
            for (int j = 0; j < g; j++) {
                double a = b[j];
                for (int k = 0; k < in; k++) a += (double)x[(s * T + t) * in + k] * w[k * g + j];
                if (deq) for (int k = 0; k < u; k++) a += (double)h[k] * ((float)q[k * g + j] * sc[j]);
                z[j] = (float)a;
            }
            if (!deq && t > 0) { ref_qmatmul(h, 1, u, g, q, sc, NULL, 0, hu); for (int j = 0; j < g; j++) z[j] += hu[j]; }
            for (int k = 0; k < u; k++) {
                const int act = u == 5 ? KERNIX_ACT_TANH : KERNIX_ACT_RELU;
                c[k] = r_sig(z[u + k]) * c[k] + r_sig(z[k]) * r_act(act, z[2 * u + k]);
                h[k] = r_sig(z[3 * u + k]) * r_act(act, c[k]);
                if (ret) out[(s * T + t) * u + k] = h[k];
            }
        }
        if (!ret) memcpy(out + s * u, h, sizeof(float) * (size_t)u);
    }
}

static void ref_qlstm(const qlstm_ref* r, const float* x, int B, int deq, float* y)
{
    float h1[40 * 4 * 5], h2[40 * 6];
    ref_qlstm_layer(x, B, 7, 5, 1, r->w1, r->b1, r->u1, r->s1, deq, h1);
    ref_qlstm_layer(h1, B, 5, 6, 0, r->w2, r->b2, r->u2, r->s2, deq, h2);
    for (int s = 0; s < B; s++) {
        if (deq) {
            for (int j = 0; j < 3; j++) {
                double a = r->bd[j];
                for (int k = 0; k < 6; k++) a += (double)h2[s * 6 + k] * ((float)r->d[k * 3 + j] * r->sd[j]);
                y[s * 3 + j] = (float)a;
            }
        } else {
            ref_qmatmul(h2 + s * 6, 1, 6, 3, r->d, r->sd, r->bd, 0, y + s * 3);
        }
    }
}

static void check_v2_forward(void)
{
    /* KNX1 vs the same weights as KNX2 F32 blocks: identical bits */
    write_lstm_model("chunk_lstm.knx");
    vbn = 0; vput(MAGIC2); vput(3);
    size_t p = 2;
    const size_t parts[3][4] = { { 6, 7 * 20, 5 * 20, 20 }, { 6, 5 * 24, 6 * 24, 24 }, { 4, 6 * 3, 0, 0 } };
    for (int op = 0; op < 3; op++) {
        for (size_t i = 0; i < parts[op][0]; i++) vput(fw[p++]);
        for (int t = 1; t < 4; t++) {
            if (parts[op][t] == 0) continue;
            if (t < 3) vput(KERNIX_DT_F32);
            for (size_t i = 0; i < parts[op][t]; i++) vput(fw[p++]);
        }
    }
    write_file("v2f.knx", vb, vbn);
    kernix_model *m1 = kernix_model_load(path_of("chunk_lstm.knx")), *m2 = kernix_model_load(path_of("v2f.knx"));
    float_tensor* x = float_zeros(40 * 4, 7);
    for (int i = 0; i < 40 * 4 * 7; i++) x->tensor[i] = (float)((i * 37) % 23 - 11) * 0.1f;
    CHECK(m1 != NULL && m2 != NULL);
    if (m1 != NULL && m2 != NULL) {
        const float_tensor* y1 = kernix_model_forward(m1, x);
        float keep[40 * 3];
        if (y1) memcpy(keep, y1->tensor, sizeof keep);
        const float_tensor* y2 = kernix_model_forward(m2, x);
        CHECK(y1 != NULL && y2 != NULL && memcmp(keep, y2->tensor, sizeof keep) == 0);
    }
    kernix_model_free(m1);
    kernix_model_free(m2);

    static qlstm_ref r;
    write_qlstm_model("qlstm.knx", &r);
    kernix_model* m = kernix_model_load(path_of("qlstm.knx"));
    if (m != NULL) {
        float want[40 * 3], y40[40 * 3];
        const int Bs[4] = { 1, KERNIX_INT8_MAX_ROWS, KERNIX_INT8_MAX_ROWS + 1, 40 };
        float err_i8 = 0.0f, err_deq = 0.0f;
        for (int bi = 0; bi < 4; bi++) {
            const int B = Bs[bi], deq = B > KERNIX_INT8_MAX_ROWS;
            const float_tensor xb = { B * 4, 7, x->tensor };
            const float_tensor* y = kernix_model_forward(m, &xb);
            CHECK(y != NULL && y->row == B);
            if (y == NULL) continue;
            ref_qlstm(&r, x->tensor, B, deq, want);
            float d = 0.0f;
            for (int i = 0; i < B * 3; i++) d = fmaxf(d, fabsf(y->tensor[i] - want[i]));
            if (deq) err_deq = fmaxf(err_deq, d); else err_i8 = fmaxf(err_i8, d);
            if (B == 40) memcpy(y40, y->tensor, sizeof y40);
            for (int i = 0; i < m->n_steps; i++)
                if (m->steps[i].q != NULL) CHECK((m->steps[i].deq != NULL) == deq); /* fp32 copy only above 2 rows */
        }
        float path = 0.0f;
        for (int s = 0; s < 40; s++) {
            const float_tensor xs = { 4, 7, x->tensor + s * 4 * 7 };
            const float_tensor* y = kernix_model_forward(m, &xs);
            for (int j = 0; y != NULL && j < 3; j++) path = fmaxf(path, fabsf(y->tensor[j] - y40[s * 3 + j]));
        }
        printf("  int8 LSTM x2 + Linear: int8 path %.1e, fp32-copy path %.1e, paths differ %.1e\n", err_i8, err_deq, path);
        CHECK(err_i8 <= 1e-5f && err_deq <= 1e-5f && path <= 1e-2f);
        check_chunk_model(m, x, "int8 LSTM", 1e-2f);
        kernix_model_set_workspace_limit(m, m->ws_fixed * sizeof(float) + m->ws_per_sample * sizeof(float) * 3);
        const float_tensor x10 = { 10 * 4, 7, x->tensor };
        CHECK(kernix_model_forward(m, &x10) != NULL && m->batch == 3 * 4);
        for (int i = 0; i < m->n_steps; i++)
            if (m->steps[i].q != NULL) CHECK(m->steps[i].deq != NULL);
    } else {
        fails++;
    }
    kernix_model_free(m);
    float_free(x);
}

int main(int argc, char** argv)
{
    if (argc != 3) { printf("usage: %s cpu|gpu <dir>\n", argv[0]); return 2; }
    snprintf(dir, sizeof dir, "%s", argv[2]);
    if (strcmp(argv[1], "cpu") == 0) {
        check_load();
        check_lstm_load();
        check_v2_load();
        check_qweight_pack();
        check_ws_fixed();
    } else {
        check_forward();
        check_lstm();
        check_chunk();
        check_qmatmul();
        check_v2_forward();
    }
    printf("%s: %d failed check(s)\n", argv[1], fails);
    return fails ? 1 : 0;
}
