/* kernix_model.h — KERNIX model runtime API (load / forward), MI355X build.
 *
 * Same public names, argument meaning and error behaviour as the reference's header-only runtime
 * (reference include/kernix_model.h); here it is a compiled library (libkernix.so) whose forward runs on one MI355X
 * through hand-written gfx950 kernels (include/knx_hip.h).  Nothing in the forward path runs on the CPU except
 * argument checks, the host→device copy of the input and the device→host copy of the output.
 *
 * Public entry points and the reference interface each one keeps:
 *   kernix_model_load                 reference include/kernix_model.h:1448   (.knx KNX1/KNX2/KNX3, untrusted input)
 *   kernix_model_forward              reference include/kernix_model.h:2023   (returns a model-owned host tensor)
 *   kernix_model_free                 reference include/kernix_model.h:367
 *   kernix_model_trim                 reference include/kernix_model.h:343    (frees the device workspace, keeps weights)
 *   kernix_model_set_workspace_limit  reference include/kernix_model.h:1691
 *   kernix_model_set_ane              reference include/kernix_model.h:1815   (always -1: no Neural Engine here)
 *   kernix_model_ane_info             reference include/kernix_model.h:1831   (all zeros)
 *   kernix_qweight_pack / _unpack     reference include/kernix_model.h:73-95
 *   kernix_qmatmul                    reference include/kernix_model.h:99-182 (runs on the GPU; host pointers)
 *
 * Values (graph edges) are channels-last per sample and stored as (batch·rows) × channels, exactly as the reference.
 * Device memory is owned by the model: weights are uploaded on the first forward and kept until free; the workspace
 * (storage buffers, attention scratch, dequantized int8 copies) is allocated per chunk size and released by trim.
 *
 * Differences that a caller can observe (all deliberate):
 *   - the default workspace limit is KERNIX_WORKSPACE_LIMIT = 1 GiB of device memory (reference: 64 MB of host memory);
 *   - ws_fixed counts only the dequantized int8 copies: convolution is an implicit GEMM and has no im2col buffer;
 *   - steps[i].buf, .tmp[] and .deq point at device memory; .deq holds the weight transposed (out × in, the
 *     device layout of every fp32 Linear weight: both GEMM operands K-contiguous).
 */
#ifndef KERNIX_MODEL_H
#define KERNIX_MODEL_H

#include "kernix.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Op ids (file ABI). */
enum {
    KERNIX_OP_LINEAR, KERNIX_OP_ACT, KERNIX_OP_LAYERNORM, KERNIX_OP_SOFTMAX, KERNIX_OP_LSTM,
    KERNIX_OP_GRU, KERNIX_OP_RNN, KERNIX_OP_CONV, KERNIX_OP_POOL, KERNIX_OP_GLOBAL_POOL,
    KERNIX_OP_RESHAPE, KERNIX_OP_PERMUTE, KERNIX_OP_BINARY, KERNIX_OP_CONCAT, KERNIX_OP_EMBEDDING,
    KERNIX_OP_AFFINE, KERNIX_OP_ADD_CONST, KERNIX_OP_ATTENTION, KERNIX_OP_SELECT, KERNIX_OP_PAD,
    KERNIX_OP_UPSAMPLE,
    KERNIX_OP_LAST = KERNIX_OP_UPSAMPLE
};
enum { KERNIX_BIN_ADD, KERNIX_BIN_SUB, KERNIX_BIN_MUL, KERNIX_BIN_DIV, KERNIX_BIN_MAX, KERNIX_BIN_MIN };
enum { KERNIX_MERGE_CONCAT, KERNIX_MERGE_SUM, KERNIX_MERGE_MUL, KERNIX_MERGE_AVE };
enum { KERNIX_POOL_MAX, KERNIX_POOL_AVG };
enum { KERNIX_AXIS_FIRST, KERNIX_AXIS_LAST };
enum { KERNIX_DT_F32, KERNIX_DT_I8_COL, KERNIX_DT_I8_ROW };

#define KERNIX_MAX_DIMS 4
#define KERNIX_MAX_INPUTS 8
#define KERNIX_MAX_GEOM 65536
#define KERNIX_MODEL_MAX_OPS 1024
#define KERNIX_CHUNK 8192          /* RNN units bound (2·units per gate pass), as the file format allows */

/* int8 limits: 128·127·K < 2³¹ keeps the int32 accumulator exact. */
#define KERNIX_INT8_MAX_K 131072
/* Rows at or below this run the int8 arithmetic in the default ("ref") mode; more rows use the fp32 copy. */
#define KERNIX_INT8_MAX_ROWS 2

#ifndef KERNIX_WORKSPACE_LIMIT
#define KERNIX_WORKSPACE_LIMIT ((size_t)1 << 30)
#endif

/* Int8 weight, symmetric per output channel: w[k][n] ≈ q·scale[n].
 * Layout (this build): q is np × kp, row n holds output channel n with k contiguous, zero padded; kp is a multiple
 * of 64 (one i8-MFMA k-step), np a multiple of 16.  scale has np entries, padded with 0. */
typedef struct kernix_qweight {
    int k, n;
    int kp, np;
    int8_t* q;
    float* scale;
} kernix_qweight;

/* One graph value (edge). Stored as (batch·r) × c. */
typedef struct {
    int nd, d[KERNIX_MAX_DIMS]; /* per-sample shape, channels-last */
    int r, c;                   /* rows per sample (product of leading axes), channels */
    int st;                     /* storage buffer index, -1 = the caller's input (read-only) */
    int last;                   /* last step that reads this value (n_steps for the model output) */
} kernix_val;

struct knx_dstep; /* device-side state of a step (uploaded weights), private to the library */

typedef struct {
    int kind;
    int act;                    /* fused activation for LINEAR/CONV, activation for ACT/RNN */
    float alpha;
    int n_in, inp[KERNIX_MAX_INPUTS];
    int in, out;
    float_tensor* w;            /* host fp32 weights (in×out layout as in the file); NULL if kept as int8 */
    float* bias;
    float* gamma;
    float* beta;
    float eps;
    float_tensor* buf;          /* device view of the output value (while a workspace is allocated) */
    float* rec;                 /* RNN recurrent weights units×G·units (host) */
    int seq;
    int ret_seq;
    int dirs, merge;
    float_tensor* w_b;
    float* rec_b;
    float* bias_b;
    kernix_qweight* q_b;
    float_tensor* deq_b;
    float_tensor* tmp[6];       /* device scratch per step (attention Q/K/V/context, RNN gates) */
    kernix_qweight* q;          /* int8 weights (LINEAR w or RNN rec) */
    float_tensor* deq;          /* device fp32 copy of q, allocated only when the chunk has > KERNIX_INT8_MAX_ROWS rows
                                   in the default int8 mode */
    int kh, kw, sh, sw, dh, dw, pt, pb, pl, pr, groups;
    int ptype, count_pad;
    int perm[KERNIX_MAX_DIMS];
    int nd, d[KERNIX_MAX_DIMS];
    int axis, start, len, squeeze;
    int bop;
    int heads, dk, dv, causal;
    float_tensor* wk;
    float_tensor* wv;
    float_tensor* wo;
    float* bk;
    float* bv;
    float* bo;
    float* cst;
    struct knx_dstep* dev;      /* uploaded weights; NULL before the first forward */
} kernix_step;

typedef struct { int segments, compiles, ane_runs, failures; } kernix_ane_info;

/* int8 execution mode for LINEAR/RNN int8 weights. */
enum {
    KERNIX_INT8_REF = 0, /* reference dispatch: int8 arithmetic at ≤ KERNIX_INT8_MAX_ROWS rows, fp32 copy above */
    KERNIX_INT8_I8 = 1   /* int8 arithmetic (i8 MFMA) at every row count */
};

struct knx_dmodel;

typedef struct kernix_model {
    int n_steps;
    int in_dim, out_dim;
    int seq_len;
    int batch;                 /* input rows the workspace is allocated for, -1 if none */
    kernix_step* steps;
    float_tensor* in_copy;     /* always NULL (kept for source compatibility) */
    float_tensor* out_all;     /* host output of a chunked forward (batch × out_dim) */
    size_t ws_limit;           /* device workspace bound in bytes, 0 = none */
    size_t ws_per_sample;      /* workspace floats per sample */
    size_t ws_fixed;           /* batch-independent workspace floats (dequantized int8 copies) */
    int n_vals;
    int out_v;
    kernix_val* vals;
    float_tensor* views;       /* views[v]: device tensor of value v in the current chunk */
    float_tensor out_view;     /* host output of an unchunked forward */
    int n_st;
    size_t* st_cap;            /* floats per sample of each storage buffer */
    float_tensor** st;         /* device storage buffers */
    size_t* st_off;            /* per-sample float offset of each storage buffer in the value region (buffers whose
                                  values are never live at the same step may overlap) */
    size_t st_span;            /* floats per sample of the value region */
    int in_nd, in_shape[KERNIX_MAX_DIMS];
    int out_nd, out_shape[KERNIX_MAX_DIMS];
    int layout;                /* 0 channels-last input, 1 PyTorch channels-first (the binding moves the axis) */
    float_tensor* col;         /* always NULL: implicit-GEMM convolution needs no im2col buffer */
    int ane;                   /* always 0 */
    int int8_mode;             /* KERNIX_INT8_REF (default) or KERNIX_INT8_I8; env KERNIX_INT8_MODE=i8 sets I8 at load */
    struct knx_dmodel* dev;    /* device state: stream, uploaded weights, input/output staging */
} kernix_model;

KERNIX_API kernix_model* kernix_model_load(const char* path);
KERNIX_API const float_tensor* kernix_model_forward(kernix_model* m, const float_tensor* x);
KERNIX_API void kernix_model_free(kernix_model* m);
KERNIX_API void kernix_model_trim(kernix_model* m);
KERNIX_API void kernix_model_set_workspace_limit(kernix_model* m, size_t bytes);
KERNIX_API int kernix_model_set_ane(kernix_model* m, int on);
KERNIX_API void kernix_model_ane_info(const kernix_model* m, kernix_ane_info* out);

/* Extensions of this build (no counterpart in the reference). */
/* Select the int8 mode (KERNIX_INT8_REF / KERNIX_INT8_I8). 0, or -1 on a bad mode. */
KERNIX_API int kernix_model_set_int8_mode(kernix_model* m, int mode);
/* Forward with the input already in device memory: d_x is rows × in_dim, d_out receives (rows/seq_len) × out_dim,
 * both device pointers; stream is a hipStream_t (NULL = the model's own stream). Work is stream-ordered; the call
 * returns after enqueueing (it synchronizes only when it has to allocate). 0 or -1. */
KERNIX_API int kernix_model_forward_device(kernix_model* m, const float* d_x, int rows, float* d_out, void* stream);
/* kernix_model_forward with each sample of x in channels-first order (C × the spatial positions, the PyTorch layout)
 * for a model whose file records layout 1: the input is copied as it is and transposed on the device, where the
 * reference's binding moves the axis on the host first.  Same rows, output and errors as kernix_model_forward; for a
 * layout-0 model, or one row per sample, it is kernix_model_forward. */
KERNIX_API const float_tensor* kernix_model_forward_cf(kernix_model* m, const float_tensor* x);
/* Waits for the model's last forward and reports the device forwards since the previous call: -1 if one of them ran a
 * Linear chain whose workgroups could not all be resident (more chains running at once than the GPU holds), so its
 * outputs are wrong and it must be run again; else 0.  Host-buffer forwards recompute such a forward themselves. */
KERNIX_API int kernix_model_device_status(kernix_model* m);

KERNIX_API kernix_qweight* kernix_qweight_pack(const int8_t* q, const float* scale, int k, int n);
KERNIX_API void kernix_qweight_unpack(const kernix_qweight* w, float* dst);
KERNIX_API void kernix_qweight_free(kernix_qweight* w);
/* y[r] = (accumulate ? y[r] : 0) + x[r]·W + bias, r < rows; host pointers, computed on the GPU with the reference's
 * int8 semantics (dynamic per-row int8 input, int32 accumulation, ((float)acc·sx)·scale + bias). 0, or -1. */
KERNIX_API int kernix_qmatmul(const float* x, int rows, const kernix_qweight* w, const float* bias, int accumulate, float* y);

#ifdef __cplusplus
}
#endif

#endif
