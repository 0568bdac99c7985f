/* knx_internal.h — private declarations shared by the host runtime files (loader, workspace/forward, C ABI). */
#ifndef KNX_INTERNAL_H
#define KNX_INTERNAL_H

#include <stdio.h>

#include "kernix_model.h"
#include "knx_hip.h"

/* Device copies of one step's parameters, uploaded on the first forward and kept until kernix_model_free. */
struct knx_dstep {
    float* w;         /* LINEAR / CONV fp32 weight and ATTENTION Wq stored transposed (out × in); EMBEDDING table;
                         RNN input weight (in × gates, as in the file) */
    float* bias;
    float* gamma;
    float* beta;
    float* cst;
    int8_t* q;        /* int8 weight, np × kp (output channel rows, k contiguous) */
    float* qscale;    /* np scales */
    float* rec;       /* RNN fp32 recurrent weight */
    float* w_b;       /* backward direction */
    float* bias_b;
    int8_t* q_b;
    float* qscale_b;
    float* rec_b;
    float* wk;        /* ATTENTION */
    float* wv;
    float* wo;
    float* bk;
    float* bv;
    float* bo;
    float* wqkv;      /* self-attention: [Wqᵀ; Wkᵀ; Wvᵀ], (2·H·dk + H·dv) × in (replaces w, wk, wv) */
    float* bqkv;      /* [bq | bk | bv] or NULL */
    float* half;      /* RNN AVE merge: u × 0.5 */
    float* zero;      /* u × 0 */
    /* per-chunk scratch inside the workspace arena */
    int8_t* xq;       /* int8 input rows (rows × kp) */
    float* sx;        /* their scales */
    int xq_rows;
};

/* Device side of a model. */
#define KNX_RING_SLOTS 4 /* pinned staging buffers of a host-buffer forward's input copies */

struct knx_dmodel {
    int device;       /* the device current at the model's first forward: every later call runs on it */
    void* stream;     /* hipStream_t owned by the model */
    int uploaded;     /* weights on the device */
    void* arena;      /* workspace: storage buffers, step scratch, dequantized copies, input staging */
    size_t arena_bytes;
    float* d_in;      /* device copy of the current chunk's input */
    void* chain;      /* scratch of knx_hip_linear_chain (barrier words, zero between launches; partial maxima) */
    size_t chain_bytes;
    int* chain_status;  /* pinned host word: set by a chain launch of this model whose barrier stopped waiting */
    int no_chain;       /* a host forward recomputing without chains after such a launch */
    float* h_out;     /* pinned host output of an unchunked forward (batch × out_dim) */
    size_t h_out_floats;
    int out_all_pinned; /* out_all->tensor was allocated pinned */
    void* done;         /* event marking the end of the last forward (see knx_forward.c, ordering between forwards) */
    int done_recorded;  /* `done` has been recorded after the last forward */
    int have_last;      /* a forward (or workspace set-up) has been enqueued */
    void* last_stream;  /* the stream it was enqueued on */
    /* host-buffer forwards of large batches: input copies on their own stream, overlapped with the compute of the
     * previous piece (created on first use) */
    void* copy_stream;
    void* ev_in[2];     /* piece's input copied into half h of d_in */
    void* ev_used[2];   /* the compute that reads half h of d_in has been enqueued before this point */
    /* pinned staging ring for input copies from pageable host memory (created on first use) */
    void* ring[KNX_RING_SLOTS];
    void* ring_ev[KNX_RING_SLOTS];   /* the copy out of slot k has completed after this event */
    int ring_next;
    /* pinned staging of a small host input, read by a copy kernel (grown on use to the largest piece, ≤ 1 MB) */
    void* stage;
    size_t stage_bytes;
    int stage_pending;  /* a copy kernel reading `stage` may not have completed (no stream synchronization since) */
    /* a channels-first host input piece on the device, before its per-sample transpose into d_in (grown on use,
     * released with the workspace) */
    float* cf_in;
    size_t cf_in_floats;
};

/* A decoded .knx file: its header and op records in file order (inputs, arguments, host weights). */
typedef struct {
    int version;                    /* 1, 2 or 3 */
    int layout;                     /* KNX3 input layout (0 channels-last, 1 channels-first) */
    int in_nd, in_d[KERNIX_MAX_DIMS]; /* KNX3 per-sample input shape */
    int n_ops;
    kernix_step* ops;
} knx_file;

/* decoder (knx_decode.c) */
int knx_decode(const char* path, knx_file* f, const char** why); /* 0, or -1 with the reason in *why */
void knx_file_release(knx_file* f);

/* graph, shapes and storage plan (knx_graph.c) */
size_t knx_conv_is_gemm(const kernix_step* s);
void knx_step_host_free(kernix_step* s);
int knx_storage_overlaps(const kernix_model* m, int a, int b); /* values a, b share storage in a chunk */

/* workspace / device (knx_forward.c) */
int knx_model_count_ws(kernix_model* m, size_t* per_sample); /* floats per sample of workspace, 0 or -1 */

/* workspace / device (knx_forward.c) */
void knx_model_release_device_ws(kernix_model* m);
void knx_model_release_device_all(kernix_model* m);
/* memcpy of n bytes on the calling thread and a process-wide pool of copying threads (plain below 256 KB) */
void knx_copy_parallel(void* dst, const void* src, size_t n);

/* messages */
#define KNX_LOG(...) fprintf(stderr, __VA_ARGS__)

#endif
