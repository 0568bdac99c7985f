/* knx_hip.h — thin C ABI between the KERNIX host runtime (C) and the hand-written gfx950 kernels (HIP).
 *
 * Every function takes plain device pointers, sizes and a stream (a hipStream_t passed as void*, NULL = the null
 * stream), enqueues its work and returns without synchronizing.  Return value: KNX_OK (0) or a negative KNX_E*
 * code; the message of the last failure is available from knx_hip_last_error().  Arguments are checked on the host
 * before any launch, so a bad shape is an error, never an out-of-bounds kernel.
 *
 * Fault injection for tests: if the environment variable KNX_HIP_FAIL names an entry point (e.g.
 * "knx_hip_sgemm_ep") or is "all", that entry point returns KNX_EINJECT without touching the device.
 *
 * Reference interfaces replaced (reference paths, file:line):
 *   knx_hip_quantize_rows   per-row int8 input quantization of kernix_qmatmul   include/kernix_model.h:112-142
 *   knx_hip_i8gemm          int32 sdot accumulation + dequant/bias epilogue     include/kernix_model.h:143-178
 *                           with the activation pass fused                      include/kernix_model.h:1854-1856
 *   knx_hip_dequant(_t)     kernix_qweight_unpack into the fp32 copy            include/kernix_model.h:91-95, :1616-1622
 *   knx_hip_sgemm_ep /      kernix_matmul_ep_into (MPS+AMX row split)          src/kernix_metal.m:161-265,
 *   knx_hip_sgemm_nt_ep
 *                           + kernix_bias_act epilogue                          include/kernix.h:951-977,
 *                                                                               include/kernix_model.h:528-550
 *   knx_hip_conv(_t)        kernix_conv_run (im2col → sgemm → bias_act)         include/kernix_model.h:711-771
 *   knx_hip_sgemm_nt_ep_res, a LINEAR (or CONV, or ATTENTION's output projection)  include/kernix_model.h:1853-1860,
 *   knx_hip_conv_t_res,     step followed by the BINARY add of another value:    :1005-1048, :877-906
 *   knx_hip_i8gemm_res      the step's epilogue adds the other operand
 *   knx_hip_layernorm       kernix_layer_norm_rows_into                         include/kernix.h:667-677
 *   knx_hip_layernorm_quantize  a LAYERNORM whose rows feed only an int8 LINEAR: include/kernix.h:667-677, then
 *                           kernix_qmatmul's row quantization               include/kernix_model.h:112-142
 *   knx_hip_softmax         floats_softmax_into                                 include/kernix.h:652-657
 *   knx_hip_bias_act        kernix_bias_act / ACT step                          include/kernix_model.h:528-541, :1866-1869
 *   knx_hip_binary          kernix_binary_run                                   include/kernix_model.h:877-906
 *   knx_hip_global_pool     kernix_global_pool_run                              include/kernix_model.h:810-830
 *   knx_hip_attention_core  per-(b,h) QKᵀ·scale, mask, softmax, ·V             include/kernix_model.h:1021-1046
 *   knx_hip_affine          AFFINE step                                         include/kernix_model.h:1882-1891
 *   knx_hip_add_const       ADD_CONST step                                      include/kernix_model.h:1892-1896
 *   knx_hip_pool            kernix_pooling_run                                  include/kernix_model.h:773-807
 *   knx_hip_permute         kernix_permute_run                                  include/kernix_model.h:833-862
 *   knx_hip_copy_cols       CONCAT (last axis) / SELECT (last axis)             include/kernix_model.h:908-949
 *   knx_hip_pad             kernix_pad_run                                      include/kernix_model.h:951-968
 *   knx_hip_upsample        kernix_upsample_run                                 include/kernix_model.h:970-984
 *   knx_hip_embedding       kernix_embedding_run                                include/kernix_model.h:987-1000
 *   knx_hip_rnn_gates       per-timestep gate update of kernix_rnn_dir          include/kernix_model.h:580-631
 *   knx_hip_rnn_recurrence  one RNN direction's timesteps in one launch         include/kernix_model.h:563-632
 *   knx_hip_rnn_recurrence_dense  the same and the LINEAR on its last state    include/kernix_model.h:563-632,
 *                                                                               :1843-1860
 *   knx_hip_linear_chain    consecutive LINEAR steps of a small batch           include/kernix_model.h:1843-1860,
 *                           (kernix_step_run layer after layer, int8 ones       :99-182
 *                           through kernix_qmatmul)
 */
#ifndef KNX_HIP_H
#define KNX_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KNX_API __attribute__((visibility("default")))

enum {
    KNX_OK = 0,
    KNX_EINVAL = -1,   /* bad argument (shape, pointer, enum) */
    KNX_EHIP = -2,     /* HIP runtime error (allocation, launch, copy) */
    KNX_ENODEV = -3,   /* no usable gfx950 device */
    KNX_EINJECT = -4   /* failure injected through KNX_HIP_FAIL */
};

/* ---- runtime ---- */
KNX_API int knx_hip_init(void);              /* checks the calling thread's current device; KNX_ENODEV unless gfx950 */
KNX_API int knx_hip_get_device(int* device); /* the current device of the calling thread */
KNX_API int knx_hip_set_device(int device);
KNX_API const char* knx_hip_last_error(void);
KNX_API int knx_hip_malloc(void** p, size_t bytes);
KNX_API int knx_hip_free(void* p);
KNX_API int knx_hip_host_malloc(void** p, size_t bytes); /* pinned host memory */
KNX_API int knx_hip_host_free(void* p);
KNX_API int knx_hip_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
KNX_API int knx_hip_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
KNX_API int knx_hip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
KNX_API int knx_hip_stream_create(void** stream);
KNX_API int knx_hip_stream_destroy(void* stream);
KNX_API int knx_hip_stream_sync(void* stream);
/* Events (hipEvent_t as void*, created without timing): the runtime orders forwards issued on different streams. */
KNX_API int knx_hip_event_create(void** event);
/* An event that only orders this device's kernels: recording it performs no system-scope cache write-back or
 * invalidation, so it must not publish data written by copies (host-to-device) or read by the host; for ordering
 * kernels of one stream after kernels of another and for the host waiting until they are done. */
KNX_API int knx_hip_event_create_ordering(void** event);
KNX_API int knx_hip_event_destroy(void* event);
KNX_API int knx_hip_event_record(void* event, void* stream);
KNX_API int knx_hip_stream_wait_event(void* stream, void* event); /* later work on stream waits for the event */
KNX_API int knx_hip_event_sync(void* event);                      /* the host waits for the event */

/* ---- int8 path ---- */
/* Per row r < rows of x (row stride ldx floats, k values): m = max|x|; a NaN or ±inf makes sx[r] = NaN (the whole
 * output row becomes NaN); else sx = m > 0 ? m/127 : 1, inv = 1/sx, xq = clamp(rint(x·inv), −127, 127).
 * xq rows have stride ldq bytes; columns [k, kp) are written as 0 (kp ≤ ldq, kp multiple of 64). */
KNX_API int knx_hip_quantize_rows(const float* x, int ldx, int rows, int k, int kp, int8_t* xq, int ldq,
                                  float* sx, void* stream);

/* Y[m][n] = act( ((float)acc[m][n] · sa[m]) · sw[n] + bias[n] (+ Y[m][n] if accumulate) ), acc = Σ_k A[m][k]·W[n][k]
 * in int32 (exact for K ≤ KERNIX_INT8_MAX_K).  A is M×K (stride lda bytes), W is N×K (stride ldw bytes), both int8 with
 * K contiguous; K must be a multiple of 64 and lda/ldw multiples of 16 (pad with zeros).  bias may be NULL, act is a
 * KERNIX_ACT_* id (−1 none).  Y (stride ldy floats) may be NULL; acc_out (stride ldacc int32) receives the raw int32
 * accumulators when not NULL.  No FMA contraction: the products and the sum are rounded separately. */
KNX_API int knx_hip_i8gemm(int M, int N, int K, const int8_t* A, int lda, const float* sa, const int8_t* W, int ldw,
                           const float* sw, const float* bias, int act, float alpha, int accumulate, float* Y, int ldy,
                           int32_t* acc_out, int ldacc, void* stream);

/* The same with an elementwise add fused after the activation: Y = act(((float)acc·sa[m])·sw[n] + bias[n]) + R
 * (R M×N, stride ldr; R may equal Y), the result of this LINEAR followed by the BINARY add of R
 * (reference include/kernix_model.h:1853-1860 then :877-906, the same two fp32 roundings). */
KNX_API int knx_hip_i8gemm_res(int M, int N, int K, const int8_t* A, int lda, const float* sa, const int8_t* W,
                               int ldw, const float* sw, const float* bias, int act, float alpha, const float* R,
                               int ldr, float* Y, int ldy, void* stream);

/* kernix_qmatmul and the activation of its LINEAR step in one call (reference include/kernix_model.h:99-182 then
 * :1854-1856): x (rows × k fp32, stride ldx) quantized per row, multiplied by W (n × kp int8), then the epilogue of
 * knx_hip_i8gemm (accumulate adds into Y; R, if not NULL, is added after the activation; not both).  At ≤ 16 rows
 * with rows·k·n ≤ 2^23 one kernel quantizes on the fly (xq and sx are not touched and may then be NULL); otherwise
 * knx_hip_quantize_rows into xq (rows × kp) and sx (rows) and then the GEMM.  Results are the same bits either way. */
KNX_API int knx_hip_qlinear(const float* x, int ldx, int rows, int k, int kp, int8_t* xq, float* sx, const int8_t* W,
                            int ldw, int n, const float* sw, const float* bias, int act, float alpha, int accumulate,
                            const float* R, int ldr, float* Y, int ldy, void* stream);

/* knx_hip_qlinear without caller scratch and without allocating: no counterpart in the reference; for callers that
 * cannot allocate device memory (code under HIP graph capture, fixed serving loops, harnesses that forbid hipMalloc).
 * The int8 rows and row scales go to a device array owned by the library (one per GPU, KNX_QLINEAR_NOALLOC_BYTES,
 * held until the process ends); a call needs ⌈4·rows/256⌉·256 + rows·kp bytes of it and is rejected (KNX_EINVAL)
 * beyond that.  Same kernels, same bits as knx_hip_qlinear.  Every call on one GPU shares the array: calls that
 * overlap on one GPU (different streams or threads) race, so the caller orders them. */
#define KNX_QLINEAR_NOALLOC_BYTES ((size_t)32 << 20)
KNX_API int knx_hip_qlinear_noalloc(const float* x, int ldx, int rows, int k, int kp, const int8_t* W, int ldw, int n,
                                    const float* sw, const float* bias, int act, float alpha, int accumulate,
                                    const float* R, int ldr, float* Y, int ldy, void* stream);

/* ---- a chain of Linear layers over a few rows, one launch ----
 * Layer 0 reads x (rows × k fp32, stride ldx), layer l > 0 reads the output of layer l − 1 (k of layer l = n of layer
 * l − 1); every layer writes y = act(x·Wᵀ + bias) (rows × n, stride ldy).  An int8 layer (i8 = 1; w: n rows of kp
 * int8, stride ldw bytes, zero past k, kp ≤ 2048; sw: n scales) quantizes its input rows as knx_hip_quantize_rows
 * and computes the epilogue of knx_hip_i8gemm, the same bits as knx_hip_qlinear; an fp32 layer (w: n rows of k
 * floats, stride ldw) sums in its own order.  1 ≤ rows ≤ 64, at most KNX_CHAIN_MAX_LAYERS layers, every k a multiple
 * of 4, x and every y but the last 16-byte aligned with strides multiple of 4 floats; a layer's output must not
 * overlap its input.  The layers are separated by barriers across the launch's workgroups (at most 64, one per CU,
 * all resident at once; more items than workgroups are taken in turn).  scratch (knx_hip_linear_chain_scratch bytes,
 * 256-byte aligned) holds the barrier words: zero before the first call (each call leaves them ready for the next);
 * calls that share a scratch must not overlap.  status is the caller's host-visible int (pinned host memory,
 * knx_hip_host_malloc): a barrier that waits ≈ 1 s without the other workgroups arriving (they could not all be
 * resident, e.g. more chains than the GPU holds running at once) stops waiting and sets it to 1 — the outputs of
 * that launch are then wrong and must be recomputed.  The kernel never clears it: the caller reads it after
 * synchronizing and clears it. */
#define KNX_CHAIN_MAX_LAYERS 8
typedef struct {
    const void* w;
    const float* sw;
    const float* bias;  /* n values or NULL */
    float* y;
    int k, kp, n, ldw, ldy;
    int act;            /* KERNIX_ACT_* id, −1 none */
    int i8;
    float alpha;        /* activation parameter */
} knx_chain_layer;
KNX_API size_t knx_hip_linear_chain_scratch(const knx_chain_layer* layers, int n_layers, int rows); /* 0: bad shape */
KNX_API int knx_hip_linear_chain(const float* x, int ldx, int rows, const knx_chain_layer* layers, int n_layers,
                                 void* scratch, size_t scratch_bytes, int* status, void* stream);
/* Fills bytes of device memory with a byte value, ordered on stream. */
KNX_API int knx_hip_memset(void* p, int value, size_t bytes, void* stream);

/* dst (K×N row-major fp32) = (float)q[n][k] · scale[n]; q is N×K int8 with row stride ldq bytes. */
KNX_API int knx_hip_dequant(const int8_t* q, int ldq, const float* scale, int K, int N, float* dst, void* stream);
/* dst (N×K row-major fp32, the layout of the fp32 weights used with knx_hip_sgemm_nt_ep) = (float)q[n][k] · scale[n]. */
KNX_API int knx_hip_dequant_t(const int8_t* q, int ldq, const float* scale, int K, int N, float* dst, void* stream);

/* ---- fp32 GEMM ---- */
/* C = act(A·W + bias): A M×K (stride lda), W K×N row-major (stride ldw), C M×N (stride ldc), all fp32.
 * K may be 0 (then C = act(bias)). */
KNX_API int knx_hip_sgemm_ep(int M, int N, int K, const float* A, int lda, const float* W, int ldw,
                             const float* bias, int act, float alpha, float* C, int ldc, void* stream);
/* Same with the weight stored transposed: Wt N×K row-major (stride ldwt ≥ K), the device layout of Linear weights
 * (both GEMM operands K-contiguous, as in kernix_matmul_ep_into with a transposed B, include/kernix.h:951-977). */
KNX_API int knx_hip_sgemm_nt_ep(int M, int N, int K, const float* A, int lda, const float* Wt, int ldwt,
                                const float* bias, int act, float alpha, float* C, int ldc, void* stream);
/* C = act(A·Wtᵀ + bias) + R (R M×N, stride ldr; R may equal C): a LINEAR followed by the BINARY add of R
 * (reference include/kernix.h:951-977 then include/kernix_model.h:877-906, the same two fp32 roundings). */
KNX_API int knx_hip_sgemm_nt_ep_res(int M, int N, int K, const float* A, int lda, const float* Wt, int ldwt,
                                    const float* bias, int act, float alpha, const float* R, int ldr, float* C, int ldc,
                                    void* stream);

/* ---- convolution (NHWC, groups, dilation, zero padding) ---- */
typedef struct {
    int B, H, W, C;        /* input: B×H×W×C */
    int Ho, Wo, Co;        /* output: B×Ho×Wo×Co */
    int kh, kw, sh, sw, dh, dw, pt, pl;
    int groups;
} knx_conv_geom;
/* y = act(conv(x, w) + bias); w is (kh·kw·C/groups) × Co with rows ordered (ky, kx, ci). */
KNX_API int knx_hip_conv(const knx_conv_geom* g, const float* x, const float* w, const float* bias, int act,
                         float alpha, float* y, void* stream);
/* Same with the weight transposed: Wt Co × (kh·kw·C/groups), the device layout of the model's convolution weights.
 * Channel counts per group that are multiples of 32 run on the pipelined implicit GEMM (LDS-DMA gathers). */
KNX_API int knx_hip_conv_t(const knx_conv_geom* g, const float* x, const float* wt, const float* bias, int act,
                           float alpha, float* y, void* stream);
/* y = act(conv(x, Wt) + bias) + R (R the same shape as y; R may equal y): a CONV followed by the BINARY add of R
 * (reference include/kernix_model.h:711-771 then :877-906). */
KNX_API int knx_hip_conv_t_res(const knx_conv_geom* g, const float* x, const float* wt, const float* bias, int act,
                               float alpha, const float* R, float* y, void* stream);

/* ---- row and elementwise ops (y may equal x unless noted) ---- */
KNX_API int knx_hip_layernorm(const float* x, float* y, int rows, int cols, const float* gamma, const float* beta,
                              float eps, void* stream);
/* layer_norm of each row followed by kernix_qmatmul's per-row int8 quantization of the normalized row (the steps of
 * knx_hip_quantize_rows): xq (rows × kp, zero past cols) and sx (rows) get the bits of knx_hip_layernorm then
 * knx_hip_quantize_rows, and the fp32 rows are not written.  cols % 4 == 0, cols ≤ 2048, kp ≥ cols, kp % 4 == 0,
 * x, gamma and beta 16-byte aligned. */
KNX_API int knx_hip_layernorm_quantize(const float* x, int rows, int cols, const float* gamma, const float* beta,
                                       float eps, int kp, int8_t* xq, float* sx, void* stream);
KNX_API int knx_hip_softmax(const float* x, float* y, int rows, int cols, void* stream);
KNX_API int knx_hip_bias_act(const float* x, float* y, int rows, int cols, const float* bias, int act, float alpha,
                             void* stream);
/* Per sample b < B and row i < R, column j < C: y = a ⊙ b with size-1 rows (ra/rb == 1) or channels (ca/cb == 1)
 * broadcast within the sample. */
KNX_API int knx_hip_binary(int op, const float* a, int ra, int ca, const float* b, int rb, int cb, float* y, int B,
                           int R, int C, void* stream);
/* Per sample, mean (type avg) or max over R rows of C channels → B×C. y must not alias x. */
KNX_API int knx_hip_global_pool(int type, const float* x, int B, int R, int C, float* y, void* stream);
/* y[r][c] = x[r][c]·scale[c] + shift[c] */
KNX_API int knx_hip_affine(const float* x, float* y, int rows, int cols, const float* scale, const float* shift,
                           void* stream);
/* y[b][i] = x[b][i] + cst[i], i < per */
KNX_API int knx_hip_add_const(const float* x, float* y, int B, int per, const float* cst, void* stream);

/* Attention core, per (b, h): S = scale·Q_h·K_hᵀ (+ causal −inf above the diagonal), P = softmax(S), ctx_h = P·V_h.
 * Q: (B·Rq) × (H·dk), K: (B·S) × (H·dk), V: (B·S) × (H·dv), ctx: (B·Rq) × (H·dv), all row-major fp32.
 * scores: scratch of B·H·Rq·S floats used when the fused kernel does not apply (may be NULL otherwise). */
KNX_API int knx_hip_attention_core(const float* Q, const float* K, const float* V, float* ctx, float* scores, int B,
                                   int H, int Rq, int S, int dk, int dv, float scale, int causal, void* stream);
/* Same with row strides ldq, ldk, ldv (≥ H·dk, H·dk, H·dv) for Q, K and V — e.g. column slices of one Q|K|V
 * projection output — and vt (H·dv × B·S floats, or NULL): scratch for Vᵀ, which lets P·V run on the pipelined
 * GEMM when the fused kernel does not apply.  Same reference loop (include/kernix_model.h:1021-1046). */
KNX_API int knx_hip_attention_core_ex(const float* Q, int ldq, const float* K, int ldk, const float* V, int ldv,
                                      float* vt, float* ctx, float* scores, int B, int H, int Rq, int S, int dk,
                                      int dv, float scale, int causal, void* stream);

/* ---- shape/copy ops for the remaining graph kinds ---- */
/* Windowed pooling over NHWC (type max/avg, count_pad as PyTorch count_include_pad). */
KNX_API int knx_hip_pool(int type, const knx_conv_geom* g, int count_pad, const float* x, float* y, void* stream);
/* Per sample of n floats with shape d[0..nd) (row-major), out axis k = in axis perm[k]. */
KNX_API int knx_hip_permute(const float* x, float* y, int B, int nd, const int* d, const int* perm, void* stream);
/* y[r][y_off + j] = x[r][x_off + j], j < n, r < rows; row strides ldx, ldy. */
KNX_API int knx_hip_copy_cols(const float* x, int ldx, int x_off, float* y, int ldy, int y_off, int rows, int n,
                              void* stream);
/* Zero padding of B×H×W×C into B×Ho×Wo×C at offset (pt, pl). */
KNX_API int knx_hip_pad(const float* x, float* y, int B, int H, int W, int C, int Ho, int Wo, int pt, int pl,
                        void* stream);
/* Nearest upsampling by (sh, sw). */
KNX_API int knx_hip_upsample(const float* x, float* y, int B, int H, int W, int C, int sh, int sw, void* stream);
/* y[i] = table[id] for integral id in [0, V), else a NaN row; n ids, D floats per row. */
KNX_API int knx_hip_embedding(const float* ids, int n, const float* table, int V, int D, float* y, void* stream);
/* RNN gate update for one timestep (see the definition for the exact per-kind formulas; the cells' sigmoid and tanh
 * on the hardware exp2 and reciprocal, ≤ 1-2 ulp each, as in knx_hip_rnn_recurrence). */
KNX_API int knx_hip_rnn_gates(int kind, int act, float alpha, int B, int u, int first_step, float* z, const float* zh,
                              float* c, float* h, float* dst, int dst_stride, void* stream);
/* The recurrence of one RNN direction over T timesteps as one launch (reference include/kernix_model.h:563-632,
 * the loop after the input projection).  kind 4 LSTM / 5 GRU / 6 simple RNN with u units; zx: the input projection
 * x·W + b, B·T rows of gates·u (row b·T + t); the recurrent weight is either int8 (q: gates·u rows of kp bytes, k
 * contiguous, with qscale per row: h·U in int8 arithmetic with the rows of h quantized as knx_hip_quantize_rows, the
 * bits of knx_hip_qlinear) or fp32 (U: u × gates·u, or gates·u × u when u_nt); brec: the GRU's recurrent bias.
 * dir 1 runs t = T−1 … 0.  Output: ret_seq: the state of timestep t of sample b at dst + (b·T + t)·stride, else the
 * last state at dst + b·stride.  h0, h1: B rows of ⌈u/4⌉·4 floats each, 16-byte aligned (scratch); scratch: 8 bytes,
 * 256-byte aligned, a multiple
 * of 256 as the chain's barrier words (the chain and this kernel may share them); status as for knx_hip_linear_chain.
 * Where U fits one workgroup's registers (gates·u ≤ 1024; LSTM and GRU up to 128 units) the batch rows are split over
 * workgroups that each run their rows alone (any B; h0, h1, scratch and status are not touched); otherwise the units are
 * split over a grid of at most 64 workgroups, which must all be resident, with a barrier per timestep.  Shapes
 * knx_hip_rnn_recurrence_fits rejects (neither form: B > 64 on the grid, u > 2048, a weight slice or h that does not
 * fit the workgroup's LDS) are KNX_EINVAL. */
KNX_API int knx_hip_rnn_recurrence_fits(int kind, int B, int u, int i8);
/* The recurrence of one direction (as knx_hip_rnn_recurrence, its last state only: ret_seq 0) and the LINEAR step that
 * reads only that state, in one launch (reference include/kernix_model.h:563-632, then the LINEAR dispatch :1843-1860
 * on its B rows): y (B rows of dn) = act(h_T·Wᵀ + b), with dq (dn rows of dkp bytes, k = u contiguous) and dqs its
 * per-output scales the int8 arithmetic of knx_hip_qlinear (the same bits), else fp32 on dw (dn rows of u floats);
 * db may be NULL.  Only the batch-split form (knx_hip_rnn_recurrence_dense_fits: U fits a workgroup, u ≤ 256);
 * dst still receives the last state. */
KNX_API int knx_hip_rnn_recurrence_dense_fits(int kind, int B, int u, int i8, int n);
KNX_API int knx_hip_rnn_recurrence_dense(int kind, int act, float alpha, int B, int T, int u, int dir, const float* zx,
                                         const float* U, int u_nt, const int8_t* q, int kp, const float* qscale,
                                         const float* brec, float* dst, int stride, const float* dw, const int8_t* dq,
                                         int dkp, const float* dqs, const float* db, int dn, int dact, float dalpha,
                                         float* dy, void* stream);
KNX_API int knx_hip_rnn_recurrence(int kind, int act, float alpha, int B, int T, int u, int dir, const float* zx,
                                   const float* U, int u_nt, const int8_t* q, int kp, const float* qscale,
                                   const float* brec, float* h0, float* h1, float* dst, int stride, int ret_seq,
                                   void* scratch, size_t scratch_bytes, int* status, void* stream);

#ifdef __cplusplus
}
#endif

#endif
