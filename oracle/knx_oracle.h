/* knx_oracle.h — CPU oracle for the KERNIX forward hot path.  TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU semantics, used by tests/ as the parity checker and by bench.py as the
 * timed CPU baseline.  The product library never links, loads or calls anything here.  Built with
 * -O3 -ffp-contract=off so that every product and sum is rounded separately, as the reference's vector (NEON/vDSP)
 * paths do.
 *
 * Every function names the reference lines it follows (reference paths relative to the reference checkout).
 * How each function is pinned (golden vectors, known-answer tests, closed forms) is listed in tests/test_oracle.py;
 * functions without such a check are marked "parity unpinned" below.
 */
#ifndef KNX_ORACLE_H
#define KNX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Thread count used by the parallel functions below (1 … 256; default 8 = the reference pool's 7 workers + caller,
 * reference include/kernix.h:63). */
void ko_set_threads(int n);
int ko_get_threads(void);

/* Symmetric per-column int8 quantization of a k×n (in×out) weight given in float64, as tools/knx_quant.py:18-25:
 * scale[c] = float32(max_k |w| / 127) (1 for an all-zero column); q = int8(clip(rint(w / (double)scale), ±127)). */
void ko_quantize_cols(const double* w, int k, int n, float* scale, int8_t* q);

/* Per-row dynamic int8 quantization of kernix_qmatmul, include/kernix_model.h:115-142.
 * bad[r] = 1 when the row holds a NaN or ±inf (the output row is then all NaN), sx[r] = the row scale. */
void ko_quantize_rows(const float* x, int rows, int k, int8_t* xq, float* sx, int* bad);

/* kernix_qmatmul, include/kernix_model.h:99-182 (scalar fallback :158-177), q given k×n row-major (file layout):
 * y = (accumulate ? y : 0) + ((float)acc·sx)·scale + bias, NaN rows as above.  acc_out (rows×n, may be NULL)
 * receives the int32 accumulators. */
void ko_qmatmul(const float* x, int rows, int k, int n, const int8_t* q, const float* scale, const float* bias,
                int accumulate, float* y, int32_t* acc_out);

/* Standalone int8 GEMM of the benchmark configuration (the second half of kernix_qmatmul with the row scale given):
 * acc[m][n] = Σ_k A[m][k]·W[n][k] (int32), Y = act(((float)acc·sa[m])·sw[n] + bias[n]).  A M×K, W N×K row-major int8.
 * Parallel over rows (ko_set_threads).  Y or acc may be NULL. */
void ko_i8gemm(int M, int N, int K, const int8_t* A, const float* sa, const int8_t* W, const float* sw,
               const float* bias, int act, float alpha, float* Y, int32_t* acc);

/* In-place activation, include/kernix_model.h:463-517 (formulas incl. the A&S 7.1.26 erf of GELU). */
void ko_act(float* o, size_t n, int act, float alpha);

/* Native float GEMM, include/kernix.h:108-124: C (M×N) = A (M×K) · W (K×N), i-k-j order, float accumulation,
 * parallel over rows.  Then per row += bias (may be NULL) and act, include/kernix_model.h:528-541. */
void ko_dense(int M, int N, int K, const float* A, const float* W, const float* bias, int act, float alpha, float* C);

/* Same GEMM with double accumulation (closed-form truth for tolerance checks). */
void ko_dense_f64(int M, int N, int K, const float* A, const float* W, const float* bias, int act, float alpha, float* C);

/* kernix_layer_norm_rows_into, include/kernix.h:667-677 (biased variance, rstd = 1/sqrtf(ss/cols + eps)). */
void ko_layernorm(const float* x, float* y, int rows, int cols, const float* gamma, const float* beta, float eps);

/* floats_softmax_into, include/kernix.h:652-657: o = exp(x − max)·(1/Σ). */
void ko_softmax(const float* x, float* y, int rows, int cols);

/* kernix_conv_run general path, include/kernix_model.h:711-771 with kernix_im2col :677-693: NHWC convolution via
 * im2col (rows (ky,kx,ci)) and the native GEMM, then bias and act.  x B×H×W×C, w (kh·kw·C/g)×Co, y B×Ho×Wo×Co. */
void ko_conv(int B, int H, int W, int C, int Ho, int Wo, int Co, int kh, int kw, int sh, int sw, int dh, int dw,
             int pt, int pl, int groups, const float* x, const float* w, const float* bias, int act, float alpha, float* y);

/* Attention core of kernix_attention_run, include/kernix_model.h:1021-1046: per (b,h), S = scale·(Q_h·K_hᵀ),
 * causal −inf for j > i, softmax as ko_softmax, ctx_h = P·V_h.  Layouts as knx_hip_attention_core. */
void ko_attention_core(const float* Q, const float* K, const float* V, float* ctx, int B, int H, int Rq, int S, int dk,
                       int dv, float scale, int causal);

/* kernix_binary_run, include/kernix_model.h:877-906. */
void ko_binary(int op, const float* a, int ra, int ca, const float* b, int rb, int cb, float* y, int B, int R, int C);

/* kernix_global_pool_run, include/kernix_model.h:810-830 (avg = Σ·(1/R), sequential sum from row 0). */
void ko_global_pool(int type, const float* x, int B, int R, int C, float* y);

#ifdef __cplusplus
}
#endif

#endif
