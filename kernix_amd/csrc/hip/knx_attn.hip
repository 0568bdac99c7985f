// knx_attn.hip — attention core of the KERNIX ATTENTION op on gfx950.
//
// Per (batch b, head h): S = scale·Q_h·K_hᵀ (causal: −inf for key j > query i), P = softmax(S), ctx_h = P·V_h,
// the loop body of kernix_attention_run (reference include/kernix_model.h:1021-1046).  The Q/K/V/O projections
// are ordinary Linear GEMMs run by the host (knx_hip_sgemm_ep).
//
// Path: one batched NT MFMA GEMM writes all B·H score matrices (alpha = scale and the causal mask fused in its
// epilogue), the wavefront softmax normalizes each row in place, one batched NN MFMA GEMM multiplies by V and writes
// the context directly in the (B·Rq) × (H·dv) layout the output projection reads.
#include "knx_common.hpp"

int knx_sgemm_batched(int M, int N, int K, const float* A, int lda, long long sAb, long long sAh, const float* B, int ldb,
                      long long sBb, long long sBh, bool transB, float* C, int ldc, long long sCb, long long sCh, int nb,
                      int nh, float alpha, int causal, hipStream_t s);

extern "C" int knx_hip_attention_core(const float* Q, const float* K, const float* V, float* ctx, float* scores, int B,
                                      int H, int Rq, int S, int dk, int dv, float scale, int causal, void* stream)
{
    const char* name = "knx_hip_attention_core";
    KNX_ENTRY(name);
    KNX_REQUIRE(B >= 0 && H >= 1 && Rq >= 1 && S >= 1 && dk >= 1 && dv >= 1, name);
    if (B == 0) return KNX_OK;
    KNX_REQUIRE(Q && K && V && ctx && scores, name);
    KNX_REQUIRE((long long)B * H * Rq * S <= (1LL << 40), name);
    hipStream_t s = knx::as_stream(stream);
    const long long hdk = (long long)H * dk, hdv = (long long)H * dv, RS = (long long)Rq * S;
    int rc = knx_sgemm_batched(Rq, S, dk, Q, (int)hdk, Rq * hdk, dk, K, (int)hdk, S * hdk, dk, true, scores, S, H * RS, RS,
                               B, H, scale, causal, s);
    if (rc != KNX_OK) return rc;
    rc = knx_hip_softmax(scores, scores, B * H * Rq, S, stream);
    if (rc != KNX_OK) return rc;
    return knx_sgemm_batched(Rq, dv, S, scores, S, H * RS, RS, V, (int)hdv, S * hdv, dv, false, ctx, (int)hdv, Rq * hdv, dv,
                             B, H, 1.0f, 0, s);
}
