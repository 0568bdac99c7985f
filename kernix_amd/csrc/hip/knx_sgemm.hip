// knx_sgemm.hip — fp32 GEMM with fused epilogue on v_mfma_f32_32x32x2_f32 (gfx950), one whole-GPU tiling.
//
// Replaces the reference's row split of one GEMM between MPS (GPU) and cblas_sgemm (AMX) with its separate bias/act
// pass (reference src/kernix_metal.m:161-265, include/kernix.h:951-977, include/kernix_model.h:528-550):
// every output tile is computed by one workgroup and leaves the chip already biased and activated.
//
// Tile: BM×BN per workgroup of WM×WN waves, K streamed in 16-float k-tiles through double-buffered LDS.  Both tiles
// are stored k-major in LDS (As[k][m], Bs[k][n]) so each MFMA operand read is 32 consecutive floats per half-wave.
// A is M×K row-major; B is K×N row-major (NN, Linear weights as stored in .knx) or N×K row-major (NT, attention
// keys).  An optional batch index (grid.y) with two-level strides serves the per-(batch, head) attention GEMMs.
#include "knx_common.hpp"

typedef float v16f __attribute__((ext_vector_type(16)));

namespace {

struct SgArgs {
    int M, N, K;
    const float* A;
    int lda;
    const float* B;
    int ldb;
    float* C;
    int ldc;
    const float* bias;
    int act;
    float act_alpha;
    float alpha;   // C = alpha·(A·B) before bias
    int causal;    // C[i][j] = −inf for j > i (attention scores)
    int tiles_n;
    int zh;        // batch index z = zb·zh + zi
    long long sAb, sAh, sBb, sBh, sCb, sCh;
};

constexpr int BK = 16;

template <int BM, int BN, int WM, int WN, bool TB>
__global__ void __launch_bounds__(WM * WN * 64) sgemm_tile(SgArgs p)
{
    constexpr int NT = WM * WN * 64;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 32, FN = TN / 32;
    constexpr int SA = BM + 4, SB = BN + 4;  // LDS row strides (floats)
    constexpr int LA = BM * BK / 4 / NT;     // float4 loads per thread (A)
    constexpr int LB = BN * BK / 4 / NT;     // float4 loads per thread (B)
    static_assert(BM * BK / 4 % NT == 0 && BN * BK / 4 % NT == 0, "load split");
    __shared__ __attribute__((aligned(16))) float As[2][BK * SA];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK * SB];

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int tm = blockIdx.x / p.tiles_n, tn = blockIdx.x % p.tiles_n;
    const int m0 = tm * BM, n0 = tn * BN;
    const int z = blockIdx.y, zb = z / p.zh, zi = z % p.zh;
    const float* A = p.A + zb * p.sAb + zi * p.sAh;
    const float* B = p.B + zb * p.sBb + zi * p.sBh;
    float* C = p.C + zb * p.sCb + zi * p.sCh;
    const int M = p.M, N = p.N, K = p.K;
    const bool a_vec = (p.lda & 3) == 0 && ((uintptr_t)A & 15) == 0;
    const bool b_vec = (p.ldb & 3) == 0 && ((uintptr_t)B & 15) == 0;

    float4 ra[LA], rb[LB];

    // A (and NT B): row r, k-chunk kc of 4 floats; zero outside the matrix.
    auto load_rows = [&](const float* X, int ld, bool vec, int r0, int rows, int k0, int i) -> float4 {
        const int idx = i * NT + t, r = idx >> 2, kc = (idx & 3) * 4;
        const int gr = r0 + r, gk = k0 + kc;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (gr < rows) {
            const float* src = X + (size_t)gr * ld + gk;
            if (vec && gk + 3 < K) v = *reinterpret_cast<const float4*>(src);
            else {
                if (gk + 0 < K) v.x = src[0];
                if (gk + 1 < K) v.y = src[1];
                if (gk + 2 < K) v.z = src[2];
                if (gk + 3 < K) v.w = src[3];
            }
        }
        return v;
    };
    // NN B: k row, n-chunk of 4 floats.
    auto load_b_nn = [&](int k0, int i) -> float4 {
        const int idx = i * NT + t, k = idx / (BN / 4), nc = (idx % (BN / 4)) * 4;
        const int gk = k0 + k, gn = n0 + nc;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (gk < K) {
            const float* src = B + (size_t)gk * p.ldb + gn;
            if (b_vec && gn + 3 < N) v = *reinterpret_cast<const float4*>(src);
            else {
                if (gn + 0 < N) v.x = src[0];
                if (gn + 1 < N) v.y = src[1];
                if (gn + 2 < N) v.z = src[2];
                if (gn + 3 < N) v.w = src[3];
            }
        }
        return v;
    };
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < LA; ++i) ra[i] = load_rows(A, p.lda, a_vec, m0, M, k0, i);
#pragma unroll
        for (int i = 0; i < LB; ++i) rb[i] = TB ? load_rows(B, p.ldb, b_vec, n0, N, k0, i) : load_b_nn(k0, i);
    };
    auto swrite = [&](int buf) {
#pragma unroll
        for (int i = 0; i < LA; ++i) {
            const int idx = i * NT + t, r = idx >> 2, kc = (idx & 3) * 4;
            float* d = &As[buf][kc * SA + r];
            d[0] = ra[i].x; d[SA] = ra[i].y; d[2 * SA] = ra[i].z; d[3 * SA] = ra[i].w;
        }
#pragma unroll
        for (int i = 0; i < LB; ++i) {
            if (TB) {
                const int idx = i * NT + t, r = idx >> 2, kc = (idx & 3) * 4;
                float* d = &Bs[buf][kc * SB + r];
                d[0] = rb[i].x; d[SB] = rb[i].y; d[2 * SB] = rb[i].z; d[3 * SB] = rb[i].w;
            } else {
                const int idx = i * NT + t, k = idx / (BN / 4), nc = (idx % (BN / 4)) * 4;
                *reinterpret_cast<float4*>(&Bs[buf][k * SB + nc]) = rb[i];
            }
        }
    };

    v16f acc[FM][FN];
#pragma unroll
    for (int fi = 0; fi < FM; ++fi)
#pragma unroll
        for (int fj = 0; fj < FN; ++fj)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[fi][fj][e] = 0.0f;

    const int rl = lane & 31, g = lane >> 5;
    const int nk = (K + BK - 1) / BK;
    if (nk > 0) {
        gload(0);
        swrite(0);
        __syncthreads();
    }
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) gload((kt + 1) * BK);
#pragma unroll
        for (int s = 0; s < BK / 2; ++s) {
            float af[FM], bf[FN];
            const int kk = 2 * s + g;
#pragma unroll
            for (int fi = 0; fi < FM; ++fi) af[fi] = As[cur][kk * SA + wm * TM + fi * 32 + rl];
#pragma unroll
            for (int fj = 0; fj < FN; ++fj) bf[fj] = Bs[cur][kk * SB + wn * TN + fj * 32 + rl];
#pragma unroll
            for (int fi = 0; fi < FM; ++fi)
#pragma unroll
                for (int fj = 0; fj < FN; ++fj)
                    acc[fi][fj] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[fi], bf[fj], acc[fi][fj], 0, 0, 0);
        }
        if (more) swrite(cur ^ 1);
        __syncthreads();
    }

    // epilogue: lane holds column (lane & 31), rows 8·(e/4) + 4·(lane/32) + e%4 of each 32×32 block
#pragma unroll
    for (int fj = 0; fj < FN; ++fj) {
        const int n = n0 + wn * TN + fj * 32 + rl;
        if (n >= N) continue;
        const float bn = p.bias ? p.bias[n] : 0.0f;
#pragma unroll
        for (int fi = 0; fi < FM; ++fi)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + wm * TM + fi * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
                if (m >= M) continue;
                float v = acc[fi][fj][e];
                if (p.alpha != 1.0f) v = p.alpha * v;
                if (p.bias) v = v + bn;
                if (p.causal && n > m) v = -INFINITY;
                C[(size_t)m * p.ldc + n] = knx_act(v, p.act, p.act_alpha);
            }
    }
}

template <int BM, int BN, int WM, int WN, bool TB>
int launch(SgArgs p, int batch, hipStream_t s, const char* name)
{
    p.tiles_n = (p.N + BN - 1) / BN;
    const unsigned tiles = (unsigned)((p.M + BM - 1) / BM) * (unsigned)p.tiles_n;
    hipLaunchKernelGGL((sgemm_tile<BM, BN, WM, WN, TB>), dim3(tiles, batch), dim3(WM * WN * 64), 0, s, p);
    return knx::check_launch(name);
}

template <bool TB>
int dispatch(SgArgs p, int batch, hipStream_t s, const char* name)
{
    const long big = (long)((p.M + 127) / 128) * ((p.N + 127) / 128) * batch;
    if (big >= knx::num_cus()) {
        if (p.N <= 64) return launch<128, 64, 2, 2, TB>(p, batch, s, name);
        return launch<128, 128, 2, 2, TB>(p, batch, s, name);
    }
    return launch<64, 64, 2, 2, TB>(p, batch, s, name);
}

}  // namespace

extern "C" int knx_hip_sgemm_ep(int M, int N, int K, const float* A, int lda, const float* W, int ldw, const float* bias,
                                int act, float alpha, float* C, int ldc, void* stream)
{
    const char* name = "knx_hip_sgemm_ep";
    KNX_ENTRY(name);
    KNX_REQUIRE(M >= 0 && N >= 0 && K >= 0 && act >= -1 && act <= 15, name);
    if (M == 0 || N == 0) return KNX_OK;
    KNX_REQUIRE(C != nullptr && ldc >= N, name);
    KNX_REQUIRE(K == 0 || (A != nullptr && W != nullptr && lda >= K && ldw >= N), name);
    SgArgs p{};
    p.M = M; p.N = N; p.K = K; p.A = A; p.lda = lda; p.B = W; p.ldb = ldw; p.C = C; p.ldc = ldc;
    p.bias = bias; p.act = act; p.act_alpha = alpha; p.alpha = 1.0f; p.causal = 0; p.zh = 1;
    return dispatch<false>(p, 1, knx::as_stream(stream), name);
}

// Batched GEMM used by the attention core (internal to this library, declared in knx_attn.hip).
int knx_sgemm_batched(int M, int N, int K, const float* A, int lda, long long sAb, long long sAh, const float* B, int ldb,
                      long long sBb, long long sBh, bool transB, float* C, int ldc, long long sCb, long long sCh, int nb,
                      int nh, float alpha, int causal, hipStream_t s)
{
    const char* name = "knx_sgemm_batched";
    SgArgs p{};
    p.M = M; p.N = N; p.K = K; p.A = A; p.lda = lda; p.B = B; p.ldb = ldb; p.C = C; p.ldc = ldc;
    p.bias = nullptr; p.act = -1; p.act_alpha = 0.0f; p.alpha = alpha; p.causal = causal; p.zh = nh;
    p.sAb = sAb; p.sAh = sAh; p.sBb = sBb; p.sBh = sBh; p.sCb = sCb; p.sCh = sCh;
    return transB ? dispatch<true>(p, nb * nh, s, name) : dispatch<false>(p, nb * nh, s, name);
}
