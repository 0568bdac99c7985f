// knx_i8gemm.hip — int8 path of the KERNIX forward on gfx950.
//
//   knx_hip_quantize_rows  dynamic per-row int8 input (reference include/kernix_model.h:112-142)
//   knx_hip_i8gemm         int32 accumulation on v_mfma_i32_32x32x32_i8 with the dequant · bias · act epilogue
//                          fused (reference include/kernix_model.h:143-178 and the activation pass :1854-1856)
//   knx_hip_dequant        fp32 copy w = q·scale (reference include/kernix_model.h:91-95)
//
// GEMM structure (one workgroup per BM×BN output tile, K streamed in 64-byte k-tiles):
//   global → VGPR (16-byte loads, fully coalesced: 4 lanes per 64-byte row segment) → LDS (double buffered,
//   16-byte chunks XOR-swizzled per row so the MFMA fragment reads are bank-conflict free) → v4i32 fragments →
//   32×32×32 i8 MFMAs into int32 accumulators → epilogue straight from the accumulators.
//   Both operands are K-contiguous (A: M×K activations, W: N×K weights), so no transposes are needed anywhere.
#include "knx_common.hpp"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

namespace {

struct I8Args {
    int M, N, K;
    const int8_t* A;
    int lda;
    const float* sa;
    const int8_t* W;
    int ldw;
    const float* sw;
    const float* bias;
    int act;
    float alpha;
    int accumulate;
    float* Y;
    int ldy;
    int32_t* acc;
    int ldacc;
    int tiles_m, tiles_n;
};

// 16-byte chunk swizzle within a 64-byte LDS row: distinct chunks for the rows that share a bank group, whether the
// LDS is serviced as 32 or 64 banks (rows r, r+2, r+4, r+6 and r, r+4, r+8, r+12 all map to different chunks).
__device__ __forceinline__ int swz(int row) { return ((row >> 1) ^ (row >> 3)) & 3; }

__device__ __forceinline__ void i8_epilogue(const I8Args& p, int m, int n, int32_t a)
{
    if (p.acc) p.acc[(size_t)m * p.ldacc + n] = a;
    if (p.Y == nullptr) return;
    // ((float)acc · sx) · scale + bias, each step rounded (reference include/kernix_model.h:167-177)
    float v = (float)a * p.sa[m];
    v = v * p.sw[n];
    if (p.bias) v = v + p.bias[n];
    float* y = p.Y + (size_t)m * p.ldy + n;
    if (p.accumulate) v = *y + v;
    *y = knx_act(v, p.act, p.alpha);
}

template <int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__(WM * WN * 64) i8gemm_tile(I8Args p)
{
    constexpr int NT = WM * WN * 64;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 32, FN = TN / 32;
    constexpr int ROWS = BM + BN;
    constexpr int LOADS = ROWS * 4 / NT;
    static_assert(ROWS * 4 % NT == 0, "load split");
    static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile");
    __shared__ __attribute__((aligned(16))) int8_t lds[2][ROWS * 64];

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int tile = blockIdx.x;
    const int tm = tile / p.tiles_n, tn = tile % p.tiles_n;
    const int m0 = tm * BM, n0 = tn * BN;

    // global → LDS assignment: chunk (row, c) with c = t & 3, rows strided by NT/4
    const int8_t* gptr[LOADS];
    bool gval[LOADS];
    int soff[LOADS];
    const int c_ld = t & 3;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int row = i * (NT / 4) + (t >> 2);
        if (row < BM) {
            const int gm = m0 + row;
            gval[i] = gm < p.M;
            gptr[i] = p.A + (size_t)(gval[i] ? gm : 0) * p.lda + c_ld * 16;
        } else {
            const int gn = n0 + row - BM;
            gval[i] = gn < p.N;
            gptr[i] = p.W + (size_t)(gval[i] ? gn : 0) * p.ldw + c_ld * 16;
        }
        soff[i] = row * 64 + ((c_ld ^ swz(row)) << 4);
    }

    // fragment read offsets: lane reads row (lane & 31) of its 32-row block, chunk 2·s + (lane >> 5)
    const int rl = lane & 31, g = lane >> 5;
    int aoff[FM][2], boff[FN][2];
#pragma unroll
    for (int fi = 0; fi < FM; ++fi) {
        const int row = wm * TM + fi * 32 + rl;
#pragma unroll
        for (int s = 0; s < 2; ++s) aoff[fi][s] = row * 64 + (((2 * s + g) ^ swz(row)) << 4);
    }
#pragma unroll
    for (int fj = 0; fj < FN; ++fj) {
        const int row = BM + wn * TN + fj * 32 + rl;
#pragma unroll
        for (int s = 0; s < 2; ++s) boff[fj][s] = row * 64 + (((2 * s + g) ^ swz(row)) << 4);
    }

    v16i acc[FM][FN];
#pragma unroll
    for (int fi = 0; fi < FM; ++fi)
#pragma unroll
        for (int fj = 0; fj < FN; ++fj)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[fi][fj][e] = 0;

    v4i pre[LOADS];
    const int nk = p.K / 64;
    if (nk > 0) {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) pre[i] = gval[i] ? *(const v4i*)gptr[i] : v4i{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < LOADS; ++i) *(v4i*)&lds[0][soff[i]] = pre[i];
        __syncthreads();
    }

    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) {
#pragma unroll
            for (int i = 0; i < LOADS; ++i)
                pre[i] = gval[i] ? *(const v4i*)(gptr[i] + (size_t)(kt + 1) * 64) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            v4i af[FM], bf[FN];
#pragma unroll
            for (int fi = 0; fi < FM; ++fi) af[fi] = *(const v4i*)&lds[cur][aoff[fi][s]];
#pragma unroll
            for (int fj = 0; fj < FN; ++fj) bf[fj] = *(const v4i*)&lds[cur][boff[fj][s]];
#pragma unroll
            for (int fi = 0; fi < FM; ++fi)
#pragma unroll
                for (int fj = 0; fj < FN; ++fj)
                    acc[fi][fj] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[fi], bf[fj], acc[fi][fj], 0, 0, 0);
        }
        if (more) {
#pragma unroll
            for (int i = 0; i < LOADS; ++i) *(v4i*)&lds[cur ^ 1][soff[i]] = pre[i];
        }
        __syncthreads();
    }

    // Epilogue.  32×32 accumulator layout: lane holds column (lane & 31) and rows 8·(e/4) + 4·(lane/32) + e%4.
    // Each wave stages 16 rows × TN of its tile at a time in LDS (row stride TN+4 ints: the two half-waves land on
    // different banks), then every lane reads 4 consecutive columns and writes them as one 16-byte store.
    constexpr int SROW = TN + 4;
    constexpr int LPR = TN / 4;   // lanes per staged row
    constexpr int RPI = 64 / LPR; // rows per read instruction
    static_assert(WM * WN * 16 * SROW * 4 <= 2 * ROWS * 64, "staging fits in the k-tile buffers");
    int* stg = reinterpret_cast<int*>(&lds[0][0]) + wave * 16 * SROW;
    const int cq = (lane % LPR) * 4, rq = lane / LPR;
    const int nb = n0 + wn * TN + cq;
    float swv[4], bv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const bool ok = nb + q < p.N;
        swv[q] = (ok && p.Y) ? p.sw[nb + q] : 0.0f;
        bv[q] = (ok && p.bias) ? p.bias[nb + q] : 0.0f;
    }
    const bool vec = nb + 3 < p.N && (p.ldy & 3) == 0 && ((uintptr_t)p.Y & 15) == 0 && (p.ldacc & 3) == 0 &&
                     ((uintptr_t)p.acc & 15) == 0;
#pragma unroll
    for (int fi = 0; fi < FM; ++fi) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            __syncthreads();
#pragma unroll
            for (int fj = 0; fj < FN; ++fj)
#pragma unroll
                for (int e = 8 * h; e < 8 * h + 8; ++e)
                    stg[(8 * ((e >> 2) - 2 * h) + 4 * g + (e & 3)) * SROW + fj * 32 + rl] = acc[fi][fj][e];
            __syncthreads();
            for (int rr = rq; rr < 16; rr += RPI) {
                const int m = m0 + wm * TM + fi * 32 + 16 * h + rr;
                if (m >= p.M) continue;
                const v4i a = *reinterpret_cast<const v4i*>(&stg[rr * SROW + cq]);
                if (vec) {
                    if (p.acc) *reinterpret_cast<v4i*>(p.acc + (size_t)m * p.ldacc + nb) = a;
                    if (p.Y) {
                        const float sx = p.sa[m];
                        float* y = p.Y + (size_t)m * p.ldy + nb;
                        float4 o = p.accumulate ? *reinterpret_cast<const float4*>(y) : make_float4(0.f, 0.f, 0.f, 0.f);
                        float r[4];
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            // ((float)acc · sx) · scale + bias, each step rounded (reference include/kernix_model.h:167-177)
                            float v = (float)a[q] * sx;
                            v = v * swv[q];
                            if (p.bias) v = v + bv[q];
                            if (p.accumulate) v = (&o.x)[q] + v;
                            r[q] = knx_act(v, p.act, p.alpha);
                        }
                        *reinterpret_cast<float4*>(y) = make_float4(r[0], r[1], r[2], r[3]);
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        if (nb + q < p.N) i8_epilogue(p, m, nb + q, a[q]);
                }
            }
        }
    }
}

template <int BM, int BN, int WM, int WN>
int launch_tile(I8Args p, hipStream_t s, const char* name)
{
    p.tiles_m = (p.M + BM - 1) / BM;
    p.tiles_n = (p.N + BN - 1) / BN;
    const unsigned grid = (unsigned)p.tiles_m * (unsigned)p.tiles_n;
    hipLaunchKernelGGL((i8gemm_tile<BM, BN, WM, WN>), dim3(grid), dim3(WM * WN * 64), 0, s, p);
    return knx::check_launch(name);
}

// ---- per-row quantization: one wave per row ----
__global__ void __launch_bounds__(256) quantize_rows_kernel(const float* __restrict__ x, int ldx, int rows, int k,
                                                             int kp, int8_t* __restrict__ xq, int ldq, float* __restrict__ sx)
{
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* xr = x + (size_t)row * ldx;
    float m = 0.0f;
    int bad = 0;
    for (int j = lane; j < k; j += 64) {
        const float a = fabsf(xr[j]);
        if (!(a <= 3.402823466e38f)) bad = 1;  // NaN or ±inf
        else m = a > m ? a : m;
    }
    m = knx_wave_max(m);
    bad = __any(bad);
    int8_t* qr = xq + (size_t)row * ldq;
    if (bad) {
        for (int j = lane; j < kp; j += 64) qr[j] = 0;
        if (lane == 0) sx[row] = __int_as_float(0x7fc00000);
        return;
    }
    const float s = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
    const float inv = __fdiv_rn(1.0f, s);
    for (int j = lane; j < kp; j += 64) {
        int8_t q = 0;
        if (j < k) {
            const float v = rintf(xr[j] * inv);
            q = (int8_t)(v > 127.0f ? 127.0f : v < -127.0f ? -127.0f : v);
        }
        qr[j] = q;
    }
    if (lane == 0) sx[row] = s;
}

// ---- dequantized copy: dst[k][n] = (float)q[n][k] · scale[n], 32×32 tiles transposed through LDS ----
__global__ void __launch_bounds__(256) dequant_kernel(const int8_t* __restrict__ q, int ldq, const float* __restrict__ scale,
                                                       int K, int N, float* __restrict__ dst)
{
    __shared__ float tile[32][33];
    const int k0 = blockIdx.x * 32, n0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 × 8
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int n = n0 + ty + 8 * i, k = k0 + tx;
        tile[ty + 8 * i][tx] = (n < N && k < K) ? (float)q[(size_t)n * ldq + k] * scale[n] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int k = k0 + ty + 8 * i, n = n0 + tx;
        if (k < K && n < N) dst[(size_t)k * N + n] = tile[tx][ty + 8 * i];
    }
}

}  // namespace

extern "C" int knx_hip_quantize_rows(const float* x, int ldx, int rows, int k, int kp, int8_t* xq, int ldq, float* sx,
                                     void* stream)
{
    const char* name = "knx_hip_quantize_rows";
    KNX_ENTRY(name);
    KNX_REQUIRE(rows >= 0 && k >= 1 && kp >= k && kp % 64 == 0 && ldq >= kp && ldx >= k, name);
    if (rows == 0) return KNX_OK;
    KNX_REQUIRE(x != nullptr && xq != nullptr && sx != nullptr, name);
    hipLaunchKernelGGL(quantize_rows_kernel, dim3((rows + 3) / 4), dim3(256), 0, knx::as_stream(stream), x, ldx, rows, k,
                       kp, xq, ldq, sx);
    return knx::check_launch(name);
}

extern "C" int knx_hip_i8gemm(int M, int N, int K, const int8_t* A, int lda, const float* sa, const int8_t* W, int ldw,
                              const float* sw, const float* bias, int act, float alpha, int accumulate, float* Y, int ldy,
                              int32_t* acc_out, int ldacc, void* stream)
{
    const char* name = "knx_hip_i8gemm";
    KNX_ENTRY(name);
    KNX_REQUIRE(M >= 0 && N >= 0 && K >= 0 && K % 64 == 0 && K <= 131072, name);
    KNX_REQUIRE(lda >= K && ldw >= K && lda % 16 == 0 && ldw % 16 == 0, name);
    KNX_REQUIRE(act >= -1 && act <= 15, name);
    if (M == 0 || N == 0) return KNX_OK;
    KNX_REQUIRE(Y != nullptr || acc_out != nullptr, name);
    KNX_REQUIRE(Y == nullptr || (ldy >= N && sa != nullptr && sw != nullptr), name);
    KNX_REQUIRE(acc_out == nullptr || ldacc >= N, name);
    KNX_REQUIRE(K == 0 || (A != nullptr && W != nullptr), name);
    KNX_REQUIRE(((uintptr_t)A & 15) == 0 && ((uintptr_t)W & 15) == 0, name);
    I8Args p{M, N, K, A, lda, sa, W, ldw, sw, bias, act, alpha, accumulate, Y, ldy, acc_out, ldacc, 0, 0};
    hipStream_t s = knx::as_stream(stream);
    if (K == 0) {
        // empty inner dimension: the accumulators are all zero; run the smallest tile (loop body never executes)
        return launch_tile<64, 64, 1, 1>(p, s, name);
    }
    const long tiles256 = (long)((M + 255) / 256) * ((N + 255) / 256);
    if (tiles256 >= knx::num_cus()) return launch_tile<256, 256, 2, 2>(p, s, name);
    const long tiles128 = (long)((M + 127) / 128) * ((N + 127) / 128);
    if (tiles128 >= knx::num_cus()) return launch_tile<128, 128, 2, 2>(p, s, name);
    return launch_tile<64, 64, 1, 1>(p, s, name);
}

extern "C" int knx_hip_dequant(const int8_t* q, int ldq, const float* scale, int K, int N, float* dst, void* stream)
{
    const char* name = "knx_hip_dequant";
    KNX_ENTRY(name);
    KNX_REQUIRE(K >= 0 && N >= 0 && ldq >= K, name);
    if (K == 0 || N == 0) return KNX_OK;
    KNX_REQUIRE(q != nullptr && scale != nullptr && dst != nullptr, name);
    hipLaunchKernelGGL(dequant_kernel, dim3((K + 31) / 32, (N + 31) / 32), dim3(256), 0, knx::as_stream(stream), q, ldq,
                       scale, K, N, dst);
    return knx::check_launch(name);
}
