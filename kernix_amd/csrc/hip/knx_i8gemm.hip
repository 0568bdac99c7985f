// knx_i8gemm.hip — int8 path of the KERNIX forward on gfx950.
//
//   knx_hip_quantize_rows  dynamic per-row int8 input (reference include/kernix_model.h:112-142)
//   knx_hip_i8gemm         int32 accumulation on v_mfma_i32_32x32x32_i8 with the dequant · bias · act epilogue
//                          fused (reference include/kernix_model.h:143-178 and the activation pass :1854-1856)
//   knx_hip_i8gemm_res     the same followed by the add of another value (a LINEAR + BINARY add pair, :877-906)
//   knx_hip_dequant        fp32 copy w = q·scale (reference include/kernix_model.h:91-95)
//
// GEMM kernels (one workgroup per output tile; both operands K-contiguous — A: M×K activations, W: N×K weights — so
// no transposes anywhere; int32 accumulation on MFMA, the dequant · bias · act epilogue fused):
//   i8gemm_k128    the default whenever its tiles fill the chip: 256×256 (or 128×128) tiles, 128-byte k-tiles moved
//                  HBM → LDS by global_load_lds (three A and two W stages at 256×256 for long K, 16-byte chunks
//                  XOR-swizzled), 32×32×32 i8 MFMAs
//   i8gemm_ring    fewer tiles than CUs at 128×128 (e.g. M = 256): 64×64 tiles on a deep ring of 128-byte k-tiles
//   i8gemm_pipe    64-byte k-tiles through a 4-stage LDS ring (shapes below 64×64; forced variants)
//   i8gemm_skinny  M ≤ 64: every W byte read once, K split across the waves of a workgroup
//   i8gemm_tile    VGPR-staged kernel (K == 0, and forced variants for tests)
#include <stdlib.h>
#include <string.h>

#include <string>
#include <mutex>
#include <unordered_map>
#include <algorithm>
#include <type_traits>
#include <utility>

#include "knx_pipe.hpp"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef unsigned v4u_t __attribute__((ext_vector_type(4)));

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
    const float* R;  // residual added after the activation (same layout as Y, stride ldr), or null
    int ldr;
    int32_t* part;   // K split across workgroups: int32 partial tiles (split kernels only)
    unsigned* cnt;   // K split: one arrival counter per output tile, a multiple of the split count between launches
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
    v = knx_act(v, p.act, p.alpha);
    if (p.R) v = v + p.R[(size_t)m * p.ldr + n];
    *y = v;
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
                            if (p.R) r[q] = r[q] + p.R[(size_t)m * p.ldr + nb + q];
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

// ---------------------------------------------------------------- pipelined tile kernel
// Same tile/fragment/epilogue structure as i8gemm_tile, but operands move HBM → LDS directly with
// global_load_lds_dwordx4 (no VGPR staging, no ds_write), through a STAGES-deep LDS ring so that STAGES−1 k-tiles are
// in flight while one is multiplied.  Each load instruction fills 1 KB of LDS = 16 rows × 64 bytes; lane l fetches
// the global 16-byte chunk (l & 3) ^ swz(row), which realizes the swizzled layout with fully coalesced loads.
// Rows past M (or N) are clamped to the last row: they only feed output rows/columns that are never stored.
#define KERNIX_ACT_RELU_ID 0

// Writes the 16 staged rows [mt0, mt0+16) of a tile: 4 consecutive columns per lane, one 16-byte store per row.
// ACT ≥ −1 is a compile-time activation for the common case (vector path, no accumulation): none, ReLU or GELU;
// −2 is the general path.
template <int ACT>
__device__ __forceinline__ void store_rows(const I8Args& p, const int* stg, const float* row_scale, int mt0, int m0, int mlo,
                                           int nlo, int rq, int rpi, int srow, int cq, int nb, const float* swv,
                                           const float* bv, bool vec = true)
{
    typedef float v4f_t __attribute__((ext_vector_type(4)));
    if (ACT >= -1 && p.R) {
        // Residual after no activation, ReLU or GELU: the round's residual rows are loaded before any store (R and Y may
        // alias, and a load after a store waits for it: one memory round trip per row).  Loading first is right when
        // R is Y, since each element is read before its own store and no other store touches it.  Unrolled, so the
        // loads sit in registers; the per-row code is a few instructions.
        // A lane owns rows rq, rq + rpi, ... < 16 of the round: at most MAXJ of them per pass (one pass when rpi ≥ 2,
        // two when rpi == 1), so every row is covered whatever the tile's lanes per row.
        constexpr int MAXJ = 8;
        const bool rvec = nb >= nlo && (nb & 3) == 0 && (p.ldr & 3) == 0 && ((uintptr_t)p.R & 15) == 0;
        for (int j0 = 0; rq + j0 * rpi < 16; j0 += MAXJ) {
            v4f_t rres[MAXJ];
#pragma unroll
            for (int j = 0; j < MAXJ; ++j) {
                const int rr = rq + (j0 + j) * rpi, m = m0 + mt0 + rr;
                rres[j] = v4f_t{0.0f, 0.0f, 0.0f, 0.0f};
                if (rr >= 16 || m < mlo || m >= p.M) continue;
                const float* rp = p.R + (size_t)m * p.ldr + nb;
                if (rvec) {
                    rres[j] = *reinterpret_cast<const v4f_t*>(rp);
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        if (nb + q >= nlo && nb + q < p.N) rres[j][q] = rp[q];
                }
            }
#pragma unroll
            for (int j = 0; j < MAXJ; ++j) {
                const int rr = rq + (j0 + j) * rpi;
                if (rr >= 16) break;
                const int mt = mt0 + rr, m = m0 + mt;
                if (m < mlo || m >= p.M) continue;
                const v4i a = *reinterpret_cast<const v4i*>(&stg[rr * srow + cq]);
                const float sx = row_scale[mt];
                v4f_t r;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float v = (float)a[q] * sx;  // ((float)acc · sx) · scale + bias, each step rounded
                    v = v * swv[q];
                    if (p.bias) v = v + bv[q];
                    r[q] = (ACT == 0 ? (v >= 0.0f ? v : 0.0f) : ACT == 1 ? knx_gelu(v) : v) + rres[j][q];
                }
                __builtin_nontemporal_store(r, reinterpret_cast<v4f_t*>(p.Y + (size_t)m * p.ldy + nb));
            }
        }
        return;
    }
    // one row per iteration, a rolled loop (the general path's activation switch appears once)
    for (int rr = rq; rr < 16; rr += rpi) {
        const int mt = mt0 + rr, m = m0 + mt;
        if (m < mlo || m >= p.M) continue;
        const v4i a = *reinterpret_cast<const v4i*>(&stg[rr * srow + cq]);
        if (ACT >= -1) {
            const float sx = row_scale[mt];
            v4f_t r;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float v = (float)a[q] * sx;  // ((float)acc · sx) · scale + bias, each step rounded
                v = v * swv[q];
                if (p.bias) v = v + bv[q];   // no bias: no addition (x + 0 would turn −0 into +0)
                r[q] = ACT == 0 ? (v >= 0.0f ? v : 0.0f) : ACT == 1 ? knx_gelu(v) : v;
            }
            // streaming store: the output is written once and never re-read by this kernel
            __builtin_nontemporal_store(r, reinterpret_cast<v4f_t*>(p.Y + (size_t)m * p.ldy + nb));
        } else if (vec) {
            if (p.acc) *reinterpret_cast<v4i*>(p.acc + (size_t)m * p.ldacc + nb) = a;
            if (p.Y) {
                const float sx = row_scale[mt];
                float* y = p.Y + (size_t)m * p.ldy + nb;
                float4 o = p.accumulate ? *reinterpret_cast<const float4*>(y) : make_float4(0.f, 0.f, 0.f, 0.f);
                float r[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float v = (float)a[q] * sx;
                    v = v * swv[q];
                    if (p.bias) v = v + bv[q];
                    if (p.accumulate) v = (&o.x)[q] + v;
                    r[q] = knx_act(v, p.act, p.alpha);
                    if (p.R) r[q] = r[q] + p.R[(size_t)m * p.ldr + nb + q];  // residual after the activation
                }
                *reinterpret_cast<float4*>(y) = make_float4(r[0], r[1], r[2], r[3]);
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (nb + q >= nlo && nb + q < p.N) i8_epilogue(p, m, nb + q, a[q]);
        }
    }
}

// Epilogue of the pipelined kernels: each wave stages 16 rows × TN of its accumulators at a time in its own LDS
// region (row stride TN+4 ints: the two half-waves land on different banks); every lane then reads 4 consecutive
// columns and writes them with one 16-byte store.  The regions are private to the wave, so after one workgroup
// barrier (nobody reads the operand ring any more) only the wave's own LDS order matters: no barrier — and so no
// wait for the stores — per round.  nb is this lane's first output column, swv/bv its 4 column scales and biases.
template <int BM, int BN, int WM, int WN>
__device__ __forceinline__ void tile_epilogue(const I8Args& p, const v16i (&acc)[BM / WM / 32][BN / WN / 32],
                                              int8_t* lds, float* row_scale, float my_sa, int m0, int nb,
                                              const float* swv, const float* bv, int mlo, int nlo)
{
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 32, FN = TN / 32;
    constexpr int SROW = TN + 4;
    constexpr int LPR = TN / 4;
    constexpr int RPI = 64 / LPR;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, wm = wave / WN;
    const int rl = lane & 31, g = lane >> 5;
    int* stg = reinterpret_cast<int*>(lds) + wave * 16 * SROW;
    const int cq = (lane % LPR) * 4, rq = lane / LPR;
    const bool vec = nb >= nlo && nb + 3 < p.N && (p.ldy & 3) == 0 && ((uintptr_t)p.Y & 15) == 0 &&
                     (p.ldacc & 3) == 0 && ((uintptr_t)p.acc & 15) == 0;
    if (t < BM) row_scale[t] = my_sa;
    KNX_WAIT_LDS();
    knx_barrier_nofence();
#pragma unroll
    for (int fi = 0; fi < FM; ++fi) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int fj = 0; fj < FN; ++fj)
#pragma unroll
                for (int e = 8 * h; e < 8 * h + 8; ++e)
                    stg[(8 * ((e >> 2) - 2 * h) + 4 * g + (e & 3)) * SROW + fj * 32 + rl] = acc[fi][fj][e];
            KNX_WAIT_LDS();
            asm volatile("" ::: "memory");
            const int mt0 = wm * TM + fi * 32 + 16 * h;
            const bool fast = vec && p.Y && !p.acc && !p.accumulate;  // plain Y store (no raw accumulators requested)
            if (fast && p.act == KERNIX_ACT_RELU_ID)
                store_rows<0>(p, stg, row_scale, mt0, m0, mlo, nlo, rq, RPI, SROW, cq, nb, swv, bv);
            else if (fast && p.act == 1)  // GELU
                store_rows<1>(p, stg, row_scale, mt0, m0, mlo, nlo, rq, RPI, SROW, cq, nb, swv, bv);
            else if (fast && p.act == -1)
                store_rows<-1>(p, stg, row_scale, mt0, m0, mlo, nlo, rq, RPI, SROW, cq, nb, swv, bv);
            else
                store_rows<-2>(p, stg, row_scale, mt0, m0, mlo, nlo, rq, RPI, SROW, cq, nb, swv, bv, vec);
            asm volatile("" ::: "memory");
        }
    }
}

template <int BM, int BN, int WM, int WN, int STAGES>
__global__ void __launch_bounds__(WM * WN * 64) i8gemm_pipe(I8Args p)
{
    constexpr int NW = WM * WN;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 32, FN = TN / 32;
    constexpr int ROWS = BM + BN;
    constexpr int STAGE = ROWS * 64;           // bytes per k-tile
    constexpr int SLOTS = ROWS / 16 / NW;      // 1-KB load instructions per wave per k-tile
    static_assert(ROWS % (16 * NW) == 0, "load split");
    static_assert(STAGES >= 2 && STAGES <= 5 && (STAGES - 2) * SLOTS <= 63, "vmcnt range");
    __shared__ __attribute__((aligned(16))) int8_t lds[STAGES * STAGE];
    __shared__ float row_scale[BM]; // sa of the tile's rows, staged once so the epilogue never waits on HBM per row

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave / WN, wn = wave % WN;
    int tm, tn;
    tile_of_best(blockIdx.x, p.tiles_m, p.tiles_n, BM, BN, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    // per-lane epilogue constants (this lane's 4 output columns), loaded now so their latency hides under the K loop
    constexpr int LPR_ = (BN / WN) / 4;
    const int nb_ = n0 + wn * (BN / WN) + (lane % LPR_) * 4;
    float swv[4], bv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const bool ok = nb_ + q < p.N;
        swv[q] = (ok && p.Y) ? p.sw[nb_ + q] : 0.0f;
        bv[q] = (ok && p.bias) ? p.bias[nb_ + q] : 0.0f;
    }

    // per slot: global row pointer (with this lane's swizzled chunk) and the LDS offset of the wave's 1-KB block
    const int8_t* gsrc[SLOTS];
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
        const int row = (i * NW + wave) * 16 + (lane >> 2);
        const int chunk = (lane & 3) ^ swz(row);
        if (row < BM) {
            const int gm = min(m0 + row, p.M - 1);
            gsrc[i] = p.A + (size_t)gm * p.lda + chunk * 16;
        } else {
            const int gn = min(n0 + row - BM, p.N - 1);
            gsrc[i] = p.W + (size_t)gn * p.ldw + chunk * 16;
        }
    }
    auto issue = [&](int kt) {
        int8_t* stage = lds + (kt % STAGES) * STAGE;
#pragma unroll
        for (int i = 0; i < SLOTS; ++i)
            __builtin_amdgcn_global_load_lds((gbl_ptr_t)(gsrc[i] + (size_t)kt * 64), (lds_ptr_t)(stage + (i * NW + wave) * 1024),
                                             16, 0, 0);
    };

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

    const int nk = p.K / 64;
    // this thread's row scale: loaded before the first k-tiles (vmcnt retires in order, so it is never waited for
    // separately), kept in a register and staged to LDS for the epilogue
    static_assert(BM <= NW * 64, "one row scale per thread");
    const float my_sa = (t < BM && p.Y && m0 + t < p.M) ? p.sa[m0 + t] : 0.0f;
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < nk) issue(s);

    // Before the barrier each wave waits until its loads of tile kt have landed (at most min(STAGES-2, nk-1-kt)
    // younger tiles may stay in flight) and until its own LDS reads have retired.  After the barrier every wave's part
    // of tile kt is in LDS and no wave still reads the stage that issue() refills: that stage last held tile
    // kt−1 (read before the previous barrier) and is the one the fragments of the previous half came from, whose
    // reads the lgkmcnt(0) of every wave retired.
    auto arrive = [&](int kt) {
        const int younger = min(STAGES - 2, nk - 1 - kt);
        if (younger >= 3) KNX_WAIT_VM_LDS(3 * SLOTS);
        else if (younger == 2) KNX_WAIT_VM_LDS(2 * SLOTS);
        else if (younger == 1) KNX_WAIT_VM_LDS(SLOTS);
        else KNX_WAIT_VM_LDS(0);
        knx_barrier_nofence();
        if (kt + STAGES - 1 < nk) issue(kt + STAGES - 1);
    };
    auto frags = [&](int kt, int s, v4i* af, v4i* bf) {
        const int8_t* cur = lds + (kt % STAGES) * STAGE;
#pragma unroll
        for (int fi = 0; fi < FM; ++fi) af[fi] = *(const v4i*)(cur + aoff[fi][s]);
#pragma unroll
        for (int fj = 0; fj < FN; ++fj) bf[fj] = *(const v4i*)(cur + boff[fj][s]);
    };
    auto mfmas = [&](const v4i* af, const v4i* bf) {
#pragma unroll
        for (int fi = 0; fi < FM; ++fi)
#pragma unroll
            for (int fj = 0; fj < FN; ++fj)
                acc[fi][fj] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[fi], bf[fj], acc[fi][fj], 0, 0, 0);
    };

    // Software pipeline over half k-tiles (32 bytes of k each): the fragments of the next half are read from LDS
    // while the MFMAs of the current half run.
    v4i a0[FM], b0[FN], a1[FM], b1[FN];
    if (nk > 0) {
        arrive(0);
        frags(0, 0, a0, b0);
    }
    for (int kt = 0; kt < nk; ++kt) {
        frags(kt, 1, a1, b1);
        mfmas(a0, b0);
        if (kt + 1 < nk) {
            arrive(kt + 1);
            frags(kt + 1, 0, a0, b0);
        }
        mfmas(a1, b1);
    }

    static_assert(NW * 16 * (TN + 4) * 4 <= STAGES * STAGE, "staging fits in the ring");
    tile_epilogue<BM, BN, WM, WN>(p, acc, lds, row_scale, my_sa, m0, nb_, swv, bv, m0, n0);
}

template <int BM, int BN, int WM, int WN, int STAGES>
int launch_pipe(I8Args p, hipStream_t s, const char* name)
{
    p.tiles_m = (p.M + BM - 1) / BM;
    p.tiles_n = (p.N + BN - 1) / BN;
    const unsigned grid = (unsigned)p.tiles_m * (unsigned)p.tiles_n;
    hipLaunchKernelGGL((i8gemm_pipe<BM, BN, WM, WN, STAGES>), dim3(grid), dim3(WM * WN * 64), 0, s, p);
    return knx::check_launch(name);
}

// ---------------------------------------------------------------- 128-byte k-tile kernel
// Each operand row contributes one whole 128-byte cache line per k-tile (a 64-byte k-tile fetches half lines, which
// wastes half of every L2 → CU transfer).  The A rows of the tile go through a ring of ASTG LDS stages, the W rows
// through a ring of two; one workgroup barrier per 128 bytes of K.
//
// Why three A stages: the L2 → LDS path of a CU moves a 64-KB k-tile (256 A + 256 W rows) in about the time the
// MFMAs need for it, so with two stages of both operands the loads of k-tile kt+2, which can only start once every
// wave is done with stage kt, arrive just when they are needed and the barrier waits for them.  160 KB of LDS holds
// three 32-KB A stages and two 32-KB W stages.  Without EARLY the loads of A k-tile kt+3 are issued after the barrier
// of k-tile kt together with those of W k-tile kt+2 (W first); with EARLY (the default for long K) the A loads of
// k-tile kt+2 go out during k-steps 0..2 of k-tile kt, into the stage k-tile kt−1 left, and only the W loads follow
// the barrier: the A loads have more than a k-tile to arrive, only 32 KB must land within one k-tile, and the loads
// are not issued as one burst.  Vector-memory loads retire in issue order, so the wait for k-tile kt+1 leaves exactly
// this wave's SA younger A loads outstanding in both schemes.
//
// LDS layout: a row holds 8 chunks of 16 bytes, global chunk c of row r at position c ^ swz8(r).  The 16 rows that
// one quarter-wave of a ds_read_b128 touches (same chunk, consecutive rows) then fall on 16 distinct 16-byte bank
// groups, and any 8 consecutive rows on 8.  swz8(r + 32) = swz8(r) ^ 4, so the fragment of row r + 32·f at k-step s
// sits at the offset of row r's k-step s ^ 2·(f & 1), plus f·4096: four offset registers per operand cover every
// fragment.
//
// Loads: global_load_lds_dwordx4 with a scalar base (tile row + slot row · ld + k) and a 32-bit lane offset
// (row-in-slot · ld + chunk).  A tile that would run past M (or N) is moved back to end at row M (column N): it
// recomputes a few rows of its neighbour and stores only the rows (columns) it owns, so every operand row it reads
// exists.  A half k-tile at the end (K % 128 == 64) loads its lower 64 bytes twice and multiplies two k-steps only.
// ---- K split across workgroups (KS > 1), for shapes whose output tiles are fewer than the CUs (M = 256,
// N = K = 4096 in 128×128 tiles: 64 tiles, 4 workgroups each over a quarter of K).  Every workgroup stores its int32
// partial tile at device scope (sc1 stores, through to the coherence point the XCDs share) into the stream's
// scratch, then increments its tile's arrival counter; the workgroup whose increment completes a multiple of KS is
// the last of the tile: it loads the other KS − 1 partial tiles (sc1 loads), adds them to its own (int32: exact in
// any order) and runs the epilogue.  No workgroup waits for another, so residency does not matter, and every
// launch adds exactly kSplitQuantum to each counter, so nothing is reset between launches.  Partial layout: unit (tile, split)
// owns FM·FN·4 × NT 16-byte pieces, piece q of thread t at (q·NT + t)·16 — each store instruction of a wave writes
// 1 KB of consecutive bytes.
constexpr unsigned kSplitRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit data format
constexpr int kSc1 = 16;                           // cache policy of a buffer access: sc1 (device scope)

constexpr unsigned kSplitQuantum = 256;            // added to a tile's arrival counter per launch

template <int FM, int FN, int NT, int KS>
__device__ __forceinline__ bool split_reduce(const I8Args& p, v16i (&acc)[FM][FN], int tile, int split, unsigned* flag)
{
    constexpr int Q = FM * FN * 4;
    static_assert(KS >= 2 && kSplitQuantum % KS == 0, "split count");
    const int t = threadIdx.x;
    const long long bytes = (long long)p.tiles_m * p.tiles_n * KS * Q * NT * 16;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(p.part, (short)0, (int)bytes, kSplitRsrcWord3);
    const int own = (tile * KS + split) * Q * NT * 16;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const v16i& a = acc[(q >> 2) / FN][(q >> 2) % FN];
        const v4i v = {a[4 * (q & 3)], a[4 * (q & 3) + 1], a[4 * (q & 3) + 2], a[4 * (q & 3) + 3]};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u_t, v), r, own + (q * NT + t) * 16, 0, kSc1);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial is at the coherence point
    __syncthreads();
    if (t == 0) {
        // the counter is a multiple of kSplitQuantum when the launch starts; the KS-th arrival completes the tile and
        // tops the counter up to the next multiple, whatever KS the next launch on this scratch uses
        const unsigned old = __hip_atomic_fetch_add(p.cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = old % kSplitQuantum == KS - 1;
        if (last) __hip_atomic_fetch_add(p.cnt + tile, kSplitQuantum - KS, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = last;
    }
    __syncthreads();
    if (!*flag) return false;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        if (s == split) continue;
        const int base = (tile * KS + s) * Q * NT * 16;
        v4i got[Q];
#pragma unroll
        for (int q = 0; q < Q; ++q)
            got[q] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, base + (q * NT + t) * 16, 0, kSc1));
#pragma unroll
        for (int q = 0; q < Q; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[(q >> 2) / FN][(q >> 2) % FN][4 * (q & 3) + e] += got[q][e];
    }
    return true;
}

template <int BM, int BN, int WM, int WN, int ASTG, bool EARLY = false, int KS = 1>
__global__ void __launch_bounds__(WM * WN * 64) i8gemm_k128(I8Args p)
{
    constexpr int NW = WM * WN;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 32, FN = TN / 32;
    constexpr int ABYTES = BM * 128, WBYTES = BN * 128;  // one k-tile of A rows / of W rows
    constexpr int WRING = ASTG * ABYTES;                 // the W ring follows the A ring
    constexpr int SLOTS = (BM + BN) / 8 / NW;            // 1-KB loads (8 rows × 128 bytes) per wave per k-tile
    constexpr int SA = BM / 8 / NW;                      // slots 0..SA-1 load A rows, the rest W rows
    constexpr int SW = SLOTS - SA;
    constexpr int STG = NW * 16 * (TN + 4) * 4;          // epilogue staging bytes (from offset 0)
    static_assert(ASTG == 2 || ASTG == 3, "A ring depth");
    static_assert(BM % (8 * NW) == 0 && BN % (8 * NW) == 0 && SLOTS <= 63, "load split");
    static_assert(TM % 32 == 0 && TN % 32 == 0 && BM % 64 == 0, "wave tile");
    static_assert(STG <= WRING + WBYTES - BM * 4, "staging below the row scales");
    static_assert(WRING + 2 * WBYTES <= 160 * 1024, "LDS");
    static_assert(BM <= NW * 64, "one row scale per thread");
    __shared__ __attribute__((aligned(16))) int8_t lds[WRING + 2 * WBYTES];

    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wave / WN, wn = wave % WN;
    int tm, tn, split = 0;
    if (KS == 1) {
        tile_of_best(blockIdx.x, p.tiles_m, p.tiles_n, BM, BN, tm, tn);
    } else {
        // consecutive workgroups go to consecutive XCDs: XCD x takes units [x·G/8, (x+1)·G/8), tm fastest, then the
        // split, then tn, so the splits of a tile and the tiles that share W rows stay on one XCD
        const int G = gridDim.x;
        const int g = G % 8 == 0 ? (blockIdx.x & 7) * (G / 8) + (blockIdx.x >> 3) : blockIdx.x;
        tm = g % p.tiles_m;
        split = (g / p.tiles_m) % KS;
        tn = g / p.tiles_m / KS;
    }
    const int mlo = tm * BM, nlo = tn * BN;                  // first row / column this tile owns
    const int m0 = min(mlo, p.M - BM), n0 = min(nlo, p.N - BN);  // first row / column it computes

    // this lane's 4 epilogue columns and its row scale, loaded first so their latency hides under the K loop
    const int nb = n0 + wn * TN + (lane % (TN / 4)) * 4;
    float swv[4], bv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        swv[q] = p.Y ? p.sw[nb + q] : 0.0f;
        bv[q] = p.bias ? p.bias[nb + q] : 0.0f;
    }
    const float my_sa = (t < BM && p.Y) ? p.sa[m0 + t] : 0.0f;

    // slot i covers rows (i·NW + wave)·8 + 0..7 of the tile's A rows then W rows; lane l loads row l >> 3 of the slot,
    // global chunk (l & 7) ^ swz8(row) = (l & 7) ^ (l >> 3) ^ ((i·NW + wave) & 7) into LDS position l & 7.  The
    // address is a scalar base (operand tile + slot row · ld + k) plus this lane's 32-bit offset.  With a K split
    // the workgroup's K range is [split·K/KS, (split+1)·K/KS), whole k-tiles (K % (128·KS) == 0).
    const int kspan = p.K / KS;
    const int8_t* tile_a = p.A + (size_t)m0 * p.lda + (size_t)split * kspan;
    const int8_t* tile_w = p.W + (size_t)n0 * p.ldw + (size_t)split * kspan;
    const int cl = (lane & 7) ^ (lane >> 3), rs = lane >> 3;
    const int nk = (kspan + 127) / 128;
    const bool half = (kspan & 127) != 0;
    auto abuf = [&](int kt) { return lds + (ASTG == 2 ? (kt & 1) : kt % 3) * ABYTES; };
    auto wbuf = [&](int kt) { return lds + WRING + (kt & 1) * WBYTES; };
    // load slot i of k-tile kt into its stage
    auto issue1 = [&](int kt, int i) {
        const int slot = i * NW + wave;
        const bool a = i < SA;
        const int ld = a ? p.lda : p.ldw;
        int chunk = cl ^ (slot & 7);
        if (half && kt == nk - 1) chunk &= 3;  // the upper 64 bytes are past K: load the lower ones again (never multiplied)
        const int8_t* base = (a ? tile_a + (size_t)(slot * 8) * ld : tile_w + (size_t)(slot * 8 - BM) * ld) + kt * 128;
        int8_t* dst = a ? abuf(kt) + slot * 1024 : wbuf(kt) + (slot - BM / 8) * 1024;
        dma16(base, (unsigned)(rs * ld + chunk * 16), dst);
    };

    const int rl = lane & 31, g = lane >> 5;
    int aoff[4], boff[4];
    {
        const int ra_ = wm * TM + rl, rb_ = wn * TN + rl;
        const int sa_ = swz8(ra_), sb_ = swz8(rb_);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            aoff[s] = ra_ * 128 + (((2 * s + g) ^ sa_) << 4);
            boff[s] = rb_ * 128 + (((2 * s + g) ^ sb_) << 4);
        }
    }
    // fragment j of k-step s of k-tile kt: j < FM an A fragment, else a W fragment
    v4i fa[2][FM], fb[2][FN];
    auto read1 = [&](int kt, int s, int j) {
        if (j < FM) fa[s & 1][j] = *(const v4i*)(abuf(kt) + aoff[s ^ (2 * (j & 1))] + j * 4096);
        else fb[s & 1][j - FM] = *(const v4i*)(wbuf(kt) + boff[s ^ (2 * ((j - FM) & 1))] + (j - FM) * 4096);
    };

    v16i acc[FM][FN];
#pragma unroll
    for (int fi = 0; fi < FM; ++fi)
#pragma unroll
        for (int fj = 0; fj < FN; ++fj)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[fi][fj][e] = 0;
    // multiply j of k-step s (fragment set s & 1)
    auto mfma1 = [&](int s, int j) {
        const int fi = j / FN, fj = j % FN;
        acc[fi][fj] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[s & 1][fi], fb[s & 1][fj], acc[fi][fj], 0, 0, 0);
    };

    // One k-tile.  K-steps 0..2: multiply fragment set s & 1 while the FM+FN fragments of k-step s+1 are read, one
    // read after each of the first FM+FN multiplies (the reads hide under the MFMA pipeline).  K-step 3: after the
    // first PRE multiplies the wave waits for its loads of tile kt+1 (WAITC younger loads may stay outstanding) and for
    // its own LDS reads (which include the last ones of tile kt), then the workgroup barrier: tile kt+1 is complete in
    // LDS and nobody reads the stages of tile kt any more, so the remaining multiplies are interleaved with the first
    // fragment reads of tile kt+1 and the loads into those stages: W rows of tile kt+2 (ISSW), then A rows of tile
    // kt+ASTG (ISSA).  The flags are compile-time so the steady-state loop has no branches (a branch merge makes the
    // compiler wait for every outstanding LDS read at the merge); the sched_barrier(0) calls pin the interleaving.
    constexpr int NM = FM * FN, NR = FM + FN, PRE = NM / 4;
    constexpr int GAPS = NM - PRE;
    auto ktile = [&](int kt, auto ARRIVE, auto ISSW, auto ISSA, auto WAITC, bool upper) {
        constexpr bool arrive = decltype(ARRIVE)::value;
        constexpr bool isw = decltype(ISSW)::value, isa = decltype(ISSA)::value;
        // EARLY: the A loads (tile kt+2, into the stage tile kt-1 left) go out during k-steps 0..2, one group per
        // k-step, instead of in the burst after the barrier
        constexpr bool early = EARLY && ASTG == 3;
        constexpr int NL = (isw ? SW : 0) + (isa && !early ? SA : 0);
        auto issue_nth = [&](int l) {  // the l-th load after the barrier: W slots first, then A slots
            if (isw && l < SW) issue1(kt + 2, SA + l);
            else issue1(kt + ASTG, l - (isw ? SW : 0));
        };
#pragma unroll
        for (int s = 0; s < 3; ++s) {
#pragma unroll
            for (int j = 0; j < NR; ++j) read1(kt, s + 1, j);
            if (s < 2 || upper)
#pragma unroll
                for (int j = 0; j < NM; ++j) mfma1(s, j);
#pragma unroll
            for (int j = 0; j < NR; ++j) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, NM - NR, 0);
            if (early && isa) {
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = SA * s / 3; i < SA * (s + 1) / 3; ++i) issue1(kt + 2, i);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (!upper) return;  // a half k-tile: k-steps 2 and 3 are past K
        if (!arrive) {
#pragma unroll
            for (int j = 0; j < NM; ++j) mfma1(3, j);
            return;
        }
#pragma unroll
        for (int j = 0; j < PRE; ++j) mfma1(3, j);
        __builtin_amdgcn_sched_barrier(0);
        KNX_WAIT_VM_LDS(decltype(WAITC)::value);
        knx_barrier_nofence();
        int r = 0, l = 0;
#pragma unroll
        for (int j = PRE; j < NM; ++j) {
            mfma1(3, j);
            const int rupto = (NR * (j - PRE + 1) + GAPS - 1) / GAPS;  // reads first: they are needed sooner
            while (r < rupto) read1(kt + 1, 0, r++);
            const int upto = (NL * (j - PRE + 1) + GAPS - 1) / GAPS;  // spread the loads over the gaps
            while (l < upto) issue_nth(l++);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    using yes = std::integral_constant<bool, true>;
    using no = std::integral_constant<bool, false>;
    using w0 = std::integral_constant<int, 0>;
    using wa = std::integral_constant<int, ASTG == 3 ? SA : 0>;
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) issue1(0, i);
    KNX_WAIT_VM_LDS(0);
    knx_barrier_nofence();
    if (nk > 1)
#pragma unroll
        for (int i = 0; i < SLOTS; ++i) issue1(1, i);
#pragma unroll
    for (int j = 0; j < NR; ++j) read1(0, 0, j);
    int kt = 0;
    if (ASTG == 3 && EARLY) {
        // tile kt issues A(kt+2) during its k-steps 0..2 and W(kt+2) after its barrier
        for (; kt < nk - 2; ++kt) ktile(kt, yes{}, yes{}, yes{}, wa{}, true);
    } else if (ASTG == 3) {
        if (nk > 2)
#pragma unroll
            for (int i = 0; i < SA; ++i) issue1(2, i);
        for (; kt < nk - 3; ++kt) ktile(kt, yes{}, yes{}, yes{}, wa{}, true);
        if (nk >= 3) ktile(kt++, yes{}, yes{}, no{}, wa{}, true);
    } else {
        for (; kt < nk - 2; ++kt) ktile(kt, yes{}, yes{}, yes{}, w0{}, true);
    }
    if (nk >= 2) ktile(kt++, yes{}, no{}, no{}, w0{}, true);
    ktile(kt, no{}, no{}, no{}, w0{}, !half);

    if constexpr (KS > 1) {
        __shared__ unsigned arrived;
        if (!split_reduce<FM, FN, NW * 64, KS>(p, acc, tm * p.tiles_n + tn, split, &arrived)) return;
    }
    // the row scales go to the W stage that the last k-tile does not use (free since the barrier of k-tile nk-2)
    float* row_scale = reinterpret_cast<float*>(wbuf(nk) + WBYTES - BM * 4);
    tile_epilogue<BM, BN, WM, WN>(p, acc, lds, row_scale, my_sa, m0, nb, swv, bv, mlo, nlo);
}

__global__ void zero_words(unsigned* w, size_t n)
{
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) w[i] = 0;
}

// Scratch of the K-split kernels, one per stream (launches on one stream are ordered, so they may share it; launches
// on different streams never do): arrival counters (zero when allocated, a multiple of the split count after every
// launch) followed by the partial tiles.  Grown when a launch needs more (the stream is synchronized first: earlier
// launches may still use the old one); kept until the process ends.
struct SplitScratch {
    char* buf = nullptr;
    size_t cnt_bytes = 0, part_bytes = 0;
};
std::mutex g_split_mu;
std::unordered_map<hipStream_t, SplitScratch> g_split;
thread_local bool g_no_alloc = false;  // inside knx_hip_qlinear_noalloc: no K split (it would allocate)

int split_scratch(hipStream_t s, size_t part_bytes, size_t cnt_words, int32_t** part, unsigned** cnt, const char* name)
{
    const size_t cb = (cnt_words * sizeof(unsigned) + 255) / 256 * 256;
    std::lock_guard<std::mutex> lock(g_split_mu);
    SplitScratch& sc = g_split[s];
    if (sc.buf == nullptr || sc.cnt_bytes < cb || sc.part_bytes < part_bytes) {
        const size_t nc = std::max(cb, sc.cnt_bytes), np = std::max(part_bytes, sc.part_bytes);
        if (sc.buf != nullptr) {
            if (hipStreamSynchronize(s) != hipSuccess || hipFree(sc.buf) != hipSuccess)
                return knx::fail(KNX_EHIP, "%s: K-split scratch release failed", name);
            sc = SplitScratch{};
        }
        void* b = nullptr;
        const hipError_t e = hipMalloc(&b, nc + np);
        if (e != hipSuccess) return knx::fail(KNX_EHIP, "%s: K-split scratch (%zu bytes): %s", name, nc + np, hipGetErrorString(e));
        hipLaunchKernelGGL(zero_words, dim3(64), dim3(256), 0, s, static_cast<unsigned*>(b), nc / sizeof(unsigned));
        if (knx::check_launch(name) != KNX_OK) {
            hipFree(b);
            return KNX_EHIP;
        }
        sc.buf = static_cast<char*>(b);
        sc.cnt_bytes = nc;
        sc.part_bytes = np;
    }
    *cnt = reinterpret_cast<unsigned*>(sc.buf);
    *part = reinterpret_cast<int32_t*>(sc.buf + sc.cnt_bytes);
    return KNX_OK;
}

template <int BM, int BN, int WM, int WN, int ASTG, bool EARLY = false, int KS = 1>
int launch_k128(I8Args p, hipStream_t s, const char* name)
{
    p.tiles_m = (p.M + BM - 1) / BM;
    p.tiles_n = (p.N + BN - 1) / BN;
    const unsigned grid = (unsigned)p.tiles_m * (unsigned)p.tiles_n * (unsigned)KS;
    if (KS > 1) {
        const size_t tiles = (size_t)p.tiles_m * (size_t)p.tiles_n;
        const int rc = split_scratch(s, tiles * KS * BM * BN * sizeof(int32_t), tiles, &p.part, &p.cnt, name);
        if (rc != KNX_OK) return rc;
    }
    hipLaunchKernelGGL((i8gemm_k128<BM, BN, WM, WN, ASTG, EARLY, KS>), dim3(grid), dim3(WM * WN * 64), 0, s, p);
    return knx::check_launch(name);
}

// ---------------------------------------------------------------- ping-pong kernel
// Same tiles, LDS layout and loads as i8gemm_k128, with the eight waves split in two groups of four (one wave of each
// group per SIMD) that take turns: while one group multiplies two k-steps from registers, the other reads its
// fragments of the next two k-steps from LDS (and group 0 also issues the loads), then a workgroup barrier and the
// roles swap.  The MFMA unit of a SIMD is always fed by the wave whose operands are already in registers, and a wave
// stalled on issuing loads or on LDS latency never holds back the multiplies of the other.  K-tile t (two halves of two
// k-steps) runs as four phases:
//   group 0 multiplies half 0 of t                 group 1 reads half 0 of t, loads its half of k-tile t+1
//   group 0 reads half 1 of t                      group 1 multiplies half 0 of t
//   group 0 multiplies half 1 of t                 group 1 reads half 1 of t (last reads of stage t & 1)
//   group 0 loads its half of k-tile t+2 into stage t & 1, reads half 0 of t+1;   group 1 multiplies half 1 of t
template <int BM, int BN>
__global__ void __launch_bounds__(512) i8gemm_pp(I8Args p)
{
    constexpr int WM = 4, WN = 2, NW = 8;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 32, FN = TN / 32;
    constexpr int ROWS = BM + BN;
    constexpr int STAGE = ROWS * 128;
    constexpr int SLOTS = ROWS / 8 / NW;   // 1-KB loads per wave per k-tile
    constexpr int SA = BM / 8 / NW;
    static_assert(BM % (8 * NW) == 0 && BN % (8 * NW) == 0, "load split");
    static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile");
    static_assert(NW * 16 * (TN + 4) * 4 <= 2 * STAGE, "staging fits in the stages");
    static_assert(BM <= NW * 64, "one row scale per thread");
    __shared__ __attribute__((aligned(16))) int8_t lds[2 * STAGE];
    __shared__ float row_scale[BM];

    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int grp = wave >> 2;
    const int wm = wave / WN, wn = wave % WN;
    int tm, tn;
    tile_of_best(blockIdx.x, p.tiles_m, p.tiles_n, BM, BN, tm, tn);
    const int mlo = tm * BM, nlo = tn * BN;
    const int m0 = min(mlo, p.M - BM), n0 = min(nlo, p.N - BN);

    const int nb = n0 + wn * TN + (lane % (TN / 4)) * 4;
    float swv[4], bv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        swv[q] = p.Y ? p.sw[nb + q] : 0.0f;
        bv[q] = p.bias ? p.bias[nb + q] : 0.0f;
    }
    const float my_sa = (t < BM && p.Y) ? p.sa[m0 + t] : 0.0f;

    const int8_t* tile_a = p.A + (size_t)m0 * p.lda;
    const int8_t* tile_w = p.W + (size_t)n0 * p.ldw;
    const int cl = (lane & 7) ^ (lane >> 3), rs = lane >> 3;
    const int nk = (p.K + 127) / 128;
    const bool half = (p.K & 127) != 0;
    // this wave's share of the loads of k-tile kt
    auto issue = [&](int kt) {
#pragma unroll
        for (int i = 0; i < SLOTS; ++i) {
            const int slot = i * NW + wave;
            const bool a = i < SA;
            const int ld = a ? p.lda : p.ldw;
            int chunk = cl ^ (slot & 7);
            if (half && kt == nk - 1) chunk &= 3;
            const int8_t* base = (a ? tile_a + (size_t)(slot * 8) * ld : tile_w + (size_t)(slot * 8 - BM) * ld) + kt * 128;
            dma16(base, (unsigned)(rs * ld + chunk * 16), lds + (kt & 1) * STAGE + slot * 1024);
        }
    };

    const int rl = lane & 31, g = lane >> 5;
    int aoff[4], boff[4];
    {
        const int ra_ = wm * TM + rl, rb_ = BM + wn * TN + rl;
        const int sa_ = swz8(ra_), sb_ = swz8(rb_);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            aoff[s] = ra_ * 128 + (((2 * s + g) ^ sa_) << 4);
            boff[s] = rb_ * 128 + (((2 * s + g) ^ sb_) << 4);
        }
    }
    // the fragments of two k-steps (half h of k-tile kt)
    v4i fa[2][FM], fb[2][FN];
    auto read_half = [&](int kt, int h) {
        const int8_t* cur = lds + (kt & 1) * STAGE;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int k = 2 * h + s;
#pragma unroll
            for (int fi = 0; fi < FM; ++fi) fa[s][fi] = *(const v4i*)(cur + aoff[k ^ (2 * (fi & 1))] + fi * 4096);
#pragma unroll
            for (int fj = 0; fj < FN; ++fj) fb[s][fj] = *(const v4i*)(cur + boff[k ^ (2 * (fj & 1))] + fj * 4096);
        }
    };
    v16i acc[FM][FN];
#pragma unroll
    for (int fi = 0; fi < FM; ++fi)
#pragma unroll
        for (int fj = 0; fj < FN; ++fj)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[fi][fj][e] = 0;
    auto compute_half = [&]() {
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int fi = 0; fi < FM; ++fi)
#pragma unroll
                for (int fj = 0; fj < FN; ++fj)
                    acc[fi][fj] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[s][fi], fb[s][fj], acc[fi][fj], 0, 0, 0);
    };

    // Both groups run the same sequence of operations — per k-tile R(t,0) C(t,0) R(t,1) C(t,1), each ending at a
    // workgroup barrier — with group 1 one barrier behind, so a barrier ends a C of one group and an R of the other and
    // no branch on the group (which would merge register values) is needed.  R(t,0) also issues the wave's share of
    // the loads of k-tile t+1 (into the stage last read in R(t-1,1) of group 1, which ended before group 0's R(t,0)
    // began); every wave waits for its loads (vmcnt) before the barrier that precedes group 0's R(t+1,0): group 0 at
    // the end of C(t,1), group 1 at the end of R(t,1).
    // A phase boundary: the accumulators pass through an empty asm statement next to the barrier, so no multiply
    // moves across it (MFMAs touch no memory, so the barrier's memory clobber alone would not hold them), and the
    // machine scheduler keeps every instruction on its side.
    static_assert(FM * FN == 8, "phase boundary pins eight accumulators");
    auto boundary = [&]() {
        asm volatile("" : "+v"(acc[0][0]), "+v"(acc[0][1]), "+v"(acc[0][2]), "+v"(acc[0][3]), "+v"(acc[1][0]),
                     "+v"(acc[1][1]), "+v"(acc[1][2]), "+v"(acc[1][3]));
        __builtin_amdgcn_sched_barrier(0);
        knx_barrier_nofence();
        __builtin_amdgcn_sched_barrier(0);
    };
    issue(0);
    KNX_WAIT_VM_LDS(0);
    boundary();
    if (grp == 1) boundary();
    for (int kt = 0; kt < nk; ++kt) {
        // R(t,0)
        if (kt + 1 < nk) issue(kt + 1);
        read_half(kt, 0);
        KNX_WAIT_LDS();
        boundary();
        // C(t,0)
        compute_half();
        boundary();
        // R(t,1)
        read_half(kt, 1);
        if (grp == 1) KNX_WAIT_VM_LDS(0);
        else KNX_WAIT_LDS();
        boundary();
        // C(t,1): a half k-tile (K % 128 == 64, last) has no k-steps 2 and 3
        if (!(half && kt == nk - 1)) compute_half();
        if (grp == 0) KNX_WAIT_VM_LDS(0);
        boundary();
    }
    if (grp == 0) boundary();

    tile_epilogue<BM, BN, WM, WN>(p, acc, lds, row_scale, my_sa, m0, nb, swv, bv, mlo, nlo);
}

template <int BM, int BN>
int launch_pp(I8Args p, hipStream_t s, const char* name)
{
    p.tiles_m = (p.M + BM - 1) / BM;
    p.tiles_n = (p.N + BN - 1) / BN;
    const unsigned grid = (unsigned)p.tiles_m * (unsigned)p.tiles_n;
    hipLaunchKernelGGL((i8gemm_pp<BM, BN>), dim3(grid), dim3(512), 0, s, p);
    return knx::check_launch(name);
}

// the 128-byte k-tile kernel needs whole tiles inside the matrices (tiles are moved back, never clipped) and each
// lane offset (at most 7 rows) inside 32 bits
template <int BM, int BN>
bool k128_fits(const I8Args& p)
{
    return p.M >= BM && p.N >= BN && (long)8 * p.lda < 0x7fffffffL && (long)8 * p.ldw < 0x7fffffffL;
}

// the K split: whole 128-byte k-tiles per split, partial tiles addressable by 32-bit buffer offsets, and no
// allocation inside knx_hip_qlinear_noalloc
template <int BM, int BN, int KS>
bool ksplit_fits(const I8Args& p)
{
    const long long tiles = (long long)((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
    return k128_fits<BM, BN>(p) && p.K % (128 * KS) == 0 && tiles * KS * BM * BN * 4 < (1LL << 31) - 256 && !g_no_alloc;
}

// f(integral_constant<int, d>) for d = 0, 1, …: a loop whose index is a compile-time constant in the body
template <typename F, int... T>
__device__ __forceinline__ void ring_unrolled(F&& f, std::integer_sequence<int, T...>)
{
    (f(std::integral_constant<int, T>{}), ...);
}

// ---------------------------------------------------------------- deep-ring kernel (mid-size M)
// Shapes whose 256×256 and 128×128 tiles would leave CUs idle (e.g. M = 256, N = K = 4096: 64×64 tiles give every CU
// one) move little MFMA work per k-tile (a 64×64×128 k-tile is 128 MFMA cycles per SIMD) against 16 KB of loads, so
// latency decides: S LDS stages of 128-byte k-tiles (whole lines, the same swizzled layout and LDS-DMA loads as
// i8gemm_k128) keep S−KPI k-tiles in flight per ring.  Per iteration of KPI k-tiles: wait until their loads have
// landed (vmcnt counts the younger ones still in flight), one workgroup barrier (every wave is done with the previous
// KPI k-tiles, whose stages are free), issue the loads of the k-tiles S−KPI ahead into those stages, read every
// fragment of the KPI k-tiles at once (one LDS round trip instead of one per k-step), multiply.
//
// KG > 1 splits K inside the workgroup: KG groups of WM×WN waves, group g streams k-tiles [g·nk/KG, (g+1)·nk/KG)
// through a ring of its own, so a CU keeps KG times the bytes in flight for the same tile.  Every group runs the
// same number of iterations (nk % KG == 0), so the workgroup barriers match.  At the end the groups g ≥ 1 hand their
// int32 partial tiles to group 0 through LDS (exact adds), and group 0 runs the epilogue.
template <int BM, int BN, int WM, int WN, int S, int KPI, int KG = 1>
__global__ void __launch_bounds__(KG * WM * WN * 64) i8gemm_ring(I8Args p)
{
    constexpr int NW = WM * WN;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 32, FN = TN / 32;
    constexpr int ROWS = BM + BN;
    constexpr int STAGE = ROWS * 128;
    constexpr int SLOTS = ROWS / 8 / NW;  // 1-KB loads per wave per k-tile
    constexpr int SA = BM / 8 / NW;
    static_assert(KPI == 1 || KPI == 2, "k-tiles per iteration");
    static_assert(BM % (8 * NW) == 0 && BN % (8 * NW) == 0, "load split");
    static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile");
    static_assert(S >= 2 * KPI && SLOTS * 6 <= 63, "ring depth and vmcnt range");
    static_assert(NW * 16 * (TN + 4) * 4 <= S * STAGE, "staging fits in the ring");
    static_assert(NW * FM * FN * 16 * 64 * 4 <= S * STAGE, "a partial tile fits in a ring");
    static_assert(BM <= NW * 64, "one row scale per thread");
    __shared__ __attribute__((aligned(16))) int8_t lds_all[KG * S * STAGE];
    __shared__ float row_scale[BM];

    const int t = threadIdx.x, lane = t & 63;
    const int wave_all = __builtin_amdgcn_readfirstlane(t >> 6);
    const int kg = wave_all / NW, wave = wave_all % NW;  // K group, wave within the group
    int8_t* const lds = lds_all + kg * S * STAGE;
    const int wm = wave / WN, wn = wave % WN;
    int tm, tn;
    tile_of_best(blockIdx.x, p.tiles_m, p.tiles_n, BM, BN, tm, tn);
    const int mlo = tm * BM, nlo = tn * BN;
    const int m0 = min(mlo, p.M - BM), n0 = min(nlo, p.N - BN);

    const int nb = n0 + wn * TN + (lane % (TN / 4)) * 4;
    float swv[4], bv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        swv[q] = p.Y ? p.sw[nb + q] : 0.0f;
        bv[q] = p.bias ? p.bias[nb + q] : 0.0f;
    }
    const float my_sa = (t < BM && p.Y) ? p.sa[m0 + t] : 0.0f;

    const int nk_all = (p.K + 127) / 128;
    const int nk = nk_all / KG;  // this group's k-tiles (KG > 1: nk_all % KG == 0 and no half k-tile)
    const int8_t* tile_a = p.A + (size_t)m0 * p.lda + (size_t)kg * nk * 128;
    const int8_t* tile_w = p.W + (size_t)n0 * p.ldw + (size_t)kg * nk * 128;
    const int cl = (lane & 7) ^ (lane >> 3), rs = lane >> 3;
    const bool half = (p.K & 127) != 0;
    auto issue = [&](int kt) {  // this wave's loads of k-tile kt into stage kt % S
        int8_t* stage = lds + (kt % S) * STAGE;
#pragma unroll
        for (int i = 0; i < SLOTS; ++i) {
            const int slot = i * NW + wave;
            const bool a = i < SA;
            const int ld = a ? p.lda : p.ldw;
            int chunk = cl ^ (slot & 7);
            if (half && kt == nk - 1) chunk &= 3;  // past K: the lower 64 bytes again (never multiplied)
            const int8_t* base = (a ? tile_a + (size_t)(slot * 8) * ld : tile_w + (size_t)(slot * 8 - BM) * ld) + kt * 128;
            dma16(base, (unsigned)(rs * ld + chunk * 16), stage + slot * 1024);
        }
    };

    const int rl = lane & 31, g = lane >> 5;
    int aoff[4], boff[4];
    {
        const int ra_ = wm * TM + rl, rb_ = BM + wn * TN + rl;
        const int sa_ = swz8(ra_), sb_ = swz8(rb_);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            aoff[s] = ra_ * 128 + (((2 * s + g) ^ sa_) << 4);
            boff[s] = rb_ * 128 + (((2 * s + g) ^ sb_) << 4);
        }
    }
    // NACC independent accumulator sets (k-step s adds into set s % NACC), so that a wave with few output blocks
    // still has independent MFMAs to issue back to back; the sets are summed (exact int32 adds) before the epilogue
    constexpr int NACC = FM * FN >= 4 ? 1 : 4 / (FM * FN);
    v16i accs[NACC][FM][FN];
#pragma unroll
    for (int c = 0; c < NACC; ++c)
#pragma unroll
        for (int fi = 0; fi < FM; ++fi)
#pragma unroll
            for (int fj = 0; fj < FN; ++fj)
#pragma unroll
                for (int e = 0; e < 16; ++e) accs[c][fi][fj][e] = 0;

    // the fragments of NT k-tiles from kt on (4 k-steps each, the last one 2 k-steps when it is a half k-tile), then
    // their multiplies
    auto multiply = [&](int kt, auto NTC, bool last_half) {
        constexpr int NT = decltype(NTC)::value;
        v4i fa[NT][4][FM], fb[NT][4][FN];
#pragma unroll
        for (int u = 0; u < NT; ++u) {
            const int8_t* stage = lds + ((kt + u) % S) * STAGE;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
#pragma unroll
                for (int fi = 0; fi < FM; ++fi) fa[u][s][fi] = *(const v4i*)(stage + aoff[s ^ (2 * (fi & 1))] + fi * 4096);
#pragma unroll
                for (int fj = 0; fj < FN; ++fj) fb[u][s][fj] = *(const v4i*)(stage + boff[s ^ (2 * (fj & 1))] + fj * 4096);
            }
        }
#pragma unroll
        for (int u = 0; u < NT; ++u)
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                if (last_half && u == NT - 1 && s >= 2) break;
#pragma unroll
                for (int fi = 0; fi < FM; ++fi)
#pragma unroll
                    for (int fj = 0; fj < FN; ++fj)
                        accs[s % NACC][fi][fj] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[u][s][fi], fb[u][s][fj],
                                                                                      accs[s % NACC][fi][fj], 0, 0, 0);
            }
    };
    using one = std::integral_constant<int, 1>;
    using kpi = std::integral_constant<int, KPI>;

    // k-tile kt lives in stage kt % S; `issued` is the next k-tile to load
    int issued = 0;
    for (; issued < min(S - KPI, nk); ++issued) issue(issued);
    int kt = 0;
    // steady state: k-tiles kt .. kt+KPI-1 are waited for while kt+KPI .. kt+S-KPI-1 stay in flight; after the
    // barrier the stages of kt-KPI .. kt-1 are free and take k-tiles kt+S-KPI .. kt+S-1
    for (; kt + S - 1 < nk; kt += KPI) {
        KNX_WAIT_VM_LDS(SLOTS * (S - 2 * KPI));
        knx_barrier_nofence();
#pragma unroll
        for (int u = 0; u < KPI; ++u) issue(kt + S - KPI + u);
        issued = kt + S;
        multiply(kt, kpi{}, false);
    }
    // tail, one k-tile at a time: issued-1-kt younger k-tiles in flight (a smaller count only waits for more)
    for (; kt < nk; ++kt) {
        const int young = min(issued - 1 - kt, 6);
        if (young >= 6) KNX_WAIT_VM_LDS(SLOTS * 6);
        else if (young == 5) KNX_WAIT_VM_LDS(SLOTS * 5);
        else if (young == 4) KNX_WAIT_VM_LDS(SLOTS * 4);
        else if (young == 3) KNX_WAIT_VM_LDS(SLOTS * 3);
        else if (young == 2) KNX_WAIT_VM_LDS(SLOTS * 2);
        else if (young == 1) KNX_WAIT_VM_LDS(SLOTS * 1);
        else KNX_WAIT_VM_LDS(0);
        knx_barrier_nofence();
        while (issued < nk && issued <= kt + S - 1) issue(issued++);  // stages of k-tiles < kt are free
        multiply(kt, one{}, half && kt == nk - 1);
    }
#pragma unroll
    for (int c = 1; c < NACC; ++c)
#pragma unroll
        for (int fi = 0; fi < FM; ++fi)
#pragma unroll
            for (int fj = 0; fj < FN; ++fj) accs[0][fi][fj] += accs[c][fi][fj];
    if (KG > 1) {
        // partial tiles of groups 1.. through their own rings (every group is past its last fragment read), lane by
        // lane: element e of block f of wave w at ((w·FM·FN + f)·16 + e)·64 + lane
        int* part = reinterpret_cast<int*>(lds);
        KNX_WAIT_LDS();
        knx_barrier_nofence();
        if (kg > 0) {
#pragma unroll
            for (int fi = 0; fi < FM; ++fi)
#pragma unroll
                for (int fj = 0; fj < FN; ++fj)
#pragma unroll
                    for (int e = 0; e < 16; ++e) part[((wave * FM * FN + fi * FN + fj) * 16 + e) * 64 + lane] = accs[0][fi][fj][e];
        }
        KNX_WAIT_LDS();
        knx_barrier_nofence();
        if (kg > 0) {
            knx_barrier_nofence();  // the one barrier of group 0's epilogue
            return;
        }
#pragma unroll
        for (int g2 = 1; g2 < KG; ++g2) {
            const int* src = reinterpret_cast<const int*>(lds_all + g2 * S * STAGE);
#pragma unroll
            for (int fi = 0; fi < FM; ++fi)
#pragma unroll
                for (int fj = 0; fj < FN; ++fj)
#pragma unroll
                    for (int e = 0; e < 16; ++e) accs[0][fi][fj][e] += src[((wave * FM * FN + fi * FN + fj) * 16 + e) * 64 + lane];
        }
    }
    tile_epilogue<BM, BN, WM, WN>(p, accs[0], lds, row_scale, my_sa, m0, nb, swv, bv, mlo, nlo);
}

template <int BM, int BN, int WM, int WN, int S, int KPI, int KG = 1>
int launch_ring(I8Args p, hipStream_t s, const char* name)
{
    p.tiles_m = (p.M + BM - 1) / BM;
    p.tiles_n = (p.N + BN - 1) / BN;
    const unsigned grid = (unsigned)p.tiles_m * (unsigned)p.tiles_n;
    hipLaunchKernelGGL((i8gemm_ring<BM, BN, WM, WN, S, KPI, KG>), dim3(grid), dim3(KG * WM * WN * 64), 0, s, p);
    return knx::check_launch(name);
}

// the in-workgroup K split needs whole 128-byte k-tiles, as many per group, and a full ring's worth per group
template <int KG, int S>
bool ring_split_fits(const I8Args& p)
{
    const int nk = p.K / 128;
    return p.K % 128 == 0 && nk % KG == 0 && nk / KG >= S;
}

// ---------------------------------------------------------------- skinny kernel (M ≤ 64)
// Bandwidth-bound shapes (a few activation rows against a whole weight matrix): every workgroup owns 16 output
// channels (16 W rows) and its KS waves split K; each wave streams its W slice HBM → VGPR with all loads issued up
// front, multiplies on v_mfma_i32_16x16x64_i8 (16 rows of A per block, up to 4 blocks), and the KS partial int32
// tiles are summed exactly through LDS before the same epilogue as the tile kernels.
// 16×16×64 operand layout: lane l holds row (l & 15), k-chunk (l >> 4) of 16 bytes; A and W use the same chunk,
// so any k order inside the instruction is consistent.  Result: lane l holds column (l & 15), rows 4·(l >> 4) + e.
typedef int v4i_t __attribute__((ext_vector_type(4)));

template <int MB, int KS, int KT>  // MB row blocks of 16, KS waves, KT 64-byte k-steps per wave per pass
__global__ void __launch_bounds__(KS * 64) i8gemm_skinny(I8Args p)
{
    __shared__ int part[KS][MB][16][17];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n0 = blockIdx.x * 16;
    const int r = lane & 15, c = lane >> 4;
    const int gn = min(n0 + r, p.N - 1);
    const int8_t* wrow = p.W + (size_t)gn * p.ldw + c * 16;
    const int8_t* arow[MB];
    bool aok[MB];
#pragma unroll
    for (int b = 0; b < MB; ++b) {
        const int gm = b * 16 + r;
        aok[b] = gm < p.M;
        arow[b] = p.A + (size_t)(aok[b] ? gm : 0) * p.lda + c * 16;
    }
    v4i acc[MB];
#pragma unroll
    for (int b = 0; b < MB; ++b) acc[b] = v4i{0, 0, 0, 0};
    const int nk = p.K / 64;
    // wave w takes k-steps w, w+KS, w+2·KS, … ; KT of them per pass, loads issued before the multiplies.  Workgroup
    // b starts its K order rot(b) k-steps in (a multiple of KS, so every wave keeps its share; int32 sums are exact
    // in any order): at a power-of-two row stride the workgroups would otherwise all read the same offsets within
    // their rows at the same time, and so the same memory channels.
    const int rot = nk >= 2 * KS ? (int)(blockIdx.x % (unsigned)(nk / KS)) * KS : 0;
    for (int k0 = wave; k0 < nk; k0 += KS * KT) {
        v4i wf[KT], af[KT][MB];
#pragma unroll
        for (int j = 0; j < KT; ++j) {
            const int kk = k0 + j * KS;
            const int kr = kk + rot < nk ? kk + rot : kk + rot - nk;
            wf[j] = kk < nk ? *(const v4i*)(wrow + (size_t)kr * 64) : v4i{0, 0, 0, 0};
#pragma unroll
            for (int b = 0; b < MB; ++b) af[j][b] = (kk < nk && aok[b]) ? *(const v4i*)(arow[b] + (size_t)kr * 64) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int j = 0; j < KT; ++j)
#pragma unroll
            for (int b = 0; b < MB; ++b) acc[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[j][b], wf[j], acc[b], 0, 0, 0);
    }
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int e = 0; e < 4; ++e) part[wave][b][4 * c + e][r] = acc[b][e];
    __syncthreads();
    // KS·64 threads finish MB·16 rows × 16 columns
    for (int i = threadIdx.x; i < MB * 256; i += KS * 64) {
        const int b = i >> 8, row = (i >> 4) & 15, col = i & 15;
        const int m = b * 16 + row, n = n0 + col;
        if (m >= p.M || n >= p.N) continue;
        int s = 0;
#pragma unroll
        for (int w = 0; w < KS; ++w) s += part[w][b][row][col];
        i8_epilogue(p, m, n, s);
    }
}

// ---------------------------------------------------------------- fused quantize + skinny GEMM (≤ 64 rows)
// kernix_qmatmul at small row counts and small weights (the reference's int8 arithmetic at ≤ 2 rows, its batch-1
// latency path, and the int8 mode at small batches) as one kernel instead of the row quantizer followed by the skinny
// GEMM.  Every
// workgroup (16 output channels, MB blocks of 16 rows) first finds the absolute maximum of each fp32 input row (all
// threads take part at every row count; partial maxima meet by exchanges and in LDS: a maximum is exact in any
// order), then runs the skinny K loop with
// each lane quantizing its 16 inputs of a k-step on the fly with the operations of knx_hip_quantize_rows (s = m/127
// or 1 for an all-zero row, inv = 1/s, rint, clamp ±127; a row holding NaN or ±inf gets s = NaN and q = 0, so its
// whole output row is NaN).  The int32 sums and outputs are therefore bit-exact against the two-kernel path.  The
// fp32 rows are read twice per workgroup from L2, which is why the fused form serves small row counts and weights
// only (see knx_hip_qlinear).
template <int KS, int KT, int MB>
__global__ void __launch_bounds__(KS * 64) i8gemm_skinny_q(I8Args p, const float* __restrict__ X, int ldx, int kx)
{
    constexpr int MR = 16 * MB;
    static_assert(MR <= 64, "at most 64 rows (one exchange group of eight or more threads per row)");
    __shared__ int part[KS][MB][16][17];
    __shared__ float pmax[1][64];  // one partial maximum per exchange group (at most 64 groups)
    __shared__ int pbad[1][64];
    __shared__ float row_s[MR], row_inv[MR];
    __shared__ int row_bad[MR];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int M = p.M;
    const bool xvec = (ldx & 3) == 0 && ((uintptr_t)X & 15) == 0;
    // row maxima: the KS·64 threads split into groups of G = KS·64 / Mp (Mp = M rounded up to a power of two), group
    // r scanning row r with G threads side by side (coalesced, four loads in flight per thread); the threads of a
    // group reduce by exchanges within at most one wave, then the ≤ KS waves of a row through LDS
    const int t = threadIdx.x;
    int mp = 1;
    while (mp < M) mp <<= 1;
    const int G = KS * 64 / mp, GW = G < 64 ? G : 64;  // threads per row, per exchange group
    {
        const int row = t / G, sub = t % G;
        float mx = 0.0f;
        int bad = 0;
        auto take = [&](float v) {
            const float a = fabsf(v);
            if (!(a <= 3.402823466e38f)) bad = 1;  // NaN or ±inf
            else mx = a > mx ? a : mx;
        };
        if (row < M) {
            const float* xr = X + (size_t)row * ldx;
            int j = 0;
            if (xvec) {
                const int n4 = kx / 4;
                for (int i = sub; i < n4; i += 4 * G) {
                    float4 f[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        f[u] = i + u * G < n4 ? *reinterpret_cast<const float4*>(xr + 4 * (i + u * G)) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        take(f[u].x); take(f[u].y); take(f[u].z); take(f[u].w);
                    }
                }
                j = 4 * n4;
            }
            for (j += sub; j < kx; j += G) take(xr[j]);
        }
        for (int off = GW / 2; off > 0; off >>= 1) {
            const float o = __shfl_xor(mx, off, 64);
            mx = o > mx ? o : mx;
            bad |= __shfl_xor(bad, off, 64);
        }
        if (t % GW == 0) {
            pmax[0][t / GW] = mx;
            pbad[0][t / GW] = bad;
        }
    }
    __syncthreads();
    if (t < M) {
        const int m = t, gpr = G / GW;  // exchange groups per row
        float mx = 0.0f;
        int bad = 0;
        for (int w = 0; w < gpr; ++w) {
            mx = pmax[0][m * gpr + w] > mx ? pmax[0][m * gpr + w] : mx;
            bad |= pbad[0][m * gpr + w];
        }
        const float sc = mx > 0.0f ? __fdiv_rn(mx, 127.0f) : 1.0f;
        row_s[m] = bad ? __int_as_float(0x7fc00000) : sc;
        row_inv[m] = __fdiv_rn(1.0f, sc);
        row_bad[m] = bad;
    }
    __syncthreads();

    // K loop of the skinny kernel over MB blocks of 16 rows (rows ≥ M are zero); lane (r, c) holds row 16b + r, bytes
    // [64·kk + 16c, +16) of k-step kk
    const int r = lane & 15, c = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int gn = min(n0 + r, p.N - 1);
    const int8_t* wrow = p.W + (size_t)gn * p.ldw + c * 16;
    bool rok[MB];
    const float* xrow[MB];
    float inv[MB];
#pragma unroll
    for (int b = 0; b < MB; ++b) {
        const int m = 16 * b + r;
        rok[b] = m < M && !row_bad[m < M ? m : 0];
        xrow[b] = X + (size_t)(m < M ? m : 0) * ldx;
        inv[b] = m < M ? row_inv[m] : 0.0f;
    }
    // the 16 inputs of k-step kk of this lane in row block b, quantized and packed four per int
    auto quant16 = [&](int b, int kk) -> v4i {
        const int j0 = kk * 64 + c * 16;
        float v[16];
        if (xvec && j0 + 16 <= kx) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float4 f = *reinterpret_cast<const float4*>(xrow[b] + j0 + 4 * u);
                v[4 * u] = f.x; v[4 * u + 1] = f.y; v[4 * u + 2] = f.z; v[4 * u + 3] = f.w;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) v[e] = j0 + e < kx ? xrow[b][j0 + e] : 0.0f;
        }
        v4i out;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            int packed = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float q = rintf(v[4 * u + e] * inv[b]);
                const int qi = (int)(q > 127.0f ? 127.0f : q < -127.0f ? -127.0f : q);
                packed |= (qi & 0xff) << (8 * e);
            }
            out[u] = packed;
        }
        return out;
    };
    v4i acc[MB];
#pragma unroll
    for (int b = 0; b < MB; ++b) acc[b] = v4i{0, 0, 0, 0};
    const v4i z = v4i{0, 0, 0, 0};
    const int nk = p.K / 64;
    const int rot = nk >= 2 * KS ? (int)(blockIdx.x % (unsigned)(nk / KS)) * KS : 0;  // as in i8gemm_skinny
    for (int k0 = wave; k0 < nk; k0 += KS * KT) {
        v4i wf[KT], af[KT][MB];
#pragma unroll
        for (int j = 0; j < KT; ++j) {
            const int kk = k0 + j * KS;
            const int kr = kk + rot < nk ? kk + rot : kk + rot - nk;
            wf[j] = kk < nk ? *(const v4i*)(wrow + (size_t)kr * 64) : z;
#pragma unroll
            for (int b = 0; b < MB; ++b) af[j][b] = (kk < nk && rok[b]) ? quant16(b, kr) : z;
        }
#pragma unroll
        for (int j = 0; j < KT; ++j)
#pragma unroll
            for (int b = 0; b < MB; ++b) acc[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[j][b], wf[j], acc[b], 0, 0, 0);
    }
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int e = 0; e < 4; ++e) part[wave][b][4 * c + e][r] = acc[b][e];
    __syncthreads();
    // rows < M × 16 columns: the exact int32 sum of the waves' partial tiles, then the epilogue with the row scale
    for (int i = threadIdx.x; i < MB * 256; i += KS * 64) {
        const int b = i >> 8, row = 16 * b + ((i >> 4) & 15), col = i & 15, n = n0 + col;
        if (row >= M || n >= p.N) continue;
        int a = 0;
#pragma unroll
        for (int w = 0; w < KS; ++w) a += part[w][b][row & 15][col];
        float v = (float)a * row_s[row];  // ((float)acc · sx) · scale + bias, each step rounded
        v = v * p.sw[n];
        if (p.bias) v = v + p.bias[n];
        float* y = p.Y + (size_t)row * p.ldy + n;
        if (p.accumulate) v = *y + v;
        v = knx_act(v, p.act, p.alpha);
        if (p.R) v = v + p.R[(size_t)row * p.ldr + n];
        *y = v;
    }
}

template <int MB>
int launch_skinny(I8Args p, hipStream_t s, const char* name)
{
    const unsigned grid = (unsigned)((p.N + 15) / 16);
    hipLaunchKernelGGL((i8gemm_skinny<MB, 8, 4>), dim3(grid), dim3(8 * 64), 0, s, p);
    return knx::check_launch(name);
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

// Register-resident variant (k % 4 == 0, k ≤ 256·NV, 16-byte aligned fp32 rows, 4-byte aligned int8 rows): x is read
// once with 16-byte loads and four int8 values are written per 32-bit store; same arithmetic as quantize_rows_kernel.
__device__ __forceinline__ float q4e(const float4& v, int e) { return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w; }

template <int NV>
__global__ void __launch_bounds__(256) quantize_rows_vec(const float* __restrict__ x, int ldx, int rows, int k, int kp,
                                                          int8_t* __restrict__ xq, int ldq, float* __restrict__ sx)
{
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float4* xr = reinterpret_cast<const float4*>(x + (size_t)row * ldx);
    const int nq = k >> 2, nqp = kp >> 2;
    float4 v[NV];
    // the row maximum of |x| as integer bits: NaN above ±inf above every finite value, so one maximum also finds a row
    // that cannot be quantized; DPP and register swaps across the wave
    unsigned mb = 0u;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int q = i * 64 + lane;
        v[i] = q < nq ? xr[q] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int e = 0; e < 4; ++e) mb = max(mb, __float_as_uint(q4e(v[i], e)) & 0x7fffffffu);
    }
    mb = knx_lane_group_max(mb, 64);
    int* qr = reinterpret_cast<int*>(xq + (size_t)row * ldq);
    if (mb >= 0x7f800000u) {  // NaN or ±inf
        for (int q = lane; q < nqp; q += 64) qr[q] = 0;
        if (lane == 0) sx[row] = __int_as_float(0x7fc00000);
        return;
    }
    const float m = __uint_as_float(mb);
    const float s = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
    const float inv = __fdiv_rn(1.0f, s);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int q = i * 64 + lane;
        if (q >= nq) continue;
        // q = clamp(rint(x·inv), ±127) by v_med3; q + 128 converts exactly to a byte, and ^ 0x80 makes it q's byte
        unsigned w = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            w = __builtin_amdgcn_cvt_pk_u8_f32(
                __builtin_amdgcn_fmed3f(rintf(q4e(v[i], e) * inv), -127.0f, 127.0f) + 128.0f, e, w);
        qr[q] = (int)(w ^ 0x80808080u);
    }
    for (int q = nq + lane; q < nqp; q += 64) qr[q] = 0;
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

// ---- dequantized copy, weight-transposed: dst[n][k] = (float)q[n][k] · scale[n] (4 elements per lane) ----
__global__ void __launch_bounds__(256) dequant_t_kernel(const int8_t* __restrict__ q, int ldq, const float* __restrict__ scale,
                                                         int K, int N, float* __restrict__ dst)
{
    const size_t n4 = (size_t)N * (K / 4);
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x) {
        const int n = (int)(i / (K / 4)), k = (int)(i % (K / 4)) * 4;
        const int w = *reinterpret_cast<const int*>(q + (size_t)n * ldq + k);
        const float s = scale[n];
        *reinterpret_cast<float4*>(dst + (size_t)n * K + k) =
            make_float4((float)(int8_t)(w & 0xff) * s, (float)(int8_t)((w >> 8) & 0xff) * s,
                        (float)(int8_t)((w >> 16) & 0xff) * s, (float)(int8_t)((w >> 24) & 0xff) * s);
    }
}

__global__ void __launch_bounds__(256) dequant_t_scalar(const int8_t* __restrict__ q, int ldq, const float* __restrict__ scale,
                                                         int K, int N, float* __restrict__ dst)
{
    const size_t n = (size_t)N * K;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(i / K), k = (int)(i % K);
        dst[i] = (float)q[(size_t)r * ldq + k] * scale[r];
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
    hipStream_t st = knx::as_stream(stream);
    const dim3 grid((rows + 3) / 4), block(256);
    if (k % 4 == 0 && ldx % 4 == 0 && ((uintptr_t)x & 15) == 0 && ldq % 4 == 0 && ((uintptr_t)xq & 3) == 0 && k <= 4096) {
        if (k <= 256) hipLaunchKernelGGL(quantize_rows_vec<1>, grid, block, 0, st, x, ldx, rows, k, kp, xq, ldq, sx);
        else if (k <= 512) hipLaunchKernelGGL(quantize_rows_vec<2>, grid, block, 0, st, x, ldx, rows, k, kp, xq, ldq, sx);
        else if (k <= 1024) hipLaunchKernelGGL(quantize_rows_vec<4>, grid, block, 0, st, x, ldx, rows, k, kp, xq, ldq, sx);
        else if (k <= 2048) hipLaunchKernelGGL(quantize_rows_vec<8>, grid, block, 0, st, x, ldx, rows, k, kp, xq, ldq, sx);
        else hipLaunchKernelGGL(quantize_rows_vec<16>, grid, block, 0, st, x, ldx, rows, k, kp, xq, ldq, sx);
        return knx::check_launch(name);
    }
    hipLaunchKernelGGL(quantize_rows_kernel, grid, block, 0, st, x, ldx, rows, k, kp, xq, ldq, sx);
    return knx::check_launch(name);
}

// the argument checks shared by the int8 GEMM entry points
static int i8gemm_check(int M, int N, int K, const int8_t* A, int lda, const float* sa, const int8_t* W, int ldw,
                        const float* sw, int act, float* Y, int ldy, int32_t* acc_out, int ldacc, const char* name)
{  // KNX_OK, 1 when there is nothing to compute (M or N is 0), or the error of the first failed check
    KNX_REQUIRE(M >= 0 && N >= 0 && K >= 0 && K % 64 == 0 && K <= 131072, name);
    KNX_REQUIRE(lda >= K && ldw >= K && lda % 16 == 0 && ldw % 16 == 0, name);
    KNX_REQUIRE(act >= -1 && act <= 15, name);
    if (M == 0 || N == 0) return 1;
    KNX_REQUIRE(Y != nullptr || acc_out != nullptr, name);
    KNX_REQUIRE(Y == nullptr || (ldy >= N && sa != nullptr && sw != nullptr), name);
    KNX_REQUIRE(acc_out == nullptr || ldacc >= N, name);
    KNX_REQUIRE(K == 0 || (A != nullptr && W != nullptr), name);
    KNX_REQUIRE(((uintptr_t)A & 15) == 0 && ((uintptr_t)W & 15) == 0, name);
    return KNX_OK;
}

static int i8gemm_run(I8Args p, hipStream_t s, const char* name)
{
    const int M = p.M, N = p.N, K = p.K;
    if (K == 0) {
        // empty inner dimension: the accumulators are all zero; run the smallest tile (loop body never executes)
        return launch_tile<64, 64, 1, 1>(p, s, name);
    }
    // KNX_I8_KERNEL forces one variant (tuning and tests) where its shape limits allow; otherwise the shape picks it
    const char* force = getenv("KNX_I8_KERNEL");
    if (force != nullptr && *force) {
        const std::string f(force);
        if (f == "tile64") return launch_tile<64, 64, 1, 1>(p, s, name);
        if (f == "pipe64") return launch_pipe<64, 64, 2, 2, 4>(p, s, name);
        if (f == "k128w8t" && k128_fits<256, 256>(p)) return launch_k128<256, 256, 4, 2, 2>(p, s, name);
        if (f == "k128w8ta3e" && k128_fits<256, 256>(p)) return launch_k128<256, 256, 4, 2, 3, true>(p, s, name);
        if (f == "k128m" && k128_fits<128, 128>(p)) return launch_k128<128, 128, 2, 2, 2>(p, s, name);
        if (f == "k128ma3" && k128_fits<128, 128>(p)) return launch_k128<128, 128, 2, 2, 3>(p, s, name);
        if (f == "k128m8a3e" && k128_fits<128, 128>(p)) return launch_k128<128, 128, 4, 2, 3, true>(p, s, name);
        if (f == "ring64s4" && k128_fits<64, 64>(p)) return launch_ring<64, 64, 2, 2, 4, 1>(p, s, name);
        if (f == "ring64g2" && k128_fits<64, 64>(p) && ring_split_fits<2, 4>(p)) return launch_ring<64, 64, 2, 2, 4, 1, 2>(p, s, name);
        if (f == "k128ms4" && ksplit_fits<128, 128, 4>(p)) return launch_k128<128, 128, 2, 2, 2, false, 4>(p, s, name);
        if (f == "k128ma3s4" && ksplit_fits<128, 128, 4>(p)) return launch_k128<128, 128, 2, 2, 3, false, 4>(p, s, name);
        if (f == "k128m8s4" && ksplit_fits<128, 128, 4>(p)) return launch_k128<128, 128, 4, 2, 2, false, 4>(p, s, name);
        if (f == "k128ms2" && ksplit_fits<128, 128, 2>(p)) return launch_k128<128, 128, 2, 2, 2, false, 2>(p, s, name);
        if (f == "k128ms8" && ksplit_fits<128, 128, 8>(p)) return launch_k128<128, 128, 2, 2, 2, false, 8>(p, s, name);
#ifdef KNX_TUNING
        // variants no shape selects (measured slower where they fit), built only for tuning (-DKNX_TUNING)
        if (f == "tile256") return launch_tile<256, 256, 2, 2>(p, s, name);
        if (f == "pipe256") return launch_pipe<256, 256, 2, 2, 4>(p, s, name);
        if (f == "pipe256w8") return launch_pipe<256, 256, 2, 4, 4>(p, s, name);
        if (f == "pipe256s3") return launch_pipe<256, 256, 2, 2, 3>(p, s, name);
        if (f == "pipe128") return launch_pipe<128, 128, 2, 2, 4>(p, s, name);
        if (f == "k128" && k128_fits<256, 256>(p)) return launch_k128<256, 256, 2, 2, 2>(p, s, name);
        if (f == "k128w8" && k128_fits<256, 256>(p)) return launch_k128<256, 256, 2, 4, 2>(p, s, name);
        if (f == "k128w8ta3" && k128_fits<256, 256>(p)) return launch_k128<256, 256, 4, 2, 3>(p, s, name);
        if (f == "k128w16" && k128_fits<256, 256>(p)) return launch_k128<256, 256, 4, 4, 2>(p, s, name);
        if (f == "pp" && k128_fits<256, 256>(p)) return launch_pp<256, 256>(p, s, name);
        if (f == "k128r" && k128_fits<256, 128>(p)) return launch_k128<256, 128, 4, 2, 3, true>(p, s, name);
        if (f == "k128c" && k128_fits<128, 256>(p)) return launch_k128<128, 256, 2, 4, 3, true>(p, s, name);
        if (f == "ring64s8k2" && k128_fits<64, 64>(p)) return launch_ring<64, 64, 2, 2, 8, 2>(p, s, name);
        if (f == "ring64s8" && k128_fits<64, 64>(p)) return launch_ring<64, 64, 2, 2, 8, 1>(p, s, name);
        if (f == "k128m8" && k128_fits<128, 128>(p)) return launch_k128<128, 128, 4, 2, 2>(p, s, name);
        if (f == "k128m8a3" && k128_fits<128, 128>(p)) return launch_k128<128, 128, 4, 2, 3>(p, s, name);
#endif
        if (f == "skinny" && M <= 64) return M <= 16 ? launch_skinny<1>(p, s, name) : M <= 32 ? launch_skinny<2>(p, s, name) : launch_skinny<4>(p, s, name);
    }
    if (M <= 16) return launch_skinny<1>(p, s, name);
    if (M <= 32) return launch_skinny<2>(p, s, name);
    if (M <= 64) return launch_skinny<4>(p, s, name);
    // the largest tile that still gives every CU a workgroup
    const long tiles256 = (long)((M + 255) / 256) * ((N + 255) / 256);
    // three A stages with the A loads spread over the k-tile pay off once the K loop is long (4096³: 67.9 against
    // 69.8-70.5 µs); for short K the deeper prologue costs more than it saves (8192×2048×512: 23.9 against 23.1 µs)
    if (tiles256 >= knx::num_cus() && k128_fits<256, 256>(p)) {
        if (K >= 2048) return launch_k128<256, 256, 4, 2, 3, true>(p, s, name);
        return launch_k128<256, 256, 4, 2, 2>(p, s, name);
    }
    const long tiles128 = (long)((M + 127) / 128) * ((N + 127) / 128);
    // 128×128 on 8 waves of 32×64, three A stages, the A loads spread over the k-tile: one workgroup per CU still has
    // two waves per SIMD (one box, µs, against 4 waves of 64×64 with two / three A stages: 8192×512×2048 + residual
    // 17.7-18.0 against 20.9-21.0 / 20.3; 8192×1536×512 17.6-18.2 against 19.6-20.3 / 19.9-20.6; two stages on the
    // 8 waves: 18.3-19.7)
    if (tiles128 >= knx::num_cus() && k128_fits<128, 128>(p)) return launch_k128<128, 128, 4, 2, 3, true>(p, s, name);
    // fewer tiles than CUs even at 128×128 (e.g. M = 256, N = 4096): one 64×64 tile per workgroup on the deep LDS
    // ring (M = 256: 13.2 µs against 16.8 for the 64-byte k-tile pipeline), K split over two rings in the workgroup
    // when the 64×64 tiles leave CUs without a second workgroup
    const long tiles64 = (long)((M + 63) / 64) * ((N + 63) / 64);
    if (tiles64 <= knx::num_cus() && k128_fits<64, 64>(p) && ring_split_fits<2, 4>(p))
        return launch_ring<64, 64, 2, 2, 4, 1, 2>(p, s, name);
    if (k128_fits<64, 64>(p)) return launch_ring<64, 64, 2, 2, 4, 1>(p, s, name);
    return launch_pipe<64, 64, 2, 2, 4>(p, s, name);
}

extern "C" int knx_hip_i8gemm(int M, int N, int K, const int8_t* A, int lda, const float* sa, const int8_t* W, int ldw,
                              const float* sw, const float* bias, int act, float alpha, int accumulate, float* Y, int ldy,
                              int32_t* acc_out, int ldacc, void* stream)
{
    const char* name = "knx_hip_i8gemm";
    KNX_ENTRY(name);
    const int rc = i8gemm_check(M, N, K, A, lda, sa, W, ldw, sw, act, Y, ldy, acc_out, ldacc, name);
    if (rc != KNX_OK) return rc == 1 ? KNX_OK : rc;
    I8Args p{M, N, K, A, lda, sa, W, ldw, sw, bias, act, alpha, accumulate, Y, ldy, acc_out, ldacc, 0, 0, nullptr, 0};
    return i8gemm_run(p, knx::as_stream(stream), name);
}

extern "C" int knx_hip_i8gemm_res(int M, int N, int K, const int8_t* A, int lda, const float* sa, const int8_t* W,
                                  int ldw, const float* sw, const float* bias, int act, float alpha, const float* R,
                                  int ldr, float* Y, int ldy, void* stream)
{
    const char* name = "knx_hip_i8gemm_res";
    KNX_ENTRY(name);
    const int rc = i8gemm_check(M, N, K, A, lda, sa, W, ldw, sw, act, Y, ldy, nullptr, 0, name);
    if (rc != KNX_OK) return rc == 1 ? KNX_OK : rc;
    KNX_REQUIRE(Y != nullptr && R != nullptr && ldr >= N, name);
    I8Args p{M, N, K, A, lda, sa, W, ldw, sw, bias, act, alpha, 0, Y, ldy, nullptr, 0, 0, 0, R, ldr};
    return i8gemm_run(p, knx::as_stream(stream), name);
}

extern "C" int knx_hip_qlinear(const float* x, int ldx, int rows, int k, int kp, int8_t* xq, float* sx, const int8_t* W,
                               int ldw, int n, const float* sw, const float* bias, int act, float alpha, int accumulate,
                               const float* R, int ldr, float* Y, int ldy, void* stream)
{
    const char* name = "knx_hip_qlinear";
    KNX_ENTRY(name);
    KNX_REQUIRE(rows >= 0 && n >= 0 && k >= 1 && kp >= k && kp % 64 == 0 && kp <= 131072 && ldx >= k, name);
    KNX_REQUIRE(ldw >= kp && ldw % 16 == 0 && act >= -1 && act <= 15, name);
    if (rows == 0 || n == 0) return KNX_OK;
    KNX_REQUIRE(x != nullptr && W != nullptr && sw != nullptr && Y != nullptr && ldy >= n, name);
    KNX_REQUIRE(((uintptr_t)W & 15) == 0 && (R == nullptr || ldr >= n) && !(R != nullptr && accumulate), name);
    hipStream_t s = knx::as_stream(stream);
    // KNX_QLINEAR=split: always the quantizer followed by the GEMM (tests)
    const char* mode = getenv("KNX_QLINEAR");
    const bool split = mode != nullptr && strcmp(mode, "split") == 0;
    // One kernel while every workgroup's own pass over the fp32 rows stays cheap: each of the n/16 workgroups reads
    // all rows twice, so the fused form loses once rows·k·n passes 2^23 (784×512 layer: 6.0 against 7.5 µs at 8 rows,
    // 9.6 against 7.4 at 32; 4096×4096: 11.6 against 10.5 µs already at 1 row)
    if (rows <= 16 && (long long)rows * k * n <= (1LL << 23) && !split) {
        I8Args p{rows, n, kp, nullptr, 0, nullptr, W, ldw, sw, bias, act, alpha, accumulate, Y, ldy, nullptr, 0, 0, 0, R, ldr};
        hipLaunchKernelGGL((i8gemm_skinny_q<8, 4, 1>), dim3((unsigned)((n + 15) / 16)), dim3(8 * 64), 0, s, p, x, ldx, k);
        return knx::check_launch(name);
    }
    KNX_REQUIRE(xq != nullptr && sx != nullptr, name);
    int rc = knx_hip_quantize_rows(x, ldx, rows, k, kp, xq, kp, sx, stream);
    if (rc != KNX_OK) return rc;
    if (R != nullptr) return knx_hip_i8gemm_res(rows, n, kp, xq, kp, sx, W, ldw, sw, bias, act, alpha, R, ldr, Y, ldy, stream);
    return knx_hip_i8gemm(rows, n, kp, xq, kp, sx, W, ldw, sw, bias, act, alpha, accumulate, Y, ldy, nullptr, 0, stream);
}

extern "C" int knx_hip_dequant_t(const int8_t* q, int ldq, const float* scale, int K, int N, float* dst, void* stream)
{
    const char* name = "knx_hip_dequant_t";
    KNX_ENTRY(name);
    KNX_REQUIRE(K >= 0 && N >= 0 && ldq >= K, name);
    if (K == 0 || N == 0) return KNX_OK;
    KNX_REQUIRE(q != nullptr && scale != nullptr && dst != nullptr, name);
    const size_t cap = (size_t)knx::num_cus() * 16;
    if (K % 4 == 0 && ldq % 4 == 0 && ((uintptr_t)q & 3) == 0 && ((uintptr_t)dst & 15) == 0) {
        const size_t n4 = (size_t)N * (K / 4), g = (n4 + 255) / 256;
        hipLaunchKernelGGL(dequant_t_kernel, dim3((unsigned)(g < cap ? g : cap)), dim3(256), 0, knx::as_stream(stream), q, ldq,
                           scale, K, N, dst);
    } else {
        const size_t n = (size_t)N * K, g = (n + 255) / 256;
        hipLaunchKernelGGL(dequant_t_scalar, dim3((unsigned)(g < cap ? g : cap)), dim3(256), 0, knx::as_stream(stream), q, ldq,
                           scale, K, N, dst);
    }
    return knx::check_launch(name);
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

// ---------------------------------------------------------------------------------------------------------------------
// knx_hip_qlinear_noalloc: knx_hip_qlinear with its int8 rows and row scales in a library-owned device array instead
// of caller scratch, for callers that cannot allocate (code under stream capture, fixed serving loops).  The array
// is file-scope device memory, one copy per GPU, held until the process ends.  Layout: the row scales (rows floats,
// rounded up to 256 bytes) at offset 0, then the int8 rows (rows × kp bytes).  Every byte a call reads is written
// by the same call first (the quantizer writes every scale and every column of [0, kp) of every row), so nothing
// needs clearing between calls.  Calls that overlap on one GPU (two streams, or two threads) share the array and
// race: the caller orders them.
constexpr size_t kNoAllocScratchBytes = KNX_QLINEAR_NOALLOC_BYTES;
static_assert(kNoAllocScratchBytes % 256 == 0, "scratch size");
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned char* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device, resolved once
}  // namespace

// The device address of `scratch` on the current device (resolved on this device's first call), or nullptr with
// the error recorded.
static unsigned char* noalloc_scratch(const char* name)
{
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        knx::fail(KNX_EHIP, "%s: no current device", name);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            knx::fail(KNX_EHIP, "%s: hipGetSymbolAddress(scratch): %s", name, hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_ptr[dev] = static_cast<unsigned char*>(p);
    }
    return g_scratch_ptr[dev];
}

// bytes of scratch a call with `rows` rows of kp int8 values uses (scales first, then the rows)
static size_t noalloc_bytes(int rows, int kp)
{
    return ((size_t)rows * sizeof(float) + 255) / 256 * 256 + (size_t)rows * (size_t)kp;
}

extern "C" int knx_hip_qlinear_noalloc(const float* x, int ldx, int rows, int k, int kp, const int8_t* W, int ldw, int n,
                                       const float* sw, const float* bias, int act, float alpha, int accumulate,
                                       const float* R, int ldr, float* Y, int ldy, void* stream)
{
    const char* name = "knx_hip_qlinear_noalloc";
    KNX_ENTRY(name);
    KNX_REQUIRE(rows >= 0 && k >= 1 && kp >= k && kp % 64 == 0 && kp <= 131072, name);
    if (noalloc_bytes(rows, kp) > kNoAllocScratchBytes)
        return knx::fail(KNX_EINVAL, "%s: %d rows of %d int8 values need %zu bytes of scratch, the limit is %zu", name,
                         rows, kp, noalloc_bytes(rows, kp), kNoAllocScratchBytes);
    int8_t* xq = nullptr;
    float* sx = nullptr;
    if (rows > 0) {
        unsigned char* base = noalloc_scratch(name);
        if (base == nullptr) return KNX_EHIP;
        sx = reinterpret_cast<float*>(base);
        xq = reinterpret_cast<int8_t*>(base + ((size_t)rows * sizeof(float) + 255) / 256 * 256);
    }
    // the same kernels and arguments as knx_hip_qlinear (its one-kernel form writes no scratch), without the K split
    // (its scratch is allocated on first use)
    g_no_alloc = true;
    const int rc = knx_hip_qlinear(x, ldx, rows, k, kp, xq, sx, W, ldw, n, sw, bias, act, alpha, accumulate, R, ldr,
                                   Y, ldy, stream);
    g_no_alloc = false;
    return rc;
}
