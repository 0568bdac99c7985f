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
#include <stdlib.h>

#include <string>

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

// ---------------------------------------------------------------- pipelined tile kernel
// Same tile/fragment/epilogue structure as i8gemm_tile, but operands move HBM → LDS directly with
// global_load_lds_dwordx4 (no VGPR staging, no ds_write), through a STAGES-deep LDS ring so that STAGES−1 k-tiles are
// in flight while one is multiplied.  Each load instruction fills 1 KB of LDS = 16 rows × 64 bytes; lane l fetches
// the global 16-byte chunk (l & 3) ^ swz(row), which realizes the swizzled layout with fully coalesced loads.
// Rows past M (or N) are clamped to the last row: they only feed output rows/columns that are never stored.
typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __attribute__((address_space(1))) const void* gbl_ptr_t;

// s_waitcnt vmcnt(n) lgkmcnt(0) (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] = 7 | lgkmcnt[11:8] | vmcnt[5:4] << 14):
// at most n vector-memory ops (LDS-DMA loads) of this wave outstanding and all of its LDS accesses retired.
#define KNX_WAIT_VM_LDS(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (0 << 8) | ((((n) >> 4) & 3) << 14))

// s_waitcnt lgkmcnt(0): all LDS accesses of this wave retired (vmcnt left unconstrained at 63).
#define KNX_WAIT_LDS() __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14))
#define KERNIX_ACT_RELU_ID 0

// Writes the 16 staged rows [mt0, mt0+16) of a tile: 4 consecutive columns per lane, one 16-byte store per row.
// ACT ≥ −1 is a compile-time activation for the common case (vector path, no accumulation); −2 is the general path.
template <int ACT>
__device__ __forceinline__ void store_rows(const I8Args& p, const int* stg, const float* row_scale, int mt0, int m0, int rq,
                                           int rpi, int srow, int cq, int nb, const float* swv, const float* bv,
                                           bool vec = true)
{
    for (int rr = rq; rr < 16; rr += rpi) {
        const int mt = mt0 + rr, m = m0 + mt;
        if (m >= p.M) continue;
        const v4i a = *reinterpret_cast<const v4i*>(&stg[rr * srow + cq]);
        if (ACT >= -1) {
            const float sx = row_scale[mt];
            float r[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float v = (float)a[q] * sx;  // ((float)acc · sx) · scale + bias, each step rounded
                v = v * swv[q];
                if (p.bias) v = v + bv[q];   // no bias: no addition (x + 0 would turn −0 into +0)
                r[q] = ACT == 0 ? (v >= 0.0f ? v : 0.0f) : v;
            }
            // streaming store: the output is written once and never re-read by this kernel
            typedef float v4f_t __attribute__((ext_vector_type(4)));
            __builtin_nontemporal_store(v4f_t{r[0], r[1], r[2], r[3]}, reinterpret_cast<v4f_t*>(p.Y + (size_t)m * p.ldy + nb));
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

// Workgroup barrier without a memory fence.  A fence (e.g. __syncthreads) would wait for every outstanding LDS-DMA
// load, which empties the prefetch ring; the caller instead waits precisely with KNX_WAIT_VM_LDS.  The empty asm
// statements keep the compiler from moving any memory access across the barrier.
__device__ __forceinline__ void knx_barrier_nofence()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Tile order: consecutive workgroups go to consecutive XCDs (8 on MI355X); when the tile grid splits evenly, each
// XCD gets one contiguous (tiles_m/2) × (tiles_n/4) block so the A and W rows it reads stay in its own L2.
__device__ __forceinline__ void tile_of(int t, int tiles_m, int tiles_n, int& tm, int& tn)
{
    if ((tiles_m & 1) == 0 && (tiles_n & 3) == 0 && tiles_m * tiles_n >= 64) {
        const int x = t & 7, j = t >> 3;
        const int bm = tiles_m >> 1, bn = tiles_n >> 2;
        tm = (x >> 2) * bm + j / bn;
        tn = (x & 3) * bn + j % bn;
    } else {
        tm = t / tiles_n;
        tn = t % tiles_n;
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
    tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
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

    // Epilogue: each wave stages 16 rows × TN of its accumulators at a time in its own LDS region (row stride TN+4
    // ints: the two half-waves land on different banks); every lane then reads 4 consecutive columns and writes them
    // with one 16-byte store.  The regions are private to the wave, so after one workgroup barrier (nobody reads the
    // ring any more) only the wave's own LDS order matters: no barrier — and so no wait for the stores — per round.
    constexpr int SROW = TN + 4;
    constexpr int LPR = TN / 4;
    constexpr int RPI = 64 / LPR;
    static_assert(NW * 16 * SROW * 4 <= STAGES * STAGE, "staging fits in the ring");
    static_assert(LPR == LPR_, "epilogue lane split");
    int* stg = reinterpret_cast<int*>(lds) + wave * 16 * SROW;
    const int cq = (lane % LPR) * 4, rq = lane / LPR;
    const int nb = nb_;
    const bool vec = nb + 3 < p.N && (p.ldy & 3) == 0 && ((uintptr_t)p.Y & 15) == 0 && (p.ldacc & 3) == 0 &&
                     ((uintptr_t)p.acc & 15) == 0;
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
                store_rows<0>(p, stg, row_scale, mt0, m0, rq, RPI, SROW, cq, nb, swv, bv);
            else if (fast && p.act == -1)
                store_rows<-1>(p, stg, row_scale, mt0, m0, rq, RPI, SROW, cq, nb, swv, bv);
            else
                store_rows<-2>(p, stg, row_scale, mt0, m0, rq, RPI, SROW, cq, nb, swv, bv, vec);
            asm volatile("" ::: "memory");
        }
    }
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
    // wave w takes k-steps w, w+KS, w+2·KS, … ; KT of them per pass, loads issued before the multiplies
    for (int k0 = wave; k0 < nk; k0 += KS * KT) {
        v4i wf[KT], af[KT][MB];
#pragma unroll
        for (int j = 0; j < KT; ++j) {
            const int kk = k0 + j * KS;
            wf[j] = kk < nk ? *(const v4i*)(wrow + (size_t)kk * 64) : v4i{0, 0, 0, 0};
#pragma unroll
            for (int b = 0; b < MB; ++b) af[j][b] = (kk < nk && aok[b]) ? *(const v4i*)(arow[b] + (size_t)kk * 64) : v4i{0, 0, 0, 0};
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
    // KNX_I8_KERNEL forces one variant (tuning and tests); otherwise the shape picks it
    const char* force = getenv("KNX_I8_KERNEL");
    if (force != nullptr && *force) {
        const std::string f(force);
        if (f == "tile256") return launch_tile<256, 256, 2, 2>(p, s, name);
        if (f == "tile64") return launch_tile<64, 64, 1, 1>(p, s, name);
        if (f == "pipe256") return launch_pipe<256, 256, 2, 2, 4>(p, s, name);
        if (f == "pipe256w8") return launch_pipe<256, 256, 2, 4, 4>(p, s, name);
        if (f == "pipe256s3") return launch_pipe<256, 256, 2, 2, 3>(p, s, name);
        if (f == "pipe128") return launch_pipe<128, 128, 2, 2, 4>(p, s, name);
        if (f == "pipe64") return launch_pipe<64, 64, 2, 2, 4>(p, s, name);
        if (f == "skinny" && M <= 64) return M <= 16 ? launch_skinny<1>(p, s, name) : M <= 32 ? launch_skinny<2>(p, s, name) : launch_skinny<4>(p, s, name);
    }
    if (M <= 16) return launch_skinny<1>(p, s, name);
    if (M <= 32) return launch_skinny<2>(p, s, name);
    if (M <= 64) return launch_skinny<4>(p, s, name);
    const long tiles256 = (long)((M + 255) / 256) * ((N + 255) / 256);
    if (tiles256 >= knx::num_cus()) return launch_pipe<256, 256, 2, 2, 4>(p, s, name);
    const long tiles128 = (long)((M + 127) / 128) * ((N + 127) / 128);
    if (tiles128 >= knx::num_cus()) return launch_pipe<128, 128, 2, 2, 4>(p, s, name);
    return launch_pipe<64, 64, 2, 2, 4>(p, s, name);
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
