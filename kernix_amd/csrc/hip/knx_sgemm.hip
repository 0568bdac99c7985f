// knx_sgemm.hip — fp32 GEMM with fused epilogue on v_mfma_f32_32x32x2_f32 (gfx950), one whole-GPU tiling.
//
// Replaces the reference's row split of one GEMM between MPS (GPU) and cblas_sgemm (AMX) with its separate bias/act
// pass (reference src/kernix_metal.m:161-265, include/kernix.h:951-977, include/kernix_model.h:528-550):
// every output tile is computed by one workgroup and leaves the chip already biased and activated.
//
// Two kernels:
//   sgemm_k32   the pipelined kernel for both operands K-contiguous (A M×K, Bt N×K: the device layout of Linear and
//               attention weights), K % 32 == 0, tiles that fill the chip (256×256 with 8 waves or 128×128 with 4):
//               128-byte k-tiles moved HBM → LDS by global_load_lds, as the int8 GEMM does;
//   sgemm_tile  the general kernel (any shape, B K×N or N×K): BM×BN per workgroup of WM×WN waves, K streamed in
//               16-float k-tiles through double-buffered LDS, both tiles stored k-major (As[k][m], Bs[k][n]) so each
//               MFMA operand read is 32 consecutive floats per half-wave.  An optional batch index (grid.y) with
//               two-level strides serves the per-(batch, head) attention GEMMs.
#include <stdlib.h>
#include <string.h>

#include <type_traits>

#include "knx_pipe.hpp"

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
    int tiles_m;
    knx_conv_geom cv;  // implicit-GEMM convolution (sgemm_k32<…, true>): A rows are output pixels gathered from x
    int cgc;           // input channels per group
    int zh;        // batch index z = zb·zh + zi
    long long sAb, sAh, sBb, sBh, sCb, sCh;
    const float* R;  // residual added after the activation (same layout as C, stride ldr), or null; batch 1 only
    int ldr;
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
                float o = knx_act(v, p.act, p.act_alpha);
                if (p.R) o = o + p.R[(size_t)m * p.ldr + n];
                C[(size_t)m * p.ldc + n] = o;
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

// ---------------------------------------------------------------- pipelined fp32 GEMM, K-contiguous operands
// C = act(alpha·A·Btᵀ + bias) with A M×K and Bt N×K row-major, K % 32 == 0: the int8 128-byte k-tile pipeline applied
// to fp32.  Each 128-byte k-tile (32 floats) of every operand row moves HBM → LDS with global_load_lds_dwordx4 into
// one of two stages, 16-byte chunks swizzled per row (chunk c of row r at c ^ swz8(r)).  K order inside a k-tile:
// lanes 0-31 take floats 0-15 and lanes 32-63 floats 16-31, one per v_mfma_f32_32x32x2_f32 k-step, so a lane reads
// its 16 operand values of a k-tile as four 16-byte chunks ("quads" of four k-steps).  Tiles that would cross M or N
// are moved back inside and store only what they own.
// 128 zero bytes: the source of the gathered rows that fall in a convolution's zero padding
__device__ __attribute__((aligned(128))) int8_t knx_zero_line[128];

template <int BM, int BN, int WM, int WN, bool CONV = false, int STG = 2>
__global__ void __launch_bounds__(WM * WN * 64) sgemm_k32(SgArgs p)
{
    static_assert(STG == 2 || STG == 3, "stages");
    constexpr int NW = WM * WN;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 32, FN = TN / 32;
    constexpr int ROWS = BM + BN;
    constexpr int STAGE = ROWS * 128;
    constexpr int SLOTS = ROWS / 8 / NW;
    constexpr int SA = BM / 8 / NW;
    static_assert(BM % (8 * NW) == 0 && BN % (8 * NW) == 0, "load split");
    static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile");
    static_assert(NW * 16 * (TN + 4) * 4 <= 2 * STAGE, "staging fits in the stages");
    __shared__ __attribute__((aligned(16))) int8_t lds[STG * STAGE];

    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wave / WN, wn = wave % WN;
    int tm, tn;
    tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const int mlo = tm * BM, nlo = tn * BN;
    const int m0 = min(mlo, p.M - BM), n0 = min(nlo, p.N - BN);
    const float* A;
    const float* B;
    float* C;
    const float* bias = p.bias;
    const float* R = p.R;  // batch 1 only (no batch offset)
    int cbase = 0;
    if (CONV) {  // grid.y = group: its channel slice of x, its rows of Wt, its columns of y and of the bias
        const int grp = blockIdx.y;
        cbase = grp * p.cgc;
        A = p.A;
        B = p.B + (size_t)grp * p.N * p.ldb;
        C = p.C + (size_t)grp * p.N;
        if (bias) bias += (size_t)grp * p.N;
        if (R) R += (size_t)grp * p.N;
    } else {
        const int z = blockIdx.y, zb = z / p.zh, zi = z % p.zh;
        A = p.A + zb * p.sAb + zi * p.sAh;
        B = p.B + zb * p.sBb + zi * p.sBh;
        C = p.C + zb * p.sCb + zi * p.sCh;
    }

    const int8_t* tile_a = reinterpret_cast<const int8_t*>(A + (size_t)m0 * p.lda);
    const int8_t* tile_b = reinterpret_cast<const int8_t*>(B + (size_t)n0 * p.ldb);
    const int lda4 = p.lda * 4, ldb4 = p.ldb * 4;  // row strides in bytes
    const int cl = (lane & 7) ^ (lane >> 3), rs = lane >> 3;
    const int nk = p.K / 32;
    // Convolution: k-tile kt is 32 consecutive channels of one tap (the group's channel count cg is a multiple of 32),
    // taps in (ky, kx) order.  Per A slot, fixed over K: the byte address of this lane's 16-byte chunk at tap (0, 0),
    // channel 0 of the group (an integer: it lies outside x when the pixel's window starts in the padding), and the
    // taps whose input pixel is inside the image as a mask, bit ky·kw + kx (at most 64 taps).  The k-tiles are issued
    // in order, so a cursor (tap, k-tile within the tap, byte offset of the k-tile from tap (0, 0), channel 0) moves
    // one k-tile per issue round: no divisions in the loop, and per slot one 64-bit add, a mask test and a select.
    constexpr int SAC = CONV ? SA : 1;
    unsigned long long at0[SAC], inside[SAC];
    int ctap = 0, ckt = 0, ckx = 0;
    long long coff = 0;
    // the zero line's address, read once: an opaque register value, so that the compiler does not load it again from
    // the global offset table in every k-tile (that load would sit in front of the k-tile's wait)
    unsigned long long zero_at;
    asm volatile("" : "=s"(zero_at) : "0"((unsigned long long)(uintptr_t)knx_zero_line));
    if (CONV) {
        const knx_conv_geom& g = p.cv;
#pragma unroll
        for (int i = 0; i < SAC; ++i) {
            const int slot = i * NW + wave;
            const int m = m0 + slot * 8 + rs;
            const int ox = m % g.Wo, oy = (m / g.Wo) % g.Ho, b = m / (g.Wo * g.Ho);
            const int iy = oy * g.sh - g.pt, ix = ox * g.sw - g.pl;
            const long long e = (((long long)b * g.H + iy) * g.W + ix) * g.C + cbase;
            at0[i] = (unsigned long long)(uintptr_t)A + (unsigned long long)(e * 4) + (unsigned)((cl ^ (slot & 7)) * 16);
            unsigned long long bits = 0;
            for (int ky = 0; ky < g.kh; ++ky) {
                const int y = iy + ky * g.dh;
                if (y < 0 || y >= g.H) continue;
                for (int kx = 0; kx < g.kw; ++kx) {
                    const int x = ix + kx * g.dw;
                    if (x >= 0 && x < g.W) bits |= 1ull << (ky * g.kw + kx);
                }
            }
            inside[i] = bits;
        }
    }
    auto conv_next = [&]() {  // cursor to the next k-tile
        const knx_conv_geom& g = p.cv;
        coff += 128;
        if (++ckt == p.cgc / 32) {
            ckt = 0;
            ++ctap;
            coff += (long long)g.dw * g.C * 4 - p.cgc * 4;
            if (++ckx == g.kw) {
                ckx = 0;
                coff += ((long long)g.dh * g.W - (long long)g.kw * g.dw) * g.C * 4;
            }
        }
    };
    auto issue1 = [&](int kt, int i) {
        const int slot = i * NW + wave;
        const bool a = i < SA;
        const int chunk = cl ^ (slot & 7);
        int8_t* dst = lds + (kt % STG) * STAGE + slot * 1024;
        if (CONV && a) {
            const bool in = (inside[i] >> ctap) & 1;
            const unsigned long long src = in ? at0[i] + (unsigned long long)coff : zero_at;
            dma16_at(reinterpret_cast<const void*>(src), dst);
            return;
        }
        const int ld = a ? lda4 : ldb4;
        const int8_t* base = (a ? tile_a + (size_t)(slot * 8) * ld : tile_b + (size_t)(slot * 8 - BM) * ld) + kt * 128;
        dma16(base, (unsigned)(rs * ld + chunk * 16), dst);
    };

    // fragment offsets: row r + 32·f has swizzle swz8(r) ^ 4·(f & 1), i.e. the chunk of half-wave g ^ (f & 1)
    const int rl = lane & 31, g = lane >> 5;
    int aoff[2][4], boff[2][4];
    {
        const int ra = wm * TM + rl, rb = BM + wn * TN + rl;
        const int sa_ = swz8(ra), sb_ = swz8(rb);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                aoff[h][c] = ra * 128 + (((4 * (g ^ h) + c) ^ sa_) << 4);
                boff[h][c] = rb * 128 + (((4 * (g ^ h) + c) ^ sb_) << 4);
            }
    }
    float4 fa[2][FM], fb[2][FN];
    auto read1 = [&](int kt, int q, int j) {  // fragment j (A if j < FM) of quad q
        const int8_t* cur = lds + (kt % STG) * STAGE;
        if (j < FM) fa[q & 1][j] = *(const float4*)(cur + aoff[j & 1][q] + j * 4096);
        else fb[q & 1][j - FM] = *(const float4*)(cur + boff[(j - FM) & 1][q] + (j - FM) * 4096);
    };
    v16f acc[FM][FN];
#pragma unroll
    for (int fi = 0; fi < FM; ++fi)
#pragma unroll
        for (int fj = 0; fj < FN; ++fj)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[fi][fj][e] = 0.0f;
    auto mfma1 = [&](int q, int j) {  // multiply j of quad q: k-step j / (FM·FN), block j % (FM·FN)
        const int s = j / (FM * FN), b = j % (FM * FN), fi = b / FN, fj = b % FN;
        acc[fi][fj] = __builtin_amdgcn_mfma_f32_32x32x2f32((&fa[q & 1][fi].x)[s], (&fb[q & 1][fj].x)[s], acc[fi][fj], 0, 0, 0);
    };

    // One k-tile, as in the int8 kernel with quads in place of k-steps: quads 0..2 multiply set q & 1 while the
    // fragments of quad q+1 are read; before quad 3's remaining multiplies the wave waits for its loads of tile kt+1
    // (with three stages the loads of tile kt+2 stay in flight: MORE) and its own LDS reads, then the barrier hands
    // stage kt % STG over to the loads of tile kt+STG.
    constexpr int NM = 4 * FM * FN, NR = FM + FN, PRE = NM / 4;
    constexpr int GAPS = NM - PRE;
    auto ktile = [&](int kt, auto ARRIVE, auto ISSUE, auto MORE) {
        constexpr bool arrive = decltype(ARRIVE)::value, iss = decltype(ISSUE)::value, more = decltype(MORE)::value;
#pragma unroll
        for (int q = 0; q < 3; ++q) {
#pragma unroll
            for (int j = 0; j < NR; ++j) read1(kt, q + 1, j);
#pragma unroll
            for (int j = 0; j < NM; ++j) mfma1(q, j);
#pragma unroll
            for (int j = 0; j < NR; ++j) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, NM - NR, 0);
        }
        if (!arrive) {
#pragma unroll
            for (int j = 0; j < NM; ++j) mfma1(3, j);
            return;
        }
#pragma unroll
        for (int j = 0; j < PRE; ++j) mfma1(3, j);
        __builtin_amdgcn_sched_barrier(0);
        if (more)
            KNX_WAIT_VM_LDS(SLOTS);
        else
            KNX_WAIT_VM_LDS(0);
        knx_barrier_nofence();
        int r = 0, l = 0;
#pragma unroll
        for (int j = PRE; j < NM; ++j) {
            mfma1(3, j);
            const int rupto = (NR * (j - PRE + 1) + GAPS - 1) / GAPS;
            while (r < rupto) read1(kt + 1, 0, r++);
            if (iss) {
                const int upto = (SLOTS * (j - PRE + 1) + GAPS - 1) / GAPS;
                while (l < upto) issue1(kt + STG, l++);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (CONV && iss) conv_next();
    };
    using yes = std::integral_constant<bool, true>;
    using no = std::integral_constant<bool, false>;
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) issue1(0, i);
    if (CONV) conv_next();
    int kt = 0;
    if (STG == 2) {
        KNX_WAIT_VM_LDS(0);
        knx_barrier_nofence();
        if (nk > 1) {
#pragma unroll
            for (int i = 0; i < SLOTS; ++i) issue1(1, i);
            if (CONV) conv_next();
        }
#pragma unroll
        for (int j = 0; j < NR; ++j) read1(0, 0, j);
        for (; kt < nk - 2; ++kt) ktile(kt, yes{}, yes{}, no{});
        if (nk >= 2) ktile(kt++, yes{}, no{}, no{});
    } else {
        // tiles 0 and 1 in flight, wait for tile 0; tile 2 goes out once every wave is past the barrier
        if (nk > 1) {
#pragma unroll
            for (int i = 0; i < SLOTS; ++i) issue1(1, i);
            if (CONV) conv_next();
            KNX_WAIT_VM_LDS(SLOTS);
        } else {
            KNX_WAIT_VM_LDS(0);
        }
        knx_barrier_nofence();
        if (nk > 2) {
#pragma unroll
            for (int i = 0; i < SLOTS; ++i) issue1(2, i);
            if (CONV) conv_next();
        }
#pragma unroll
        for (int j = 0; j < NR; ++j) read1(0, 0, j);
        for (; kt < nk - 3; ++kt) ktile(kt, yes{}, yes{}, yes{});
        if (kt < nk - 2) ktile(kt++, yes{}, no{}, yes{});
        if (kt < nk - 1) ktile(kt++, yes{}, no{}, no{});
    }
    ktile(kt, no{}, no{}, no{});

    // Epilogue: each wave stages 16 rows × TN of its accumulators at a time in its own LDS region (row stride TN+4),
    // then every lane writes 4 consecutive columns of a row with one 16-byte store.
    constexpr int SROW = TN + 4, LPR = TN / 4, RPI = 64 / LPR;
    float* stg = reinterpret_cast<float*>(lds) + wave * 16 * SROW;
    // lanes from LPR·RPI on (when LPR does not divide 64) would repeat rows of other lanes: they store nothing, so with
    // R aliasing C no lane reads a residual element that another lane has already overwritten
    const int cq = (lane % LPR) * 4, rq = lane < LPR * RPI ? lane / LPR : 16;
    const int nb = n0 + wn * TN + cq;
    float bv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) bv[q] = bias ? bias[nb + q] : 0.0f;
    const bool vec = nb >= nlo && (p.ldc & 3) == 0 && ((uintptr_t)C & 15) == 0;
    const bool rvec = nb >= nlo && (nb & 3) == 0 && (p.ldr & 3) == 0 && ((uintptr_t)R & 15) == 0;
    const bool relu = p.act == 0;
    const bool fast_res = R && p.alpha == 1.0f && !p.causal && (p.act == -1 || relu);
    static_assert(16 % RPI == 0, "rows per store instruction");
    KNX_WAIT_LDS();
    knx_barrier_nofence();  // nobody reads the operand stages any more
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
            const int mt0 = m0 + wm * TM + fi * 32 + 16 * h;
            if (fast_res) {
                // Residual with no activation or ReLU: the round's residual rows are loaded before any store (R and C
                // may alias, and a load after a store waits for it: one memory round trip per row).  Loading first is
                // right when R is C, since each element is read before its own store and no other store touches it.
                // Unrolled, so the loads sit in registers; the per-row code is a few instructions.
                constexpr int NJ = (16 + RPI - 1) / RPI;
                float4 rres[NJ];
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const int rr = rq + j * RPI, m = mt0 + rr;
                    rres[j] = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (rr >= 16 || m < mlo) continue;
                    const float* rp = R + (size_t)m * p.ldr + nb;
                    if (rvec) {
                        rres[j] = *reinterpret_cast<const float4*>(rp);
                    } else {
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            if (nb + q >= nlo) (&rres[j].x)[q] = rp[q];
                    }
                }
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const int rr = rq + j * RPI;  // idle lanes have rq = 16
                    if (rr >= 16) break;
                    const int m = mt0 + rr;
                    if (m < mlo) continue;
                    const float4 a = *reinterpret_cast<const float4*>(&stg[rr * SROW + cq]);
                    float r[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        float v = (&a.x)[q];
                        if (bias) v = v + bv[q];
                        if (relu) v = v >= 0.0f ? v : 0.0f;  // the ReLU of knx_act (NaN → 0)
                        r[q] = v + (&rres[j].x)[q];
                    }
                    float* y = C + (size_t)m * p.ldc + nb;
                    if (vec) {
                        *reinterpret_cast<float4*>(y) = make_float4(r[0], r[1], r[2], r[3]);
                    } else {
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            if (nb + q >= nlo) y[q] = r[q];
                    }
                }
            } else {
                // General epilogue: one row per iteration, a rolled loop; GELU, ReLU and no activation are
                // compile-time cases (an activation switch per element costs as much as GELU itself), any other
                // activation goes through the switch
                auto rows = [&](auto actc) {
                    constexpr int ACT = decltype(actc)::value;
                    for (int rr = rq; rr < 16; rr += RPI) {
                        const int m = mt0 + rr;
                        if (m < mlo) continue;
                        const float4 a = *reinterpret_cast<const float4*>(&stg[rr * SROW + cq]);
                        float r[4];
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            float v = (&a.x)[q];
                            if (p.alpha != 1.0f) v = p.alpha * v;
                            if (bias) v = v + bv[q];
                            if (p.causal && nb + q > m) v = -INFINITY;
                            r[q] = ACT == 1 ? knx_gelu(v) : ACT == 0 ? (v >= 0.0f ? v : 0.0f) : ACT == -1 ? v
                                                                        : knx_act(v, p.act, p.act_alpha);
                        }
                        float* y = C + (size_t)m * p.ldc + nb;
                        if (R) {  // residual after the activation; each element is read before its own store
#pragma unroll
                            for (int q = 0; q < 4; ++q)
                                if (nb + q >= nlo) r[q] = r[q] + R[(size_t)m * p.ldr + nb + q];
                        }
                        if (vec) {
                            *reinterpret_cast<float4*>(y) = make_float4(r[0], r[1], r[2], r[3]);
                        } else {
#pragma unroll
                            for (int q = 0; q < 4; ++q)
                                if (nb + q >= nlo) y[q] = r[q];
                        }
                    }
                };
                if (p.act == 1) rows(std::integral_constant<int, 1>{});
                else if (p.act == 0) rows(std::integral_constant<int, 0>{});
                else if (p.act == -1) rows(std::integral_constant<int, -1>{});
                else rows(std::integral_constant<int, -2>{});
            }
            asm volatile("" ::: "memory");
        }
    }
}

typedef float v4f __attribute__((ext_vector_type(4)));

// Small NT GEMMs (a few dozen 64×64 tiles at most, e.g. a batch of 64 rows through a Linear layer): a 16×16 output
// tile per block so that the grid still spreads over the chip, K split over the 4 waves (wave w takes the 16-wide
// k-chunks w, w + 4, …), the partial sums added in wave order through LDS.  Both operands are K-contiguous and read
// straight from global memory as 16-byte vectors; 16×16×4 fp32 MFMA.  Needs lda, ldb % 4 == 0 and 16-byte aligned
// A and B (the tail K % 16 is read element by element).
__global__ void __launch_bounds__(256) sgemm_skinny(SgArgs p)
{
    __shared__ float part[4][64 * 4];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, kq = lane >> 4;
    const int m0 = blockIdx.y * 16, n0 = blockIdx.x * 16;
    const float* a = p.A + (size_t)min(m0 + r, p.M - 1) * p.lda + 4 * kq;
    const float* b = p.B + (size_t)min(n0 + r, p.N - 1) * p.ldb + 4 * kq;
    // step c of a chunk: half-row kq of the lanes contracts over k = 16·chunk + 4·kq + c, for A and B alike
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const int nk = p.K / 16;
    int kc = wave;
    for (; kc + 12 < nk; kc += 16) {  // four chunks in flight
        float4 x[4], y[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            x[u] = *reinterpret_cast<const float4*>(a + 16 * (kc + 4 * u));
            y[u] = *reinterpret_cast<const float4*>(b + 16 * (kc + 4 * u));
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int c = 0; c < 4; ++c) acc = __builtin_amdgcn_mfma_f32_16x16x4f32((&x[u].x)[c], (&y[u].x)[c], acc, 0, 0, 0);
    }
    for (; kc < nk; kc += 4) {
        const float4 x = *reinterpret_cast<const float4*>(a + 16 * kc);
        const float4 y = *reinterpret_cast<const float4*>(b + 16 * kc);
#pragma unroll
        for (int c = 0; c < 4; ++c) acc = __builtin_amdgcn_mfma_f32_16x16x4f32((&x.x)[c], (&y.x)[c], acc, 0, 0, 0);
    }
    if (p.K % 16 != 0 && wave == nk % 4) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int k = 16 * nk + 4 * kq + c;  // relative to the row starts below
            const bool in = k < p.K;
            const float xa = in ? a[16 * nk + c] : 0.0f, yb = in ? b[16 * nk + c] : 0.0f;
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa, yb, acc, 0, 0, 0);
        }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) part[wave][lane * 4 + e] = acc[e];
    __syncthreads();
    if (wave != 0) return;
    // element e of a lane is row 4·kq + e, column r of the tile
    const int n = n0 + r;
    if (n >= p.N) return;
    const float bv = p.bias ? p.bias[n] : 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int m = m0 + 4 * kq + e;
        if (m >= p.M) break;
        float v = ((part[0][lane * 4 + e] + part[1][lane * 4 + e]) + part[2][lane * 4 + e]) + part[3][lane * 4 + e];
        if (p.alpha != 1.0f) v = p.alpha * v;
        if (p.bias) v = v + bv;
        if (p.causal && n > m) v = -INFINITY;
        float o = knx_act(v, p.act, p.act_alpha);
        if (p.R) o = o + p.R[(size_t)m * p.ldr + n];
        p.C[(size_t)m * p.ldc + n] = o;
    }
}

bool skinny_ok(const SgArgs& p, int batch)
{
    return batch == 1 && p.K >= 16 && (p.lda & 3) == 0 && (p.ldb & 3) == 0 && ((uintptr_t)p.A & 15) == 0 &&
           ((uintptr_t)p.B & 15) == 0 && (p.N + 15) / 16 <= 0x7fffffff && (p.M + 15) / 16 <= 65535;
}

int launch_skinny(SgArgs p, hipStream_t s, const char* name)
{
    hipLaunchKernelGGL(sgemm_skinny, dim3((p.N + 15) / 16, (p.M + 15) / 16), dim3(256), 0, s, p);
    return knx::check_launch(name);
}

template <int BM, int BN, int WM, int WN, int STG = 2>
int launch_k32(SgArgs p, int batch, hipStream_t s, const char* name)
{
    p.tiles_m = (p.M + BM - 1) / BM;
    p.tiles_n = (p.N + BN - 1) / BN;
    const unsigned tiles = (unsigned)p.tiles_m * (unsigned)p.tiles_n;
    hipLaunchKernelGGL((sgemm_k32<BM, BN, WM, WN, false, STG>), dim3(tiles, batch), dim3(WM * WN * 64), 0, s, p);
    return knx::check_launch(name);
}

// the pipelined kernel needs K % 32 == 0, 16-byte aligned rows and whole tiles inside M and N
bool k32_ok(const SgArgs& p, int bm, int bn)
{
    // batch offsets keep every operand base 16-byte aligned
    const bool strides = ((p.sAb | p.sAh | p.sBb | p.sBh) & 3) == 0;
    return p.K > 0 && p.K % 32 == 0 && p.M >= bm && p.N >= bn && (p.lda & 3) == 0 && (p.ldb & 3) == 0 && strides &&
           ((uintptr_t)p.A & 15) == 0 && ((uintptr_t)p.B & 15) == 0 && (long)8 * p.lda * 4 < 0x7fffffffL &&
           (long)8 * p.ldb * 4 < 0x7fffffffL;
}

// NT dispatch: the pipelined kernel when its tiles fill the chip, else the general kernel
int dispatch_nt(SgArgs p, int batch, hipStream_t s, const char* name)
{
    const long cus = knx::num_cus();
    const long t256 = (long)((p.M + 255) / 256) * ((p.N + 255) / 256) * batch;
    const long t128 = (long)((p.M + 127) / 128) * ((p.N + 127) / 128) * batch;
    // KNX_SGEMM_KERNEL forces the general kernel ("general"), one pipelined tile ("t256", "t128", "t128w8", "t64",
    // "t64x64") or the small-GEMM kernel ("skinny") where the shape allows it, else the general kernel (tests, tuning)
    const char* force = getenv("KNX_SGEMM_KERNEL");
    if (force != nullptr && *force) {
        if (strcmp(force, "t256") == 0 && k32_ok(p, 256, 256)) return launch_k32<256, 256, 4, 2>(p, batch, s, name);
        if (strcmp(force, "t128") == 0 && k32_ok(p, 128, 128)) return launch_k32<128, 128, 2, 2>(p, batch, s, name);
        if (strcmp(force, "t128w8") == 0 && k32_ok(p, 128, 128)) return launch_k32<128, 128, 4, 2>(p, batch, s, name);
        if (strcmp(force, "t64") == 0 && k32_ok(p, 128, 64)) return launch_k32<128, 64, 4, 1>(p, batch, s, name);
        if (strcmp(force, "t64x64") == 0 && k32_ok(p, 64, 64)) return launch_k32<64, 64, 2, 2>(p, batch, s, name);
#ifdef KNX_TUNING
        // variants no shape selects (measured slower where they fit), built only for tuning (-DKNX_TUNING)
        if (strcmp(force, "t128s3") == 0 && k32_ok(p, 128, 128)) return launch_k32<128, 128, 2, 2, 3>(p, batch, s, name);
        if (strcmp(force, "t64s3") == 0 && k32_ok(p, 128, 64)) return launch_k32<128, 64, 4, 1, 3>(p, batch, s, name);
        if (strcmp(force, "t64w2") == 0 && k32_ok(p, 128, 64)) return launch_k32<128, 64, 2, 2>(p, batch, s, name);
        if (strcmp(force, "t256x128") == 0 && k32_ok(p, 256, 128)) return launch_k32<256, 128, 4, 2>(p, batch, s, name);
        if (strcmp(force, "t256x192") == 0 && k32_ok(p, 256, 192)) return launch_k32<256, 192, 4, 2>(p, batch, s, name);
        if (strcmp(force, "t128x256") == 0 && k32_ok(p, 128, 256)) return launch_k32<128, 256, 2, 4>(p, batch, s, name);
        if (strcmp(force, "t64x64s3") == 0 && k32_ok(p, 64, 64)) return launch_k32<64, 64, 2, 2, 3>(p, batch, s, name);
#endif
        if (strcmp(force, "skinny") == 0 && skinny_ok(p, batch)) return launch_skinny(p, s, name);
        return dispatch<true>(p, batch, s, name);
    }
    // fewer 64×64 tiles than a quarter of the CUs: 16×16 tiles with split K
    const long t64x64 = (long)((p.M + 63) / 64) * ((p.N + 63) / 64) * batch;
    if (t64x64 * 4 < cus && skinny_ok(p, batch)) return launch_skinny(p, s, name);
    const long t64 = (long)((p.M + 127) / 128) * ((p.N + 63) / 64) * batch;
    // short K with 128×128 tiles enough for three or more workgroups per CU: those tiles on 8 waves of 32×64 (one box,
    // same process: 8192×2048×512 + GELU 138.7 µs against 142.5 on the 128×64 tiles below, 8192×4096×1024 492.4
    // against 499.4, 4096×4096×512 131.7 against 133.9, 8192×3072×768 282.8 against 287.7, 8192×1536×512 100.0
    // against 100.3; the same bits: every tile of this kernel sums each output in the same order)
    if (p.K <= 2048 && t128 >= 3 * cus && k32_ok(p, 128, 128)) return launch_k32<128, 128, 4, 2>(p, batch, s, name);
    // short K: 128×64 tiles, at least two per CU, so that several workgroups share a CU and one's prologue and
    // epilogue overlap another's multiplies (Transformer layers at 8192 rows, one box after a 2 s warm-up:
    // 8192×1536×512 105 µs against 113 for 128×128, 8192×512×512 41 against 47, 8192×2048×512 + GELU 145 against
    // 153, 8192×512×2048 131 against 137; 2×2 waves of 64×32 time the same as these 4×1 waves of 32×64)
    if (p.K <= 2048 && t64 >= 2 * cus && k32_ok(p, 128, 64)) return launch_k32<128, 64, 4, 1>(p, batch, s, name);
    if (t256 >= cus && k32_ok(p, 256, 256)) return launch_k32<256, 256, 4, 2>(p, batch, s, name);
    if (t128 >= cus && k32_ok(p, 128, 128)) return launch_k32<128, 128, 2, 2>(p, batch, s, name);
    if (t64 >= cus && k32_ok(p, 128, 64)) return launch_k32<128, 64, 4, 1>(p, batch, s, name);
    // mid shapes that leave CUs idle on the tiles above: 64×64 tiles on 2×2 waves of 32×32 (one box, µs, against the
    // general kernel and 128×64 tiles: the LSTM input projection at batch 64, 2048×512×128, 6.6 / 11.7 / 9.2;
    // 1024×512×128 6.3 / 11.2 / 9.2; 2048×512×256 8.3 / 16.3 / 13.2)
    if (k32_ok(p, 64, 64)) return launch_k32<64, 64, 2, 2>(p, batch, s, name);
    return dispatch<true>(p, batch, s, name);
}

template <int BM, int BN, int WM, int WN, int STG = 2>
int launch_conv_k32(SgArgs p, hipStream_t s, const char* name)
{
    p.tiles_m = (p.M + BM - 1) / BM;
    p.tiles_n = (p.N + BN - 1) / BN;
    const unsigned tiles = (unsigned)p.tiles_m * (unsigned)p.tiles_n;
    hipLaunchKernelGGL((sgemm_k32<BM, BN, WM, WN, true, STG>), dim3(tiles, p.cv.groups), dim3(WM * WN * 64), 0, s, p);
    return knx::check_launch(name);
}

}  // namespace

// Convolution on the pipelined kernel (internal to this library, declared in knx_conv.hip): A rows are the output
// pixels (M = B·Ho·Wo), K = kh·kw·cg with cg % 32 == 0 so a k-tile is 32 channels of one tap, Wt is Co × K.
// Returns 1 without launching when the shape does not qualify (the caller then runs the general kernel).
int knx_conv_k32(const knx_conv_geom* g, const float* x, const float* wt, const float* bias, int act, float alpha,
                 const float* R, float* y, hipStream_t s, const char* name)
{
    const int cg = g->C / g->groups, N = g->Co / g->groups;
    const long M = (long)g->B * g->Ho * g->Wo;
    if (cg % 32 != 0 || ((uintptr_t)x & 15) != 0 || ((uintptr_t)wt & 15) != 0 || M > 0x7fffffffL || g->kh * g->kw > 64)
        return 1;
    const char* force = getenv("KNX_SGEMM_KERNEL");
    if (force != nullptr && strcmp(force, "general") == 0) return 1;
    SgArgs p{};
    p.M = (int)M; p.N = N; p.K = g->kh * g->kw * cg;
    p.A = x; p.lda = 0; p.B = wt; p.ldb = p.K; p.C = y; p.ldc = g->Co;
    p.bias = bias; p.act = act; p.act_alpha = alpha; p.alpha = 1.0f; p.causal = 0; p.zh = 1;
    p.R = R; p.ldr = g->Co;
    p.cv = *g; p.cgc = cg;
    const long cus = knx::num_cus(), groups = g->groups;
    auto tiles = [&](int bm, int bn) { return (long)((M + bm - 1) / bm) * ((N + bn - 1) / bn) * groups; };
    // KNX_CONV_TILE forces one tile of the pipelined convolution where the shape allows it (tests, tuning)
    const char* tile = getenv("KNX_CONV_TILE");
    if (tile != nullptr && *tile) {
        if (strcmp(tile, "256x256") == 0 && N >= 256 && M >= 256) return launch_conv_k32<256, 256, 4, 2>(p, s, name);
        if (strcmp(tile, "256x128") == 0 && N >= 128 && M >= 256) return launch_conv_k32<256, 128, 4, 2>(p, s, name);
        if (strcmp(tile, "128x128") == 0 && N >= 128 && M >= 128) return launch_conv_k32<128, 128, 2, 2>(p, s, name);
        if (strcmp(tile, "128x128w8") == 0 && N >= 128 && M >= 128) return launch_conv_k32<128, 128, 4, 2>(p, s, name);
        if (strcmp(tile, "64x128") == 0 && N >= 128 && M >= 64) return launch_conv_k32<64, 128, 2, 4>(p, s, name);
        if (strcmp(tile, "256x64") == 0 && N >= 64 && M >= 256) return launch_conv_k32<256, 64, 4, 1>(p, s, name);
        if (strcmp(tile, "128x64") == 0 && N >= 64 && M >= 128) return launch_conv_k32<128, 64, 4, 2>(p, s, name);
    }
    if (N >= 256 && M >= 256 && tiles(256, 256) >= cus) return launch_conv_k32<256, 256, 4, 2>(p, s, name);
    // Below that, 8 waves of 32×32 or 32×64 outputs per workgroup and two or more workgroups per CU: the tap gathers
    // of 16 to 24 waves per CU hide each other's latency (CNN 3×3 convolutions over 256 images, 16 and 32 KB of
    // weights: conv3, 32×32×64 → 128 stride 2, 80.3 µs on 128×128 tiles of 4×2 waves against 84.0 on 64×128 of 2×2;
    // conv4, 16×16×128 → 256 stride 2, 77.7 µs on 64×128 of 2×4 waves against 80.0; 3 stages: 83-89 µs)
    if (N >= 128 && M >= 128 && tiles(128, 128) >= 2 * cus) return launch_conv_k32<128, 128, 4, 2>(p, s, name);
    if (N >= 128 && M >= 64 && tiles(64, 128) >= 2 * cus) return launch_conv_k32<64, 128, 2, 4>(p, s, name);
    if (N >= 128 && M >= 256 && tiles(256, 128) >= cus) return launch_conv_k32<256, 128, 4, 2>(p, s, name);
    if (N >= 128 && M >= 128 && tiles(128, 128) >= cus) return launch_conv_k32<128, 128, 2, 2>(p, s, name);
    // 64 output channels: 128×64 tiles on 4×2 waves (CNN conv2, 32×32×64 → 64: 161.7 µs, against 168.4 on 2×2 waves,
    // 167.2 for 64×64 and 174 for 256×64)
    if (N >= 64 && M >= 128 && tiles(128, 64) >= 2 * cus) return launch_conv_k32<128, 64, 4, 2>(p, s, name);
    if (N >= 64 && M >= 256 && tiles(256, 64) >= cus) return launch_conv_k32<256, 64, 4, 1>(p, s, name);
    return 1;
}

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

extern "C" int knx_hip_sgemm_nt_ep(int M, int N, int K, const float* A, int lda, const float* Wt, int ldwt,
                                   const float* bias, int act, float alpha, float* C, int ldc, void* stream)
{
    const char* name = "knx_hip_sgemm_nt_ep";
    KNX_ENTRY(name);
    KNX_REQUIRE(M >= 0 && N >= 0 && K >= 0 && act >= -1 && act <= 15, name);
    if (M == 0 || N == 0) return KNX_OK;
    KNX_REQUIRE(C != nullptr && ldc >= N, name);
    KNX_REQUIRE(K == 0 || (A != nullptr && Wt != nullptr && lda >= K && ldwt >= K), name);
    SgArgs p{};
    p.M = M; p.N = N; p.K = K; p.A = A; p.lda = lda; p.B = Wt; p.ldb = ldwt; p.C = C; p.ldc = ldc;
    p.bias = bias; p.act = act; p.act_alpha = alpha; p.alpha = 1.0f; p.causal = 0; p.zh = 1;
    return dispatch_nt(p, 1, knx::as_stream(stream), name);
}

extern "C" int knx_hip_sgemm_nt_ep_res(int M, int N, int K, const float* A, int lda, const float* Wt, int ldwt,
                                       const float* bias, int act, float alpha, const float* R, int ldr, float* C, int ldc,
                                       void* stream)
{
    const char* name = "knx_hip_sgemm_nt_ep_res";
    KNX_ENTRY(name);
    KNX_REQUIRE(M >= 0 && N >= 0 && K >= 0 && act >= -1 && act <= 15, name);
    if (M == 0 || N == 0) return KNX_OK;
    KNX_REQUIRE(C != nullptr && ldc >= N && R != nullptr && ldr >= N, name);
    KNX_REQUIRE(K == 0 || (A != nullptr && Wt != nullptr && lda >= K && ldwt >= K), name);
    SgArgs p{};
    p.M = M; p.N = N; p.K = K; p.A = A; p.lda = lda; p.B = Wt; p.ldb = ldwt; p.C = C; p.ldc = ldc;
    p.bias = bias; p.act = act; p.act_alpha = alpha; p.alpha = 1.0f; p.causal = 0; p.zh = 1;
    p.R = R; p.ldr = ldr;
    return dispatch_nt(p, 1, knx::as_stream(stream), name);
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
    return transB ? dispatch_nt(p, nb * nh, s, name) : dispatch<false>(p, nb * nh, s, name);
}
