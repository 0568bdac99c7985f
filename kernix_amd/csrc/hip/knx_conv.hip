// knx_conv.hip — NHWC convolution as an implicit GEMM on v_mfma_f32_32x32x2_f32 (gfx950).
//
// Replaces kernix_conv_run's tiled im2col → cblas_sgemm → bias_act (reference include/kernix_model.h:711-771,
// im2col :677-693): the GEMM is out[m][n] = Σ_k A[m][k]·W[k][n] with m = (b, oy, ox), k = (ky, kx, ci) and
// A[m][k] = x[b, oy·sh − pt + ky·dh, ox·sw − pl + kx·dw, ci] (0 outside the image).  Each workgroup gathers its
// BM×16 slice of A directly from the input into LDS, so the column matrix never exists in HBM; bias and activation
// are applied in the epilogue.  Groups run as grid.y (each group is an independent GEMM over its channel slice).
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "knx_common.hpp"

typedef float v16f __attribute__((ext_vector_type(16)));

// the pipelined implicit-GEMM kernel (knx_sgemm.hip): returns 1 without launching when the shape does not qualify
int knx_conv_k32(const knx_conv_geom* g, const float* x, const float* wt, const float* bias, int act, float alpha,
                 const float* R, float* y, hipStream_t s, const char* name);

namespace {

struct ConvArgs {
    knx_conv_geom g;
    const float* x;
    const float* w;
    const float* bias;
    int act;
    float alpha;
    float* y;
    int M, N, K, cg;
    int tiles_n;
    const float* R;  // residual added after the activation (same layout as y), or null
};

constexpr int BK = 16;

// TB: the weight is given transposed (Wt, Co × K, the device layout of the model's convolution weights)
template <int BM, int BN, int WM, int WN, bool VEC, bool TB = false>
__global__ void __launch_bounds__(WM * WN * 64) conv_tile(ConvArgs p)
{
    constexpr int NT = WM * WN * 64;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 32, FN = TN / 32;
    constexpr int SA = BM + 4, SB = BN + 4;
    constexpr int LA = BM * BK / 4 / NT;
    constexpr int LB = BN * BK / 4 / NT;
    static_assert(BM * BK / 4 % NT == 0 && BN * BK / 4 % NT == 0, "load split");
    __shared__ __attribute__((aligned(16))) float As[2][BK * SA];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK * SB];

    const knx_conv_geom& g = p.g;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int tm = blockIdx.x / p.tiles_n, tn = blockIdx.x % p.tiles_n;
    const int m0 = tm * BM, n0 = tn * BN;
    const int grp = blockIdx.y;
    const int M = p.M, N = p.N, K = p.K, cg = p.cg;
    const int cbase = grp * cg;                 // first input channel of the group
    // the group's weight columns in W (K × Co), or its rows in Wt (Co × K)
    const float* W = TB ? p.w + (size_t)grp * N * K : p.w + (size_t)grp * N;
    const bool b_vec = TB ? (K & 3) == 0 && ((uintptr_t)p.w & 15) == 0 : (g.Co & 3) == 0 && (N & 3) == 0;

    // per load slot: the output pixel this thread gathers for (fixed over the whole K loop)
    int sb[LA], siy[LA], six[LA];
    bool sok[LA];
#pragma unroll
    for (int i = 0; i < LA; ++i) {
        const int idx = i * NT + t, r = idx >> 2, m = m0 + r;
        sok[i] = m < M;
        const int mm = sok[i] ? m : 0;
        const int ox = mm % g.Wo, oy = (mm / g.Wo) % g.Ho, b = mm / (g.Wo * g.Ho);
        sb[i] = b;
        siy[i] = oy * g.sh - g.pt;
        six[i] = ox * g.sw - g.pl;
    }

    // The k index of this thread's first gathered element is k0 + kc (kc = 4·(t & 3), the same for every load
    // slot); its tap (ky, kx) and channel ci are tracked incrementally as k0 advances, so the K loop does no integer
    // division.
    const int kc0 = (t & 3) * 4;
    int tci, tkx, tky;
    {
        const int seg = kc0 / cg;
        tci = kc0 - seg * cg;
        tky = seg / g.kw;
        tkx = seg - tky * g.kw;
    }
    auto advance = [&](int& ci, int& kx, int& ky, int d) {
        ci += d;
        while (ci >= cg) {
            ci -= cg;
            if (++kx == g.kw) { kx = 0; ++ky; }
        }
    };
    auto tap = [&](int i, int ci, int kx, int ky) -> const float* {
        const int iy = siy[i] + ky * g.dh, ix = six[i] + kx * g.dw;
        if (iy < 0 || iy >= g.H || ix < 0 || ix >= g.W) return nullptr;
        return p.x + (((size_t)sb[i] * g.H + iy) * g.W + ix) * g.C + cbase + ci;
    };

    float4 ra[LA], rb[LB];
    auto gload = [&](int k0) {  // k0: first k of the tile; (tci, tkx, tky) describe k0 + kc0 on entry
        const int gk = k0 + kc0;
#pragma unroll
        for (int i = 0; i < LA; ++i) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (sok[i]) {
                if (VEC) {
                    // cg % 4 == 0: the 4 consecutive k share one (ky, kx) tap and are 4 consecutive channels
                    if (gk < K) {
                        const float* src = tap(i, tci, tkx, tky);
                        if (src) v = *reinterpret_cast<const float4*>(src);
                    }
                } else {
                    int ci = tci, kx = tkx, ky = tky;
                    float e[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const float* src = gk + u < K ? tap(i, ci, kx, ky) : nullptr;
                        e[u] = src ? *src : 0.0f;
                        advance(ci, kx, ky, 1);
                    }
                    v = make_float4(e[0], e[1], e[2], e[3]);
                }
            }
            ra[i] = v;
        }
        advance(tci, tkx, tky, BK);
#pragma unroll
        for (int i = 0; i < LB; ++i) {
            if (TB) {  // row r of Wt (output channel n0 + r), k-chunk kc
                const int idx = i * NT + t, r = idx >> 2, kc = (idx & 3) * 4;
                const int gn = n0 + r, gkb = k0 + kc;
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (gn < N) {
                    const float* src = W + (size_t)gn * K + gkb;
                    if (b_vec && gkb + 3 < K) v = *reinterpret_cast<const float4*>(src);
                    else {
                        if (gkb + 0 < K) v.x = src[0];
                        if (gkb + 1 < K) v.y = src[1];
                        if (gkb + 2 < K) v.z = src[2];
                        if (gkb + 3 < K) v.w = src[3];
                    }
                }
                rb[i] = v;
                continue;
            }
            const int idx = i * NT + t, k = idx / (BN / 4), nc = (idx % (BN / 4)) * 4;
            const int gkb = k0 + k, gn = n0 + nc;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (gkb < K) {
                const float* src = W + (size_t)gkb * g.Co + gn;
                if (b_vec && gn + 3 < N) v = *reinterpret_cast<const float4*>(src);
                else {
                    if (gn + 0 < N) v.x = src[0];
                    if (gn + 1 < N) v.y = src[1];
                    if (gn + 2 < N) v.z = src[2];
                    if (gn + 3 < N) v.w = src[3];
                }
            }
            rb[i] = v;
        }
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

    const int rl = lane & 31, gl = lane >> 5;
    const int nk = (K + BK - 1) / BK;
    gload(0);
    swrite(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) gload((kt + 1) * BK);
#pragma unroll
        for (int s = 0; s < BK / 2; ++s) {
            float af[FM], bf[FN];
            const int kk = 2 * s + gl;
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

#pragma unroll
    for (int fj = 0; fj < FN; ++fj) {
        const int n = n0 + wn * TN + fj * 32 + rl;
        if (n >= N) continue;
        const int co = grp * N + n;
        const float bn = p.bias ? p.bias[co] : 0.0f;
#pragma unroll
        for (int fi = 0; fi < FM; ++fi)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + wm * TM + fi * 32 + 8 * (e >> 2) + 4 * gl + (e & 3);
                if (m >= M) continue;
                float v = acc[fi][fj][e];
                if (p.bias) v = v + bn;
                v = knx_act(v, p.act, p.alpha);
                if (p.R) v = v + p.R[(size_t)m * g.Co + co];
                p.y[(size_t)m * g.Co + co] = v;
            }
    }
}

// ---------------------------------------------------------------- convolution with few inputs per output
// A first layer such as 3×3 over RGB (K = 27) is a poor fit for the k-tiled kernels: K pads to whole k-tiles of
// LDS-staged operands while the output, Co fp32 channels per pixel, is what costs.  Here each wave owns 32 output
// pixels at a time and multiplies its gathered inputs straight from registers on v_mfma_f32_32x32x2f32: lane l
// gathers, for pixel l & 31, the inputs k = 2p + (l >> 5) of every k pair p (the A fragments, K ≤ 32 so at most 16
// pairs); the weights are staged once per workgroup in LDS and read from there as the B fragments (Co = 32·NB,
// NB ≤ 4; holding them in registers cost a wave per SIMD of occupancy); every accumulator register is stored
// directly (two 128-byte row segments per instruction).  Epilogue: bias, then ReLU or nothing, then the residual,
// each an fp32 rounding as in the other convolution kernels.
constexpr int SMALL_K = 32;

struct SmallConvArgs {
    const float* x;
    const float* w;
    const float* bias;
    const float* R;  // residual added after the activation (same layout as y), or null
    float* y;
    int H, W, C, Ho, Wo, Co, sh, sw, pt, pl;
    int relu;
    int M;                          // B·Ho·Wo
    int K;                          // kh·kw·C ≤ 32
    int wsc, wsk;                   // weight element (co, k) at w[co·wsc + k·wsk]
    int dyx[SMALL_K];               // per k: input row and column offset of its tap, ky·dh << 16 | kx·dw
    int off[SMALL_K];               // per k: element offset from the pixel's top-left input element
};

__device__ float conv_zero_word = 0.0f;  // what the gather reads for padding: never written

template <int NB, bool RES, int KP = SMALL_K / 2>  // KP: the k pairs multiplied (⌈K/2⌉ ≤ KP ≤ 16)
__global__ void __launch_bounds__(256) conv_small(SmallConvArgs a)
{
    constexpr int CO = 32 * NB;
    __shared__ float wl[SMALL_K * CO];  // the weights, [k][co]: staged once per workgroup with coalesced loads
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rl = lane & 31, g = lane >> 5;
    // y (and R) as buffers of M·Co floats (< 2^31 bytes, checked at launch)
    const int ybytes = (int)((long long)a.M * CO * 4);
    const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(a.y, (short)0, ybytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(RES ? a.R : a.y), (short)0,
                                                                        ybytes, 0x00020000);
    constexpr int kPast = 0x7ffffff0;
    for (int i = threadIdx.x; i < a.K * CO; i += 256) {
        // i walks the weight in memory order: Wt rows (co, then k) or W rows (k, then co)
        const int co = a.wsk == 1 ? i / a.K : i % CO, k = a.wsk == 1 ? i % a.K : i / CO;
        wl[k * CO + co] = a.w[i];
    }
    __syncthreads();
    // rows k ≥ K of the staged weights are zero, so every k pair can be multiplied
    for (int i = a.K * CO + threadIdx.x; i < SMALL_K * CO; i += 256) wl[i] = 0.0f;
    __syncthreads();
    float bv[NB];
    int dyx[KP], off[KP];
#pragma unroll
    for (int p = 0; p < KP; ++p) {
        dyx[p] = g ? a.dyx[2 * p + 1] : a.dyx[2 * p];
        off[p] = g ? a.off[2 * p + 1] : a.off[2 * p];
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) bv[nb] = a.bias ? a.bias[32 * nb + rl] : 0.0f;
    // A row of lane rl: pixel m0 + rl (rows past M gather zeros and are not stored)
    // Branch-free: a lane whose k is padding, past K or of a pixel past M loads the zero word instead, so the loads
    // issue back to back under one exec mask and their values feed the MFMAs unchanged (no select after the load).
    auto gather = [&](long long m0, float (&av)[KP]) {
        const long long mp = m0 + rl;
        const bool pok = mp < a.M;
        const int m = pok ? (int)mp : 0;
        const int ox = m % a.Wo, r = m / a.Wo, oy = r % a.Ho, b = r / a.Ho;
        const int iy0 = oy * a.sh - a.pt, ix0 = ox * a.sw - a.pl;
        const float* px = a.x + (((long long)b * a.H + iy0) * a.W + ix0) * a.C;  // never read at a padded corner
#pragma unroll
        for (int p = 0; p < KP; ++p) {
            const int iy = iy0 + (dyx[p] >> 16), ix = ix0 + (dyx[p] & 0xffff);
            const bool in = pok & (2 * p + g < a.K) & ((unsigned)iy < (unsigned)a.H) & ((unsigned)ix < (unsigned)a.W);
            av[p] = *(in ? px + off[p] : &conv_zero_word);
        }
    };
    // multiply the gathered group at m0 and write it (full: the whole group is inside M, known at the call site)
    auto group = [&](long long m0, const float (&av)[KP], bool full) {
        v16f acc[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[nb][e] = 0.0f;
#pragma unroll
        for (int p = 0; p < KP; ++p)  // every pair up to KP: pairs past K multiply zeros (no branch between the MFMAs)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)  // B fragment: weight (k = 2p + g, channel 32·nb + rl) from LDS
                acc[nb] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[p], wl[(2 * p + g) * CO + 32 * nb + rl], acc[nb], 0, 0, 0);
        // accumulator e of block nb: pixel m0 + 8·(e >> 2) + 4·g + (e & 3), channel 32·nb + rl; Co = 32·NB, so
        // every element's offset from this lane's first one is a constant
        // Every store is issued, rows past M with an offset past the buffer's end (the hardware drops them): a
        // fixed count of stores per group, so the compiler's count of memory operations in flight stays exact
        // across the loop and the next group's inputs are waited for without waiting for these stores.
        const int first = (int)((m0 + 4 * g) * CO + rl) * 4;
        const int left = (int)std::min<long long>(a.M - m0 - 4 * g, 32);  // rows of this lane's half still in M
        float rres[NB][16];
        if (RES) {  // every residual element this lane adds is loaded before its stores (R may be y)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int row = 8 * (e >> 2) + (e & 3);
                    rres[nb][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                        rr, full || row < left ? first + 4 * (row * CO + 32 * nb) : kPast, 0, 0));
                }
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = 8 * (e >> 2) + (e & 3);
                float v = acc[nb][e];
                if (a.bias) v = v + bv[nb];
                if (a.relu) v = v >= 0.0f ? v : 0.0f;  // the ReLU of knx_act (NaN → 0)
                if (RES) v = v + rres[nb][e];
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, v), yr,
                                                      full || row < left ? first + 4 * (row * CO + 32 * nb) : kPast, 0, 0);
            }
    };
    // Each wave takes the groups of 32 pixels m0, m0 + step, …; the next group's inputs are in flight while one
    // multiplies and stores (two input buffers, alternating).
    const long long step = (long long)gridDim.x * 128;
    long long m0 = ((long long)blockIdx.x * 4 + wave) * 32;
    float av0[KP], av1[KP];
    gather(m0, av0);
    // the first group's inputs waited for here, so that at the loop's head the only loads in flight are those of
    // the iterations before (followed by their stores) and the waits inside the loop count those stores
    __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // vmcnt(0)
    while (m0 < a.M) {
        gather(m0 + step, av1);
        group(m0, av0, m0 + 32 <= a.M);  // m0 is the same in every lane: a scalar branch
        m0 += step;
        if (m0 >= a.M) break;
        gather(m0 + step, av0);
        group(m0, av1, m0 + 32 <= a.M);
        m0 += step;
    }
}

// Runs the MFMA kernel above when the shape qualifies (one group, K ≤ 32, Co ∈ {32, 64, 96, 128}, no activation or
// ReLU, offsets within int); returns 1 without launching otherwise.  KNX_CONV_SMALL=0 turns it off, "g<N>" launches
// N workgroups per CU instead of 3 (tests, tuning).  3×3 over 3 channels to 64, 256×32×32 pixels: 24.5 µs with 3 per
// CU (2: 25.1, 4: 26.1, 6: 27.7) against 43 µs for the tile kernel.
int conv_small_entry(const knx_conv_geom* g, const float* x, const float* w, bool transposed, const float* bias,
                     int act, const float* R, float* y, hipStream_t s, const char* name)
{
    const char* env = getenv("KNX_CONV_SMALL");
    if (env != nullptr && strcmp(env, "0") == 0) return 1;
    const int K = g->kh * g->kw * g->C;
    if (g->groups != 1 || K > SMALL_K || g->Co % 32 != 0 || g->Co > 128 || (act != -1 && act != 0)) return 1;
    const long long span = ((long long)(g->kh - 1) * g->dh * g->W + (long long)(g->kw - 1) * g->dw + 1) * g->C;
    if (span > 0x7fffffffLL || (g->kh - 1) * g->dh > 0x7fff || (g->kw - 1) * g->dw > 0xffff) return 1;
    if ((long long)g->B * g->Ho * g->Wo * g->Co * 4 >= (1LL << 31) - 16) return 1;  // y as a buffer: 32-bit offsets
    SmallConvArgs a{};
    a.x = x; a.w = w; a.bias = bias; a.R = R; a.y = y;
    a.H = g->H; a.W = g->W; a.C = g->C; a.Ho = g->Ho; a.Wo = g->Wo; a.Co = g->Co;
    a.sh = g->sh; a.sw = g->sw; a.pt = g->pt; a.pl = g->pl; a.relu = act == 0;
    a.M = g->B * g->Ho * g->Wo;
    a.K = K;
    a.wsc = transposed ? K : 1;
    a.wsk = transposed ? 1 : g->Co;
    for (int k = 0; k < K; ++k) {  // k = (ky, kx, ci), the im2col order
        const int tap = k / g->C, ci = k % g->C, ky = tap / g->kw, kx = tap % g->kw;
        a.dyx[k] = ky * g->dh << 16 | kx * g->dw;
        a.off[k] = (int)(((long long)ky * g->dh * g->W + (long long)kx * g->dw) * g->C + ci);
    }
    const long groups32 = ((long)a.M + 31) / 32;
    long per_cu = 3;  // about the resident workgroups
    if (env != nullptr && env[0] == 'g') per_cu = std::max(1L, strtol(env + 1, nullptr, 10));
    const long blocks = std::min<long>((groups32 + 3) / 4, per_cu * knx::num_cus());
    const dim3 grid((unsigned)blocks);
    // K = 27 (3×3 over RGB): 14 k pairs instead of 16
    const bool k14 = K <= 28 && (env == nullptr || strcmp(env, "k16") != 0);
    if (k14 && g->Co == 64) {
        if (R) hipLaunchKernelGGL((conv_small<2, true, 14>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((conv_small<2, false, 14>), grid, dim3(256), 0, s, a);
        return knx::check_launch(name);
    }
    switch (g->Co / 32 * 2 + (R != nullptr)) {
    case 2: hipLaunchKernelGGL((conv_small<1, false>), grid, dim3(256), 0, s, a); break;
    case 3: hipLaunchKernelGGL((conv_small<1, true>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((conv_small<2, false>), grid, dim3(256), 0, s, a); break;
    case 5: hipLaunchKernelGGL((conv_small<2, true>), grid, dim3(256), 0, s, a); break;
    case 6: hipLaunchKernelGGL((conv_small<3, false>), grid, dim3(256), 0, s, a); break;
    case 7: hipLaunchKernelGGL((conv_small<3, true>), grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((conv_small<4, false>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((conv_small<4, true>), grid, dim3(256), 0, s, a); break;
    }
    return knx::check_launch(name);
}

template <int BM, int BN, int WM, int WN, bool TB>
int launch(ConvArgs p, bool vec, hipStream_t s, const char* name)
{
    p.tiles_n = (p.N + BN - 1) / BN;
    const unsigned tiles = (unsigned)((p.M + BM - 1) / BM) * (unsigned)p.tiles_n;
    if (vec) hipLaunchKernelGGL((conv_tile<BM, BN, WM, WN, true, TB>), dim3(tiles, p.g.groups), dim3(WM * WN * 64), 0, s, p);
    else hipLaunchKernelGGL((conv_tile<BM, BN, WM, WN, false, TB>), dim3(tiles, p.g.groups), dim3(WM * WN * 64), 0, s, p);
    return knx::check_launch(name);
}

template <bool TB>
int conv_entry(const knx_conv_geom* g, const float* x, const float* w, const float* bias, int act, float alpha,
               const float* R, float* y, void* stream, const char* name)
{
    KNX_ENTRY(name);
    KNX_REQUIRE(g != nullptr, name);
    KNX_REQUIRE(g->B >= 0 && g->H >= 1 && g->W >= 1 && g->C >= 1 && g->Ho >= 1 && g->Wo >= 1 && g->Co >= 1, name);
    KNX_REQUIRE(g->kh >= 1 && g->kw >= 1 && g->sh >= 1 && g->sw >= 1 && g->dh >= 1 && g->dw >= 1, name);
    KNX_REQUIRE(g->pt >= 0 && g->pl >= 0 && g->groups >= 1 && g->C % g->groups == 0 && g->Co % g->groups == 0, name);
    KNX_REQUIRE(act >= -1 && act <= 15, name);
    // every gathered (oy, ox, ky, kx) must come from a finite geometry; the kernel bounds-checks each input pixel
    KNX_REQUIRE((long long)g->B * g->Ho * g->Wo <= 0x7fffffffLL && (long long)g->B * g->H * g->W * g->C <= (1LL << 40), name);
    if (g->B == 0) return KNX_OK;
    KNX_REQUIRE(x && w && y && x != y, name);
    hipStream_t s = knx::as_stream(stream);
    {
        const int rc = conv_small_entry(g, x, w, TB, bias, act, R, y, s, name);
        if (rc != 1) return rc;
    }
    if (TB) {
        const int rc = knx_conv_k32(g, x, w, bias, act, alpha, R, y, s, name);
        if (rc != 1) return rc;
    }
    ConvArgs p{};
    p.g = *g; p.x = x; p.w = w; p.bias = bias; p.act = act; p.alpha = alpha; p.y = y; p.R = R;
    p.cg = g->C / g->groups;
    p.M = g->B * g->Ho * g->Wo;
    p.N = g->Co / g->groups;
    p.K = g->kh * g->kw * p.cg;
    const bool vec = (p.cg & 3) == 0 && (((uintptr_t)x) & 15) == 0;
    const long tiles = (long)((p.M + 127) / 128) * g->groups;
    if (tiles >= knx::num_cus()) {
        // narrow outputs: 256 pixels × 64 channels, each wave 64 × 64 (four MFMAs per four fragment reads)
        if (vec && p.N <= 64 && tiles >= 2L * knx::num_cus()) return launch<256, 64, 4, 1, TB>(p, vec, s, name);
        if (p.N <= 64) return launch<128, 64, 2, 2, TB>(p, vec, s, name);
        return launch<128, 128, 2, 2, TB>(p, vec, s, name);
    }
    return launch<64, 64, 2, 2, TB>(p, vec, s, name);
}

}  // namespace

extern "C" int knx_hip_conv(const knx_conv_geom* g, const float* x, const float* w, const float* bias, int act,
                            float alpha, float* y, void* stream)
{
    return conv_entry<false>(g, x, w, bias, act, alpha, nullptr, y, stream, "knx_hip_conv");
}

extern "C" int knx_hip_conv_t(const knx_conv_geom* g, const float* x, const float* wt, const float* bias, int act,
                              float alpha, float* y, void* stream)
{
    return conv_entry<true>(g, x, wt, bias, act, alpha, nullptr, y, stream, "knx_hip_conv_t");
}

extern "C" int knx_hip_conv_t_res(const knx_conv_geom* g, const float* x, const float* wt, const float* bias, int act,
                                  float alpha, const float* R, float* y, void* stream)
{
    const char* name = "knx_hip_conv_t_res";
    KNX_ENTRY(name);
    KNX_REQUIRE(R != nullptr, name);
    return conv_entry<true>(g, x, wt, bias, act, alpha, R, y, stream, name);
}
