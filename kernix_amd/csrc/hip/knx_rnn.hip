// knx_rnn.hip — the recurrence of one RNN direction (LSTM, GRU, simple RNN) as one launch.
//
// Reference include/kernix_model.h:563-632 (kernix_rnn_dir): the input projection x·W + b of every timestep is one
// GEMM (done before this kernel, zx); then for t in order (reversed for the backward direction) the recurrent term
// h_{t−1}·U is added and the cell applied, int8 (kernix_qmatmul on the B rows of h) or fp32.  Run as a launch per
// timestep for the product and another for the cell, a small batch is all launch latency; here one grid does every
// timestep: workgroup w owns units [w·uw, (w+1)·uw), keeps the U columns of those units' gates in LDS for the whole
// sequence and its cells' c in registers, and per timestep
//   1. loads h_{t−1} (all B rows, written by every workgroup at t−1) into LDS — int8: quantizes each row there with
//      the quantizer's operations (s = max|h|/127, 1 for an all-zero row, NaN for a row holding NaN or ±inf;
//      q = clamp(rint(h·(1/s)), ±127)), as knx_hip_quantize_rows;
//   2. forms its gate columns of h_{t−1}·U: fp32 dot products, or exact int32 sums of int8 products dequantized as the
//      int8 GEMM's epilogue, ((float)acc·s)·scale (+ the GRU's recurrent bias);
//   3. applies the cells (knx_lstm_cell / knx_gru_cell, the same functions as knx_hip_rnn_gates) to its (row, unit)
//      pairs, writes h_t (at device scope, for the other workgroups) and the output;
//   4. waits at a grid barrier (knx_grid.hpp: one 64-bit word, every barrier adds 256; at most 64 workgroups, all
//      resident).
// The int8 results are the bits of the per-timestep path (same quantizer, exact int32 sums, same epilogue and cell
// order); fp32 sums run in this kernel's own order.
#include <float.h>
#include <math.h>
#include <algorithm>
#include <mutex>

#include "knx_common.hpp"
#include "knx_grid.hpp"

namespace {

constexpr int kThreads = 256, kWaves = 4;
constexpr int kMaxPairs = 2;             // (row, unit) pairs per thread in the cell phase: B·uw ≤ 512
constexpr int kMaxGrid = 64;
constexpr int kLoads = 8;                // float4 loads of h in flight per thread
constexpr size_t kMaxLds = 120 * 1024;

struct RnnArgs {
    int kind, act;
    float alpha;
    int B, T, u, gu, gates, dir, ret_seq, stride, uw, up;
    const float* zx;      // B·T × gu (row b·T + t), the input projection with its bias
    const float* U;       // fp32 recurrent weight: u × gu (u_nt = 0) or gu × u (u_nt = 1)
    int u_nt;
    const int8_t* q;      // int8 recurrent weight: gu rows of kp bytes (k contiguous), or null
    int kp;
    const float* qs;      // its gu scales
    const float* brec;    // GRU recurrent bias (gu), or null
    float* h0;            // hidden states of even / odd timesteps (B × u each)
    float* h1;
    float* dst;
    knx::GridSync gs;
};

__host__ __device__ inline size_t round16(size_t b) { return (b + 15) / 16 * 16; }

// Dot products of a timestep: each thread sums CB adjacent gate columns of one row over a slice of K (P consecutive
// lanes split K, their partial sums reduced by lane exchanges), so a row value read from LDS serves CB products.
constexpr int CB = 4;

// LDS layout (bytes): weight slice [ncp][upp] (fp32: upp = up + 1 floats; int8: upp = up/4 + 1 words), rows of h
// [B][upp] fp32, int8 rows [B][up/4 + 1] words and their scales [B] (int8 only), recurrent terms [B][gates·uw].
// The odd row pitches put the rows that one wave reads at the same k on different banks.  ncp: the workgroup's gate
// columns rounded up to CB (the extra columns are zero).
struct Lds {
    size_t us, hs, hq, sx, r, total;
    int upp, hwp, ncp;
};
__host__ __device__ inline Lds lds_layout(int B, int gates, int uw, int up, bool i8)
{
    Lds l;
    l.ncp = (gates * uw + CB - 1) / CB * CB;
    l.upp = i8 ? up / 4 + 1 : up + 1;
    l.hwp = up / 4 + 1;
    l.us = 0;
    l.hs = round16((size_t)l.ncp * l.upp * 4);
    l.hq = l.hs + round16((size_t)B * (up + 1) * 4);
    l.sx = l.hq + (i8 ? round16((size_t)B * l.hwp * 4) : 0);
    l.r = l.sx + (i8 ? round16((size_t)B * 4) : 0);
    l.total = l.r + round16((size_t)B * gates * uw * 4);
    return l;
}

__device__ __forceinline__ float mag(float v)
{
    const float a = fabsf(v);
    return a <= FLT_MAX ? a : INFINITY;
}

__global__ void __launch_bounds__(kThreads) rnn_recurrence(RnnArgs a)
{
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const bool i8 = a.q != nullptr;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int B = a.B, T = a.T, u = a.u, up = a.up, gu = a.gu, G = a.gates;
    const int j0 = blockIdx.x * a.uw;
    const int nwu = min(a.uw, u - j0);  // ≥ 1: the grid has ⌈u / uw⌉ workgroups
    const int NC = G * nwu, NCM = G * a.uw;
    const Lds L = lds_layout(B, G, a.uw, up, i8);
    const int upp = L.upp, hp = up + 1, hwp = L.hwp, ncp = L.ncp;
    float* usf = reinterpret_cast<float*>(smem + L.us);
    int* usw = reinterpret_cast<int*>(smem + L.us);
    float* hs = reinterpret_cast<float*>(smem + L.hs);
    int* hqw = reinterpret_cast<int*>(smem + L.hq);
    float* sxs = reinterpret_cast<float*>(smem + L.sx);
    float* r = reinterpret_cast<float*>(smem + L.r);
    auto column = [&](int cc) { return (cc / nwu) * u + j0 + cc % nwu; };  // gate column of local column cc

    // the weight slice, once: local column cc = g·nwu + jj is gate g of unit j0 + jj; k ≥ u and columns ≥ NC are zero
    if (i8) {
        for (int e = tid; e < ncp * (up / 4); e += kThreads) {
            const int cc = e / (up / 4), w = e % (up / 4);
            unsigned v = 0;
            if (cc < NC) {
                const int8_t* src = a.q + (size_t)column(cc) * a.kp + 4 * w;
#pragma unroll
                for (int i = 0; i < 4; ++i) v |= (unsigned)(uint8_t)(4 * w + i < u ? src[i] : 0) << (8 * i);
            }
            usw[cc * upp + w] = (int)v;
        }
    } else {
        for (int e = tid; e < ncp * up; e += kThreads) {
            const int cc = e / up, k = e % up;
            float v = 0.0f;
            if (cc < NC && k < u) {
                const int col = column(cc);
                v = a.u_nt ? a.U[(size_t)col * u + k] : a.U[(size_t)k * gu + col];
            }
            usf[cc * upp + k] = v;
        }
    }
    // this thread's (row, unit) pairs of the cell phase and their per-column constants
    const int npairs = B * nwu;
    float cst[kMaxPairs];
    for (int i = 0; i < kMaxPairs; ++i) cst[i] = 0.0f;

    // dot products: O groups of CB columns of one row, P consecutive lanes each (a power of two ≤ 64)
    const int ncg = ncp / CB, O = B * ncg;
    int P = 1;
    while (P < 64 && P * 2 * O <= kThreads) P *= 2;
    const int groups = kThreads / P, gl = tid % P;
    int qlpr = 1;  // lanes per row of the int8 quantizer
    while (qlpr < 64 && qlpr * 8 < u) qlpr *= 2;

    // the input-side gate values of this thread's pairs, one timestep ahead (they do not depend on h)
    auto load_z = [&](int st, float (&z)[kMaxPairs][4]) {
        const int tt = a.dir ? T - 1 - st : st;
#pragma unroll
        for (int i = 0; i < kMaxPairs; ++i) {
            const int pr = tid + kThreads * i;
            const int b = pr / nwu, jj = pr % nwu;
#pragma unroll
            for (int g = 0; g < 4; ++g)
                z[i][g] = pr < npairs && g < G ? a.zx[((size_t)b * T + tt) * gu + (size_t)g * u + j0 + jj] : 0.0f;
        }
    };
    float zn[kMaxPairs][4];
    load_z(0, zn);
    for (int step = 0; step < T; ++step) {
        const int t = a.dir ? T - 1 - step : step;
        const float* hin = (step & 1) ? a.h0 : a.h1;  // h_{t−1}: written at the previous step
        float* hout = (step & 1) ? a.h1 : a.h0;
        float zv[kMaxPairs][4];
#pragma unroll
        for (int i = 0; i < kMaxPairs; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) zv[i][g] = zn[i][g];
        if (step + 1 < T) load_z(step + 1, zn);
        if (step > 0) {
            // h_{t−1} into LDS: the B·u floats as float4s (the buffers are 16-byte aligned and padded to 256 bytes),
            // up to kLoads in flight per thread, all issued before the first is stored
            {
                const int n = B * u, n4 = (n + 3) / 4;
                const float4* src = reinterpret_cast<const float4*>(hin);
                for (int f0 = 0; f0 < n4; f0 += kLoads * kThreads) {
                    float4 v[kLoads];
#pragma unroll
                    for (int i = 0; i < kLoads; ++i) {
                        const int f = f0 + tid + i * kThreads;
                        v[i] = f < n4 ? src[f] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    }
#pragma unroll
                    for (int i = 0; i < kLoads; ++i) {
                        const int f = f0 + tid + i * kThreads;
                        if (f >= n4) continue;
                        int b = 4 * f / u, k = 4 * f - b * u;  // element 4f is (b, k); the next ones may wrap
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            if (b * u + k < n) hs[b * hp + k] = (&v[i].x)[q];
                            if (++k == u) k = 0, ++b;
                        }
                    }
                }
            }
            __syncthreads();
            if (i8) {
                // LPR lanes per row (a power of two, about 8 values each): maximum, scale, quantized values packed
                // four to a word (bytes past u are 0)
                const int rl = lane % qlpr;
                for (int b = wave * (64 / qlpr) + lane / qlpr; b - lane / qlpr < B; b += kWaves * (64 / qlpr)) {
                    const int bb = min(b, B - 1);  // lanes past the last row repeat it, unstored
                    float mx = 0.0f;
                    for (int k = rl; k < u; k += qlpr) mx = fmaxf(mx, mag(hs[bb * hp + k]));
                    for (int off = qlpr / 2; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
                    if (b >= B) continue;
                    const bool bad = !(mx <= FLT_MAX);
                    const float sc = (!bad && mx > 0.0f) ? __fdiv_rn(mx, 127.0f) : 1.0f;
                    const float inv = __fdiv_rn(1.0f, sc);
                    if (rl == 0) sxs[b] = bad ? __int_as_float(0x7fc00000) : sc;
                    for (int w = rl; w < up / 4; w += qlpr) {
                        // a row that cannot be quantized stores zeros: its outputs are NaN through its scale
                        unsigned pk = 0;
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int k = 4 * w + i;
                            const float v = k < u && !bad ? __builtin_amdgcn_fmed3f(rintf(hs[b * hp + k] * inv), -127.0f, 127.0f) : 0.0f;
                            pk |= (unsigned)(uint8_t)(int8_t)(int)v << (8 * i);
                        }
                        hqw[b * hwp + w] = (int)pk;
                    }
                }
                __syncthreads();
            }
            // the recurrent terms of this workgroup's columns
            for (int o0 = 0; o0 < O; o0 += groups) {
                const int o = min(o0 + tid / P, O - 1);  // lanes past the end repeat the last group, unstored
                const int b = o / ncg, c0 = (o % ncg) * CB;
                float v[CB];
                if (i8) {
                    int acc[CB] = {};
                    const int* hw = hqw + b * hwp;
                    for (int w = gl; w < up / 4; w += P) {
                        const int hv = hw[w];
#pragma unroll
                        for (int c = 0; c < CB; ++c) acc[c] = __builtin_amdgcn_sdot4(hv, usw[(c0 + c) * upp + w], acc[c], false);
                    }
#pragma unroll
                    for (int c = 0; c < CB; ++c) {
                        for (int off = P / 2; off > 0; off >>= 1) acc[c] += __shfl_xor(acc[c], off, 64);
                        v[c] = (float)acc[c] * sxs[b];  // ((float)acc · sx) · scale, the int8 GEMM's epilogue
                    }
                } else {
#pragma unroll
                    for (int c = 0; c < CB; ++c) v[c] = 0.0f;
                    const float* hr = hs + b * hp;
                    for (int k = gl; k < u; k += P) {
                        const float hv = hr[k];
#pragma unroll
                        for (int c = 0; c < CB; ++c) v[c] = fmaf(hv, usf[(c0 + c) * upp + k], v[c]);
                    }
#pragma unroll
                    for (int c = 0; c < CB; ++c)
                        for (int off = P / 2; off > 0; off >>= 1) v[c] += __shfl_xor(v[c], off, 64);
                }
                if (gl == 0 && o0 + tid / P < O) {
#pragma unroll
                    for (int c = 0; c < CB; ++c) {
                        const int cc = c0 + c;
                        if (cc >= NC) break;
                        const int col = column(cc);
                        float x = v[c];
                        if (i8) x = x * a.qs[col];
                        if (a.brec) x = x + a.brec[col];
                        r[b * NCM + cc] = x;
                    }
                }
            }
            __syncthreads();
        }
        // the cells
#pragma unroll
        for (int i = 0; i < kMaxPairs; ++i) {
            const int pr = tid + kThreads * i;
            if (pr >= npairs) continue;
            const int b = pr / nwu, jj = pr % nwu, j = j0 + jj;
            const bool first = step == 0;
            auto rec = [&](int g) { return r[b * NCM + g * nwu + jj]; };
            float hv;
            if (a.kind == 4) {  // LSTM: i, f, g, o
                float zi = zv[i][0], zf = zv[i][1], zg = zv[i][2], zo = zv[i][3];
                if (!first) { zi = zi + rec(0); zf = zf + rec(1); zg = zg + rec(2); zo = zo + rec(3); }
                hv = knx_lstm_cell(zi, zf, zg, zo, a.act, a.alpha, first, cst[i]);
            } else if (a.kind == 5) {  // GRU: z, r, h~; at the first step (h = 0) the recurrent term is its bias
                const float hz = first ? a.brec[j] : rec(0);
                const float hr = first ? a.brec[u + j] : rec(1);
                const float hh = first ? a.brec[2 * u + j] : rec(2);
                const float prev = first ? 0.0f : hs[b * hp + j];
                hv = knx_gru_cell(zv[i][0], zv[i][1], zv[i][2], hz, hr, hh, a.act, a.alpha, first, prev);
            } else {
                float v = zv[i][0];
                if (!first) v = v + rec(0);
                hv = knx_act(v, a.act, a.alpha);
            }
            if (step + 1 < T) __hip_atomic_store(hout + (size_t)b * u + j, hv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (a.ret_seq) a.dst[((size_t)b * T + t) * a.stride + j] = hv;
            else if (step + 1 == T) a.dst[(size_t)b * a.stride + j] = hv;
        }
        if (step + 1 < T) knx::grid_barrier(a.gs, 0);  // also: every thread is done with hs and r of this step
    }
}

// ---- one workgroup for the whole recurrence (B ≤ 2: batch 1, and the reference's int8 dispatch at ≤ 2 rows) ----
// With a few rows the per-timestep work is tiny and the cost of a multi-workgroup step is its round trips through
// memory (h stores, the barrier, h reloads).  One workgroup of 1024 threads keeps all of U in registers — thread t owns
// column c = t / KS and its k-slice [s·KSL, (s+1)·KSL), s = t % KS, KS lanes per column (consecutive lanes, so their
// partial sums are reduced by exchanges; the lanes of one slice read the same h values, 16 bytes at a time) — and h in
// LDS, so a timestep is two workgroup barriers and no global synchronization.  Same quantizer, int32 sums, epilogue
// and cells as above.
constexpr int kSoloThreads = 1024;
constexpr int kSoloRegs = 64;   // U values per thread (fp32; int8: kSoloRegs / 2 words of four values)
constexpr int kSoloRows = 2;

template <bool I8>
__global__ void __launch_bounds__(kSoloThreads) rnn_solo(RnnArgs a, int KS)
{
    __shared__ __attribute__((aligned(16))) float hs[kSoloRows][2048];  // h_{t−1}, fp32 (u ≤ 2048), zero past u
    __shared__ __attribute__((aligned(16))) int hq[kSoloRows][512];     // its int8 rows, four to a word
    __shared__ float sxs[kSoloRows];
    __shared__ float r[kSoloRows][kSoloThreads];                        // recurrent terms (gates·u ≤ 1024)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int B = a.B, T = a.T, u = a.u, gu = a.gu, G = a.gates, uw4 = (u + 3) / 4;
    const int c = tid / KS, ks = tid % KS;
    const bool active = c < gu;
    const int cc = active ? c : gu - 1;
    constexpr int REGS = I8 ? kSoloRegs / 2 : kSoloRegs;
    const int k0 = ks * REGS;  // first k (fp32) or word (int8) of this lane's slice
    // this thread's part of U; h is zero past u, so the slice runs over whole 16-byte groups
    for (int e = tid; e < kSoloRows * 2048; e += kSoloThreads) (&hs[0][0])[e] = 0.0f;
    for (int e = tid; e < kSoloRows * 512; e += kSoloThreads) (&hq[0][0])[e] = 0;
    float uf[I8 ? 4 : REGS];
    int uq[I8 ? REGS : 4];
#pragma unroll
    for (int i = 0; i < REGS; ++i) {
        if (I8) {
            const int w = k0 + i;
            unsigned v = 0;
            if (w < uw4) {
                const int8_t* src = a.q + (size_t)cc * a.kp + 4 * w;
#pragma unroll
                for (int e = 0; e < 4; ++e) v |= (unsigned)(uint8_t)(4 * w + e < u ? src[e] : 0) << (8 * e);
            }
            uq[i] = (int)v;
        } else {
            const int k = k0 + i;
            uf[i] = k < u ? (a.u_nt ? a.U[(size_t)cc * u + k] : a.U[(size_t)k * gu + cc]) : 0.0f;
        }
    }
    __syncthreads();
    const float col_scale = I8 ? a.qs[cc] : 1.0f;
    const float col_bias = a.brec ? a.brec[cc] : 0.0f;
    // cell phase: thread tid < B·u owns row b = tid / u, unit j = tid % u
    const bool cell = tid < B * u;
    const int cb = cell ? tid / u : 0, cj = cell ? tid % u : 0;
    float cst = 0.0f;
    int qlpr = 1;
    while (qlpr < 64 && qlpr * 8 < u) qlpr *= 2;
    // the input-side gate values of this thread's cell, one timestep ahead (they do not depend on h)
    auto load_z = [&](int st, float (&z)[4]) {
        const int tt = a.dir ? T - 1 - st : st;
#pragma unroll
        for (int g = 0; g < 4; ++g) z[g] = cell && g < G ? a.zx[((size_t)cb * T + tt) * gu + (size_t)g * u + cj] : 0.0f;
    };
    float zn[4];
    load_z(0, zn);
    for (int step = 0; step < T; ++step) {
        const int t = a.dir ? T - 1 - step : step;
        float zv[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) zv[g] = zn[g];
        if (step + 1 < T) load_z(step + 1, zn);
        if (step > 0) {
            if (I8) {
                const int rl = lane % qlpr, b = wave * (64 / qlpr) + lane / qlpr;
                if (wave * (64 / qlpr) < B) {  // the waves that hold a row (uniform over the wave)
                    const int bb = min(b, B - 1);
                    float mx = 0.0f;
                    for (int k = rl; k < u; k += qlpr) mx = fmaxf(mx, mag(hs[bb][k]));
                    for (int off = qlpr / 2; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
                    if (b < B) {
                        const bool bad = !(mx <= FLT_MAX);
                        const float sc = (!bad && mx > 0.0f) ? __fdiv_rn(mx, 127.0f) : 1.0f;
                        const float inv = __fdiv_rn(1.0f, sc);
                        if (rl == 0) sxs[b] = bad ? __int_as_float(0x7fc00000) : sc;
                        for (int w = rl; w < uw4; w += qlpr) {
                            unsigned pk = 0;
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const int k = 4 * w + e;
                                const float v = k < u && !bad ? __builtin_amdgcn_fmed3f(rintf(hs[b][k] * inv), -127.0f, 127.0f) : 0.0f;
                                pk |= (unsigned)(uint8_t)(int8_t)(int)v << (8 * e);
                            }
                            hq[b][w] = (int)pk;
                        }
                    }
                }
                __syncthreads();
            }
            for (int b = 0; b < B; ++b) {
                float v;
                if (I8) {
                    int acc = 0;
                    const int4* hrow = reinterpret_cast<const int4*>(&hq[b][k0]);
#pragma unroll
                    for (int i = 0; i < REGS / 4; ++i) {
                        if (k0 + 4 * i >= uw4) break;  // past u: zero words
                        const int4 hv = hrow[i];
                        acc = __builtin_amdgcn_sdot4(hv.x, uq[4 * i], acc, false);
                        acc = __builtin_amdgcn_sdot4(hv.y, uq[4 * i + 1], acc, false);
                        acc = __builtin_amdgcn_sdot4(hv.z, uq[4 * i + 2], acc, false);
                        acc = __builtin_amdgcn_sdot4(hv.w, uq[4 * i + 3], acc, false);
                    }
                    for (int off = KS / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
                    v = (float)acc * sxs[b];  // ((float)acc · sx) · scale (+ bias), the int8 GEMM's epilogue
                    v = v * col_scale;
                } else {
                    v = 0.0f;
                    const float4* hrow = reinterpret_cast<const float4*>(&hs[b][k0]);
#pragma unroll
                    for (int i = 0; i < REGS / 4; ++i) {
                        if (k0 + 4 * i >= u) break;  // past u: zeros
                        const float4 hv = hrow[i];
                        v = fmaf(hv.x, uf[4 * i], v);
                        v = fmaf(hv.y, uf[4 * i + 1], v);
                        v = fmaf(hv.z, uf[4 * i + 2], v);
                        v = fmaf(hv.w, uf[4 * i + 3], v);
                    }
                    for (int off = KS / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
                }
                if (a.brec) v = v + col_bias;
                if (active && ks == 0) r[b][c] = v;
            }
        }
        __syncthreads();  // r complete; every read of hs done
        if (cell) {
            const bool first = step == 0;
            auto rec = [&](int g) { return r[cb][g * u + cj]; };
            float hv;
            if (a.kind == 4) {
                float zi = zv[0], zf = zv[1], zg = zv[2], zo = zv[3];
                if (!first) { zi = zi + rec(0); zf = zf + rec(1); zg = zg + rec(2); zo = zo + rec(3); }
                hv = knx_lstm_cell(zi, zf, zg, zo, a.act, a.alpha, first, cst);
            } else if (a.kind == 5) {
                const float hz = first ? a.brec[cj] : rec(0);
                const float hr = first ? a.brec[u + cj] : rec(1);
                const float hh = first ? a.brec[2 * u + cj] : rec(2);
                hv = knx_gru_cell(zv[0], zv[1], zv[2], hz, hr, hh, a.act, a.alpha, first, first ? 0.0f : hs[cb][cj]);
            } else {
                float v = zv[0];
                if (!first) v = v + rec(0);
                hv = knx_act(v, a.act, a.alpha);
            }
            hs[cb][cj] = hv;
            if (a.ret_seq) a.dst[((size_t)cb * T + t) * a.stride + cj] = hv;
            else if (step + 1 == T) a.dst[(size_t)cb * a.stride + cj] = hv;
        }
        __syncthreads();  // h_t complete in LDS
    }
}

// lanes per column of the single-workgroup kernel: the most (a power of two ≤ 64) that the 1024 threads hold, if
// each lane's slice of its column then fits the registers; else 0 (no single-workgroup kernel for the shape)
int solo_lanes(int B, int gu, int u, bool i8)
{
    if (B > kSoloRows || (long)B * u > kSoloThreads || u > 2048 || gu > kSoloThreads) return 0;
    const char* e = getenv("KNX_RNN_SOLO");  // 0: the multi-workgroup kernel for every shape (tests, tuning)
    if (e != nullptr && *e == '0') return 0;
    int ks = 1;
    while (ks < 64 && (long)gu * ks * 2 <= kSoloThreads) ks *= 2;
    const int len = i8 ? (u + 3) / 4 : u;
    return len <= ks * (i8 ? kSoloRegs / 2 : kSoloRegs) ? ks : 0;  // lane s covers [s·R, (s+1)·R)
}

// units per workgroup: the grid's workgroups each take ⌈u / G⌉ units, G as large as the barrier allows while each
// workgroup still has at least one unit and its (row, unit) pairs fit the threads
int units_per_wg(int B, int u)
{
    int uw = (u + kMaxGrid - 1) / kMaxGrid;
    if (const char* e = getenv("KNX_RNN_UNITS")) {  // tuning: units per workgroup
        const int v = atoi(e);
        if (v >= 1) uw = std::max(uw, v);
    }
    while (B * uw > kThreads * kMaxPairs && uw > 1) --uw;  // cannot happen for B ≤ 64 (uw ≤ 8 then)
    return uw;
}

}  // namespace

extern "C" int knx_hip_rnn_recurrence_fits(int kind, int B, int u, int i8)
{
    if ((kind != 4 && kind != 5 && kind != 6) || B < 1 || B > 64 || u < 1 || u > 65536) return 0;
    const int gates = kind == 4 ? 4 : kind == 5 ? 3 : 1;
    if (solo_lanes(B, gates * u, u, i8 != 0) > 0) return 1;
    const int uw = units_per_wg(B, u);
    if ((u + uw - 1) / uw > kMaxGrid || B * uw > kThreads * kMaxPairs) return 0;
    const int up = (u + 3) / 4 * 4;
    return lds_layout(B, gates, uw, up, i8 != 0).total <= kMaxLds ? 1 : 0;
}

extern "C" int knx_hip_rnn_recurrence(int kind, int act, float alpha, int B, int T, int u, int dir, const float* zx,
                                      const float* U, int u_nt, const int8_t* q, int kp, const float* qscale,
                                      const float* brec, float* h0, float* h1, float* dst, int stride, int ret_seq,
                                      void* scratch, size_t scratch_bytes, int* status, void* stream)
{
    const char* name = "knx_hip_rnn_recurrence";
    KNX_ENTRY(name);
    KNX_REQUIRE(T >= 1 && act >= -1 && act <= 15 && (dir == 0 || dir == 1), name);
    KNX_REQUIRE(knx_hip_rnn_recurrence_fits(kind, B, u, q != nullptr), name);
    const int gates = kind == 4 ? 4 : kind == 5 ? 3 : 1;
    KNX_REQUIRE(zx != nullptr && h0 != nullptr && h1 != nullptr && dst != nullptr && stride >= u, name);
    KNX_REQUIRE(kind != 5 || brec != nullptr, name);
    KNX_REQUIRE(q != nullptr ? (qscale != nullptr && kp >= (u + 3) / 4 * 4 && ((uintptr_t)q & 3) == 0 && kp % 4 == 0)
                             : U != nullptr, name);
    KNX_REQUIRE(scratch != nullptr && ((uintptr_t)scratch & 255) == 0 && scratch_bytes >= 8, name);
    KNX_REQUIRE(status != nullptr && ((uintptr_t)status & 3) == 0, name);
    RnnArgs a{};
    a.kind = kind; a.act = act; a.alpha = alpha;
    a.B = B; a.T = T; a.u = u; a.gu = gates * u; a.gates = gates; a.dir = dir; a.ret_seq = ret_seq != 0;
    a.stride = stride; a.uw = units_per_wg(B, u); a.up = (u + 3) / 4 * 4;
    a.zx = zx; a.U = U; a.u_nt = u_nt != 0; a.q = q; a.kp = kp; a.qs = qscale; a.brec = brec;
    a.h0 = h0; a.h1 = h1; a.dst = dst;
    a.gs = knx::GridSync{static_cast<unsigned long long*>(scratch), status, knx::grid_spin_limit()};
    const int ks = solo_lanes(B, a.gu, u, q != nullptr);
    if (ks > 0) {
        if (q != nullptr) hipLaunchKernelGGL(rnn_solo<true>, dim3(1), dim3(kSoloThreads), 0, knx::as_stream(stream), a, ks);
        else hipLaunchKernelGGL(rnn_solo<false>, dim3(1), dim3(kSoloThreads), 0, knx::as_stream(stream), a, ks);
        return knx::check_launch(name);
    }
    const int G = (u + a.uw - 1) / a.uw;
    const size_t lds = lds_layout(B, gates, a.uw, a.up, q != nullptr).total;
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] {
        attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&rnn_recurrence),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds);
    });
    if (attr != hipSuccess) return knx::fail(KNX_EHIP, "%s: %s", name, hipGetErrorString(attr));
    hipLaunchKernelGGL(rnn_recurrence, dim3((unsigned)G), dim3(kThreads), lds, knx::as_stream(stream), a);
    return knx::check_launch(name);
}
