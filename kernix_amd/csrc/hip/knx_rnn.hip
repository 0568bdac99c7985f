// knx_rnn.hip — the recurrence of one RNN direction (LSTM, GRU, simple RNN) as one launch.
//
// Reference include/kernix_model.h:563-632 (kernix_rnn_dir): the input projection x·W + b of every timestep is one
// GEMM (done before this kernel, zx); then for t in order (reversed for the backward direction) the recurrent term
// h_{t−1}·U is added and the cell applied, int8 (kernix_qmatmul on the B rows of h) or fp32.  Run as a launch per
// timestep for the product and another for the cell, a small batch is all launch latency; here one grid does every
// timestep: workgroup w owns units [w·uw, (w+1)·uw), keeps the U columns of those units' gates in LDS for the whole
// sequence and its cells' c in registers, and per timestep
//   1. loads h_{t−1} (all B rows, written by every workgroup at t−1) into LDS, a row's float4s over a group of
//      lanes — int8: quantizes each row from those registers with the quantizer's operations (s = max|h|/127, 1 for
//      an all-zero row, NaN for a row holding NaN or ±inf; q = clamp(rint(h·(1/s)), ±127)), as
//      knx_hip_quantize_rows;
//   2. forms its gate columns of h_{t−1}·U on the matrix cores in 16 × 16 tiles: v_mfma_f32_16x16x4f32, or exact
//      int32 sums from v_mfma_i32_16x16x64_i8 dequantized as the int8 GEMM's epilogue, ((float)acc·s)·scale (+ the
//      GRU's recurrent bias);
//   3. applies the cells (knx_lstm_cell / knx_gru_cell, the same functions as knx_hip_rnn_gates) to its (row, unit)
//      pairs, writes h_t (at device scope, for the other workgroups) and the output;
//   4. waits at a grid barrier (knx_grid.hpp: one 64-bit word, every barrier adds 256; at most 64 workgroups, all
//      resident).
// Where one workgroup can hold all of U (rnn_solo, below) the batch is split over workgroups instead, each running
// its rows' timesteps alone: the rows of a recurrence never meet, so nothing is exchanged and nothing synchronizes
// across workgroups.
// The int8 results are the bits of the per-timestep path (same quantizer, exact int32 sums, same epilogue and cell
// order); fp32 sums run in this kernel's own order.
#include <float.h>
#include <math.h>
#include <algorithm>

#include "knx_common.hpp"
#include "knx_grid.hpp"
#include "knx_pipe.hpp"

namespace {

constexpr int kThreads = 256, kWaves = 4;
constexpr int kMaxPairs = 2;             // (row, unit) pairs per thread in the cell phase: B·uw ≤ 512
constexpr int kMaxGrid = 64;
constexpr int kLoads = 8;                // float4 loads of h in flight per thread
constexpr int kMaxUnits = 2048;          // the multi-workgroup kernel: a row of h is at most kLoads float4s per lane
constexpr size_t kMaxLds = 120 * 1024;

typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));

struct RnnArgs {
    int kind, act;
    float alpha;
    int B, T, u, gu, gates, dir, ret_seq, stride, uw, up, ldh;
    const float* zx;      // B·T × gu (row b·T + t), the input projection with its bias
    const float* U;       // fp32 recurrent weight: u × gu (u_nt = 0) or gu × u (u_nt = 1)
    int u_nt;
    const int8_t* q;      // int8 recurrent weight: gu rows of kp bytes (k contiguous), or null
    int kp;
    const float* qs;      // its gu scales
    const float* brec;    // GRU recurrent bias (gu), or null
    float* h0;            // hidden states of even / odd timesteps (B rows of ldh floats each)
    float* h1;
    float* dst;
    knx::GridSync gs;
    // the row-split kernel only: the LINEAR step that reads only the last state, at the end of the same launch
    // (dn > 0): y = act(h_T·Wᵀ + b) over dn outputs, int8 (dq: dn rows of dkp bytes, dqs their scales) or fp32 (dw:
    // dn rows of u floats); dy: B rows of dn
    const float* dw;
    const int8_t* dq;
    const float* dqs;
    const float* db;
    int dn, dkp, dact;
    float dalpha;
    float* dy;
};

__host__ __device__ inline size_t round16(size_t b) { return (b + 15) / 16 * 16; }

// Row pitch (4-byte words) of the LDS matrices that the MFMAs read: ≥ n and ≡ 4 (mod 32), so that the rows that 8
// consecutive lanes read 16 bytes of at the same k start 4 banks apart.
__host__ __device__ inline int mfma_pitch(int n) { return (n + 31) / 32 * 32 + 4; }

// k extent of the products: fp32 in 16-wide chunks (four v_mfma_f32_16x16x4f32, lane quarter q taking k = 4q…4q+3 of
// each chunk), int8 in 64-wide chunks (one v_mfma_i32_16x16x64_i8, lane quarter q taking bytes 16q…16q+15); h and U
// are zero past u
__host__ __device__ inline int k_extent(int u, bool i8) { return i8 ? (u + 63) / 64 * 64 : (u + 15) / 16 * 16; }

// LDS layout (bytes): weight slice [ncp][upp] (fp32 values or int8 words, k contiguous), column scales and biases
// [ncp] each, h_{t−1} [b16][hp] fp32 (not for the int8 LSTM / RNN, whose cells do not read it), its int8 rows
// [b16][hwp] words and their scales [b16] (int8), the K-split partial tiles [kWaves][256], recurrent terms
// [B][gates·uw].  ncp: the workgroup's gate columns rounded up to 16, b16: B rounded up to 16 (zero columns and rows).
struct Lds {
    size_t us, cs, hs, hq, sx, pt, r, total;
    int upp, hp, hwp, ncp, b16;
};
__host__ __device__ inline Lds lds_layout(int B, int gates, int uw, int up, bool i8, bool h32)
{
    Lds l;
    l.ncp = (gates * uw + 15) / 16 * 16;
    l.b16 = (B + 15) / 16 * 16;
    l.upp = mfma_pitch(i8 ? up / 4 : up);
    l.hp = mfma_pitch(up);
    l.hwp = mfma_pitch(up / 4);
    l.us = 0;
    l.cs = round16((size_t)l.ncp * l.upp * 4);
    l.hs = l.cs + round16((size_t)l.ncp * 2 * 4);
    l.hq = l.hs + (h32 ? round16((size_t)l.b16 * l.hp * 4) : 0);
    l.sx = l.hq + (i8 ? round16((size_t)l.b16 * l.hwp * 4) : 0);
    l.pt = l.sx + (i8 ? round16((size_t)l.b16 * 4) : 0);
    l.r = l.pt + (size_t)kWaves * 256 * 4;
    l.total = l.r + round16((size_t)B * gates * uw * 4);
    return l;
}

// The kernels are instantiated per cell kind (KIND 4 LSTM, 5 GRU, 6 simple RNN) and for the tanh activation (ACT 4,
// the recurrent layers' default) or any (kActAny: the activation read from the arguments): with the cell's branches
// and the activation's switch resolved at compile time a timestep's cells took 0.46 against 0.70 µs.
constexpr int kActAny = -100;

template <bool I8, int KIND, int ACT>
__global__ void __launch_bounds__(kThreads) rnn_recurrence(RnnArgs a)
{
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    constexpr bool i8 = I8;  // a.q != nullptr
    constexpr bool h32 = !i8 || KIND == 5;
    const int act = ACT == kActAny ? a.act : ACT;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);  // the same value, known to the compiler as uniform
    const int B = a.B, T = a.T, u = a.u, up = a.up, gu = a.gu, G = a.gates, ldh = a.ldh;
    const int j0 = blockIdx.x * a.uw;
    const int nwu = min(a.uw, u - j0);  // ≥ 1: the grid has ⌈u / uw⌉ workgroups
    const int NC = G * nwu, NCM = G * a.uw;
    const Lds L = lds_layout(B, G, a.uw, up, i8, h32);
    const int upp = L.upp, hp = L.hp, hwp = L.hwp, ncp = L.ncp;
    float* usf = reinterpret_cast<float*>(smem + L.us);
    int* usw = reinterpret_cast<int*>(smem + L.us);
    float* csc = reinterpret_cast<float*>(smem + L.cs);  // per local column: int8 scale, recurrent bias
    float* cbi = csc + ncp;
    float* hs = reinterpret_cast<float*>(smem + L.hs);
    int* hqw = reinterpret_cast<int*>(smem + L.hq);
    float* sxs = reinterpret_cast<float*>(smem + L.sx);
    int* pt = reinterpret_cast<int*>(smem + L.pt);
    float* r = reinterpret_cast<float*>(smem + L.r);
    auto column = [&](int cc) { return (cc / nwu) * u + j0 + cc % nwu; };  // gate column of local column cc

    // h rows (and the rows past B, k past u, which stay zero) cleared; the weight slice, once: local column
    // cc = g·nwu + jj is gate g of unit j0 + jj; k ≥ u and columns ≥ NC are zero
    for (size_t e = tid; e < (L.pt - L.hs) / 4; e += kThreads) reinterpret_cast<int*>(smem + L.hs)[e] = 0;
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
    for (int cc = tid; cc < ncp; cc += kThreads) {
        const int col = cc < NC ? column(cc) : 0;
        csc[cc] = i8 && cc < NC ? a.qs[col] : 1.0f;
        cbi[cc] = a.brec && cc < NC ? a.brec[col] : 0.0f;
    }
    // this thread's (row, unit) pairs of the cell phase and their per-column constants
    const int npairs = B * nwu;
    float cst[kMaxPairs];
    for (int i = 0; i < kMaxPairs; ++i) cst[i] = 0.0f;

    // loading h_{t−1}: a row is W4 float4s over LR lanes (a power of two: as many as keep every row within one pass
    // of the four waves, at least enough for kLoads float4s per lane to cover the row, at most one per float4), RPW
    // rows per wave-wide load; lane (rsub, lr) of row group g takes row g·RPW + rsub, float4s lr + LR·s, s < NWL
    const int W4 = (u + 3) / 4;
    int LR = 1;
    while (LR < 64 && LR < W4 && (LR * kLoads < W4 || 2 * LR * B <= kThreads)) LR *= 2;
    const int RPW = 64 / LR, NWL = (W4 + LR - 1) / LR, ngr = (B + RPW - 1) / RPW;
    const int lr = lane % LR, rsub = lane / LR;

    // products: RB × NCT output tiles of 16 × 16 (rows of h × local columns); with fewer tiles than waves the k
    // chunks of a tile are split over kparts waves, whose partial tiles are summed in LDS in wave order
    const int RB = L.b16 / 16, NCT = ncp / 16, tiles = RB * NCT;
    const int kparts = tiles >= kWaves ? 1 : tiles == 1 ? kWaves : tiles == 2 ? 2 : 1;
    const int part = wave % kparts, fr = lane & 15, fq = lane >> 4;
    const int nkc = i8 ? up / 64 : up / 16;

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
    // the recurrent term of row b, local column cc from its product (fp32 sum, or int32 sum dequantized as the int8
    // GEMM's epilogue ((float)acc · sx) · scale), plus the GRU's recurrent bias
    auto put = [&](int b, int cc, int bits) {
        float x = i8 ? (float)bits * sxs[b] * csc[cc] : __int_as_float(bits);
        if (a.brec) x = x + cbi[cc];
        r[b * NCM + cc] = x;
    };
    __syncthreads();
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
            // h_{t−1} into LDS, a batch of up to kLoads float4s per lane issued before the first is used; int8: each
            // row quantized from the registers (s = max|h|/127, 1 for an all-zero row, NaN for a row holding NaN or
            // ±inf; q = clamp(rint(h·(1/s)), ±127), four to a word; the bytes of a row that cannot be quantized do
            // not matter: its products are NaN through its scale)
            for (int g = wave_u; g < ngr; g += kWaves) {
                const int b = g * RPW + rsub;
                float4 v[kLoads];
                bool ok[kLoads];
#pragma unroll
                for (int s = 0; s < kLoads; ++s) {
                    const int w = lr + LR * s;
                    ok[s] = s < NWL && b < B && w < W4;
                    v[s] = ok[s] ? *reinterpret_cast<const float4*>(hin + (size_t)b * ldh + 4 * w)
                                 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                }
#pragma unroll
                for (int s = 0; s < kLoads; ++s) {
                    if (s >= NWL) break;
                    const int w = lr + LR * s;
                    if (4 * w + 4 > u) {  // the float4 reaching past u: the row padding is not h
                        if (4 * w + 1 >= u) v[s].y = 0.0f;
                        if (4 * w + 2 >= u) v[s].z = 0.0f;
                        v[s].w = 0.0f;
                    }
                    if (h32 && ok[s]) *reinterpret_cast<float4*>(hs + b * hp + 4 * w) = v[s];
                }
                if (i8) {
                    // the row's max |h| as bits (NaN above +inf above every finite value) over its LR lanes, the
                    // quantizer's scale (max/127, 1 for an all-zero row, NaN for a row holding NaN or ±inf) and
                    // q = clamp(rint(h·(1/s)), ±127), four to a word; + 128 is an exact integer that converts
                    // exactly to a byte; the bytes of a row that cannot be quantized do not matter: its products are
                    // NaN through its scale
                    unsigned m = 0;
#pragma unroll
                    for (int s = 0; s < kLoads; ++s) {
                        if (s >= NWL) break;
                        const unsigned x = __float_as_uint(v[s].x) & 0x7fffffffu, y = __float_as_uint(v[s].y) & 0x7fffffffu;
                        const unsigned z = __float_as_uint(v[s].z) & 0x7fffffffu, w = __float_as_uint(v[s].w) & 0x7fffffffu;
                        m = max(m, max(max(x, y), max(z, w)));
                    }
                    m = knx_lane_group_max(m, LR);
                    const bool bad = m >= 0x7f800000u;
                    const float mx = __uint_as_float(m);
                    const float sc = (!bad && mx > 0.0f) ? __fdiv_rn(mx, 127.0f) : 1.0f;
                    const float inv = bad ? 0.0f : __fdiv_rn(1.0f, sc);
                    if (lr == 0 && b < B) sxs[b] = bad ? __int_as_float(0x7fc00000) : sc;
#pragma unroll
                    for (int s = 0; s < kLoads; ++s) {
                        if (s >= NWL) break;
                        if (!ok[s]) continue;
                        unsigned pk = 0;
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            pk = __builtin_amdgcn_cvt_pk_u8_f32(
                                __builtin_amdgcn_fmed3f(rintf((&v[s].x)[e] * inv), -127.0f, 127.0f) + 128.0f, e, pk);
                        hqw[b * hwp + lr + LR * s] = (int)(pk ^ 0x80808080u);
                    }
                }
            }
            __syncthreads();
            // the recurrent terms of this workgroup's columns on the matrix cores: tile (rt, ct), lane (fr, fq) holds
            // rows 16·rt + 4·fq + e, e < 4, of local column 16·ct + fr
            for (int ti = wave / kparts; ti < tiles; ti += kWaves / kparts) {
                const int rt = ti % RB, ct = ti / RB;
                v4i acc = {0, 0, 0, 0};
                if (i8) {
                    const int* ar = hqw + (16 * rt + fr) * hwp + 4 * fq;
                    const int* br = usw + (16 * ct + fr) * upp + 4 * fq;
                    for (int kc = part; kc < nkc; kc += 2 * kparts) {
                        const bool two = kc + kparts < nkc;
                        const v4i a0 = *reinterpret_cast<const v4i*>(ar + 16 * kc);
                        const v4i b0 = *reinterpret_cast<const v4i*>(br + 16 * kc);
                        const v4i a1 = two ? *reinterpret_cast<const v4i*>(ar + 16 * (kc + kparts)) : v4i{0, 0, 0, 0};
                        const v4i b1 = two ? *reinterpret_cast<const v4i*>(br + 16 * (kc + kparts)) : v4i{0, 0, 0, 0};
                        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, acc, 0, 0, 0);
                    }
                } else {
                    v4f f = {0.0f, 0.0f, 0.0f, 0.0f};
                    const float* ar = hs + (16 * rt + fr) * hp + 4 * fq;
                    const float* br = usf + (16 * ct + fr) * upp + 4 * fq;
                    for (int kc = part; kc < nkc; kc += 4 * kparts) {
                        float4 av[4], bv[4];
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int kk = kc + i * kparts;
                            const bool in = kk < nkc;
                            av[i] = in ? *reinterpret_cast<const float4*>(ar + 16 * kk) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                            bv[i] = in ? *reinterpret_cast<const float4*>(br + 16 * kk) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                        }
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            f = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i].x, bv[i].x, f, 0, 0, 0);
                            f = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i].y, bv[i].y, f, 0, 0, 0);
                            f = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i].z, bv[i].z, f, 0, 0, 0);
                            f = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i].w, bv[i].w, f, 0, 0, 0);
                        }
                    }
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[e] = __float_as_int(f[e]);
                }
                if (kparts == 1) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int b = 16 * rt + 4 * fq + e, cc = 16 * ct + fr;
                        if (b < B && cc < NC) put(b, cc, acc[e]);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) pt[wave * 256 + (4 * fq + e) * 16 + fr] = acc[e];
                }
            }
            if (kparts > 1) {  // the partial tiles of tile ti are those of waves ti·kparts … ti·kparts + kparts − 1
                __syncthreads();
                for (int e = tid; e < tiles * 256; e += kThreads) {
                    const int ti = e / 256, i = e % 256;
                    const int b = 16 * (ti % RB) + i / 16, cc = 16 * (ti / RB) + i % 16;
                    if (b >= B || cc >= NC) continue;
                    const int* p = pt + ti * kparts * 256 + i;
                    int bits;
                    if (i8) {
                        int s = 0;
                        for (int w = 0; w < kparts; ++w) s += p[256 * w];
                        bits = s;
                    } else {
                        float s = __int_as_float(p[0]);
                        for (int w = 1; w < kparts; ++w) s = s + __int_as_float(p[256 * w]);
                        bits = __float_as_int(s);
                    }
                    put(b, cc, bits);
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
            if (KIND == 4) {  // LSTM: i, f, g, o
                float zi = zv[i][0], zf = zv[i][1], zg = zv[i][2], zo = zv[i][3];
                if (!first) { zi = zi + rec(0); zf = zf + rec(1); zg = zg + rec(2); zo = zo + rec(3); }
                hv = knx_lstm_cell(zi, zf, zg, zo, act, a.alpha, first, cst[i]);
            } else if (KIND == 5) {  // GRU: z, r, h~; at the first step (h = 0) the recurrent term is its bias
                const float hz = first ? a.brec[j] : rec(0);
                const float hr = first ? a.brec[u + j] : rec(1);
                const float hh = first ? a.brec[2 * u + j] : rec(2);
                const float prev = first ? 0.0f : hs[b * hp + j];
                hv = knx_gru_cell(zv[i][0], zv[i][1], zv[i][2], hz, hr, hh, act, a.alpha, first, prev);
            } else {
                float v = zv[i][0];
                if (!first) v = v + rec(0);
                hv = knx_gate_act(v, act, a.alpha);
            }
            if (step + 1 < T) __hip_atomic_store(hout + (size_t)b * ldh + j, hv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (a.ret_seq) a.dst[((size_t)b * T + t) * a.stride + j] = hv;
            else if (step + 1 == T) a.dst[(size_t)b * a.stride + j] = hv;
        }
        if (step + 1 < T) knx::grid_barrier(a.gs, 0);  // also: every thread is done with hs and r of this step
    }
}

// Barrier for the LDS hand-offs of a timestep (h, its int8 rows, the recurrent terms, the row maxima): this wave's LDS
// accesses retired, then s_barrier.  __syncthreads would also wait for the wave's global stores (the output h) and
// loads (the next timestep's gate inputs), which no other wave reads.
__device__ __forceinline__ void lds_barrier()
{
    KNX_WAIT_LDS();
    knx_barrier_nofence();
}

// ---- the batch split over workgroups, each running the whole recurrence of its rows ----
// The rows of a recurrence never meet (h, its int8 row scale and the cells are per row), so a workgroup that holds all
// of U runs its rows' timesteps alone: no h exchange through memory and no barrier across workgroups, whose round trips
// are the cost of a multi-workgroup step at these sizes, and no workgroup waits for another (nothing needs to be
// resident together).  One workgroup of 1024 threads keeps all of U in registers and h in LDS, so a timestep is two
// workgroup barriers and no global synchronization.  fp32: thread t owns column
// c = t / KS and its 64-value k-slice s = t % KS, KS lanes per column (consecutive lanes, so their partial sums are
// reduced by exchanges; the lanes of one slice read the same h values, 16 bytes at a time), FMAs on the VALU.  int8:
// the products on the matrix cores, the rows of h as the rows of A of v_mfma_i32_16x16x64_i8 (one or two of its 16:
// at u = 128 a wave still needs only four per timestep, against 32 dot4 instructions per lane and the reduction).  Same
// quantizer, int32 sums, epilogue and cells as above; with int8 arithmetic one wave holds a row's cells (two units per
// lane), takes the row maximum of h_t by lane exchanges and quantizes the row right after the cells.
constexpr int kSoloThreads = 1024;
constexpr int kSoloRegs = 64;   // fp32: U values per thread
constexpr int kSoloRows = 2;
constexpr int kSoloBlocks = 2;  // int8: 16-column blocks per wave (gates·u ≤ 512)
constexpr int kSoloChunks = 2;  // int8: 64-byte k-chunks (u ≤ 128); 4 × 4 fragments spilled registers

template <bool I8, int KIND, int ACT>
__global__ void __launch_bounds__(kSoloThreads) rnn_solo(RnnArgs a, int KS, int R)
{
    const int act = ACT == kActAny ? a.act : ACT;
    __shared__ __attribute__((aligned(16))) float hs[kSoloRows][2048];  // h_{t−1}, fp32 (u ≤ 2048), zero past u
    __shared__ __attribute__((aligned(16))) int hq[kSoloRows][512];     // its int8 rows, four to a word
    __shared__ float sxs[kSoloRows];
    __shared__ float r[kSoloRows][kSoloThreads];                        // recurrent terms (gates·u ≤ 1024)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // this workgroup's rows of the batch: [row0, row0 + B) (the rows of a recurrence never meet)
    const int row0 = blockIdx.x * R;
    const int B = min(R, a.B - row0), T = a.T, u = a.u, gu = a.gu, G = a.gates;
    const float* zx = a.zx + (size_t)row0 * T * gu;
    float* dst = a.dst + (size_t)row0 * (a.ret_seq ? (size_t)T * a.stride : (size_t)a.stride);
    // fp32: thread t owns column c = t / KS and its k-slice [k0, k0 + 64), KS lanes per column
    const int c = tid / KS, ks = tid % KS;
    const bool active = c < gu;
    const int cc = active ? c : gu - 1;
    constexpr int REGS = kSoloRegs;
    const int k0 = ks * REGS;
    // int8: the products on the matrix cores (v_mfma_i32_16x16x64_i8, rows of h in the rows of A): wave w owns the
    // 16-column blocks w, w + 16, …; lane (fr, fq) holds bytes 64·kc + 16·fq … + 15 of column 16·block + fr
    const int fr = lane & 15, fq = lane >> 4;
    const int nb = (gu + 15) / 16, nkc = (u + 63) / 64;
    for (int e = tid; e < kSoloRows * 2048; e += kSoloThreads) (&hs[0][0])[e] = 0.0f;
    for (int e = tid; e < kSoloRows * 512; e += kSoloThreads) (&hq[0][0])[e] = 0;
    float uf[I8 ? 1 : REGS];
    v4i ub[I8 ? kSoloBlocks : 1][I8 ? kSoloChunks : 1];
    float csc[I8 ? kSoloBlocks : 1], cbi[I8 ? kSoloBlocks : 1];
    if (I8) {
        // U's bytes past u are zeroed (those of h are zero too); rows of kp bytes, kp ≥ u rounded up to 4: 16 bytes at
        // a time where kp is a multiple of 16 and q 16-byte aligned, else four words
        const bool vec16 = a.kp % 16 == 0 && ((uintptr_t)a.q & 15) == 0;
#pragma unroll
        for (int i = 0; i < kSoloBlocks; ++i) {
            const int n = 16 * (wave + 16 * i) + fr;
            const bool col = n < gu;
            csc[i] = col ? a.qs[n] : 0.0f;
            cbi[i] = col && a.brec ? a.brec[n] : 0.0f;
#pragma unroll
            for (int kc = 0; kc < kSoloChunks; ++kc) {
                const int kb = 64 * kc + 16 * fq;  // this lane's first byte
                v4i v = {0, 0, 0, 0};
                if (col && kb < u) {
                    const int8_t* src = a.q + (size_t)n * a.kp + kb;
                    if (vec16) {
                        v = *reinterpret_cast<const v4i*>(src);
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            if (kb + 4 * j < u) v[j] = *reinterpret_cast<const int*>(src + 4 * j);
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int left = u - (kb + 4 * j);  // bytes of word j inside u
                        if (left <= 0) v[j] = 0;
                        else if (left < 4) v[j] &= (int)((1u << (8 * left)) - 1u);
                    }
                }
                ub[i][kc] = v;
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < REGS; ++i) {
            const int k = k0 + i;
            uf[i] = k < u ? (a.u_nt ? a.U[(size_t)cc * u + k] : a.U[(size_t)k * gu + cc]) : 0.0f;
        }
    }
    __syncthreads();
    const float col_bias = !I8 && a.brec ? a.brec[cc] : 0.0f;  // fp32 (int8: cbi)
    // cell phase: fp32 — thread tid < B·u owns row tid / u, unit tid % u; int8 — wave b < B owns row b, lane l its
    // units l and l + 64 (u ≤ 128), so the wave that writes a row of h_t also takes its maximum by lane exchanges and
    // quantizes it for the next timestep's products, before the timestep's last barrier
    constexpr int NU = I8 ? 2 : 1;  // units per thread
    const bool cell = I8 ? wave < B : tid < B * u;
    const int cb = cell ? (I8 ? wave : tid / u) : 0;
    const int cj0 = I8 ? lane : (cell ? tid % u : 0);  // unit of slot 0 (int8: slot i is unit cj0 + 64·i)
    float cst[NU];  // the cells' c
#pragma unroll
    for (int i = 0; i < NU; ++i) cst[i] = 0.0f;
    // the input-side gate values of this thread's cells, one timestep ahead (they do not depend on h)
    auto load_z = [&](int st, float (&z)[NU][4]) {
        const int tt = a.dir ? T - 1 - st : st;
#pragma unroll
        for (int i = 0; i < NU; ++i) {
            const int j = cj0 + 64 * i;
#pragma unroll
            for (int g = 0; g < 4; ++g)
                z[i][g] = cell && j < u && g < G ? zx[((size_t)cb * T + tt) * gu + (size_t)g * u + j] : 0.0f;
        }
    };
    float zn[NU][4];
    load_z(0, zn);
    for (int step = 0; step < T; ++step) {
        const int t = a.dir ? T - 1 - step : step;
        float zv[NU][4];
#pragma unroll
        for (int i = 0; i < NU; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) zv[i][g] = zn[i][g];
        if (step + 1 < T) load_z(step + 1, zn);
        if (step > 0) {
            if (I8) {
                // the rows of h_{t−1} (quantized by the cells that wrote them) as rows of A (rows from B on repeat row
                // B − 1; their sums are not used), exact int32 sums in lanes fq = 0 (row b in element b), then the
                // int8 GEMM's epilogue ((float)acc · sx) · scale (+ bias)
                const int arow = fr < B ? fr : B - 1;
                v4i af[kSoloChunks];
#pragma unroll
                for (int kc = 0; kc < kSoloChunks; ++kc)
                    af[kc] = kc < nkc ? *reinterpret_cast<const v4i*>(&hq[arow][16 * kc + 4 * fq]) : v4i{0, 0, 0, 0};
#pragma unroll
                for (int i = 0; i < kSoloBlocks; ++i) {
                    if (wave + 16 * i >= nb) break;
                    v4i acc = {0, 0, 0, 0};
#pragma unroll
                    for (int kc = 0; kc < kSoloChunks; ++kc)
                        if (kc < nkc) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[kc], ub[i][kc], acc, 0, 0, 0);
                    const int n = 16 * (wave + 16 * i) + fr;
                    if (fq == 0 && n < gu) {
#pragma unroll
                        for (int b = 0; b < kSoloRows; ++b) {
                            if (b >= B) break;
                            float v = (float)acc[b] * sxs[b];
                            v = v * csc[i];
                            if (a.brec) v = v + cbi[i];
                            r[b][n] = v;
                        }
                    }
                }
            } else {
                for (int b = 0; b < B; ++b) {
                    // a slice that starts inside u is read whole (zeros past u in hs and in uf; it ends inside the
                    // 2048-float row, k0 being a multiple of 64), so its loads go out together
                    float v = 0.0f;
                    const float4* hrow = reinterpret_cast<const float4*>(&hs[b][k0]);
#pragma unroll
                    for (int i = 0; i < REGS / 4; ++i) {
                        if (k0 >= u) break;  // the whole slice past u
                        const float4 hv = hrow[i];
                        v = fmaf(hv.x, uf[4 * i], v);
                        v = fmaf(hv.y, uf[4 * i + 1], v);
                        v = fmaf(hv.z, uf[4 * i + 2], v);
                        v = fmaf(hv.w, uf[4 * i + 3], v);
                    }
                    v = knx_lane_group_sum(v, KS);
                    if (a.brec) v = v + col_bias;
                    if (active && ks == 0) r[b][c] = v;
                }
            }
        }
        lds_barrier();  // r complete; every read of hs, hq and sxs done
        if (cell) {
            const bool first = step == 0;
            auto rec = [&](int g, int j) { return r[cb][g * u + j]; };
            float hv[NU];
            unsigned mb = 0u;  // int8: the row maximum of |h_t| as bits (NaN above +inf above every finite value)
#pragma unroll
            for (int i = 0; i < NU; ++i) {
                const int j = cj0 + 64 * i;
                hv[i] = 0.0f;
                if (j >= u) continue;
                if (KIND == 4) {
                    float zi = zv[i][0], zf = zv[i][1], zg = zv[i][2], zo = zv[i][3];
                    if (!first) { zi = zi + rec(0, j); zf = zf + rec(1, j); zg = zg + rec(2, j); zo = zo + rec(3, j); }
                    hv[i] = knx_lstm_cell(zi, zf, zg, zo, act, a.alpha, first, cst[i]);
                } else if (KIND == 5) {
                    const float hz = first ? a.brec[j] : rec(0, j);
                    const float hr = first ? a.brec[u + j] : rec(1, j);
                    const float hh = first ? a.brec[2 * u + j] : rec(2, j);
                    hv[i] = knx_gru_cell(zv[i][0], zv[i][1], zv[i][2], hz, hr, hh, act, a.alpha, first,
                                         first ? 0.0f : hs[cb][j]);
                } else {
                    float v = zv[i][0];
                    if (!first) v = v + rec(0, j);
                    hv[i] = knx_gate_act(v, act, a.alpha);
                }
                hs[cb][j] = hv[i];
                if (I8) mb = max(mb, __float_as_uint(hv[i]) & 0x7fffffffu);
                if (a.ret_seq) dst[((size_t)cb * T + t) * a.stride + j] = hv[i];
                else if (step + 1 == T) dst[(size_t)cb * a.stride + j] = hv[i];
            }
            if (I8 && step + 1 < T) {
                // h_t's int8 row for the next timestep: s = max|h|/127, 1 for an all-zero row, NaN for a row holding
                // NaN or ±inf; q = clamp(rint(h·(1/s)), ±127); bytes past u stay 0; the bytes of a row that cannot be
                // quantized do not matter (its products are NaN through its scale)
                mb = knx_lane_group_max(mb, 64);
                const bool bad = mb >= 0x7f800000u;
                const float mx = __uint_as_float(mb);
                const float sc = (!bad && mx > 0.0f) ? __fdiv_rn(mx, 127.0f) : 1.0f;
                const float inv = bad ? 0.0f : __fdiv_rn(1.0f, sc);
                if (lane == 0) sxs[cb] = bad ? __int_as_float(0x7fc00000) : sc;
#pragma unroll
                for (int i = 0; i < NU; ++i) {
                    const int j = cj0 + 64 * i;
                    if (j < u)
                        reinterpret_cast<int8_t*>(&hq[cb][0])[j] =
                            (int8_t)(int)__builtin_amdgcn_fmed3f(rintf(hv[i] * inv), -127.0f, 127.0f);
                }
            }
        }
        lds_barrier();  // h_t (and its int8 row and scale) complete in LDS
    }
    if (a.dn > 0) {
        // The LINEAR after the recurrence, on h_T still in LDS (zero past u).  int8: each row quantized by one wave with
        // the quantizer's operations (as above) into hq and sxs, exact int32 sums, ((float)acc · sx) · scale (+ bias),
        // then the activation — the bits of knx_hip_qlinear; fp32: lane sums of h·w (+ bias), then the activation.
        const bool di8 = a.dq != nullptr;
        if (di8) {
            if (wave < B) {
                float hv[4];  // u ≤ 256 on the row-split kernel
                unsigned mb = 0u;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int j = lane + 64 * i;
                    hv[i] = j < u ? hs[wave][j] : 0.0f;
                    mb = max(mb, __float_as_uint(hv[i]) & 0x7fffffffu);
                }
                mb = knx_lane_group_max(mb, 64);
                const bool bad = mb >= 0x7f800000u;
                const float mx = __uint_as_float(mb);
                const float sc = (!bad && mx > 0.0f) ? __fdiv_rn(mx, 127.0f) : 1.0f;
                const float inv = bad ? 0.0f : __fdiv_rn(1.0f, sc);
                if (lane == 0) sxs[wave] = bad ? __int_as_float(0x7fc00000) : sc;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int j = lane + 64 * i;
                    if (j < u)
                        reinterpret_cast<int8_t*>(&hq[wave][0])[j] =
                            (int8_t)(int)__builtin_amdgcn_fmed3f(rintf(hv[i] * inv), -127.0f, 127.0f);
                }
            }
            lds_barrier();
        }
        for (int pr = wave; pr < B * a.dn; pr += kSoloThreads / 64) {  // (row, output) pairs, one per wave
            const int b = pr / a.dn, c = pr % a.dn;
            float v;
            if (di8) {
                int acc = 0;  // lane: bytes 4·lane … 4·lane + 3 (hq is zero past u, so the weight's bytes there do not count)
                if (4 * lane < u)
                    acc = __builtin_amdgcn_sdot4(hq[b][lane], *reinterpret_cast<const int*>(a.dq + (size_t)c * a.dkp + 4 * lane),
                                                 0, false);
#pragma unroll
                for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
                v = (float)acc * sxs[b];
                v = v * a.dqs[c];
            } else {
                float part = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int j = lane + 64 * i;
                    if (j < u) part = fmaf(hs[b][j], a.dw[(size_t)c * u + j], part);
                }
                v = knx_lane_group_sum(part, 64);
            }
            if (a.db) v = v + a.db[c];
            v = knx_act(v, a.dact, a.dalpha);
            if (lane == 0) a.dy[(size_t)(row0 + b) * a.dn + c] = v;
        }
    }
}

// rows per workgroup of the row-split kernel: one while there is a CU for every row (a workgroup's timestep grows with
// its rows), two above
int solo_rows(int B)
{
    return B <= 256 ? 1 : kSoloRows;
}

// lanes per column of the row-split kernel: the most (a power of two ≤ 64) that the 1024 threads hold, if each lane's
// slice of its column then fits the registers; else 0 (no row-split kernel for the shape)
int solo_lanes(int B, int gu, int u, bool i8)
{
    if ((long)solo_rows(B) * u > kSoloThreads || u > 2048 || gu > kSoloThreads) return 0;
    const char* e = getenv("KNX_RNN_SOLO");  // 0: the grid kernel wherever it fits (tests, tuning)
    if (e != nullptr && *e == '0') return 0;
    if (i8) return u <= 64 * kSoloChunks && gu <= 16 * 16 * kSoloBlocks ? 1 : 0;  // the products on the matrix cores
    int ks = 1;
    while (ks < 64 && (long)gu * ks * 2 <= kSoloThreads) ks *= 2;
    return u <= ks * kSoloRegs ? ks : 0;  // lane s covers [s·64, (s+1)·64)
}

// units per workgroup: enough that the workgroup's gate columns fill a 16-wide tile of the products (LSTM 4, GRU 5,
// simple RNN 16 units), more where u needs it to stay within kMaxGrid workgroups, fewer where the (row, unit) pairs
// would not fit the threads
int units_per_wg(int B, int u, int gates)
{
    const int least = (u + kMaxGrid - 1) / kMaxGrid;
    int uw = std::max(least, 16 / gates);
    if (const char* e = getenv("KNX_RNN_UNITS")) {  // tuning: units per workgroup
        const int v = atoi(e);
        if (v >= 1) uw = std::max(least, v);
    }
    while (B * uw > kThreads * kMaxPairs && uw > least) --uw;
    return uw;
}

// one launch of the instantiation for (I8, KIND, ACT): the row-split kernel when ks > 0, else the grid of G
// workgroups with lds bytes of dynamic LDS (its limit raised once per instantiation)
template <bool I8, int KIND, int ACT>
int launch_rnn(const RnnArgs& a, int ks, int G, size_t lds, hipStream_t s, const char* name)
{
    if (ks > 0) {
        const int R = solo_rows(a.B);
        hipLaunchKernelGGL((rnn_solo<I8, KIND, ACT>), dim3((unsigned)((a.B + R - 1) / R)), dim3(kSoloThreads), 0, s, a,
                           ks, R);
        return knx::check_launch(name);
    }
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&rnn_recurrence<I8, KIND, ACT>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds);
    if (attr != hipSuccess) return knx::fail(KNX_EHIP, "%s: %s", name, hipGetErrorString(attr));
    hipLaunchKernelGGL((rnn_recurrence<I8, KIND, ACT>), dim3((unsigned)G), dim3(kThreads), lds, s, a);
    return knx::check_launch(name);
}

template <bool I8, int KIND>
int launch_act(const RnnArgs& a, int ks, int G, size_t lds, hipStream_t s, const char* name)
{
    return a.act == 4 ? launch_rnn<I8, KIND, 4>(a, ks, G, lds, s, name) : launch_rnn<I8, KIND, kActAny>(a, ks, G, lds, s, name);
}

template <bool I8>
int launch_kind(const RnnArgs& a, int ks, int G, size_t lds, hipStream_t s, const char* name)
{
    if (a.kind == 4) return launch_act<I8, 4>(a, ks, G, lds, s, name);
    if (a.kind == 5) return launch_act<I8, 5>(a, ks, G, lds, s, name);
    return launch_act<I8, 6>(a, ks, G, lds, s, name);
}

}  // namespace

extern "C" int knx_hip_rnn_recurrence_fits(int kind, int B, int u, int i8)
{
    if ((kind != 4 && kind != 5 && kind != 6) || B < 1 || u < 1 || u > 65536) return 0;
    const int gates = kind == 4 ? 4 : kind == 5 ? 3 : 1;
    if (solo_lanes(B, gates * u, u, i8 != 0) > 0) return 1;
    if (B > 64 || u > kMaxUnits) return 0;
    const int uw = units_per_wg(B, u, gates);
    if ((u + uw - 1) / uw > kMaxGrid || B * uw > kThreads * kMaxPairs) return 0;
    return lds_layout(B, gates, uw, k_extent(u, i8 != 0), i8 != 0, !i8 || kind == 5).total <= kMaxLds ? 1 : 0;
}

extern "C" int knx_hip_rnn_recurrence_dense_fits(int kind, int B, int u, int i8, int n)
{
    if ((kind != 4 && kind != 5 && kind != 6) || B < 1 || u < 1 || u > 65536 || n < 1) return 0;
    const int gates = kind == 4 ? 4 : kind == 5 ? 3 : 1;
    return solo_lanes(B, gates * u, u, i8 != 0) > 0 && u <= 256 ? 1 : 0;
}

extern "C" int knx_hip_rnn_recurrence_dense(int kind, int act, float alpha, int B, int T, int u, int dir, const float* zx,
                                            const float* U, int u_nt, const int8_t* q, int kp, const float* qscale,
                                            const float* brec, float* dst, int stride, const float* dw, const int8_t* dq,
                                            int dkp, const float* dqs, const float* db, int dn, int dact, float dalpha,
                                            float* dy, void* stream)
{
    const char* name = "knx_hip_rnn_recurrence_dense";
    KNX_ENTRY(name);
    KNX_REQUIRE(T >= 1 && act >= -1 && act <= 15 && dact >= -1 && dact <= 15 && (dir == 0 || dir == 1), name);
    KNX_REQUIRE(knx_hip_rnn_recurrence_dense_fits(kind, B, u, q != nullptr, dn), name);
    const int gates = kind == 4 ? 4 : kind == 5 ? 3 : 1;
    KNX_REQUIRE(zx != nullptr && dst != nullptr && stride >= u && dy != nullptr, name);
    KNX_REQUIRE(kind != 5 || brec != nullptr, name);
    KNX_REQUIRE(q != nullptr ? (qscale != nullptr && kp >= (u + 3) / 4 * 4 && ((uintptr_t)q & 3) == 0 && kp % 4 == 0)
                             : U != nullptr, name);
    KNX_REQUIRE(dq != nullptr ? (dqs != nullptr && dkp >= (u + 3) / 4 * 4 && ((uintptr_t)dq & 3) == 0 && dkp % 4 == 0)
                              : dw != nullptr, name);
    RnnArgs a{};
    a.kind = kind; a.act = act; a.alpha = alpha;
    a.B = B; a.T = T; a.u = u; a.gu = gates * u; a.gates = gates; a.dir = dir; a.ret_seq = 0;
    a.stride = stride; a.uw = units_per_wg(B, u, gates);
    a.up = k_extent(u, q != nullptr); a.ldh = (u + 3) / 4 * 4;
    a.zx = zx; a.U = U; a.u_nt = u_nt != 0; a.q = q; a.kp = kp; a.qs = qscale; a.brec = brec;
    a.dst = dst;
    a.dw = dq != nullptr ? nullptr : dw; a.dq = dq; a.dkp = dkp; a.dqs = dqs; a.db = db;
    a.dn = dn; a.dact = dact; a.dalpha = dalpha; a.dy = dy;
    const int ks = solo_lanes(B, a.gu, u, q != nullptr);
    const hipStream_t s = knx::as_stream(stream);
    if (q != nullptr) return launch_kind<true>(a, ks, 0, 0, s, name);
    return launch_kind<false>(a, ks, 0, 0, s, name);
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
    KNX_REQUIRE((((uintptr_t)h0 | (uintptr_t)h1) & 15) == 0, name);
    KNX_REQUIRE(kind != 5 || brec != nullptr, name);
    KNX_REQUIRE(q != nullptr ? (qscale != nullptr && kp >= (u + 3) / 4 * 4 && ((uintptr_t)q & 3) == 0 && kp % 4 == 0)
                             : U != nullptr, name);
    KNX_REQUIRE(scratch != nullptr && ((uintptr_t)scratch & 255) == 0 && scratch_bytes >= 8, name);
    KNX_REQUIRE(status != nullptr && ((uintptr_t)status & 3) == 0, name);
    RnnArgs a{};
    a.kind = kind; a.act = act; a.alpha = alpha;
    a.B = B; a.T = T; a.u = u; a.gu = gates * u; a.gates = gates; a.dir = dir; a.ret_seq = ret_seq != 0;
    a.stride = stride; a.uw = units_per_wg(B, u, gates);
    a.up = k_extent(u, q != nullptr); a.ldh = (u + 3) / 4 * 4;
    a.zx = zx; a.U = U; a.u_nt = u_nt != 0; a.q = q; a.kp = kp; a.qs = qscale; a.brec = brec;
    a.h0 = h0; a.h1 = h1; a.dst = dst;
    a.gs = knx::GridSync{static_cast<unsigned long long*>(scratch), status, knx::grid_spin_limit()};
    const int ks = solo_lanes(B, a.gu, u, q != nullptr);
    const int G = (u + a.uw - 1) / a.uw;
    const size_t lds = ks > 0 ? 0 : lds_layout(B, gates, a.uw, a.up, q != nullptr, q == nullptr || kind == 5).total;
    const hipStream_t s = knx::as_stream(stream);
    if (q != nullptr) return launch_kind<true>(a, ks, G, lds, s, name);
    return launch_kind<false>(a, ks, G, lds, s, name);
}
