// knx_chain.hip — a run of Linear layers over a few rows (≤ 64) as one launch.
//
// At small batches a Linear layer is a few µs of memory latency (weights and input rows fetched, a handful of
// MFMAs, outputs written) and a launch costs about as much again, so a chain of layers (the int8 MLP at batch 1 to
// 64: reference kernix_step_run, include/kernix_model.h:1843-1860, layer after layer) runs here as one grid: the
// layers one after the other, separated by barriers across the grid (knx_grid.hpp: one workgroup per CU at most,
// all resident at once).  Inside a layer the work is split into items of 16 rows × 16 output channels (int8 layers:
// × 1, 2 or 4 adjacent blocks of 16 channels, so that at more rows the grid, and with it the cost of each barrier,
// stays small while an item's input rows are loaded and quantized once for all of its channels); an item's K range
// is split over the 8 waves of its workgroup (16×16×64 int8 or 16×16×4 fp32 MFMA, the partial tiles summed through
// LDS in wave order), and its epilogue applies bias and activation.
//
// Latency is the whole cost here (one memory round trip ≈ 1.2–1.8 µs on MI355X), so each item issues all of its
// loads at once — weight fragments, input rows, per-channel scales and bias — and waits once.
//
// int8 layers (reference kernix_qmatmul, include/kernix_model.h:99-182): an item loads its 16 input rows in full
// (k ≤ 2048), 32 threads per row; the threads of a row reduce its maximum by lane exchanges and quantize the row
// into LDS — s = max|x|/127 (1 for an all-zero row), q = clamp(rint(x·(1/s)), ±127), a row holding NaN or ±inf gets
// s = NaN — the arithmetic of knx_hip_quantize_rows, so the results are the bits of the quantizer followed by
// knx_hip_i8gemm, with no quantizer pass and no int8 copy of the rows in memory.
//
// The layers' outputs cross the grid: they are stored at device scope (sc1, through to the coherence point the
// XCDs share), and after each barrier the workgroup drops its cached copies of other agents' data (knx_grid.hpp),
// so every input row is read with ordinary loads: each line once per XCD from memory, then from the XCD's L2.
#include <float.h>
#include <algorithm>
#include <math.h>
#include <mutex>
#include <string.h>

#include "knx_common.hpp"
#include "knx_grid.hpp"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));

namespace {

constexpr int kThreads = 512, kWaves = 8;
constexpr int kMaxRows = 64;
constexpr int kMaxBlocks = 8;                   // 16-channel blocks per int8 item (at most 2 when kp > 1024)
constexpr int kTargetItems = 16;                // items per int8 layer the grid aims for, per row block (≤ 2)
constexpr int kI8Steps = 4;                     // 64-wide k-steps per wave of an int8 item: k ≤ 8·4·64
constexpr int kMaxI8K = kWaves * kI8Steps * 64;
constexpr int kF32Chunks = 8;                   // 16-wide k-chunks per wave and pass of an fp32 item
constexpr unsigned kBufferWord3 = 0x00020000u;  // raw buffer, 32-bit data format

struct LayerDev {
    const void* w;
    const float* sw;
    const float* bias;
    const float* x;     // input rows (layer 0: the caller's x, then the previous layer's y)
    float* y;
    int k, kp, n, ldw, ldx, ldy, act, i8, last;
    int cb;             // 16-channel blocks per item (int8: 1, 2 or 4; fp32: 1)
    float alpha;
};

struct ChainArgs {
    LayerDev L[KNX_CHAIN_MAX_LAYERS];
    int layers, rows;
    knx::GridSync gs;
};

// Buffer resources: a load at an offset past num_records returns zeros, so every load of an item is issued
// unconditionally (out-of-range rows, k-steps and channels get an offset past the end) — no exec-masked branches,
// whose zero-filled destinations make the compiler wait for loads already in flight.
constexpr int kOut = 0x7ffffff0;  // an offset past every buffer (buffers are < 2^31 bytes)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, long long bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kBufferWord3);
}
__device__ __forceinline__ float4 ld4(__amdgpu_buffer_rsrc_t r, int off)
{
    const v4u u = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
    return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
}
__device__ __forceinline__ v4i ld4i(__amdgpu_buffer_rsrc_t r, int off)
{
    return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ float ld1(__amdgpu_buffer_rsrc_t r, int off)
{
    return __uint_as_float((unsigned)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ void st_dev(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
// |v|, or +inf for NaN and ±inf: a row whose maximum is +inf cannot be quantized
__device__ __forceinline__ float mag(float v)
{
    const float a = fabsf(v);
    return a <= FLT_MAX ? a : INFINITY;
}

constexpr int kQPitch = kMaxI8K + 16;  // bytes per quantized row in LDS

struct Shared {
    int part[kWaves][kMaxBlocks][16][17];   // per-wave partial tiles (int32, or fp32 bits), per channel block
    float rsx[16];                          // row scales of an int8 item's rows
    alignas(16) int8_t q[16][kQPitch];      // an int8 item's rows, quantized
};

// The item's output tile (16 rows × 16·CB channels) from the wave-partial tiles (summed in wave order), then bias,
// activation and the store.  Output o = t + 512·p of the tile is row o / (16·CB), channel o % (16·CB) (a row's
// channels to consecutive threads); sw_n[p] / b_n[p] are that channel's scale and bias, loaded early.
template <bool I8, int CB>
__device__ __forceinline__ void tile_epilogue(const LayerDev& L, int rows, int rb, int cg, const float* sw_n, const float* b_n,
                              Shared& sh)
{
    constexpr int W16 = 16 * CB, EP = (16 * W16 + kThreads - 1) / kThreads;
    __syncthreads();
    const int t = threadIdx.x;
#pragma unroll
    for (int p = 0; p < EP; ++p) {
        const int o = t + kThreads * p;
        if (o >= 16 * W16) break;
        const int i = o / W16, cc = o % W16, b = cc >> 4, col = cc & 15, m = 16 * rb + i, n = W16 * cg + cc;
        if (m < rows && n < L.n) {
            float v;
            if (I8) {
                int s = 0;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) s += sh.part[w][b][i][col];
                // ((float)acc · sx) · scale + bias, each step rounded (reference include/kernix_model.h:167-177)
                v = (float)s * sh.rsx[i];
                v = v * sw_n[p];
            } else {
                v = __int_as_float(sh.part[0][b][i][col]);
#pragma unroll
                for (int w = 1; w < kWaves; ++w) v = v + __int_as_float(sh.part[w][b][i][col]);
            }
            if (L.bias) v = v + b_n[p];
            v = knx_act(v, L.act, L.alpha);
            float* y = L.y + (size_t)m * L.ldy + n;
            if (L.last) *y = v;
            else st_dev(y, v);
        }
    }
    __syncthreads();  // the partial tiles are reused by the next item
}

// int8 item: rows 16·rb … and the CB channel blocks CB·cg … of 16 channels, at most KS 64-wide k-steps per wave
// (kp ≤ 512·KS).  Loads: the 16 rows' fp32 values, thread t taking row t / 32 and the float4s t % 32, + 32, …
// (coalesced, at most 4·KS per thread); per block b the weight fragments of lane (r, c) of wave w — output channel
// 16·(CB·cg + b) + r, bytes [16c, 16c + 16) of the k-steps w, w + 8, …; the scales and biases of the channels the
// thread stores.  The 32 threads of a row reduce its maximum by lane exchanges (a half-wave) and quantize their values
// into the row's LDS copy; the waves then read their MFMA fragments from there, each fragment serving all blocks.
template <int CB, int KS>
__device__ __forceinline__ void item_i8(const LayerDev& L, int rows, __amdgpu_buffer_rsrc_t xr, int rb, int cg, Shared& sh)
{
    constexpr int W16 = 16 * CB, EP = (16 * W16 + kThreads - 1) / kThreads, kXS = KS * kWaves * 64 / 4 / 32;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, r = lane & 15, c = lane >> 4;
    const __amdgpu_buffer_rsrc_t wr = rsrc(L.w, (long long)L.n * L.ldw);
    const int nk = L.kp / 64;
    const int i = t >> 5, s0 = t & 31, m = 16 * rb + i;  // the row this thread quantizes
    const bool mok = m < rows;
    const int K4 = L.k / 4, xbase = (mok ? m : 0) * L.ldx * 4;
    // every load of the item at once
    float4 xv[kXS];
#pragma unroll
    for (int q = 0; q < kXS; ++q) {
        const int j = s0 + 32 * q;
        xv[q] = ld4(xr, mok && j < K4 ? xbase + 16 * j : kOut);
    }
    v4i wf[CB][KS];
#pragma unroll
    for (int b = 0; b < CB; ++b) {
        const int n = W16 * cg + 16 * b + r;
        const bool nok = n < L.n;
        const int wbase = (nok ? n : 0) * L.ldw + c * 16;  // offsets of channels that exist only (no overflow)
#pragma unroll
        for (int j = 0; j < KS; ++j) {
            const int kk = wave + j * kWaves;
            wf[b][j] = ld4i(wr, nok && kk < nk ? wbase + kk * 64 : kOut);
        }
    }
    const __amdgpu_buffer_rsrc_t swr = rsrc(L.sw, (long long)L.n * 4), br = rsrc(L.bias, L.bias ? (long long)L.n * 4 : 0);
    float sw_n[EP], b_n[EP];
#pragma unroll
    for (int p = 0; p < EP; ++p) {
        const int ne = min(W16 * cg + (t + kThreads * p) % W16, L.n - 1);
        sw_n[p] = ld1(swr, ne * 4);
        b_n[p] = ld1(br, ne * 4);
    }
    // all of the above issued before the first wait: the scheduler would otherwise move the weight and scale loads
    // down to their first use, after the input rows' wait, for a second round trip
    __builtin_amdgcn_sched_barrier(0);
    // The row's maximum over its 32 threads (|x|, +inf for NaN and ±inf; values past k were loaded as 0), then the
    // quantized values.  Only the float4 slots that reach into k (a condition uniform over the workgroup) and the
    // waves that hold a row of the item (wave w: rows 2w, 2w + 1) do this work.
    if (16 * rb + 2 * wave < rows) {
        float mx = 0.0f;
#pragma unroll
        for (int q = 0; q < kXS; ++q)
            if (32 * q < K4) mx = fmaxf(fmaxf(fmaxf(mx, mag(xv[q].x)), fmaxf(mag(xv[q].y), mag(xv[q].z))), mag(xv[q].w));
        mx = __uint_as_float(knx_lane_group_max(__float_as_uint(mx), 32));  // the half-wave's 32 lanes
        const bool bad = !(mx <= FLT_MAX);
        const float sc = (!bad && mx > 0.0f) ? __fdiv_rn(mx, 127.0f) : 1.0f;
        const float inv = __fdiv_rn(1.0f, sc);
        if (s0 == 0) sh.rsx[i] = bad ? __int_as_float(0x7fc00000) : sc;
        // q = clamp(rint(x·inv), ±127), packed four per int (an exact integer + 128 converts exactly to a byte; the
        // bytes of a row that cannot be quantized do not matter: its outputs are NaN through its scale)
#pragma unroll
        for (int q = 0; q < kXS; ++q) {
            const int j = s0 + 32 * q;
            if (32 * q < K4 && j < K4) {
                unsigned p = 0;
                p = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_amdgcn_fmed3f(rintf(xv[q].x * inv), -127.0f, 127.0f) + 128.0f, 0, p);
                p = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_amdgcn_fmed3f(rintf(xv[q].y * inv), -127.0f, 127.0f) + 128.0f, 1, p);
                p = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_amdgcn_fmed3f(rintf(xv[q].z * inv), -127.0f, 127.0f) + 128.0f, 2, p);
                p = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_amdgcn_fmed3f(rintf(xv[q].w * inv), -127.0f, 127.0f) + 128.0f, 3, p);
                *reinterpret_cast<unsigned*>(&sh.q[i][4 * j]) = p ^ 0x80808080u;
            }
        }
    }
    __syncthreads();
    // rows past the block's and bytes in [k, kp) hold stale LDS values: the former are never stored, the latter meet
    // the weight's zero padding
    v4i acc[CB];
#pragma unroll
    for (int b = 0; b < CB; ++b) acc[b] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < KS; ++j) {
        const int kk = wave + j * kWaves;
        if (kk < nk) {
            const v4i af = *reinterpret_cast<const v4i*>(&sh.q[r][64 * kk + 16 * c]);
#pragma unroll
            for (int b = 0; b < CB; ++b) acc[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, wf[b][j], acc[b], 0, 0, 0);
        }
    }
    // lane (r, c) holds rows 4c + e of channel r of each block
#pragma unroll
    for (int b = 0; b < CB; ++b)
#pragma unroll
        for (int e = 0; e < 4; ++e) sh.part[wave][b][4 * c + e][r] = acc[b][e];
    tile_epilogue<true, CB>(L, rows, rb, cg, sw_n, b_n, sh);
}

// fp32 item: lane (r, q) of wave w holds row 16·rb + r and channel 16·ct + r, k = 16·kc + 4q + (0..3) of the
// 16-wide k-chunks kc = w, w + 8, …, kF32Chunks of them per pass.
__device__ __forceinline__ void item_f32(const LayerDev& L, int rows, __amdgpu_buffer_rsrc_t xr, int rb, int ct, Shared& sh)
{
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, r = lane & 15, q = lane >> 4;
    const __amdgpu_buffer_rsrc_t wr = rsrc(L.w, (long long)L.n * L.ldw * 4);
    const int n = 16 * ct + r, m = 16 * rb + r;
    const bool nok = n < L.n, mok = m < rows;
    const int wbase = (nok ? n : 0) * L.ldw * 4 + 16 * q, xbase = (mok ? m : 0) * L.ldx * 4 + 16 * q;
    const int nkc = (L.k + 15) / 16;
    const int ne = min(16 * ct + (t & 15), L.n - 1);
    const __amdgpu_buffer_rsrc_t br = rsrc(L.bias, L.bias ? (long long)L.n * 4 : 0);
    float b_n = 0.0f;
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = wave; k0 < nkc; k0 += kWaves * kF32Chunks) {
        float4 wf[kF32Chunks], xf[kF32Chunks];
#pragma unroll
        for (int j = 0; j < kF32Chunks; ++j) {
            const int kc = k0 + j * kWaves;
            const bool in = kc < nkc && 16 * kc + 4 * q < L.k;
            wf[j] = ld4(wr, in && nok ? wbase + 64 * kc : kOut);
            xf[j] = ld4(xr, in && mok ? xbase + 64 * kc : kOut);
        }
        if (k0 == wave) b_n = ld1(br, ne * 4);  // with the first pass's loads
        __builtin_amdgcn_sched_barrier(0);  // the pass's loads all issued before the first wait
#pragma unroll
        for (int j = 0; j < kF32Chunks; ++j) {
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[j].x, wf[j].x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[j].y, wf[j].y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[j].z, wf[j].z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[j].w, wf[j].w, acc, 0, 0, 0);
        }
    }
    if (wave >= nkc) b_n = ld1(br, ne * 4);  // a wave without k-chunks (k < 128)
#pragma unroll
    for (int e = 0; e < 4; ++e) sh.part[wave][0][4 * q + e][r] = __float_as_int(acc[e]);
    const float one = 1.0f;
    tile_epilogue<false, 1>(L, rows, rb, ct, &one, &b_n, sh);
}

__global__ void __launch_bounds__(kThreads) linear_chain(ChainArgs a)
{
    __shared__ Shared sh;
    const int rows = a.rows, RB = (rows + 15) / 16;
    for (int l = 0; l < a.layers; ++l) {
        const LayerDev& L = a.L[l];
        const int items = RB * ((L.n + 16 * L.cb - 1) / (16 * L.cb));
        const __amdgpu_buffer_rsrc_t xr = rsrc(L.x, (long long)rows * L.ldx * 4);
        for (int it = blockIdx.x; it < items; it += gridDim.x) {
            const int rb = it % RB, cg = it / RB;
            if (!L.i8) item_f32(L, rows, xr, rb, cg, sh);
            else if (L.kp > 1024) {
                if (L.cb == 2) item_i8<2, 4>(L, rows, xr, rb, cg, sh);
                else item_i8<1, 4>(L, rows, xr, rb, cg, sh);
            } else if (L.kp > 512) {
                if (L.cb == 8) item_i8<8, 2>(L, rows, xr, rb, cg, sh);
                else if (L.cb == 4) item_i8<4, 2>(L, rows, xr, rb, cg, sh);
                else if (L.cb == 2) item_i8<2, 2>(L, rows, xr, rb, cg, sh);
                else item_i8<1, 2>(L, rows, xr, rb, cg, sh);
            } else {
                if (L.cb == 8) item_i8<8, 1>(L, rows, xr, rb, cg, sh);
                else if (L.cb == 4) item_i8<4, 1>(L, rows, xr, rb, cg, sh);
                else if (L.cb == 2) item_i8<2, 1>(L, rows, xr, rb, cg, sh);
                else item_i8<1, 1>(L, rows, xr, rb, cg, sh);
            }
        }
        if (l + 1 < a.layers) knx::grid_barrier(a.gs, (unsigned)l);
    }
}

bool overlaps(const void* a, size_t na, const void* b, size_t nb)
{
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return x < y + nb && y < x + na;
}

constexpr size_t kScratchBytes = 256;  // the barrier words (one 64-bit word per barrier, layers − 1 of them)
constexpr int kMaxGrid = 64;           // workgroups of a chain launch at most

}  // namespace

extern "C" size_t knx_hip_linear_chain_scratch(const knx_chain_layer* layers, int n_layers, int rows)
{
    if (layers == nullptr || n_layers < 1 || n_layers > KNX_CHAIN_MAX_LAYERS || rows < 1 || rows > kMaxRows) return 0;
    return kScratchBytes;
}

extern "C" int knx_hip_linear_chain(const float* x, int ldx, int rows, const knx_chain_layer* layers, int n_layers,
                                    void* scratch, size_t scratch_bytes, int* status, void* stream)
{
    const char* name = "knx_hip_linear_chain";
    KNX_ENTRY(name);
    KNX_REQUIRE(layers != nullptr && n_layers >= 1 && n_layers <= KNX_CHAIN_MAX_LAYERS, name);
    KNX_REQUIRE(rows >= 1 && rows <= kMaxRows, name);
    KNX_REQUIRE(x != nullptr && ((uintptr_t)x & 15) == 0 && ldx % 4 == 0 && ldx >= layers[0].k, name);
    for (int l = 0; l < n_layers; ++l) {
        const knx_chain_layer& L = layers[l];
        KNX_REQUIRE(L.k >= 4 && L.k % 4 == 0 && L.n >= 1 && L.n <= 1 << 20 && L.act >= -1 && L.act <= 15, name);
        KNX_REQUIRE(L.w != nullptr && ((uintptr_t)L.w & 15) == 0 && L.y != nullptr && L.ldy >= L.n, name);
        // an output that the next layer reads as 16-byte vectors
        KNX_REQUIRE(l + 1 == n_layers || (((uintptr_t)L.y & 15) == 0 && L.ldy % 4 == 0), name);
        KNX_REQUIRE((long long)L.n * L.ldw * (L.i8 ? 1 : 4) < (1LL << 31) - 16, name);  // buffer offsets are 32-bit
        if (L.i8) {
            KNX_REQUIRE(L.kp >= L.k && L.kp % 64 == 0 && L.kp <= kMaxI8K && L.ldw >= L.kp && L.ldw % 16 == 0, name);
            KNX_REQUIRE(L.sw != nullptr, name);
        } else {
            KNX_REQUIRE(L.k <= 1 << 20 && L.ldw >= L.k && L.ldw % 4 == 0, name);
        }
        // the layer's input: x or the previous layer's output, which must not share memory with this layer's output
        const float* in = l == 0 ? x : layers[l - 1].y;
        const int ldin = l == 0 ? ldx : layers[l - 1].ldy;
        KNX_REQUIRE(l == 0 || layers[l - 1].n == L.k, name);
        KNX_REQUIRE((long long)rows * ldin * 4 < (1LL << 31) - 16, name);
        KNX_REQUIRE(!overlaps(in, (size_t)rows * ldin * 4, L.y, (size_t)rows * L.ldy * 4), name);
    }
    KNX_REQUIRE(scratch != nullptr && ((uintptr_t)scratch & 255) == 0 && scratch_bytes >= kScratchBytes, name);
    KNX_REQUIRE(status != nullptr && ((uintptr_t)status & 3) == 0, name);

    // measured on the int8 MLP 784-512-256-10: 16 items at one row (14.3 µs against 15.2 at 32), 32 at 64 rows
    // (16.8 µs against 19.1 at 16: with 16 workgroups each loads 156 KB of rows and weights in the first layer)
    int target = kTargetItems * std::min((rows + 15) / 16, 2);
    if (const char* e = getenv("KNX_CHAIN_ITEMS")) target = atoi(e) > 0 ? atoi(e) : target;  // tuning and tests
    ChainArgs a{};
    a.layers = n_layers;
    a.rows = rows;
    a.gs = knx::GridSync{static_cast<unsigned long long*>(scratch), status, knx::grid_spin_limit()};
    for (int l = 0; l < n_layers; ++l) {
        const knx_chain_layer& L = layers[l];
        LayerDev& d = a.L[l];
        d.w = L.w; d.sw = L.sw; d.bias = L.bias; d.y = L.y;
        d.x = l == 0 ? x : layers[l - 1].y;
        d.ldx = l == 0 ? ldx : layers[l - 1].ldy;
        d.k = L.k; d.kp = L.kp; d.n = L.n; d.ldw = L.ldw; d.ldy = L.ldy; d.act = L.act; d.i8 = L.i8 != 0;
        d.alpha = L.alpha;
        d.last = l + 1 == n_layers;
    }
    // Items: an int8 layer's items take 1, 2, 4 or 8 blocks of 16 channels (at most 2 when kp > 1024).  A barrier
    // costs more the more workgroups arrive at it (1.1 µs at 16, 1.2 at 32, 1.9 at 64, 3.1 at 128), and an item's
    // input rows are loaded and quantized once for all of its blocks, so the grid is the largest layer's item count
    // with the fewest blocks that bring each layer within the target (or as close as it gets), and then every layer
    // takes the fewest blocks that fit that grid, i.e. as many workgroups as the barriers are paid for anyway.
    const int RB = (rows + 15) / 16;
    auto items_of = [&](const LayerDev& d, int cb) { return RB * (((d.n + 15) / 16 + cb - 1) / cb); };
    auto max_blocks = [&](const LayerDev& d) { return !d.i8 ? 1 : d.kp > 1024 ? 2 : kMaxBlocks; };
    int items_max = 1;
    for (int l = 0; l < n_layers; ++l) {
        int cb = 1;
        while (cb < max_blocks(a.L[l]) && items_of(a.L[l], cb) > target) cb *= 2;
        items_max = std::max(items_max, items_of(a.L[l], cb));
    }
    for (int l = 0; l < n_layers; ++l) {
        LayerDev& d = a.L[l];
        d.cb = 1;
        while (d.cb < max_blocks(d) && items_of(d, d.cb) > items_max) d.cb *= 2;
    }
    // one workgroup per item of the widest layer, at most kMaxGrid (a quarter of the CUs: four chains launched at the
    // same time from different threads or processes still find all of their workgroups resident; above it the
    // workgroups take several items each, and a barrier at 64 workgroups costs 1.9 µs against 3.1 at 128)
    int G = std::min(std::min(items_max, kMaxGrid), knx::num_cus());
    if (const char* e = getenv("KNX_CHAIN_WG")) {  // tuning and tests: fewer workgroups (each then takes several items)
        const int g = atoi(e);
        if (g >= 1 && g < G) G = g;
    }
    hipLaunchKernelGGL(linear_chain, dim3((unsigned)G), dim3(kThreads), 0, knx::as_stream(stream), a);
    return knx::check_launch(name);
}
