// knx_attn.hip — attention core of the KERNIX ATTENTION op on gfx950.
//
// Per (batch b, head h): S = scale·Q_h·K_hᵀ (causal: −inf for key j > query i), P = softmax(S), ctx_h = P·V_h,
// the loop body of kernix_attention_run (reference include/kernix_model.h:1021-1046).  The Q/K/V/O projections
// are ordinary Linear GEMMs run by the host (knx_hip_sgemm_ep).
//
// Paths: for dk = dv ∈ {32, 64, 128} and S ≤ 256 (S ≤ 128 at 128) one fused kernel keeps each head's K and V in
// LDS and the scores in registers, so nothing but Q, K, V and the context touches HBM.  Otherwise one batched NT
// MFMA GEMM writes all B·H score matrices (alpha = scale and the causal mask fused in its epilogue), the wavefront
// softmax normalizes each row in place, and one batched GEMM multiplies by V and writes the context directly in the
// (B·Rq) × (H·dv) layout the output projection reads; given scratch for Vᵀ, V is transposed once so that both
// products have K-contiguous operands and run on the pipelined kernel.
#include <stdlib.h>
#include <string.h>

#include <utility>

#include "knx_pipe.hpp"

int knx_sgemm_batched(int M, int N, int K, const float* A, int lda, long long sAb, long long sAh, const float* B, int ldb,
                      long long sBb, long long sBh, bool transB, float* C, int ldc, long long sCb, long long sCh, int nb,
                      int nh, float alpha, int causal, hipStream_t s);

namespace {

// Vt (C × R) = Vᵀ for V (R × C, row stride ldv), 32 × 32 tiles through LDS
__global__ void __launch_bounds__(256) transpose_kernel(const float* __restrict__ v, int R, int C, int ldv,
                                                        float* __restrict__ vt)
{
    __shared__ float tile[32][33];
    const int r0 = blockIdx.x * 32, c0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 × 8
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = r0 + ty + 8 * i, c = c0 + tx;
        tile[ty + 8 * i][tx] = (r < R && c < C) ? v[(size_t)r * ldv + c] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = c0 + ty + 8 * i, r = r0 + tx;
        if (c < C && r < R) vt[(size_t)c * R + r] = tile[tx][ty + 8 * i];
    }
}

typedef float v16f __attribute__((ext_vector_type(16)));

// f(integral_constant<int, t>) for t = 0, 1, …: a loop whose index is a compile-time constant in the body
template <typename F, int... T>
__device__ __forceinline__ void unrolled(F&& f, std::integer_sequence<int, T...>)
{
    (f(std::integral_constant<int, T>{}), ...);
}

// 16 zero bytes: the source of the staged chunks of keys beyond S
__device__ __attribute__((aligned(16))) float knx_attn_zero[4];

// Fused attention for sequences of at most 32·NS keys, dk = dv = D ∈ {32, 64, 128}.  One block per (b·h, 128
// queries), each wave owns 32 queries.  K_h and V_h of the whole sequence (zero beyond S) are staged in LDS by
// LDS-DMA (global_load_lds, 16 bytes per lane), both row-major in 16-byte chunks with a per-row chunk swizzle, one
// 32-key tile after another: the K tiles first, then the V tiles.  The wave computes Sᵀ = K_h·Q_hᵀ on 32×32×2 fp32
// MFMA tile by tile, each tile as soon as its keys have arrived, while the later K tiles and all of V are still in
// flight; its accumulators hold, per lane, one query (lane & 31) and 16 keys of each 32-key tile, so the row max and
// sum of the softmax need one exchange between the two half-waves, and the normalized probabilities are already the
// B operand of ctxᵀ = V_hᵀ·Pᵀ, whose A operand is read from the row-major V one float at a time.  Keys beyond S
// count as −inf, which leaves max, sum and probabilities as they are over the S keys alone.
//
// LDS layout (16-byte chunk c of key row r), conflict-free for both products:
//   K: chunk position r·CPR + (c ^ sk(r)), sk(r) = r mod 16 (CPR = D/4 ≥ 16) or (r/2) mod 8 (CPR = 8): the 16 rows
//      one quarter-wave reads at one logical chunk fall on 16 distinct 16-byte bank groups;
//   V: chunk position vrow(r)·CPR + (c ^ sv(r)), sv(r) = 8·((r/4) mod 2) (CPR ≥ 16) or 0, vrow(r) = r ^ ((r/4) mod
//      2) (CPR = 8) or r: the two half-waves read rows 4 apart, which then occupy disjoint halves of the banks.
template <int NS, int DK, int DV, int DEPTH = 2 * NS>  // DEPTH: staging tiles in flight before the first product
__global__ void __launch_bounds__(256) attention_fused(const float* __restrict__ Q, int ldq, const float* __restrict__ K,
                                                       int ldk, const float* __restrict__ V, int ldv,
                                                       float* __restrict__ ctx, int H, int Rq, int S, float scale,
                                                       int causal)
{
    static_assert(DK == DV && (DK == 32 || DK == 64 || DK == 128), "head sizes");
    constexpr int D = DK, SK = 32 * NS, CPR = D / 4, TILE = 32 * CPR, PW = TILE / 256;  // PW: DMA ops per wave per tile
    __shared__ __attribute__((aligned(16))) float ks[SK * D];
    __shared__ __attribute__((aligned(16))) float vs[SK * D];
    const int z = blockIdx.y, b = z / H, h = z % H;
    const int tid = threadIdx.x, lane = tid & 63, col = lane & 31, hf = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const float* Kh = K + (size_t)b * S * ldk + (size_t)h * DK;
    const float* Vh = V + (size_t)b * S * ldv + (size_t)h * DV;
    auto sk = [](int r) { return CPR >= 16 ? (r & 15) : ((r >> 1) & 7); };
    auto sv = [](int r) { return CPR >= 16 ? ((r >> 2) & 1) << 3 : 0; };
    auto vrow = [](int r) { return CPR == 8 ? (r ^ ((r >> 2) & 1)) : r; };

    // this lane's 32 Q values of query qi (rows beyond Rq read row Rq − 1 and store nothing): at step c of group g,
    // half-wave hf contracts over d = 8g + 4hf + c (K fragments likewise)
    const int qi = blockIdx.x * 128 + wave * 32 + col;
    const float* Qr = Q + ((size_t)b * Rq + (qi < Rq ? qi : Rq - 1)) * ldq + (size_t)h * DK;
    float4 qf[DK / 8];
#pragma unroll
    for (int g = 0; g < DK / 8; ++g) qf[g] = *reinterpret_cast<const float4*>(Qr + 8 * g + 4 * hf);
    // The staging loads are inline assembly the compiler does not count: have it wait for Q here, before any of them
    // is issued, so that its own wait before the first product does not also wait for the staging.
#pragma unroll
    for (int g = 0; g < DK / 8; ++g) asm volatile("" ::"v"(qf[g].x), "v"(qf[g].y), "v"(qf[g].z), "v"(qf[g].w));

    // staging: LDS-DMA op k of this wave in tile t fills chunk positions p0 .. p0 + 63, lane l position p0 + l
    auto stage = [&](bool isv, int t) {
#pragma unroll
        for (int k = 0; k < PW; ++k) {
            const int p0 = t * TILE + (k * 4 + wave) * 64, p = p0 + lane;
            const int rl = p / CPR, cp = p % CPR;
            const int r = isv ? vrow(rl) : rl, c = cp ^ (isv ? sv(r) : sk(r));
            const float* src = r < S ? (isv ? Vh + (size_t)r * ldv : Kh + (size_t)r * ldk) + 4 * c : knx_attn_zero;
            dma16_at(src, (isv ? vs : ks) + (size_t)p0 * 4);
        }
    };
    // tile i of the staging order: K tile i (i < NS), then V tile i − NS; DEPTH of them issued up front, then one
    // more each time a K tile has been consumed, the rest after the last K tile
    static_assert(DEPTH >= 1 && DEPTH <= 2 * NS, "staging depth");
    auto stage_tile = [&](int i) { stage(i >= NS, i >= NS ? i - NS : i); };
#pragma unroll
    for (int i = 0; i < DEPTH; ++i) stage_tile(i);

    // K fragment of group g: row 32t + col, logical chunk 2g + hf (byte offset within the tile)
    int kb[DK / 8];
#pragma unroll
    for (int g = 0; g < DK / 8; ++g) kb[g] = (col * CPR + ((2 * g + hf) ^ sk(col))) * 16;
    v16f sc[NS];
    unrolled([&](auto tc) {
        constexpr int t = decltype(tc)::value;
#pragma unroll
        for (int e = 0; e < 16; ++e) sc[t][e] = 0.0f;
        // the tiles issued after tile t may stay in flight (DEPTH + t issued so far, at most all 2·NS)
        constexpr int issued = DEPTH + t < 2 * NS ? DEPTH + t : 2 * NS;
        KNX_WAIT_VM_LDS((issued - t - 1) * PW);
        knx_barrier_nofence();
        if (DEPTH + t < 2 * NS) stage_tile(DEPTH + t);  // its LDS region is its own: no wait needed
        if (t == NS - 1)
#pragma unroll
            for (int i = DEPTH + NS; i < 2 * NS; ++i) stage_tile(i);  // the V tiles not issued yet
        const int8_t* kt = reinterpret_cast<const int8_t*>(ks) + t * TILE * 16;
#pragma unroll
        for (int g = 0; g < DK / 8; ++g) {
            const float4 kf = *reinterpret_cast<const float4*>(kt + kb[g]);
#pragma unroll
            for (int c = 0; c < 4; ++c)
                sc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32((&kf.x)[c], (&qf[g].x)[c], sc[t], 0, 0, 0);
        }
    }, std::make_integer_sequence<int, NS>{});

    // element e of tile t is key 32t + 8(e/4) + 4hf + e%4 of query qi
    float m = -INFINITY;
#pragma unroll
    for (int t = 0; t < NS; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int j = 32 * t + 8 * (e >> 2) + 4 * hf + (e & 3);
            float v = scale * sc[t][e];
            if (j >= S || (causal && j > qi)) v = -INFINITY;
            sc[t][e] = v;
            m = v > m ? v : m;
        }
    {
        const float w = __shfl_xor(m, 32, 64);
        m = w > m ? w : m;
    }
    // exp(x − max) as the hardware exp2 of (x − max)·log2(e) (≤ 1-2 ulp): a libm expf is some twenty instructions, and
    // with 64 of them per lane the softmax took as long as the two products; masked keys give exp2(−inf) = 0
    float sum = 0.0f;
#pragma unroll
    for (int t = 0; t < NS; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            sc[t][e] = __builtin_amdgcn_exp2f((sc[t][e] - m) * 1.44269504f);
            sum += sc[t][e];
        }
    sum += __shfl_xor(sum, 32, 64);
    const float inv = 1.0f / sum;
#pragma unroll
    for (int t = 0; t < NS; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) sc[t][e] = sc[t][e] * inv;

    // V value of key j = J + 4hf (J = 32t + 8e4 + c, bit 2 of J clear) and column 32u + col: byte offset
    // J·CPR·16 + vb[J & 1][u]
    int vb[2][DV / 32];
#pragma unroll
    for (int par = 0; par < 2; ++par)
#pragma unroll
        for (int u = 0; u < DV / 32; ++u) {
            const int j = par + 4 * hf;  // the row's low bits; vrow and sv depend on bits 0-2 only
            vb[par][u] = ((vrow(j) - par) * CPR + ((8 * u + (col >> 2)) ^ sv(j))) * 16 + (col & 3) * 4;
        }
    KNX_WAIT_VM_LDS(0);
    knx_barrier_nofence();
    v16f o[DV / 32];
#pragma unroll
    for (int u = 0; u < DV / 32; ++u)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[u][e] = 0.0f;
    const int8_t* vbase = reinterpret_cast<const int8_t*>(vs);
#pragma unroll
    for (int t = 0; t < NS; ++t)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4)
#pragma unroll
            for (int u = 0; u < DV / 32; ++u)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int J = 32 * t + 8 * e4 + c;
                    const float vv = *reinterpret_cast<const float*>(vbase + J * CPR * 16 + vb[c & 1][u]);
                    o[u] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv, sc[t][4 * e4 + c], o[u], 0, 0, 0);
                }
    if (qi >= Rq) return;
    // element e of o[u] is ctx column 32u + 8(e/4) + 4hf + e%4 of query qi
    float* y = ctx + ((size_t)b * Rq + qi) * ((size_t)H * DV) + (size_t)h * DV + 4 * hf;
#pragma unroll
    for (int u = 0; u < DV / 32; ++u)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4)
            *reinterpret_cast<float4*>(y + 32 * u + 8 * e4) =
                make_float4(o[u][4 * e4], o[u][4 * e4 + 1], o[u][4 * e4 + 2], o[u][4 * e4 + 3]);
}

struct AttnArgs {
    const float* Q;
    int ldq;
    const float* K;
    int ldk;
    const float* V;
    int ldv;
    float* ctx;
    int B, H, Rq, S, dk, dv;
    float scale;
    int causal;
};

template <int NS, int D, int DEPTH>
int launch_fused_d(const AttnArgs& a, hipStream_t s, const char* name)
{
    constexpr int DP = DEPTH < 2 * NS ? DEPTH : 2 * NS;
    hipLaunchKernelGGL((attention_fused<NS, D, D, DP>), dim3((a.Rq + 127) / 128, a.B * a.H), dim3(256), 0, s, a.Q, a.ldq,
                       a.K, a.ldk, a.V, a.ldv, a.ctx, a.H, a.Rq, a.S, a.scale, a.causal);
    return knx::check_launch(name);
}

template <int NS, int D>
int launch_fused(const AttnArgs& a, hipStream_t s, const char* name)
{
    // three 32-key tiles in flight up front, one more per consumed K tile: with all of K and V requested at once by
    // every workgroup (64 KB each at S = 128, d = 64) a workgroup's first tile arrives anywhere in the 32 MB stream
    // (B 64, H 8, S 128, d 64: 26.5 µs at depth 3, 26.7 at 2 and 4, 27.3 at 6, 27.8 with everything up front)
    const char* dep = getenv("KNX_ATTN_DEPTH");  // tuning and tests: 2, 4, 6, or "all"
    if (dep != nullptr && strcmp(dep, "all") == 0) return launch_fused_d<NS, D, 2 * NS>(a, s, name);
    const int d = dep != nullptr ? atoi(dep) : 3;
    if (d == 2) return launch_fused_d<NS, D, 2>(a, s, name);
    if (d == 4) return launch_fused_d<NS, D, 4>(a, s, name);
    if (d == 6) return launch_fused_d<NS, D, 6>(a, s, name);
    return launch_fused_d<NS, D, 3>(a, s, name);
}

// the fused kernel when dk = dv ∈ {32, 64, 128}, S fits its LDS tiles and every row is 16-byte aligned; 1 = not eligible
int try_fused(const AttnArgs& a, hipStream_t s, const char* name)
{
    const char* force = getenv("KNX_ATTN_KERNEL");
    if (force != nullptr && strcmp(force, "unfused") == 0) return 1;
    if (a.dk != a.dv || (((uintptr_t)a.Q | (uintptr_t)a.K | (uintptr_t)a.V | (uintptr_t)a.ctx) & 15) != 0 ||
        ((a.ldq | a.ldk | a.ldv) & 3) != 0)
        return 1;
    if ((long long)a.B * a.H > 65535) return 1;  // grid.y
    const int ns = a.S <= 32 ? 1 : a.S <= 64 ? 2 : a.S <= 128 ? 4 : a.S <= 256 ? 8 : 0;
    if (ns == 0 || (a.dk == 128 && ns == 8)) return 1;
#define KNX_FUSED_NS(D)                                         \
    switch (ns) {                                              \
    case 1: return launch_fused<1, D>(a, s, name);             \
    case 2: return launch_fused<2, D>(a, s, name);             \
    case 4: return launch_fused<4, D>(a, s, name);             \
    default: return launch_fused<8, D>(a, s, name);            \
    }
    switch (a.dk) {
    case 32: KNX_FUSED_NS(32)
    case 64: KNX_FUSED_NS(64)
    case 128:
        switch (ns) {
        case 1: return launch_fused<1, 128>(a, s, name);
        case 2: return launch_fused<2, 128>(a, s, name);
        default: return launch_fused<4, 128>(a, s, name);
        }
    default: return 1;
    }
#undef KNX_FUSED_NS
}

}  // namespace

extern "C" int knx_hip_attention_core_ex(const float* Q, int ldq, const float* K, int ldk, const float* V, int ldv,
                                         float* vt, float* ctx, float* scores, int B, int H, int Rq, int S, int dk,
                                         int dv, float scale, int causal, void* stream)
{
    const char* name = "knx_hip_attention_core";
    KNX_ENTRY(name);
    KNX_REQUIRE(B >= 0 && H >= 1 && Rq >= 1 && S >= 1 && dk >= 1 && dv >= 1, name);
    if (B == 0) return KNX_OK;
    KNX_REQUIRE(Q && K && V && ctx, name);
    KNX_REQUIRE((long long)ldq >= (long long)H * dk && (long long)ldk >= (long long)H * dk &&
                    (long long)ldv >= (long long)H * dv, name);
    KNX_REQUIRE((long long)B * H * Rq * S <= (1LL << 40) && (long long)B * S * H * dv <= 0x7fffffffLL, name);
    hipStream_t s = knx::as_stream(stream);
    const AttnArgs a{Q, ldq, K, ldk, V, ldv, ctx, B, H, Rq, S, dk, dv, scale, causal};
    int rc = try_fused(a, s, name);
    if (rc != 1) return rc;
    KNX_REQUIRE(scores != nullptr, name);
    const long long hdv = (long long)H * dv, RS = (long long)Rq * S;
    rc = knx_sgemm_batched(Rq, S, dk, Q, ldq, Rq * (long long)ldq, dk, K, ldk, S * (long long)ldk, dk, true, scores, S,
                           H * RS, RS, B, H, scale, causal, s);
    if (rc != KNX_OK) return rc;
    rc = knx_hip_softmax(scores, scores, B * H * Rq, S, stream);
    if (rc != KNX_OK) return rc;
    if (vt == nullptr)
        return knx_sgemm_batched(Rq, dv, S, scores, S, H * RS, RS, V, ldv, S * (long long)ldv, dv, false, ctx, (int)hdv,
                                 Rq * hdv, dv, B, H, 1.0f, 0, s);
    // P·V as an NT product against Vᵀ: head h of batch b is rows h·dv.. of Vt, columns b·S.. (row stride B·S)
    const int R = B * S, C = (int)hdv;
    KNX_REQUIRE((C + 31) / 32 <= 65535, name);
    hipLaunchKernelGGL(transpose_kernel, dim3((R + 31) / 32, (C + 31) / 32), dim3(256), 0, s, V, R, C, ldv, vt);
    rc = knx::check_launch(name);
    if (rc != KNX_OK) return rc;
    return knx_sgemm_batched(Rq, dv, S, scores, S, H * RS, RS, vt, R, S, (long long)dv * R, true, ctx, (int)hdv, Rq * hdv,
                             dv, B, H, 1.0f, 0, s);
}

extern "C" int knx_hip_attention_core(const float* Q, const float* K, const float* V, float* ctx, float* scores, int B,
                                      int H, int Rq, int S, int dk, int dv, float scale, int causal, void* stream)
{
    return knx_hip_attention_core_ex(Q, H * dk, K, H * dk, V, H * dv, nullptr, ctx, scores, B, H, Rq, S, dk, dv, scale,
                                     causal, stream);
}
