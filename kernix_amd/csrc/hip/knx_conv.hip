// knx_conv.hip — NHWC convolution as an implicit GEMM on v_mfma_f32_32x32x2_f32 (gfx950).
//
// Replaces kernix_conv_run's tiled im2col → cblas_sgemm → bias_act (reference include/kernix_model.h:711-771,
// im2col :677-693): the GEMM is out[m][n] = Σ_k A[m][k]·W[k][n] with m = (b, oy, ox), k = (ky, kx, ci) and
// A[m][k] = x[b, oy·sh − pt + ky·dh, ox·sw − pl + kx·dw, ci] (0 outside the image).  Each workgroup gathers its
// BM×16 slice of A directly from the input into LDS, so the column matrix never exists in HBM; bias and activation
// are applied in the epilogue.  Groups run as grid.y (each group is an independent GEMM over its channel slice).
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
