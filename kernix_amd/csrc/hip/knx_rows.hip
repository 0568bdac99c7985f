// knx_rows.hip — bandwidth-bound row and elementwise kernels of the KERNIX forward (gfx950).
//
// Row ops (layer_norm, softmax) run one 64-lane wavefront per row with DPP/permute reductions; elementwise ops are
// grid-stride loops with one element per lane per iteration (consecutive lanes → consecutive addresses, so each
// wave moves 256 contiguous bytes per access).  Formulas follow the reference CPU path line for line (file:line at
// each kernel); summation order inside a row is the wave's tree order, which is why fp32 parity is by tolerance.
#include "knx_common.hpp"

namespace {

inline unsigned grid_for(size_t n, unsigned block = 256)
{
    size_t g = (n + block - 1) / block;
    const size_t cap = (size_t)knx::num_cus() * 16;
    return (unsigned)(g < 1 ? 1 : g > cap ? cap : g);
}

// ---- layer_norm: reference include/kernix.h:667-677 (biased variance, rstd = 1/sqrtf(ss/cols + eps)) ----
__global__ void __launch_bounds__(256) layernorm_kernel(const float* __restrict__ x, float* y, int rows, int cols,
                                                         const float* __restrict__ gamma, const float* __restrict__ beta,
                                                         float eps)
{
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* xr = x + (size_t)row * cols;
    float* yr = y + (size_t)row * cols;
    float s = 0.0f;
    for (int j = lane; j < cols; j += 64) s += xr[j];
    const float mean = knx_wave_sum(s) / (float)cols;
    float ss = 0.0f;
    for (int j = lane; j < cols; j += 64) { const float d = xr[j] - mean; ss += d * d; }
    const float rstd = 1.0f / sqrtf(knx_wave_sum(ss) / (float)cols + eps);
    for (int j = lane; j < cols; j += 64) {
        float v = (xr[j] - mean) * rstd;
        if (gamma && beta) v = v * gamma[j] + beta[j];
        else if (gamma) v = v * gamma[j];
        else if (beta) v = v + beta[j];
        yr[j] = v;
    }
}

// ---- softmax: reference include/kernix.h:652-657 (exp(x − max) · (1/Σ)) ----
__global__ void __launch_bounds__(256) softmax_kernel(const float* __restrict__ x, float* y, int rows, int cols)
{
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* xr = x + (size_t)row * cols;
    float* yr = y + (size_t)row * cols;
    float m = -INFINITY;
    for (int j = lane; j < cols; j += 64) m = xr[j] > m ? xr[j] : m;
    m = knx_wave_max(m);
    float s = 0.0f;
    for (int j = lane; j < cols; j += 64) s += expf(xr[j] - m);
    const float inv = 1.0f / knx_wave_sum(s);
    for (int j = lane; j < cols; j += 64) yr[j] = expf(xr[j] - m) * inv;
}

// ---- register-resident row kernels ----
// G lanes per row (16, 32 or 64), NV float4 per lane: used when cols % 4 == 0, cols ≤ 4·G·NV and the rows are 16-byte
// aligned.  Each row is read from memory once (16-byte loads) and kept in registers for every pass over it.
template <int G>
__device__ __forceinline__ float group_sum(float v)
{
    return knx_lane_group_sum(v, G);  // DPP and gfx950's register swaps (every lane of the group gets the sum)
}
template <int G>
__device__ __forceinline__ float group_max(float v)
{
#pragma unroll
    for (int o = G / 2; o >= 1; o >>= 1) { const float w = __shfl_xor(v, o, 64); v = w > v ? w : v; }
    return v;
}
__device__ __forceinline__ float f4(const float4& v, int e) { return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w; }

// layer_norm of one row, same formulas as layernorm_kernel: lane l of the row's G lanes gets its float4 chunks
// l, l + G, … of the normalized row in o (chunks past the row are left unset)
template <int G, int NV>
__device__ __forceinline__ void ln_row(const float* x, int row, int cols, int l, const float* __restrict__ gamma,
                                       const float* __restrict__ beta, float eps, float4 (&o)[NV])
{
    const float4* xr = reinterpret_cast<const float4*>(x + (size_t)row * cols);
    const int nq = cols >> 2;
    float4 v[NV];
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int q = i * G + l;
        v[i] = q < nq ? xr[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    }
    const float mean = group_sum<G>(s) / (float)cols;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
        if (i * G + l < nq)
#pragma unroll
            for (int e = 0; e < 4; ++e) { const float d = f4(v[i], e) - mean; ss += d * d; }
    const float rstd = 1.0f / sqrtf(group_sum<G>(ss) / (float)cols + eps);
    const float4* g4 = reinterpret_cast<const float4*>(gamma);  // 16-byte aligned (checked by the caller)
    const float4* b4 = reinterpret_cast<const float4*>(beta);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int q = i * G + l;
        if (q >= nq) continue;
        const float4 gq = gamma ? g4[q] : make_float4(1.f, 1.f, 1.f, 1.f);
        const float4 bq = beta ? b4[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        float t4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float t = (f4(v[i], e) - mean) * rstd;
            if (gamma && beta) t = t * f4(gq, e) + f4(bq, e);
            else if (gamma) t = t * f4(gq, e);
            else if (beta) t = t + f4(bq, e);
            t4[e] = t;
        }
        o[i] = make_float4(t4[0], t4[1], t4[2], t4[3]);
    }
}

// layer_norm (x may alias y: every lane reads its whole row before writing)
template <int G, int NV>
__global__ void __launch_bounds__(256) layernorm_vec(const float* x, float* y, int rows, int cols,
                                                      const float* __restrict__ gamma, const float* __restrict__ beta,
                                                      float eps)
{
    const int row = blockIdx.x * (256 / G) + (int)threadIdx.x / G, l = threadIdx.x % G;
    if (row >= rows) return;
    float4 o[NV];
    ln_row<G, NV>(x, row, cols, l, gamma, beta, eps, o);
    float4* yr = reinterpret_cast<float4*>(y + (size_t)row * cols);
    const int nq = cols >> 2;
#pragma unroll
    for (int i = 0; i < NV; ++i)
        if (i * G + l < nq) yr[i * G + l] = o[i];
}

// layer_norm followed by the per-row int8 quantization of kernix_qmatmul (the steps of knx_hip_quantize_rows: s = m/127
// from the row's largest magnitude m, or 1 for an all-zero row; inv = 1/s; rint(x·inv) clamped to ±127; a row with
// NaN or ±inf gets s = NaN and zeros) on the normalized row while it is still in registers: the int8 row (kp bytes,
// zero past cols) and its scale are the result, the fp32 row is never written.  Same G, NV and arithmetic as
// layernorm_vec and a maximum is exact in any order, so the bits are those of layer_norm then quantize_rows.
template <int G, int NV>
__global__ void __launch_bounds__(256) layernorm_quant_vec(const float* x, int rows, int cols,
                                                            const float* __restrict__ gamma,
                                                            const float* __restrict__ beta, float eps, int kp,
                                                            int8_t* __restrict__ xq, float* __restrict__ sx)
{
    const int row = blockIdx.x * (256 / G) + (int)threadIdx.x / G, l = threadIdx.x % G;
    if (row >= rows) return;
    float4 o[NV];
    ln_row<G, NV>(x, row, cols, l, gamma, beta, eps, o);
    const int nq = cols >> 2, nqp = kp >> 2;
    // the quantizer's operations as knx_hip_quantize_rows: the row maximum of |x| as integer bits (NaN above ±inf above
    // every finite value), q = clamp(rint(x·inv), ±127) by v_med3, bytes by cvt_pk_u8 of q + 128, ^ 0x80
    unsigned mb = 0u;
#pragma unroll
    for (int i = 0; i < NV; ++i)
        if (i * G + l < nq)
#pragma unroll
            for (int e = 0; e < 4; ++e) mb = max(mb, __float_as_uint(f4(o[i], e)) & 0x7fffffffu);
    mb = knx_lane_group_max(mb, G);
    int* qr = reinterpret_cast<int*>(xq + (size_t)row * kp);
    if (mb >= 0x7f800000u) {  // NaN or ±inf
        for (int q = l; q < nqp; q += G) qr[q] = 0;
        if (l == 0) sx[row] = __int_as_float(0x7fc00000);
        return;
    }
    const float m = __uint_as_float(mb);
    const float s = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
    const float inv = __fdiv_rn(1.0f, s);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int q = i * G + l;
        if (q >= nq) continue;
        unsigned w = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            w = __builtin_amdgcn_cvt_pk_u8_f32(
                __builtin_amdgcn_fmed3f(rintf(f4(o[i], e) * inv), -127.0f, 127.0f) + 128.0f, e, w);
        qr[q] = (int)(w ^ 0x80808080u);
    }
    for (int q = nq + l; q < nqp; q += G) qr[q] = 0;
    if (l == 0) sx[row] = s;
}

// softmax, same formulas as softmax_kernel; exp(x − max) is computed once and kept
template <int G, int NV>
__global__ void __launch_bounds__(256) softmax_vec(const float* x, float* y, int rows, int cols)
{
    const int row = blockIdx.x * (256 / G) + (int)threadIdx.x / G, l = threadIdx.x % G;
    if (row >= rows) return;
    const float4* xr = reinterpret_cast<const float4*>(x + (size_t)row * cols);
    const int nq = cols >> 2;
    float4 v[NV];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int q = i * G + l;
        v[i] = q < nq ? xr[q] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
#pragma unroll
        for (int e = 0; e < 4; ++e) m = f4(v[i], e) > m ? f4(v[i], e) : m;
    }
    m = group_max<G>(m);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        if (i * G + l >= nq) continue;
        v[i] = make_float4(expf(v[i].x - m), expf(v[i].y - m), expf(v[i].z - m), expf(v[i].w - m));
        s += v[i].x;
        s += v[i].y;
        s += v[i].z;
        s += v[i].w;
    }
    const float inv = 1.0f / group_sum<G>(s);
    float4* yr = reinterpret_cast<float4*>(y + (size_t)row * cols);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int q = i * G + l;
        if (q < nq) yr[q] = make_float4(v[i].x * inv, v[i].y * inv, v[i].z * inv, v[i].w * inv);
    }
}

// picks G and NV for a row of nq float4 (nq ≤ 512) and launches K<G, NV>
#define KNX_ROWVEC_DISPATCH(K, nq, rows, stream, ...)                                                                \
    do {                                                                                                            \
        hipStream_t st_ = knx::as_stream(stream);                                                                   \
        if ((nq) <= 16) hipLaunchKernelGGL((K<16, 1>), dim3(((rows) + 15) / 16), dim3(256), 0, st_, __VA_ARGS__);   \
        else if ((nq) <= 32) hipLaunchKernelGGL((K<32, 1>), dim3(((rows) + 7) / 8), dim3(256), 0, st_, __VA_ARGS__); \
        else if ((nq) <= 64) hipLaunchKernelGGL((K<64, 1>), dim3(((rows) + 3) / 4), dim3(256), 0, st_, __VA_ARGS__); \
        else if ((nq) <= 128) hipLaunchKernelGGL((K<64, 2>), dim3(((rows) + 3) / 4), dim3(256), 0, st_, __VA_ARGS__); \
        else if ((nq) <= 256) hipLaunchKernelGGL((K<64, 4>), dim3(((rows) + 3) / 4), dim3(256), 0, st_, __VA_ARGS__); \
        else hipLaunchKernelGGL((K<64, 8>), dim3(((rows) + 3) / 4), dim3(256), 0, st_, __VA_ARGS__);                \
    } while (0)

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// ---- bias + activation, 4 consecutive elements per lane (cols % 4 == 0, 16-byte aligned); ACT ≥ −1 compile time ----
template <int ACT>
__global__ void __launch_bounds__(256) bias_act_vec(const float* x, float* y, size_t n4, int cols,
                                                     const float* __restrict__ bias, int act, float alpha)
{
    const float4* x4 = reinterpret_cast<const float4*>(x);
    float4* y4 = reinterpret_cast<float4*>(y);
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x) {
        float4 v = x4[i];
        if (bias) {
            const float4 b = *reinterpret_cast<const float4*>(bias + (i * 4) % cols);
            v = make_float4(v.x + b.x, v.y + b.y, v.z + b.z, v.w + b.w);
        }
        if (ACT == -2) v = make_float4(knx_act(v.x, act, alpha), knx_act(v.y, act, alpha), knx_act(v.z, act, alpha),
                                       knx_act(v.w, act, alpha));
        else if (ACT >= 0) v = make_float4(knx_act(v.x, ACT, alpha), knx_act(v.y, ACT, alpha), knx_act(v.z, ACT, alpha),
                                           knx_act(v.w, ACT, alpha));
        y4[i] = v;
    }
}

// ---- same-shape binary (no broadcast), 4 elements per lane ----
__global__ void __launch_bounds__(256) binary_vec(int op, const float* a, const float* b, float* y, size_t n4);

// ---- bias + activation: reference include/kernix_model.h:528-541 ----
__global__ void __launch_bounds__(256) bias_act_kernel(const float* x, float* y, size_t n, int cols,
                                                        const float* __restrict__ bias, int act, float alpha)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        float v = x[i];
        if (bias) v = v + bias[i % cols];
        y[i] = knx_act(v, act, alpha);
    }
}

// ---- broadcast binary: reference include/kernix_model.h:864-906 ----
__device__ __forceinline__ float bin1(int op, float a, float b)
{
    switch (op) {
    case 0: return a + b;
    case 1: return a - b;
    case 2: return a * b;
    case 3: return a / b;
    case 4: return a > b ? a : b;
    default: return a < b ? a : b;
    }
}

__global__ void __launch_bounds__(256) binary_vec(int op, const float* a, const float* b, float* y, size_t n4)
{
    const float4* a4 = reinterpret_cast<const float4*>(a);
    const float4* b4 = reinterpret_cast<const float4*>(b);
    float4* y4 = reinterpret_cast<float4*>(y);
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x) {
        const float4 u = a4[i], w = b4[i];
        y4[i] = make_float4(bin1(op, u.x, w.x), bin1(op, u.y, w.y), bin1(op, u.z, w.z), bin1(op, u.w, w.w));
    }
}

__global__ void __launch_bounds__(256) binary_kernel(int op, const float* a, int ra, int ca, const float* b, int rb, int cb,
                                                      float* y, size_t n, int R, int C)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const size_t row = i / C, j = i % C, bi = row / R, ri = row % R;
        const float av = a[(bi * ra + (ra == 1 ? 0 : ri)) * ca + (ca == 1 ? 0 : j)];
        const float bv = b[(bi * rb + (rb == 1 ? 0 : ri)) * cb + (cb == 1 ? 0 : j)];
        y[i] = bin1(op, av, bv);
    }
}

// ---- global pool: reference include/kernix_model.h:810-830 (sequential over rows, avg = Σ·(1/R)) ----
__global__ void __launch_bounds__(256) global_pool_kernel(int type, const float* __restrict__ x, int B, int R, int C,
                                                           float* __restrict__ y)
{
    const size_t n = (size_t)B * C;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const size_t b = i / C, c = i % C;
        const float* xp = x + b * (size_t)R * C + c;
        float o = xp[0];
        int r = 1;
        // 32 loads in flight (there is one thread per output, too few to cover the memory latency with less),
        // combined in row order (the reference's sequential order)
        for (; r + 32 <= R; r += 32) {
            float v[32];
#pragma unroll
            for (int u = 0; u < 32; ++u) v[u] = xp[(size_t)(r + u) * C];
#pragma unroll
            for (int u = 0; u < 32; ++u) o = type == 0 ? (o > v[u] ? o : v[u]) : o + v[u];
        }
        for (; r + 8 <= R; r += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = xp[(size_t)(r + u) * C];
#pragma unroll
            for (int u = 0; u < 8; ++u) o = type == 0 ? (o > v[u] ? o : v[u]) : o + v[u];
        }
        for (; r < R; ++r) {
            const float v = xp[(size_t)r * C];
            o = type == 0 ? (o > v ? o : v) : o + v;
        }
        if (type == 1) o = o * (1.0f / (float)R);
        y[i] = o;
    }
}

// ---- affine / add_const: reference include/kernix_model.h:1882-1896 ----
__global__ void __launch_bounds__(256) affine_kernel(const float* x, float* y, size_t n, int cols,
                                                      const float* __restrict__ scale, const float* __restrict__ shift)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const int c = (int)(i % cols);
        y[i] = x[i] * scale[c] + shift[c];
    }
}

__global__ void __launch_bounds__(256) add_const_kernel(const float* x, float* y, size_t n, int per,
                                                         const float* __restrict__ cst)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        y[i] = x[i] + cst[i % per];
}

// ---- windowed pooling: reference include/kernix_model.h:773-807 ----
__global__ void __launch_bounds__(256) pool_kernel(int type, knx_conv_geom g, int count_pad, const float* __restrict__ x,
                                                    float* __restrict__ y)
{
    const size_t n = (size_t)g.B * g.Ho * g.Wo * g.C;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const size_t c = i % g.C, r = i / g.C;
        const size_t b = r / ((size_t)g.Ho * g.Wo), oy = (r / g.Wo) % g.Ho, ox = r % g.Wo;
        float o = type == 0 ? -INFINITY : 0.0f;
        int cnt = 0;
        for (int ky = 0; ky < g.kh; ++ky) {
            const long iy = (long)oy * g.sh - g.pt + ky;
            if (iy < 0 || iy >= g.H) continue;
            for (int kx = 0; kx < g.kw; ++kx) {
                const long ix = (long)ox * g.sw - g.pl + kx;
                if (ix < 0 || ix >= g.W) continue;
                const float v = x[(((size_t)b * g.H + iy) * g.W + ix) * g.C + c];
                o = type == 0 ? (o > v ? o : v) : o + v;
                cnt++;
            }
        }
        if (type == 1) o = o * (1.0f / (float)(count_pad ? g.kh * g.kw : (cnt ? cnt : 1)));
        y[i] = o;
    }
}

// ---- permute: reference include/kernix_model.h:833-862 ----
struct PermArgs { int nd; int od[4]; int ist[4]; };

__global__ void __launch_bounds__(256) permute_kernel(const float* __restrict__ x, float* __restrict__ y, size_t total,
                                                       size_t per, PermArgs a)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const size_t b = i / per;
        size_t rem = i % per, src = 0;
        for (int k = a.nd - 1; k >= 0; --k) {
            src += (rem % (size_t)a.od[k]) * (size_t)a.ist[k];
            rem /= (size_t)a.od[k];
        }
        y[i] = x[b * per + src];
    }
}

// ---- column block copy (CONCAT / SELECT): reference include/kernix_model.h:908-949 ----
__global__ void __launch_bounds__(256) copy_cols_kernel(const float* __restrict__ x, int ldx, int x_off, float* __restrict__ y,
                                                         int ldy, int y_off, int rows, int n)
{
    const size_t total = (size_t)rows * n;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / n, j = i % n;
        y[r * ldy + y_off + j] = x[r * ldx + x_off + j];
    }
}

// ---- zero padding / nearest upsampling: reference include/kernix_model.h:951-984 ----
__global__ void __launch_bounds__(256) pad_kernel(const float* __restrict__ x, float* __restrict__ y, int B, int H, int W,
                                                   int C, int Ho, int Wo, int pt, int pl)
{
    const size_t n = (size_t)B * Ho * Wo * C;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const size_t c = i % C, r = i / C;
        const size_t b = r / ((size_t)Ho * Wo);
        const long iy = (long)((r / Wo) % Ho) - pt, ix = (long)(r % Wo) - pl;
        y[i] = (iy >= 0 && iy < H && ix >= 0 && ix < W) ? x[(((size_t)b * H + iy) * W + ix) * C + c] : 0.0f;
    }
}

__global__ void __launch_bounds__(256) upsample_kernel(const float* __restrict__ x, float* __restrict__ y, int B, int H,
                                                        int W, int C, int sh, int sw)
{
    const int Ho = H * sh, Wo = W * sw;
    const size_t n = (size_t)B * Ho * Wo * C;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const size_t c = i % C, r = i / C;
        const size_t b = r / ((size_t)Ho * Wo), oy = (r / Wo) % Ho, ox = r % Wo;
        y[i] = x[(((size_t)b * H + oy / sh) * W + ox / sw) * C + c];
    }
}

// ---- embedding: reference include/kernix_model.h:987-1000 ----
__global__ void __launch_bounds__(256) embedding_kernel(const float* __restrict__ ids, int n, const float* __restrict__ table,
                                                         int V, int D, float* __restrict__ y)
{
    const size_t total = (size_t)n * D;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / D, j = i % D;
        const float id = ids[r];
        y[i] = (id >= 0.0f && id < (float)V && id == floorf(id)) ? table[(size_t)id * D + j] : __int_as_float(0x7fc00000);
    }
}

// ---- RNN gates for one timestep: reference include/kernix_model.h:594-627 ----
// kind 4 LSTM (i f g o), 5 GRU (z r h, reset_after), 6 SimpleRNN.  z: B×gu input projection of this step (+ h·U for
// LSTM/RNN when hu == NULL it is already included); hu: B×gu recurrent term to add (LSTM/RNN) or the GRU recurrent
// term zh = brec + h·U (GRU).  c, h: B×u state.  dst: h written at dst + b·dst_stride when dst != NULL.

__global__ void __launch_bounds__(256) rnn_gates_kernel(int kind, int act, float alpha, int B, int u, int step0, float* z,
                                                         const float* hu, float* c, float* h, float* dst, int dst_stride)
{
    const int n = B * u;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const int b = i / u, j = i % u;
        if (kind == 4) {
            float* zb = z + (size_t)b * 4 * u;
            float zi = zb[j], zf = zb[u + j], zg = zb[2 * u + j], zo = zb[3 * u + j];
            if (hu) {
                const float* hb = hu + (size_t)b * 4 * u;
                zi = zi + hb[j]; zf = zf + hb[u + j]; zg = zg + hb[2 * u + j]; zo = zo + hb[3 * u + j];
            }
            float cv = step0 ? 0.0f : c[i];
            const float hv = knx_lstm_cell(zi, zf, zg, zo, act, alpha, step0, cv);
            c[i] = cv;
            h[i] = hv;
            if (dst) dst[(size_t)b * dst_stride + j] = hv;
        } else if (kind == 5) {
            float* zb = z + (size_t)b * 3 * u;
            const float* hz = hu + (size_t)b * 3 * u;
            const float prev = step0 ? 0.0f : h[i];
            const float hv = knx_gru_cell(zb[j], zb[u + j], zb[2 * u + j], hz[j], hz[u + j], hz[2 * u + j], act, alpha,
                                          step0, prev);
            h[i] = hv;
            if (dst) dst[(size_t)b * dst_stride + j] = hv;
        } else {
            float v = z[(size_t)b * u + j];
            if (hu) v = v + hu[(size_t)b * u + j];
            const float hv = knx_gate_act(v, act, alpha);
            h[i] = hv;
            if (dst) dst[(size_t)b * dst_stride + j] = hv;
        }
    }
}

}  // namespace

#define KNX_LAUNCH(name, kernel, grid, ...)                                                   \
    do {                                                                                      \
        hipLaunchKernelGGL(kernel, dim3(grid), dim3(256), 0, knx::as_stream(stream), __VA_ARGS__); \
        return knx::check_launch(name);                                                       \
    } while (0)

extern "C" int knx_hip_layernorm(const float* x, float* y, int rows, int cols, const float* gamma, const float* beta,
                                 float eps, void* stream)
{
    const char* name = "knx_hip_layernorm";
    KNX_ENTRY(name);
    KNX_REQUIRE(rows >= 0 && cols >= 1, name);
    if (rows == 0) return KNX_OK;
    KNX_REQUIRE(x && y, name);
    if (cols % 4 == 0 && cols / 4 <= 512 && aligned16(x) && aligned16(y) && aligned16(gamma) && aligned16(beta)) {
        KNX_ROWVEC_DISPATCH(layernorm_vec, cols / 4, rows, stream, x, y, rows, cols, gamma, beta, eps);
        return knx::check_launch(name);
    }
    KNX_LAUNCH(name, layernorm_kernel, (rows + 3) / 4, x, y, rows, cols, gamma, beta, eps);
}

extern "C" int knx_hip_layernorm_quantize(const float* x, int rows, int cols, const float* gamma, const float* beta,
                                          float eps, int kp, int8_t* xq, float* sx, void* stream)
{
    const char* name = "knx_hip_layernorm_quantize";
    KNX_ENTRY(name);
    KNX_REQUIRE(rows >= 0 && cols >= 4 && cols % 4 == 0 && cols / 4 <= 512 && kp >= cols && kp % 4 == 0, name);
    if (rows == 0) return KNX_OK;
    KNX_REQUIRE(x && xq && sx && aligned16(x) && aligned16(gamma) && aligned16(beta) && ((uintptr_t)xq & 3) == 0, name);
    KNX_ROWVEC_DISPATCH(layernorm_quant_vec, cols / 4, rows, stream, x, rows, cols, gamma, beta, eps, kp, xq, sx);
    return knx::check_launch(name);
}

extern "C" int knx_hip_softmax(const float* x, float* y, int rows, int cols, void* stream)
{
    const char* name = "knx_hip_softmax";
    KNX_ENTRY(name);
    KNX_REQUIRE(rows >= 0 && cols >= 1, name);
    if (rows == 0) return KNX_OK;
    KNX_REQUIRE(x && y, name);
    if (cols % 4 == 0 && cols / 4 <= 512 && aligned16(x) && aligned16(y)) {
        KNX_ROWVEC_DISPATCH(softmax_vec, cols / 4, rows, stream, x, y, rows, cols);
        return knx::check_launch(name);
    }
    KNX_LAUNCH(name, softmax_kernel, (rows + 3) / 4, x, y, rows, cols);
}

extern "C" int knx_hip_bias_act(const float* x, float* y, int rows, int cols, const float* bias, int act, float alpha,
                                void* stream)
{
    const char* name = "knx_hip_bias_act";
    KNX_ENTRY(name);
    KNX_REQUIRE(rows >= 0 && cols >= 1 && act >= -1 && act <= 15, name);
    const size_t n = (size_t)rows * cols;
    if (n == 0) return KNX_OK;
    KNX_REQUIRE(x && y, name);
    if (cols % 4 == 0 && aligned16(x) && aligned16(y) && (bias == nullptr || aligned16(bias))) {
        const size_t n4 = n / 4;
        // activation ids of the file format: 0 relu, 1 gelu
        if (act == 0) KNX_LAUNCH(name, bias_act_vec<0>, grid_for(n4), x, y, n4, cols, bias, act, alpha);
        if (act == 1) KNX_LAUNCH(name, bias_act_vec<1>, grid_for(n4), x, y, n4, cols, bias, act, alpha);
        if (act == -1) KNX_LAUNCH(name, bias_act_vec<-1>, grid_for(n4), x, y, n4, cols, bias, act, alpha);
        KNX_LAUNCH(name, bias_act_vec<-2>, grid_for(n4), x, y, n4, cols, bias, act, alpha);
    }
    KNX_LAUNCH(name, bias_act_kernel, grid_for(n), x, y, n, cols, bias, act, alpha);
}

extern "C" int knx_hip_binary(int op, const float* a, int ra, int ca, const float* b, int rb, int cb, float* y, int B,
                              int R, int C, void* stream)
{
    const char* name = "knx_hip_binary";
    KNX_ENTRY(name);
    KNX_REQUIRE(op >= 0 && op <= 5 && B >= 0 && R >= 1 && C >= 1, name);
    KNX_REQUIRE((ra == R || ra == 1) && (rb == R || rb == 1) && (ca == C || ca == 1) && (cb == C || cb == 1), name);
    const size_t n = (size_t)B * R * C;
    if (n == 0) return KNX_OK;
    KNX_REQUIRE(a && b && y, name);
    if (ra == R && rb == R && ca == C && cb == C && n % 4 == 0 && aligned16(a) && aligned16(b) && aligned16(y))
        KNX_LAUNCH(name, binary_vec, grid_for(n / 4), op, a, b, y, n / 4);
    KNX_LAUNCH(name, binary_kernel, grid_for(n), op, a, ra, ca, b, rb, cb, y, n, R, C);
}

extern "C" int knx_hip_global_pool(int type, const float* x, int B, int R, int C, float* y, void* stream)
{
    const char* name = "knx_hip_global_pool";
    KNX_ENTRY(name);
    KNX_REQUIRE((type == 0 || type == 1) && B >= 0 && R >= 1 && C >= 1 && x != y, name);
    if (B == 0) return KNX_OK;
    KNX_REQUIRE(x && y, name);
    KNX_LAUNCH(name, global_pool_kernel, grid_for((size_t)B * C), type, x, B, R, C, y);
}

extern "C" int knx_hip_affine(const float* x, float* y, int rows, int cols, const float* scale, const float* shift,
                              void* stream)
{
    const char* name = "knx_hip_affine";
    KNX_ENTRY(name);
    KNX_REQUIRE(rows >= 0 && cols >= 1, name);
    const size_t n = (size_t)rows * cols;
    if (n == 0) return KNX_OK;
    KNX_REQUIRE(x && y && scale && shift, name);
    KNX_LAUNCH(name, affine_kernel, grid_for(n), x, y, n, cols, scale, shift);
}

extern "C" int knx_hip_add_const(const float* x, float* y, int B, int per, const float* cst, void* stream)
{
    const char* name = "knx_hip_add_const";
    KNX_ENTRY(name);
    KNX_REQUIRE(B >= 0 && per >= 1, name);
    const size_t n = (size_t)B * per;
    if (n == 0) return KNX_OK;
    KNX_REQUIRE(x && y && cst, name);
    KNX_LAUNCH(name, add_const_kernel, grid_for(n), x, y, n, per, cst);
}

extern "C" int knx_hip_pool(int type, const knx_conv_geom* g, int count_pad, const float* x, float* y, void* stream)
{
    const char* name = "knx_hip_pool";
    KNX_ENTRY(name);
    KNX_REQUIRE(g != nullptr && (type == 0 || type == 1) && x != y, name);
    const size_t n = (size_t)g->B * g->Ho * g->Wo * g->C;
    if (n == 0) return KNX_OK;
    KNX_REQUIRE(x && y, name);
    KNX_LAUNCH(name, pool_kernel, grid_for(n), type, *g, count_pad, x, y);
}

extern "C" int knx_hip_permute(const float* x, float* y, int B, int nd, const int* d, const int* perm, void* stream)
{
    const char* name = "knx_hip_permute";
    KNX_ENTRY(name);
    KNX_REQUIRE(nd >= 1 && nd <= 4 && B >= 0 && d && perm && x != y, name);
    PermArgs a{};
    a.nd = nd;
    size_t st[4], per = 1;  // row-major strides of the input axes
    for (int k = nd - 1; k >= 0; --k) { st[k] = per; per *= (size_t)d[k]; }
    for (int k = 0; k < nd; ++k) {
        KNX_REQUIRE(perm[k] >= 0 && perm[k] < nd, name);
        a.od[k] = d[perm[k]];        // output axis k has the size of input axis perm[k]
        a.ist[k] = (int)st[perm[k]]; // and walks with that axis' stride
    }
    const size_t total = per * (size_t)B;
    if (total == 0) return KNX_OK;
    KNX_LAUNCH(name, permute_kernel, grid_for(total), x, y, total, per, a);
}

extern "C" int knx_hip_copy_cols(const float* x, int ldx, int x_off, float* y, int ldy, int y_off, int rows, int n,
                                 void* stream)
{
    const char* name = "knx_hip_copy_cols";
    KNX_ENTRY(name);
    KNX_REQUIRE(rows >= 0 && n >= 0 && x_off >= 0 && y_off >= 0 && x_off + n <= ldx && y_off + n <= ldy, name);
    if ((size_t)rows * n == 0) return KNX_OK;
    KNX_REQUIRE(x && y, name);
    KNX_LAUNCH(name, copy_cols_kernel, grid_for((size_t)rows * n), x, ldx, x_off, y, ldy, y_off, rows, n);
}

extern "C" int knx_hip_pad(const float* x, float* y, int B, int H, int W, int C, int Ho, int Wo, int pt, int pl,
                           void* stream)
{
    const char* name = "knx_hip_pad";
    KNX_ENTRY(name);
    KNX_REQUIRE(B >= 0 && H >= 1 && W >= 1 && C >= 1 && Ho >= H && Wo >= W && pt >= 0 && pl >= 0 && x != y, name);
    const size_t n = (size_t)B * Ho * Wo * C;
    if (n == 0) return KNX_OK;
    KNX_LAUNCH(name, pad_kernel, grid_for(n), x, y, B, H, W, C, Ho, Wo, pt, pl);
}

extern "C" int knx_hip_upsample(const float* x, float* y, int B, int H, int W, int C, int sh, int sw, void* stream)
{
    const char* name = "knx_hip_upsample";
    KNX_ENTRY(name);
    KNX_REQUIRE(B >= 0 && H >= 1 && W >= 1 && C >= 1 && sh >= 1 && sw >= 1 && x != y, name);
    const size_t n = (size_t)B * H * sh * W * sw * C;
    if (n == 0) return KNX_OK;
    KNX_LAUNCH(name, upsample_kernel, grid_for(n), x, y, B, H, W, C, sh, sw);
}

extern "C" int knx_hip_embedding(const float* ids, int n, const float* table, int V, int D, float* y, void* stream)
{
    const char* name = "knx_hip_embedding";
    KNX_ENTRY(name);
    KNX_REQUIRE(n >= 0 && V >= 1 && D >= 1, name);
    if (n == 0) return KNX_OK;
    KNX_REQUIRE(ids && table && y, name);
    KNX_LAUNCH(name, embedding_kernel, grid_for((size_t)n * D), ids, n, table, V, D, y);
}

extern "C" int knx_hip_rnn_gates(int kind, int act, float alpha, int B, int u, int first_step, float* z, const float* zh,
                                 float* c, float* h, float* dst, int dst_stride, void* stream)
{
    const char* name = "knx_hip_rnn_gates";
    KNX_ENTRY(name);
    KNX_REQUIRE((kind == 4 || kind == 5 || kind == 6) && B >= 0 && u >= 1 && act >= -1 && act <= 15, name);
    KNX_REQUIRE(kind != 5 || zh != nullptr, name);
    KNX_REQUIRE(kind != 4 || c != nullptr, name);
    if (B == 0) return KNX_OK;
    KNX_REQUIRE(z && h, name);
    KNX_LAUNCH(name, rnn_gates_kernel, grid_for((size_t)B * u), kind, act, alpha, B, u, first_step, z, zh, c, h, dst,
               dst_stride);
}
