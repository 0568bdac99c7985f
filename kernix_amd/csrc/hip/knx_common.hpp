// knx_common.hpp — shared device helpers and host-side error plumbing for the gfx950 kernels.
// All HIP sources are compiled with -ffp-contract=off: a·b + c is two rounded operations everywhere, which is what
// the reference's vector paths (vDSP / NEON, no FMA) compute and what makes the int8 epilogue bit-exact.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "knx_hip.h"

namespace knx {

// Records a formatted error message (thread-local) and returns code.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// KNX_HIP_FAIL fault injection: true if the entry point `name` must fail.
bool injected(const char* name);
// Checks the last launch; returns KNX_OK or KNX_EHIP with the kernel name recorded.
int check_launch(const char* what);
// Number of compute units of the current device (cached).
int num_cus();
// Polls of a grid barrier (knx_grid.hpp) before it stops waiting: KNX_GRID_SPIN_LIMIT, or KNX_GRID_SPIN (tests).
unsigned grid_spin_limit();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace knx

#define KNX_ENTRY(name)                                                           \
    do {                                                                          \
        if (knx::injected(name)) return knx::fail(KNX_EINJECT, "%s: injected failure", name); \
    } while (0)

#define KNX_REQUIRE(cond, name)                                                   \
    do {                                                                          \
        if (!(cond)) return knx::fail(KNX_EINVAL, "%s: %s", name, #cond);         \
    } while (0)

// ---- activations (ids as the .knx file format); formulas of the reference's kernix_act_chunk
//      (reference include/kernix_model.h:463-517) ----
__device__ __forceinline__ float knx_relu6(float v) { return v < 0.0f ? 0.0f : v > 6.0f ? 6.0f : v; }
__device__ __forceinline__ float knx_softplus(float v) { return v > 20.0f ? v : log1pf(expf(v)); }

// GELU with Abramowitz–Stegun 7.1.26 erf; exp and 1/(1 + p·z) on the hardware exp2 / reciprocal (≤ 1-2 ulp each; the
// formula's own error is 1.5e-7), as the epilogue of large GEMMs evaluates it once per output element
__device__ __forceinline__ float knx_gelu(float x)
{
    const float z = fabsf(x) * 0.70710678f;
    const float t = __builtin_amdgcn_exp2f(-(z * z) * 1.44269504f);
    const float k = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * z);
    const float p = k * (0.254829592f + k * (-0.284496736f + k * (1.421413741f + k * (-1.453152027f + k * 1.061405429f))));
    const float e = 1.0f - p * t;
    return 0.5f * x * (1.0f + (x < 0.0f ? -e : e));
}

__device__ __forceinline__ float knx_act(float x, int act, float alpha)
{
    switch (act) {
    case 0: return x >= 0.0f ? x : 0.0f;  // threshold at 0 (NaN → 0, as vDSP_vthr and Metal max)
    case 1: return knx_gelu(x);
    case 2: { const float s = 1.0f / (1.0f + expf(-x)); return x * s; }
    case 3: return 1.0f / (1.0f + expf(-x));
    case 4: return tanhf(x);
    case 5: return x < 0.0f ? alpha * x : x;
    case 6: return x < 0.0f ? alpha * expm1f(x) : x;
    case 7: return 1.0507009873554805f * (x < 0.0f ? 1.6732632423543772f * expm1f(x) : x);
    case 8: return knx_softplus(x);
    case 9: return knx_relu6(x);
    case 10: return knx_relu6(x + 3.0f) / 6.0f;
    case 11: return x * knx_relu6(x + 3.0f) / 6.0f;
    case 12: return 0.5f * x * (1.0f + tanhf(0.7978845608028654f * (x + 0.044715f * x * x * x)));
    case 13: return expf(x);
    case 14: return x * tanhf(knx_softplus(x));
    case 15: return x / (1.0f + fabsf(x));
    default: return x;
    }
}

// The recurrent cells' sigmoid and tanh on the hardware exp2 and reciprocal (≤ 1-2 ulp each, as the GELU above): with
// libm expf / tanhf and IEEE divisions an LSTM cell is some 150 instructions, and the cells are the serial part of every
// timestep.  sigmoid(x) = 1 / (1 + 2^(−x·log2 e)); tanh(x) = 1 − 2 / (1 + 2^(2x·log2 e)), ±1 at the extremes, an absolute
// error of ≈ 1e-7 near 0.  The other activations of a cell stay those of knx_act.
__device__ __forceinline__ float knx_gate_sigmoid(float x)
{
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.44269504f));
}
__device__ __forceinline__ float knx_gate_act(float x, int act, float alpha)
{
    if (act == 4) return 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * 2.88539008f));
    return knx_act(x, act, alpha);
}

// Recurrent cells on the summed gate inputs (x·W + b + h·U; reference include/kernix_model.h:595-626), shared by the
// per-timestep gates kernel and the persistent recurrence so that both give the same bits.
// LSTM (gates i, f, g, o): c = f·c + i·g (c = i·g at the first step), h = o·act(c).
__device__ __forceinline__ float knx_lstm_cell(float zi, float zf, float zg, float zo, int act, float alpha, bool step0,
                                               float& c)
{
    const float ig = knx_gate_sigmoid(zi), fg = knx_gate_sigmoid(zf), gg = knx_gate_act(zg, act, alpha);
    const float og = knx_gate_sigmoid(zo);
    float cv = step0 ? ig * gg : fg * c;
    if (!step0) cv = ig * gg + cv;
    c = cv;
    return knx_gate_act(cv, act, alpha) * og;
}
// GRU (reset after; gates z, r, h~): x* the input side, h* the recurrent side with its bias; h = z·(h − h~) + h~.
__device__ __forceinline__ float knx_gru_cell(float xz, float xr, float xh, float hz, float hr, float hh_in, int act,
                                              float alpha, bool step0, float prev)
{
    const float zg = knx_gate_sigmoid(xz + hz);
    const float rg = knx_gate_sigmoid(xr + hr);
    const float hh = knx_gate_act(rg * hh_in + xh, act, alpha);
    return step0 ? (-hh) * zg + hh : (prev - hh) * zg + hh;
}

// Unsigned maximum over aligned groups of n lanes (n a power of two ≤ 64, uniform; every lane active), every lane of a
// group getting it: DPP within rows of 16 lanes (the quad swaps, then the half-row and row mirrors), gfx950's register
// swaps across rows and halves (each lane's value and its partner's in the pair of results), no exchange through the
// LDS.  Non-negative floats compare as their bits.
__device__ __forceinline__ unsigned knx_lane_group_max(unsigned v, int n)
{
    if (n > 1) v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));  // quad [1,0,3,2]
    if (n > 2) v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));  // quad [2,3,0,1]
    if (n > 4) v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false)); // half-row mirror
    if (n > 8) v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false)); // row mirror
    if (n > 16) {
        const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        v = max((unsigned)p[0], (unsigned)p[1]);
    }
    if (n > 32) {
        const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        v = max((unsigned)p[0], (unsigned)p[1]);
    }
    return v;
}

// Sum over aligned groups of n lanes, the same exchanges as knx_lane_group_max (every lane of a group ends with the
// same value: a + b and b + a are the same float).
template <int CTRL>
__device__ __forceinline__ float knx_dpp_f32(float x)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float knx_lane_group_sum(float v, int n)
{
    if (n > 1) v = v + knx_dpp_f32<0xB1>(v);
    if (n > 2) v = v + knx_dpp_f32<0x4E>(v);
    if (n > 4) v = v + knx_dpp_f32<0x141>(v);
    if (n > 8) v = v + knx_dpp_f32<0x140>(v);
    if (n > 16) {
        const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
    if (n > 32) {
        const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
    return v;
}

// Wave-wide (64 lanes) reductions through DPP/permute; every lane gets the result.
__device__ __forceinline__ float knx_wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float knx_wave_max(float v)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) { const float w = __shfl_xor(v, o, 64); v = w > v ? w : v; }
    return v;
}
