// knx_pipe.hpp — building blocks of the LDS-pipelined GEMM kernels (int8 and fp32) on gfx950.
#pragma once

#include "knx_common.hpp"

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __attribute__((address_space(1))) const void* gbl_ptr_t;

// s_waitcnt vmcnt(n) lgkmcnt(0) (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] = 7 | lgkmcnt[11:8] | vmcnt[5:4] << 14):
// at most n vector-memory ops (LDS-DMA loads) of this wave outstanding and all of its LDS accesses retired.
#define KNX_WAIT_VM_LDS(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (0 << 8) | ((((n) >> 4) & 3) << 14))

// s_waitcnt lgkmcnt(0): all LDS accesses of this wave retired (vmcnt left unconstrained at 63).
#define KNX_WAIT_LDS() __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14))

// Workgroup barrier without a memory fence.  A fence (e.g. __syncthreads) would wait for every outstanding LDS-DMA
// load, which empties the prefetch ring; the caller instead waits precisely with KNX_WAIT_VM_LDS.  The empty asm
// statements keep the compiler from moving any memory access across the barrier.
static __device__ __forceinline__ void knx_barrier_nofence()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Tile order: consecutive workgroups go to consecutive XCDs (8 on MI355X); when the tile grid splits evenly, each
// XCD gets one contiguous (tiles_m/2) × (tiles_n/4) block so the operand rows it reads stay in its own L2.
static __device__ __forceinline__ void tile_of(int t, int tiles_m, int tiles_n, int& tm, int& tn)
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

// Tile order with the XCD split chosen per shape: consecutive workgroups go to consecutive XCDs, and the tile grid is
// cut into px × (8/px) equal blocks, one per XCD, with the px (of 2, 4, 1, 8 in that order of preference) that gives
// each XCD the fewest operand rows to hold in its L2 (bm·BM A rows + bn·BN W rows).  M = 256, N = 4096 in 64×64
// tiles: px = 1 (every XCD holds all 256 A rows and 512 W rows, 3 MB) instead of px = 2 (128 + 1024 rows, 4.5 MB).
static __device__ __forceinline__ void tile_of_best(int t, int tiles_m, int tiles_n, int BM, int BN, int& tm, int& tn)
{
    int px = 0;
    long best = 0;
    if (tiles_m * tiles_n >= 64) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int x = c == 0 ? 2 : c == 1 ? 4 : c == 2 ? 1 : 8, y = 8 / x;
            if (tiles_m % x != 0 || tiles_n % y != 0) continue;
            const long rows = (long)(tiles_m / x) * BM + (long)(tiles_n / y) * BN;
            if (px == 0 || rows < best) px = x, best = rows;
        }
    }
    if (px > 0) {
        const int py = 8 / px, x = t & 7, j = t >> 3;
        const int bm = tiles_m / px, bn = tiles_n / py;
        tm = (x / py) * bm + j / bn;
        tn = (x % py) * bn + j % bn;
    } else {
        tm = t / tiles_n;
        tn = t % tiles_n;
    }
}

// 16-byte chunk swizzle of a 128-byte LDS row: chunk c of row r is stored at position c ^ swz8(r).  The 16 rows that
// one quarter-wave of a ds_read_b128 touches (same chunk, consecutive rows) then fall on 16 distinct 16-byte bank
// groups, and any 8 consecutive rows on 8; swz8(r + 32) = swz8(r) ^ 4.
static __device__ __forceinline__ int swz8(int row) { return (row ^ (row >> 3)) & 7; }

// LDS-DMA load of 16 bytes per lane, global (base + voff) → LDS (dst + 16·lane), with base and dst wave-uniform.
// Inline assembly, so that the compiler does not treat it as an LDS store: it cannot tell the stages apart and
// would make every later LDS read wait for all outstanding loads.  The loads are waited for explicitly (vmcnt) and
// published with a workgroup barrier; the compiler's own vmcnt waits stay correct, only stricter (vmcnt retires
// loads in order, so loads it does not know about only add younger entries).
static __device__ __forceinline__ void dma16(const void* base, unsigned voff, void* dst)
{
    const unsigned l = (unsigned)(uintptr_t)(lds_ptr_t)dst;
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(l), "v"(voff), "s"(base) : "memory");
}

// The same load with a per-lane 64-bit source address (gathers: every lane's row may live anywhere).
static __device__ __forceinline__ void dma16_at(const void* src, void* dst)
{
    const unsigned l = (unsigned)(uintptr_t)(lds_ptr_t)dst;
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(l), "v"(src) : "memory");
}
