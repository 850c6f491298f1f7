// Shared device helpers for the CDNA4 (gfx950) kernels of the hot path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nq_abi.h"

#define NQ_CHECK_ARG(cond)                                                                     \
    do {                                                                                       \
        if (!(cond)) return NQ_ERR_INVALID_ARGUMENT;                                           \
    } while (0)

#define NQ_LAUNCH_STATUS() ((hipGetLastError() == hipSuccess) ? NQ_OK : NQ_ERR_LAUNCH)

namespace nq {

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
    return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

// Round-to-nearest-even float -> bfloat16, quiet NaN preserved (matches torch).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// Unpack 8 bf16 held in a 128-bit vector into floats.
__device__ __forceinline__ void unpack8(const uint4 &p, float (&x)[8]) {
    x[0] = __uint_as_float(p.x << 16);
    x[1] = __uint_as_float(p.x & 0xffff0000u);
    x[2] = __uint_as_float(p.y << 16);
    x[3] = __uint_as_float(p.y & 0xffff0000u);
    x[4] = __uint_as_float(p.z << 16);
    x[5] = __uint_as_float(p.z & 0xffff0000u);
    x[6] = __uint_as_float(p.w << 16);
    x[7] = __uint_as_float(p.w & 0xffff0000u);
}

__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
    return static_cast<uint32_t>(f32_to_bf16(a)) | (static_cast<uint32_t>(f32_to_bf16(b)) << 16);
}

// DPP lane permutations (gfx9 encodings): quad_perm [1,0,3,2], [2,3,0,1],
// row_half_mirror (reverse 8 lanes), row_mirror (reverse 16 lanes).
constexpr int kDppQuadXor1 = 0xB1;
constexpr int kDppQuadXor2 = 0x4E;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

template <int Ctrl>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), Ctrl, 0xF, 0xF, false));
}

// Sum over aligned groups of Width lanes, result in every lane of the group.
// Widths up to 16 stay inside a DPP row (one VALU op per step); wider groups
// fall back to cross-row shuffles.
template <int Width>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(Width >= 1 && Width <= kWave && (Width & (Width - 1)) == 0, "power of two");
    if constexpr (Width >= 2) v += dpp_f32<kDppQuadXor1>(v);
    if constexpr (Width >= 4) v += dpp_f32<kDppQuadXor2>(v);
    if constexpr (Width >= 8) v += dpp_f32<kDppHalfMirror>(v);
    if constexpr (Width >= 16) v += dpp_f32<kDppMirror>(v);
#pragma unroll
    for (int m = 16; m < Width; m <<= 1) v += __shfl_xor(v, m, kWave);
    return v;
}

// Inclusive prefix sum over the 64 lanes of a wave (every lane active):
// row_shr 1, 2, 4, 8 inside each 16-lane row (lanes shifted in from outside
// the row add 0), then row_bcast:15 into rows 1 and 3 and row_bcast:31 into
// rows 2 and 3.  Six DPP adds, no LDS round trips.
__device__ __forceinline__ int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);
    return v;
}

// Exclusive prefix sums of N values per thread over the workgroup (all of its
// threads active) in one pass: three barriers for all N.  tmp holds
// N * (kWave + 1) ints; total[i] receives the workgroup sum of value i.
template <int N>
__device__ void block_exclusive_scan_n(const int (&v)[N], int *tmp, int (&excl)[N], int (&total)[N]) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    int incl[N];
#pragma unroll
    for (int i = 0; i < N; ++i) incl[i] = wave_incl_scan(v[i]);
    if (lane == kWave - 1) {
#pragma unroll
        for (int i = 0; i < N; ++i) tmp[i * (kWave + 1) + wave] = incl[i];
    }
    __syncthreads();
    if (wave == 0) {
        const int nw = blockDim.x / kWave;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const int w = lane < nw ? tmp[i * (kWave + 1) + lane] : 0;
            const int wi = wave_incl_scan(w);
            if (lane < nw) tmp[i * (kWave + 1) + lane] = wi - w;  // exclusive wave offsets
            if (lane == nw - 1) tmp[i * (kWave + 1) + kWave] = wi;
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < N; ++i) {
        excl[i] = tmp[i * (kWave + 1) + wave] + incl[i] - v[i];
        total[i] = tmp[i * (kWave + 1) + kWave];
    }
    __syncthreads();
}

template <int Width>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int m = 1; m < Width; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
    return v;
}

}  // namespace nq
