// Pieces shared between translation units of the library: the split-K
// partial-plane reader and the launchers that fuse a projection's reduction
// into the kernel that consumes it.
#pragma once

#include "nq_common.h"

namespace nq {

// x[0..8) = sum over s = 0..S-1 (in that order) of p[s * plane + 0..8); the
// planes are fp32, 16-byte aligned at p; kGroup planes are loaded per round
// (each round waits for its loads before the next is issued).
template <int kGroup = 4>
__device__ __forceinline__ void sum_partials8(const float *__restrict__ p, int S, int64_t plane,
                                              float (&x)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = 0.f;
    for (int s0 = 0; s0 < S; s0 += kGroup) {
        float4 v[kGroup][2];
#pragma unroll
        for (int u = 0; u < kGroup; ++u) {
            if (s0 + u < S) {
                const float4 *q = reinterpret_cast<const float4 *>(p + (s0 + u) * plane);
                v[u][0] = q[0];
                v[u][1] = q[1];
            } else {
                v[u][0] = make_float4(0.f, 0.f, 0.f, 0.f);
                v[u][1] = v[u][0];
            }
        }
#pragma unroll
        for (int u = 0; u < kGroup; ++u) {
            if (s0 + u < S) {
                x[0] += v[u][0].x;
                x[1] += v[u][0].y;
                x[2] += v[u][0].z;
                x[3] += v[u][0].w;
                x[4] += v[u][1].x;
                x[5] += v[u][1].y;
                x[6] += v[u][1].z;
                x[7] += v[u][1].w;
            }
        }
    }
}

// e4m3fn code of x (round to nearest even; |x| beyond 448 saturates to 448).
// Exponents >= -6 keep three mantissa bits by the carry-propagating rounding
// add; smaller magnitudes are multiples of 2^-9 (subnormal codes 0..8, where
// 8 is the smallest normal).
__device__ __forceinline__ uint32_t e4m3_code(float x) {
    const uint32_t u = __float_as_uint(x);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t au = u & 0x7fffffffu;
    const int exp = static_cast<int>(au >> 23) - 127;
    uint32_t code;
    if (exp >= -6) {
        const uint32_t mant = au & 0x7fffffu;
        const uint32_t r = (mant + 0x7ffffu + ((mant >> 20) & 1u)) >> 20;
        code = (static_cast<uint32_t>(exp + 7) << 3) + r;
        code = code > 0x7eu ? 0x7eu : code;
    } else {
        code = static_cast<uint32_t>(rintf(__uint_as_float(au) * 512.0f));
    }
    return code | sign;
}

// Eight codes of x[0..8) / s (s > 0) packed little-endian into two words.
__device__ __forceinline__ uint2 e4m3_pack8(const float (&x)[8], float s) {
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int e = 0; e < 8; ++e) w[e / 4] |= e4m3_code(x[e] / s) << (8 * (e % 4));
    return make_uint2(w[0], w[1]);
}

// Activation scale of a 128-column group: max |x| / 448, or 1 for an all-zero
// group (whose codes are then all zero).
__device__ __forceinline__ float row_group_scale(float amax) { return amax > 0.f ? amax / 448.0f : 1.0f; }

// q/k RMSNorm (with weight) and rotate-half RoPE of one head of D values held
// as lane pairs: lane i < D/2 holds elements i and i + D/2 (x1, x2) and their
// norm weights (w1, w2, loaded by the caller with its inputs); lanes at or
// above D/2 pass on = false.  inv_freq = exp(-ln(theta) * 2i / D), the
// normalised values are rounded to bf16 first when round_to_input is set.
// Every caller (the rope kernel and the fused decode attention) goes through
// this one sequence of operations, so their q and K agree bit for bit.
template <int D>
__device__ __forceinline__ void norm_rope_pair(float x1, float x2, bool on, float w1, float w2, int lane, float eps,
                                               float log_theta, float position, int round_to_input, uint16_t &o1,
                                               uint16_t &o2) {
    constexpr int HALF = D / 2;
    const float ss = group_sum<(HALF < kWave ? HALF : kWave)>(on ? x1 * x1 + x2 * x2 : 0.f);
    if (!on) return;
    const float inv_rms = 1.0f / sqrtf(ss / static_cast<float>(D) + eps);
    float f = x1 * inv_rms * w1;
    float s = x2 * inv_rms * w2;
    if (round_to_input) {
        f = bf16_to_f32(f32_to_bf16(f));
        s = bf16_to_f32(f32_to_bf16(s));
    }
    const float inv_freq = expf(-log_theta * (static_cast<float>(lane) * 2.0f / static_cast<float>(D)));
    float sn, cs;
    sincosf(position * inv_freq, &sn, &cs);
    o1 = f32_to_bf16(f * cs - s * sn);
    o2 = f32_to_bf16(s * cs + f * sn);
}

// Bands (64 output columns each) per GEMM workgroup for `splits` K slices.
int bands_per_wg(int bands, int splits);

// out = bf16(sum over the S planes of part (+ bias)), planes added in index order.
int launch_reduce_partials(const float *part, int S, int M, int N, uint16_t *out, int64_t o_s0,
                           const uint16_t *bias, hipStream_t st);

// residual[r] = bf16(residual[r] + bf16(sum_s part[s][r])); hidden_out[r] =
// rmsnorm(residual[r]) * weight, for rows r < rows of width `width`.
int launch_add_rmsnorm_partials(const float *part, int S, int rows, int width, uint16_t *hidden_out,
                                int64_t ho_s0, uint16_t *residual, const uint16_t *weight, float eps,
                                hipStream_t st);

// As launch_add_rmsnorm_partials, with the normalised row stored as e4m3fn
// codes xq [rows, width] and per-128-column scales sx [rows, width / 128].
int launch_add_rmsnorm_partials_fp8(const float *part, int S, int rows, int width, uint16_t *residual,
                                    const uint16_t *weight, float eps, uint8_t *xq, int64_t xq_s0, float *sx,
                                    int64_t sx_s0, hipStream_t st);

// out[r, j] = silu(g) * u with g, u = bf16(sum_s part[s][r][j]), bf16(.. [width + j]).
int launch_silu_mul_partials(const float *part, int S, int rows, int width, uint16_t *out, int64_t o_s0,
                             hipStream_t st);

}  // namespace nq
