// Pieces shared between translation units of the library: the split-K
// partial-plane reader and the launchers that fuse a projection's reduction
// into the kernel that consumes it.
#pragma once

#include "nq_common.h"

namespace nq {

// x[0..8) = sum over s = 0..S-1 (in that order) of p[s * plane + 0..8); the
// planes are fp32, 16-byte aligned at p; four planes are loaded per round.
__device__ __forceinline__ void sum_partials8(const float *__restrict__ p, int S, int64_t plane,
                                              float (&x)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = 0.f;
    for (int s0 = 0; s0 < S; s0 += 4) {
        float4 v[4][2];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
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
        for (int u = 0; u < 4; ++u) {
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

// residual[r] = bf16(residual[r] + bf16(sum_s part[s][r])); hidden_out[r] =
// rmsnorm(residual[r]) * weight, for rows r < rows of width `width`.
int launch_add_rmsnorm_partials(const float *part, int S, int rows, int width, uint16_t *hidden_out,
                                int64_t ho_s0, uint16_t *residual, const uint16_t *weight, float eps,
                                hipStream_t st);

// out[r, j] = silu(g) * u with g, u = bf16(sum_s part[s][r][j]), bf16(.. [width + j]).
int launch_silu_mul_partials(const float *part, int S, int rows, int width, uint16_t *out, int64_t o_s0,
                             hipStream_t st);

}  // namespace nq
